// Dense dequant-fused linear: C[M, N] = A[M, K] (bf16) x dequant(W)[N, K]^T,
// W in MXFP8 (E4M3) or MXFP4 (E2M1) with per-32 E8M0 scales, fp32
// accumulation on v_mfma_f32_32x32x16_bf16, bf16 or fp32 output.
//
// This is the A16 operand contract of kquant's MXFP8 closure oracle
// (scripts/closure_mxfp8_mlp.py:146-187: fp32 matmul over the dequantized
// weights) and of the W4A16 expert linears.
//
// Workgroup tile 256 x 256, 8 waves of 64 x 128 (2 x 4 MFMA 32x32 blocks),
// K step 64, LDS double buffered.  Weights are staged in LDS still packed
// (E4M3: 64 B per row and step, E2M1: 32 B) and expanded to bf16 per fragment.
#include "kq_gemm.h"
#include "kq_internal.h"

namespace kq {

namespace lin {
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int THREADS = 512;
constexpr int A_ROW = BK * 2 + 16;                  // 144 B: bf16 row + pad
template <int FMT> constexpr int b_row() { return FMT == 0 ? 72 : 36; }  // packed row + pad
constexpr int A_BYTES = BM * A_ROW;                 // 36 KiB
template <int FMT> constexpr int b_bytes() { return BN * b_row<FMT>(); }
constexpr int S_BYTES = BN * 2;                     // 2 scale bytes per row per step
template <int FMT> constexpr int stage_bytes() { return A_BYTES + b_bytes<FMT>() + S_BYTES; }
}  // namespace lin

using gemm::bf16x8_t;
using gemm::u32x2_t;
using gemm::u32x4_t;

template <int FMT, int OUT>
__global__ __launch_bounds__(512, 1) void mx_linear_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, void* __restrict__ c, int64_t ldc, int M, int N, int K, int KB) {
  using namespace lin;
  constexpr int BROW = b_row<FMT>();
  constexpr int WBYTES = FMT == 0 ? BK : BK / 2;  // packed bytes per row per step
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  // A has K columns; the weights have KB (K is a multiple of KB, and A's
  // column k multiplies weight column k % KB: the split-fp32 operand).
  const int64_t kw = FMT == 0 ? KB : KB / 2;  // packed bytes per weight row
  const int64_t ks = KB / 32;                 // scale bytes per weight row

  // ---- global -> register staging
  u32x4_t ra[4], rb[2];
  uint32_t rs = 0;
  auto load = [&](int k0) {
    const int kb0 = k0 % KB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + THREADS * i;  // 2048 chunks of 16 B
      const int row = ch >> 3, col = (ch & 7) * 8;
      const int gm = m0 + row;
      ra[i] = gm < M ? *reinterpret_cast<const u32x4_t*>(a + (int64_t)gm * lda + k0 + col)
                     : u32x4_t{0u, 0u, 0u, 0u};
    }
    constexpr int BCH = BN * WBYTES / 16;  // chunks of 16 B
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = tid + THREADS * i;
      if (ch < BCH) {
        const int row = ch / (WBYTES / 16), col = (ch % (WBYTES / 16)) * 16;
        const int gn = n0 + row;
        rb[i] = gn < N ? *reinterpret_cast<const u32x4_t*>(wq + (int64_t)gn * kw + (FMT == 0 ? kb0 : kb0 / 2) + col)
                       : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    if (tid < BN) {
      const int gn = n0 + tid;
      rs = gn < N ? *reinterpret_cast<const uint16_t*>(ws + (int64_t)gn * ks + kb0 / 32) : 0u;
    }
  };
  auto store = [&](int buf) {
    unsigned char* base = lds + buf * stage_bytes<FMT>();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + THREADS * i;
      const int row = ch >> 3, col = (ch & 7) * 16;
      *reinterpret_cast<u32x4_t*>(base + row * A_ROW + col) = ra[i];
    }
    unsigned char* bb = base + A_BYTES;
    constexpr int BCH = BN * WBYTES / 16;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = tid + THREADS * i;
      if (ch < BCH) {
        const int row = ch / (WBYTES / 16), col = (ch % (WBYTES / 16)) * 16;
        if (FMT == 0) {
          *reinterpret_cast<u32x2_t*>(bb + row * BROW + col) = u32x2_t{rb[i][0], rb[i][1]};
          *reinterpret_cast<u32x2_t*>(bb + row * BROW + col + 8) = u32x2_t{rb[i][2], rb[i][3]};
        } else {
#pragma unroll
          for (int d = 0; d < 4; ++d) *reinterpret_cast<uint32_t*>(bb + row * BROW + col + 4 * d) = rb[i][d];
        }
      }
    }
    if (tid < BN) *reinterpret_cast<uint16_t*>(base + A_BYTES + b_bytes<FMT>() + tid * 2) = (uint16_t)rs;
  };

  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
  float16_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int frow = lane & 31, fk = lane >> 5;  // fragment row, k half (8 elements)
  const int steps = K / BK;
  load(0);
  store(0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < steps) load((s + 1) * BK);
    const unsigned char* base = lds + buf * stage_bytes<FMT>();
    const unsigned char* bb = base + A_BYTES;
    const unsigned char* sb = bb + b_bytes<FMT>();
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8_t fa[2], fb[4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        fa[i] = *reinterpret_cast<const bf16x8_t*>(base + (wm + i * 32 + frow) * A_ROW + kk * 32 + fk * 16);
      // this lane's 8 k values lie in scale block (kk * 16 + fk * 8) / 32 = kk / 2
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = wn + j * 32 + frow;
        const uint32_t sc = sb[row * 2 + (kk >> 1)];
        u32x2_t w;
        if (FMT == 0) {
          w = *reinterpret_cast<const u32x2_t*>(bb + row * BROW + kk * 16 + fk * 8);
        } else {
          w[0] = *reinterpret_cast<const uint32_t*>(bb + row * BROW + kk * 8 + fk * 4);
          w[1] = 0u;
        }
        fb[j] = gemm::dequant8<FMT>(w, sc);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < steps) store(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: C[32x32] lane layout col = lane % 32, row = 8(r/4) + 4(lane/32) + r%4
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
        const int gn = n0 + wn + j * 32 + frow;
        if (gm < M && gn < N) {
          if (OUT == 2) static_cast<float*>(c)[(int64_t)gm * ldc + gn] = acc[i][j][r];
          else static_cast<__bf16*>(c)[(int64_t)gm * ldc + gn] = (__bf16)acc[i][j][r];
        }
      }
}

// Exact three-term bf16 split of fp32 A: a = a0 + a1 + a2 (each step keeps
// the next 8 significant bits and leaves an exactly representable residual),
// written as row [a0 | a1 | a2] of a [rows, 3k] bf16 matrix.  Four columns
// per thread.
__global__ __launch_bounds__(256) void split3_bf16_kernel(const float* __restrict__ a, int64_t lda,
                                                          int64_t rows, int64_t k,
                                                          uint16_t* __restrict__ out) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = k / 4;
  if (q >= rows * per_row) return;
  const int64_t r = q / per_row, c = (q - r * per_row) * 4;
  const float4_t x = *reinterpret_cast<const float4_t*>(a + r * lda + c);
  uint32_t t0[2], t1[2], t2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float h0[2], h1[2], h2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float v = x[2 * h + j];
      h0[j] = (float)(__bf16)v;
      const float r1 = v - h0[j];
      h1[j] = (float)(__bf16)r1;
      h2[j] = r1 - h1[j];
    }
    t0[h] = f32x2_to_bf16x2_bits(h0[0], h0[1]);
    t1[h] = f32x2_to_bf16x2_bits(h1[0], h1[1]);
    t2[h] = f32x2_to_bf16x2_bits(h2[0], h2[1]);
  }
  uint16_t* o = out + r * 3 * k + c;
  *reinterpret_cast<gemm::u32x2_t*>(o) = gemm::u32x2_t{t0[0], t0[1]};
  *reinterpret_cast<gemm::u32x2_t*>(o + k) = gemm::u32x2_t{t1[0], t1[1]};
  *reinterpret_cast<gemm::u32x2_t*>(o + 2 * k) = gemm::u32x2_t{t2[0], t2[1]};
}

}  // namespace kq

using namespace kq;

template <int FMT, int OUT>
static hipError_t launch_linear(const uint16_t* a, int64_t lda, const uint8_t* wq, const uint8_t* ws,
                                void* c, int64_t ldc, int M, int N, int K, int KB, hipStream_t st) {
  const size_t lds = 2 * (size_t)lin::stage_bytes<FMT>();
  auto kern = mx_linear_kernel<FMT, OUT>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid((N + lin::BN - 1) / lin::BN, (M + lin::BM - 1) / lin::BM);
  kern<<<grid, lin::THREADS, lds, st>>>(a, lda, wq, ws, c, ldc, M, N, K, KB);
  return hipGetLastError();
}

extern "C" int kq_mx_linear(int w_fmt, const void* a, int64_t lda, const void* w_q,
                            const uint8_t* w_scale, int64_t m, int64_t n, int64_t k,
                            int out_dtype, void* c, int64_t ldc, void* stream) {
  if (w_fmt != KQ_FMT_MXFP8_E4M3 && w_fmt != KQ_FMT_MXFP4_E2M1)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear: unknown weight format %d", w_fmt);
  if (out_dtype != KQ_DT_BF16 && out_dtype != KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear: output dtype must be bf16 or f32");
  if (m < 0 || n < 0 || k <= 0 || k % 64 != 0 || lda < k || lda % 8 != 0 || ldc < n)
    return kq_fail(KQ_ERR_INVALID,
                   "kq_mx_linear: need k %% 64 == 0, lda >= k, lda %% 8 == 0, ldc >= n "
                   "(m=%lld n=%lld k=%lld lda=%lld ldc=%lld)",
                   (long long)m, (long long)n, (long long)k, (long long)lda, (long long)ldc);
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2)
    return kq_fail(KQ_ERR_LIMIT, "kq_mx_linear: dimension too large");
  if (kq_misaligned(a, 16) || kq_misaligned(w_q, 16) || kq_misaligned(w_scale, 2))
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear: a and w_q must be 16-byte aligned");
  if (m == 0 || n == 0) return KQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* ap = (const uint16_t*)a;
  const uint8_t* wp = (const uint8_t*)w_q;
  hipError_t e;
  if (w_fmt == KQ_FMT_MXFP8_E4M3)
    e = out_dtype == KQ_DT_BF16 ? launch_linear<0, 0>(ap, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, (int)k, st)
                                : launch_linear<0, 2>(ap, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, (int)k, st);
  else
    e = out_dtype == KQ_DT_BF16 ? launch_linear<1, 0>(ap, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, (int)k, st)
                                : launch_linear<1, 2>(ap, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, (int)k, st);
  return kq_check_launch(e, "kq_mx_linear");
}

extern "C" int64_t kq_mx_linear_f32_workspace_size(int64_t m, int64_t k) {
  if (m < 0 || k < 0) return -1;
  return m * 3 * k * 2;
}

extern "C" int kq_mx_linear_f32(int w_fmt, const float* a, int64_t lda, const void* w_q,
                                const uint8_t* w_scale, int64_t m, int64_t n, int64_t k, float* c,
                                int64_t ldc, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (w_fmt != KQ_FMT_MXFP8_E4M3 && w_fmt != KQ_FMT_MXFP4_E2M1)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear_f32: unknown weight format %d", w_fmt);
  if (m < 0 || n < 0 || k <= 0 || k % 64 != 0 || lda < k || lda % 4 != 0 || ldc < n)
    return kq_fail(KQ_ERR_INVALID,
                   "kq_mx_linear_f32: need k %% 64 == 0, lda >= k, lda %% 4 == 0, ldc >= n "
                   "(m=%lld n=%lld k=%lld lda=%lld ldc=%lld)",
                   (long long)m, (long long)n, (long long)k, (long long)lda, (long long)ldc);
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || 3 * k > INT32_MAX / 2)
    return kq_fail(KQ_ERR_LIMIT, "kq_mx_linear_f32: dimension too large");
  if (workspace_bytes < m * 3 * k * 2)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear_f32: workspace needs %lld bytes",
                   (long long)(m * 3 * k * 2));
  if (kq_misaligned(a, 16) || kq_misaligned(w_q, 16) || kq_misaligned(w_scale, 2) ||
      kq_misaligned(workspace, 16))
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear_f32: a, w_q and workspace must be 16-byte aligned");
  if (m == 0 || n == 0) return KQ_OK;
  hipStream_t st = (hipStream_t)stream;
  uint16_t* a3 = static_cast<uint16_t*>(workspace);
  const int64_t quads = m * (k / 4);
  split3_bf16_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, st>>>(a, lda, m, k, a3);
  if (int rc = kq_check_launch(hipGetLastError(), "kq_mx_linear_f32")) return rc;
  const uint8_t* wp = (const uint8_t*)w_q;
  const hipError_t e =
      w_fmt == KQ_FMT_MXFP8_E4M3
          ? launch_linear<0, 2>(a3, 3 * k, wp, w_scale, c, ldc, (int)m, (int)n, (int)(3 * k), (int)k, st)
          : launch_linear<1, 2>(a3, 3 * k, wp, w_scale, c, ldc, (int)m, (int)n, (int)(3 * k), (int)k, st);
  return kq_check_launch(e, "kq_mx_linear_f32");
}
