// Calibration Hessian: H += X^T diag(w) X over token rows, fp32 accumulate.
//
// kquant accumulates H with chunked fp32 addmm_ (kquant/candidate_hessian.py:
// 98-105, kquant/capture.py:713-730).  Here bf16 activations go straight into
// bf16 MFMA (v_mfma_f32_32x32x16_bf16): bf16 x bf16 products are exact in
// fp32, so only the summation order differs from the reference.  fp16 / fp32
// rows and row weights are split into a bf16 high part and a bf16 residual
// (x*w = hi + lo to 16 significant bits), costing one more MFMA per step.
//
// Tiling: the K x K output is cut into 128 x 128 tiles and only tiles with
// row-tile <= col-tile are computed (the other half is the mirror image).
// A 256-thread workgroup owns one tile and streams every token row through
// it in steps of 64 tokens.  Each thread loads an 8-token x 8-feature block
// (eight 16-byte row loads), transposes it in registers with v_perm so that
// each feature's 8 tokens are contiguous, and stores it into an LDS slab laid
// out [feature][token] -- the MFMA operand order (8 consecutive reduction
// elements per lane).  LDS is double buffered: the global loads of step s+1
// are in flight while step s runs on the matrix cores.
#include <type_traits>

#include "kq_dma.h"
#include "kq_common.h"
#include "kq_internal.h"

namespace kq {

namespace syrk {
constexpr int TILE = 128;          // output tile edge
constexpr int BK = 64;             // tokens per pipeline step
constexpr int ROW_BYTES = BK * 2 + 16;  // LDS row (one feature): 64 bf16 + pad
constexpr int SLAB_BYTES = TILE * ROW_BYTES;  // 18 KiB
}  // namespace syrk

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 8x8 transpose of 16-bit elements held as 8 rows of 4 dwords.
// in[t] = elements (t, 0..7) packed two per dword; out[f] = (0..7, f).
__device__ __forceinline__ void transpose8x8_b16(const u32x4_t in[8], u32x4_t out[8]) {
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    const uint32_t sel = (f & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      out[f][e] = __builtin_amdgcn_perm(in[2 * e + 1][f >> 1], in[2 * e][f >> 1], sel);
  }
}

// w times a packed pair of bf16 values, split into packed bf16 hi (round to
// nearest) and bf16 lo = the fp32 residual rounded: one v_cvt_pk_bf16_f32 per
// part and pair.
__device__ __forceinline__ void split_bf16_pair(uint32_t pair, float w, uint32_t& hi, uint32_t& lo) {
  float2_t v;
  v[0] = __builtin_bit_cast(float, pair << 16) * w;
  v[1] = __builtin_bit_cast(float, pair & 0xffff0000u) * w;
  const bf16x2_t h = __builtin_convertvector(v, bf16x2_t);
  const uint32_t hb = __builtin_bit_cast(uint32_t, h);
  float2_t r;
  r[0] = v[0] - __builtin_bit_cast(float, hb << 16);
  r[1] = v[1] - __builtin_bit_cast(float, hb & 0xffff0000u);
  hi = hb;
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2_t));
}

// Split fp32 values into bf16 hi (round to nearest) and bf16 lo = fp32 residual.
__device__ __forceinline__ void split_bf16(float v, uint32_t& hi, uint32_t& lo) {
  __bf16 h = (__bf16)v;
  float r = v - (float)h;
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, (__bf16)r);
}

// Group of grid row r for the grouped kernels: groups in descending order of
// their row count (ties by index), so the longest tiles start first and the
// short ones fill in behind them (longest-processing-time-first order; the
// result of each group does not depend on it).  Every thread ranks a few
// groups against all others with uniform (scalar) reads of offsets; for more
// than LPT_MAX_GROUPS groups the quadratic ranking costs more than it saves
// and row r is group r.
constexpr int LPT_MAX_GROUPS = 1024;
__device__ __forceinline__ int64_t group_of_row(const int64_t* __restrict__ offsets, int groups, int r) {
  if (groups > LPT_MAX_GROUPS) return r;
  __shared__ int s_group;
  for (int g = threadIdx.x; g < groups; g += blockDim.x) {
    const int64_t ng = offsets[g + 1] - offsets[g];
    int rank = 0;
    for (int h = 0; h < groups; ++h) {
      const int64_t nh = offsets[h + 1] - offsets[h];
      rank += (nh > ng || (nh == ng && h < g)) ? 1 : 0;
    }
    if (rank == r) s_group = g;
  }
  __syncthreads();
  return s_group;
}

// IN: 0 bf16, 1 f16, 2 f32.  SPLIT: operands carry a bf16 residual part
// (needed for weights or non-bf16 inputs).  GROUPED: blockIdx.y is a group
// (an expert; grid row order from group_of_row) whose rows are list positions [offsets[g], offsets[g+1]), row
// index[p] of x (or p itself without an index), weight w[p] (squared when
// square_w), and whose k x k result sits at acc + g * acc_stride.
template <int IN, bool SPLIT, bool WEIGHTED, bool GROUPED>
__global__ __launch_bounds__(256, 1) void syrk_upper_kernel(
    const void* __restrict__ x, int64_t ld, int64_t n, int64_t k,
    const float* __restrict__ w, float* __restrict__ acc, int64_t ld_acc, int ntiles,
    int overwrite, const int64_t* __restrict__ offsets, const int32_t* __restrict__ index,
    int64_t acc_stride, int square_w) {
  using namespace syrk;
  int64_t list0 = 0;
  if (GROUPED) {
    const int64_t g = group_of_row(offsets, gridDim.y, blockIdx.y);
    list0 = offsets[g];
    n = offsets[g + 1] - list0;
    acc += g * acc_stride;
  }
  // ---- tile coordinates: linear index -> (ti <= tj) over the upper triangle
  int rem = blockIdx.x, ti = 0;
  while (rem >= ntiles - ti) { rem -= ntiles - ti; ++ti; }
  const int tj = ti + rem;
  const int64_t row0 = (int64_t)ti * TILE, col0 = (int64_t)tj * TILE;

  // LDS: [buffer][slab] with slabs A(hi) B(hi) [A(lo) B(lo)]
  constexpr int NSLAB = SPLIT ? 4 : 2;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // loader role: 256 threads cover 2 slabs x (16 feature groups x 8 token groups)
  const int slab = tid >> 7;              // 0: rows of A (ti), 1: rows of B (tj)
  const int fg = tid & 15;                // feature group (8 features)
  const int tg = (tid >> 4) & 7;          // token group (8 tokens)
  const int64_t feat0 = (slab == 0 ? row0 : col0) + fg * 8;
  const bool feat_ok = feat0 < k;         // k % 8 == 0: whole groups in or out

  u32x4_t regs[8];
  u32x4_t regs_lo[8];

  auto load_step = [&](int64_t t0) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int64_t pos = t0 + tg * 8 + t;
      u32x4_t v = {0u, 0u, 0u, 0u};
      u32x4_t vlo = {0u, 0u, 0u, 0u};
      if (feat_ok && pos < n) {
        const int64_t tok = !GROUPED ? pos : (index ? (int64_t)index[list0 + pos] : list0 + pos);
        float wt = 1.0f;
        if (WEIGHTED && slab == 1) {
          wt = w[GROUPED ? list0 + pos : pos];
          if (GROUPED && square_w) wt *= wt;
        }
        if (IN == 0 && !SPLIT) {
          v = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + tok * ld + feat0);
        } else {
          float f[8];
          if (IN == 2) {
            const float4_t* p = reinterpret_cast<const float4_t*>(static_cast<const float*>(x) + tok * ld + feat0);
            float4_t a = p[0], b = p[1];
            f[0] = a[0]; f[1] = a[1]; f[2] = a[2]; f[3] = a[3];
            f[4] = b[0]; f[5] = b[1]; f[6] = b[2]; f[7] = b[3];
          } else {
            u32x4_t r = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + tok * ld + feat0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              f[2 * i] = IN == 0 ? bf16_bits_to_f32(r[i] & 0xffffu) : f16_bits_to_f32(r[i] & 0xffffu);
              f[2 * i + 1] = IN == 0 ? bf16_bits_to_f32(r[i] >> 16) : f16_bits_to_f32(r[i] >> 16);
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            uint32_t h0, l0, h1, l1;
            split_bf16(f[2 * i] * wt, h0, l0);
            split_bf16(f[2 * i + 1] * wt, h1, l1);
            v[i] = h0 | (h1 << 16);
            vlo[i] = l0 | (l1 << 16);
          }
        }
      }
      regs[t] = v;
      if (SPLIT) regs_lo[t] = vlo;
    }
  };

  auto store_step = [&](int buf) {
    unsigned char* base = lds + (size_t)buf * NSLAB * SLAB_BYTES;
    u32x4_t tr[8];
    transpose8x8_b16(regs, tr);
#pragma unroll
    for (int f = 0; f < 8; ++f)
      *reinterpret_cast<u32x4_t*>(base + slab * SLAB_BYTES + (fg * 8 + f) * ROW_BYTES + tg * 16) = tr[f];
    if (SPLIT) {
      transpose8x8_b16(regs_lo, tr);
#pragma unroll
      for (int f = 0; f < 8; ++f)
        *reinterpret_cast<u32x4_t*>(base + (2 + slab) * SLAB_BYTES + (fg * 8 + f) * ROW_BYTES + tg * 16) = tr[f];
    }
  };

  // wave tile: 64 x 64 at (wm, wn) inside the 128 x 128 tile, 2 x 2 MFMA 32x32
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  float16_t accv[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) accv[i][j][r] = 0.0f;

  const int arow = lane & 31;          // operand row inside a 32-block
  const int koff = (lane >> 5) * 16;   // byte offset of this lane's 8 tokens

  const int64_t steps = (n + BK - 1) / BK;
  if (steps > 0) {
    load_step(0);
    store_step(0);
  }
  __syncthreads();
  for (int64_t s = 0; s < steps; ++s) {
    const int buf = (int)(s & 1);
    if (s + 1 < steps) load_step((s + 1) * BK);
    const unsigned char* base = lds + (size_t)buf * NSLAB * SLAB_BYTES;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8_t a[2], b[2], alo[2], blo[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = *reinterpret_cast<const bf16x8_t*>(base + 0 * SLAB_BYTES + (wm + i * 32 + arow) * ROW_BYTES + kk * 32 + koff);
        b[i] = *reinterpret_cast<const bf16x8_t*>(base + 1 * SLAB_BYTES + (wn + i * 32 + arow) * ROW_BYTES + kk * 32 + koff);
        if (SPLIT) {
          alo[i] = *reinterpret_cast<const bf16x8_t*>(base + 2 * SLAB_BYTES + (wm + i * 32 + arow) * ROW_BYTES + kk * 32 + koff);
          blo[i] = *reinterpret_cast<const bf16x8_t*>(base + 3 * SLAB_BYTES + (wn + i * 32 + arow) * ROW_BYTES + kk * 32 + koff);
        }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          accv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], accv[i][j], 0, 0, 0);
          if (SPLIT) {
            // (a_hi + a_lo)(b_hi + b_lo) ~ a_hi b_hi + a_hi b_lo + a_lo b_hi
            accv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], blo[j], accv[i][j], 0, 0, 0);
            accv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo[i], b[j], accv[i][j], 0, 0, 0);
          }
        }
    }
    if (s + 1 < steps) {
      store_step(buf ^ 1);
    }
    __syncthreads();
  }

  // ---- epilogue: C[32x32] lane layout: col = lane % 32,
  //      row = 8 * (r / 4) + 4 * (lane / 32) + r % 4
  const int ccol = lane & 31, crow = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gr = row0 + wm + i * 32 + 8 * (r >> 2) + crow + (r & 3);
        const int64_t gc = col0 + wn + j * 32 + ccol;
        if (gr < k && gc < k) {
          float* p = acc + gr * ld_acc + gc;
          *p = overwrite ? accv[i][j][r] : *p + accv[i][j][r];
        }
      }
}

// ---------------------------------------------------------------------------
// bf16 SYRK on 256 x 256 upper tiles.  X stays in LDS in its natural
// [token][feature] layout (16-byte row loads go straight in, no register
// transpose) and the MFMA operands, which need 8 consecutive tokens per lane,
// are read with the transposing ds_read_b64_tr_b16: in a 16-lane group, lane
// s points at token s/4 and features 4(s%4)..+3 of one 16-feature strip, and
// lane i receives the 4 tokens of feature i.  Two such reads give the 8
// tokens of a 32x32x16 bf16 MFMA operand.  8 waves of 64 x 128 (2 x 4 MFMA
// blocks), double-buffered LDS stages of BK tokens.  WEIGHTED: the B side is
// w * x split into bf16 hi + lo (two more slabs, BK = 32), A stays exact, so
// each product is a_hi * (b_hi + b_lo) (two MFMAs).  Diagonal tiles of an
// unweighted call read B from the A slab.
namespace syrk2 {
constexpr int TILE = 256;
constexpr int THREADS = 512;
#ifndef KQ_SYRK_PAD
#define KQ_SYRK_PAD 64
#endif
#ifndef KQ_SYRK_BK
#define KQ_SYRK_BK 32
#endif
constexpr int ROW_BYTES = TILE * 2 + KQ_SYRK_PAD;  // one token row of 256 features + pad
template <bool W> constexpr int bk() { return W ? 32 : KQ_SYRK_BK; }
template <bool W> constexpr int slab_bytes() { return bk<W>() * ROW_BYTES; }
template <bool W> constexpr int nslab() { return W ? 3 : 2; }
template <bool W> constexpr int stage_bytes() { return nslab<W>() * slab_bytes<W>(); }
}  // namespace syrk2

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

__device__ __forceinline__ s16x4_t lds_read_tr16(const unsigned char* base, int byte_off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4_t*)((__attribute__((address_space(3))) unsigned char*)base + byte_off));
}

// Upper tile (ti <= tj) of an nt x nt tile grid for workgroup b.  Ungrouped
// launches are XCD-aware: workgroups are dispatched to the 8 XCDs round-robin
// (b % 8), so XCD x is given the contiguous run [x * per, (x + 1) * per) of a
// blocked order of the triangle (4 x 4 tile blocks, block rows then block
// columns), and the ~32 tiles an XCD runs at once share a few row and column
// slabs in its L2.  Returns false for the spare blocks of the last run.
constexpr int SYRK_XCDS = 8;
constexpr int SYRK_BLOCK = 4;
__device__ __forceinline__ bool upper_tile_for_block(int b, int nt, bool grouped, int& ti, int& tj) {
  const int total = nt * (nt + 1) / 2;
  int t = b;
  if (!grouped) {
    const int per = (total + SYRK_XCDS - 1) / SYRK_XCDS;
    t = (b % SYRK_XCDS) * per + b / SYRK_XCDS;
    if (t >= total) return false;
  }
  const int nb = (nt + SYRK_BLOCK - 1) / SYRK_BLOCK;
  for (int R = 0; R < nb; ++R) {
    const int r0 = R * SYRK_BLOCK, r1 = min(r0 + SYRK_BLOCK, nt);
    for (int C = R; C < nb; ++C) {
      const int c0 = C * SYRK_BLOCK, c1 = min(c0 + SYRK_BLOCK, nt);
      int cnt = 0;  // tiles (i, j) of this block with i <= j
      for (int i = r0; i < r1; ++i) cnt += max(0, c1 - max(c0, i));
      if (t < cnt) {
        for (int i = r0; i < r1; ++i) {
          const int jlo = max(c0, i), row = max(0, c1 - jlo);
          if (t < row) {
            ti = i;
            tj = jlo + t;
            return true;
          }
          t -= row;
        }
      }
      t -= cnt;
    }
  }
  return false;
}

template <bool WEIGHTED, bool GROUPED>
__global__ __launch_bounds__(512, 1) void syrk256_kernel(
    const uint16_t* __restrict__ x, int64_t ld, int64_t n, int64_t k, const float* __restrict__ w,
    float* __restrict__ acc, int64_t ld_acc, int ntiles, int overwrite,
    const int64_t* __restrict__ offsets, const int32_t* __restrict__ index, int64_t acc_stride,
    int square_w) {
  using namespace syrk2;
  constexpr int BK = bk<WEIGHTED>();
  constexpr int SLAB = slab_bytes<WEIGHTED>();
  constexpr int STAGE = stage_bytes<WEIGHTED>();
  constexpr int CPT = BK * 32 / THREADS;  // 16-byte chunks per thread per slab
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

  int64_t list0 = 0;
  if (GROUPED) {
    const int64_t g = group_of_row(offsets, gridDim.y, blockIdx.y);
    list0 = offsets[g];
    n = offsets[g + 1] - list0;
    acc += g * acc_stride;
  }
  int ti, tj;
  if (!upper_tile_for_block(blockIdx.x, ntiles, GROUPED, ti, tj)) return;  // spare block
  const bool share_b = !WEIGHTED && ti == tj;
  const int64_t row0 = (int64_t)ti * TILE, col0 = (int64_t)tj * TILE;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // ---- global -> registers: chunk c = tid + THREADS * i: token c / 32, features 8 (c % 32)
  u32x4_t ra[CPT], rb[CPT], rbl[CPT];
  auto load = [&](int64_t t0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + THREADS * i;
      const int64_t pos = t0 + (c >> 5);
      const int fc = (c & 31) * 8;
      u32x4_t va = {0u, 0u, 0u, 0u}, vb = {0u, 0u, 0u, 0u}, vl = {0u, 0u, 0u, 0u};
      if (pos < n) {
        const int64_t tok = !GROUPED ? pos : (index ? (int64_t)index[list0 + pos] : list0 + pos);
        const uint16_t* rowp = x + tok * ld;
        if (row0 + fc < k) va = *reinterpret_cast<const u32x4_t*>(rowp + row0 + fc);
        if (!share_b && col0 + fc < k) {
          const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(rowp + col0 + fc);
          if (WEIGHTED) {
            float wt = w[GROUPED ? list0 + pos : pos];
            if (GROUPED && square_w) wt *= wt;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              uint32_t h0, l0, h1, l1;
              split_bf16(bf16_bits_to_f32(raw[e] & 0xffffu) * wt, h0, l0);
              split_bf16(bf16_bits_to_f32(raw[e] >> 16) * wt, h1, l1);
              vb[e] = h0 | (h1 << 16);
              vl[e] = l0 | (l1 << 16);
            }
          } else {
            vb = raw;
          }
        }
      }
      ra[i] = va;
      rb[i] = vb;
      if (WEIGHTED) rbl[i] = vl;
    }
  };
  auto store = [&](int buf) {
    unsigned char* base = lds + buf * STAGE;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + THREADS * i;
      const int off = (c >> 5) * ROW_BYTES + (c & 31) * 16;
      *reinterpret_cast<u32x4_t*>(base + off) = ra[i];
      if (!share_b) *reinterpret_cast<u32x4_t*>(base + SLAB + off) = rb[i];
      if (WEIGHTED) *reinterpret_cast<u32x4_t*>(base + 2 * SLAB + off) = rbl[i];
    }
  };

  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
  float16_t accv[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) accv[i][j][r] = 0.0f;

  // transposed-read address of this lane inside a 32-feature x 16-token block:
  // 16-lane group g covers features 16 (g % 2) + [0, 16) and tokens 8 (g / 2) + [0, 8)
  const int g16 = lane >> 4, s16 = lane & 15;
  const int lane_off = (8 * (g16 >> 1) + (s16 >> 2)) * ROW_BYTES + (16 * (g16 & 1) + 4 * (s16 & 3)) * 2;

  const int64_t steps = (n + BK - 1) / BK;
  if (steps > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int64_t s = 0; s < steps; ++s) {
    const int buf = (int)(s & 1);
    if (s + 1 < steps) load((s + 1) * BK);
    const unsigned char* a_base = lds + buf * STAGE;
    const unsigned char* b_base = share_b ? a_base : a_base + SLAB;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int koff = kk * 16 * ROW_BYTES + lane_off;
      bf16x8_t fa[2], fb[4], fbl[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int o = koff + (wm + i * 32) * 2;
        const s16x4_t lo = lds_read_tr16(a_base, o);
        const s16x4_t hi = lds_read_tr16(a_base, o + 4 * ROW_BYTES);
        fa[i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int o = koff + (wn + j * 32) * 2;
        const s16x4_t lo = lds_read_tr16(b_base, o);
        const s16x4_t hi = lds_read_tr16(b_base, o + 4 * ROW_BYTES);
        fb[j] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        if (WEIGHTED) {
          const s16x4_t l2 = lds_read_tr16(a_base + 2 * SLAB, o);
          const s16x4_t h2 = lds_read_tr16(a_base + 2 * SLAB, o + 4 * ROW_BYTES);
          fbl[j] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(l2, h2, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          accv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], accv[i][j], 0, 0, 0);
      if (WEIGHTED) {  // residual products after all high parts: no back-to-back accumulator updates
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            accv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fbl[j], accv[i][j], 0, 0, 0);
      }
    }
    if (s + 1 < steps) store(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: C[32x32] lane layout col = lane % 32, row = 8 (r/4) + 4 (lane/32) + r%4
  const int ccol = lane & 31, crow = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gr = row0 + wm + i * 32 + 8 * (r >> 2) + crow + (r & 3);
        const int64_t gc = col0 + wn + j * 32 + ccol;
        if (gr < k && gc < k) {
          float* p = acc + gr * ld_acc + gc;
          *p = overwrite ? accv[i][j][r] : *p + accv[i][j][r];
        }
      }
}

// ---------------------------------------------------------------------------
// Unweighted bf16 SYRK with direct-to-LDS loads.  Same tiles, waves and
// transposed operand reads as syrk256_kernel, but X rows go from HBM into LDS
// by buffer_load_dwordx4 ... lds (no register staging), double-buffered in
// steps of 64 tokens: a step's loads are issued one step ahead, so the
// memory latency is covered by one step of MFMA work (32 MFMAs per wave
// between barriers: 4-5 % faster than four stages of 32 tokens, and as fast
// as two of 80).  A wave's load writes 1 KiB of LDS contiguously (two token
// rows), so rows are not padded:
// 16-byte chunk c of token row r is stored at slot c ^ 4 (r % 4), which puts
// the four rows of each transposed read on distinct LDS banks.  Tokens past n
// get an out-of-range buffer offset and read as zeros; features past k only
// reach output rows and columns past k, which are not stored.
namespace syrk3 {
constexpr int TILE = 256;
constexpr int BK = 64;
constexpr int ROW = TILE * 2;      // bytes per token row
constexpr int SLAB = BK * ROW;     // 32 KiB
constexpr int NST = 2;             // ring stages
constexpr int QPW = BK / 16;       // load instructions per wave and slab (two token rows each)
}  // namespace syrk3

__shared__ __attribute__((aligned(16))) unsigned char syrk3_lds[syrk3::NST * 2 * syrk3::SLAB];

using dma::i32x4_t;
using dma::load_to_lds16;
using dma::lds_offset_of;
using dma::make_rsrc;
using dma::waitcnt_vm;

// One tile's token range [t_begin, t_end) through the two-stage ring into
// accv.  Every wave of the workgroup calls it with the same arguments; it
// starts and ends with the ring idle (all loads landed, all reads done).
__device__ __forceinline__ void syrk3_range(const i32x4_t rsrc, uint32_t nbytes, int64_t ld, int64_t t_begin,
                                            int64_t t_end, int64_t row0, int64_t col0, bool share_b,
                                            float16_t (&accv)[2][4], int wave, int lane) {
  using namespace syrk3;
  const uint32_t lds0 = lds_offset_of(syrk3_lds);
  // Loads: wave w, part q < QPW: token rows 2 (QPW w + q) + lane / 32 of a
  // stage, this lane's 16-byte slot lane % 32 holds global chunk slot ^ 4 (row % 4).
  int drow[QPW], dchunk[QPW];
#pragma unroll
  for (int q = 0; q < QPW; ++q) {
    drow[q] = 2 * (QPW * wave + q) + (lane >> 5);
    dchunk[q] = (lane & 31) ^ (4 * (drow[q] & 3));
  }
  // stage s lives at [2 SLAB s, 2 SLAB s + SLAB) (A) and the next SLAB bytes (B)
  auto issue = [&](int stage, int64_t t0) {
#pragma unroll
    for (int q = 0; q < QPW; ++q) {
      const int64_t tok = t0 + drow[q];
      const bool ok = tok < t_end;
      const uint32_t base = ok ? (uint32_t)(tok * ld * 2) : nbytes;  // nbytes: first offset past the range
      const uint32_t dst = lds0 + (uint32_t)(2 * SLAB * stage + (QPW * wave + q) * 1024);
      load_to_lds16(rsrc, ok ? base + (uint32_t)((row0 + dchunk[q] * 8) * 2) : base, dst);
      if (!share_b)
        load_to_lds16(rsrc, ok ? base + (uint32_t)((col0 + dchunk[q] * 8) * 2) : base, dst + SLAB);
    }
  };

  // Transposed reads: 16-lane group g covers features 16 (g % 2) of a 32-feature
  // block and tokens 8 (g / 2) + [0, 8); lane s16 reads token s16 / 4 (+4 for
  // the second half) and features 4 (s16 % 4) .. +3.
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
  const int g16 = lane >> 4, s16 = lane & 15;
  const int trow = 8 * (g16 >> 1) + (s16 >> 2);
  const int xorv = 4 * (s16 >> 2);
  int offa[2], offb[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int f = wm + i * 32 + 16 * (g16 & 1) + 4 * (s16 & 3);
    offa[i] = trow * ROW + (((f >> 3) ^ xorv) << 4) + (f & 7) * 2;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = wn + j * 32 + 16 * (g16 & 1) + 4 * (s16 & 3);
    offb[j] = trow * ROW + (((f >> 3) ^ xorv) << 4) + (f & 7) * 2;
  }

  // Step s on stage s % NST: wait for this step's loads (NST - 2 later steps'
  // may still be in flight), barrier (every wave's loads have landed; every
  // wave is done with the stage the next loads overwrite), issue the loads of
  // step s + NST - 1, compute.  Steps past the end load zeros, which keeps the
  // per-step count of outstanding loads fixed.
  const int64_t steps = (t_end - t_begin + BK - 1) / BK;
  for (int p = 0; p < NST - 1; ++p) issue(p, t_begin + p * BK);
  int stage = 0;
  for (int64_t s = 0; s < steps; ++s) {
    asm volatile("" ::: "memory");  // the barrier builtin alone does not order LDS accesses
    if (share_b) __builtin_amdgcn_s_waitcnt(waitcnt_vm((NST - 2) * QPW));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm((NST - 2) * 2 * QPW));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(stage == 0 ? NST - 1 : stage - 1, t_begin + (s + NST - 1) * BK);
    const unsigned char* a_base = syrk3_lds + 2 * SLAB * stage;
    const unsigned char* b_base = share_b ? a_base : a_base + SLAB;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8_t fa[2], fb[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int o = offa[i] + kk * 16 * ROW;
        const s16x4_t lo = lds_read_tr16(a_base, o);
        const s16x4_t hi = lds_read_tr16(a_base, o + 4 * ROW);
        fa[i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int o = offb[j] + kk * 16 * ROW;
        const s16x4_t lo = lds_read_tr16(b_base, o);
        const s16x4_t hi = lds_read_tr16(b_base, o + 4 * ROW);
        fb[j] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          accv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], accv[i][j], 0, 0, 0);
    }
    stage = stage == NST - 1 ? 0 : stage + 1;
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // the loads issued past the end have landed
  __syncthreads();                            // every wave is done reading the ring
}

// Store a wave's 64 x 128 part of a 256 x 256 tile: dst[r][c] (row stride
// ld) for r < rlim, c < clim, written or added.
__device__ __forceinline__ void syrk3_store(const float16_t (&accv)[2][4], float* dst, int64_t ld, int64_t rlim,
                                            int64_t clim, bool overwrite, int wave, int lane) {
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
  const int ccol = lane & 31, crow = (lane >> 5) * 4;
  // opaque to the optimiser: keeps a persistent caller from hoisting (and
  // spilling) the 128 element offsets out of its item loop
  asm volatile("" : "+s"(ld));
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gr = wm + i * 32 + 8 * (r >> 2) + crow + (r & 3);
        const int64_t gc = wn + j * 32 + ccol;
        if (gr < rlim && gc < clim) {
          float* p = dst + gr * ld + gc;
          *p = overwrite ? accv[i][j][r] : *p + accv[i][j][r];
        }
      }
}

// Chunked tail.  Tiles go to XCDs in contiguous runs of per = ceil(tiles / 8)
// (tile x per + j on XCD x = workgroup % 8).  The workgroups of an XCD take
// its tiles j < j1 whole, j1 a multiple of the XCD's CU count, so those
// rounds are full.  With chunks > 1 the remaining tiles of each XCD (at most
// nmax) are cut by 64-token steps into `chunks` equal parts, and the XCD's
// workgroups take them chunk-major (chunk 0 of every tail tile, then chunk 1
// ...), so the workgroups that run together stream the same token rows, as
// the whole tiles of a round do.  Chunk 0 writes (or adds to) the tile; chunk
// c >= 1 writes partial slot (x nmax + i)(chunks - 1) + c - 1 for tail tile
// i; the fix-up kernel then adds slots 1 .. chunks - 1, in that order.
struct TailPlan {
  int j1, nmax, chunks;
};

__global__ __launch_bounds__(512, 1) void syrk256_dma_kernel(
    const uint16_t* __restrict__ x, int64_t ld, int64_t n, int64_t k, float* __restrict__ acc,
    int64_t ld_acc, int nt, int overwrite, uint32_t nbytes, float* __restrict__ partial, TailPlan plan) {
  using namespace syrk3;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const i32x4_t rsrc = make_rsrc(x, nbytes);
  const int total = nt * (nt + 1) / 2, per = (total + SYRK_XCDS - 1) / SYRK_XCDS;
  const int b = blockIdx.x;
  const int64_t steps = (n + BK - 1) / BK;
  int xcd = b % SYRK_XCDS, j = b / SYRK_XCDS;
  int64_t s0 = 0, s1 = steps;
  int slot = -1;
  if (plan.chunks > 1 && j >= plan.j1) {
    const int nx = min(per, total - xcd * per) - plan.j1;
    if (nx <= 0) return;  // spare block
    const int q = j - plan.j1, c = q / nx, i = q - c * nx;
    if (c >= plan.chunks) return;
    j = plan.j1 + i;
    s0 = c * steps / plan.chunks;
    s1 = (c + 1) * steps / plan.chunks;
    if (c > 0) slot = (xcd * plan.nmax + i) * (plan.chunks - 1) + c - 1;
  }
  const int t = xcd * per + j;
  int ti, tj;
  if (t >= total || !upper_tile_for_block(t, nt, true, ti, tj)) return;  // spare block
  const int64_t row0 = (int64_t)ti * TILE, col0 = (int64_t)tj * TILE;
  float16_t accv[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int q = 0; q < 16; ++q) accv[i][jj][q] = 0.0f;
  const int64_t t_end = s1 * BK < n ? s1 * BK : n;
  syrk3_range(rsrc, nbytes, ld, s0 * BK, t_end, row0, col0, ti == tj, accv, wave, lane);
  const bool to_slot = slot >= 0;
  float* dst = to_slot ? partial + (int64_t)slot * (TILE * TILE) : acc + row0 * ld_acc + col0;
  syrk3_store(accv, dst, to_slot ? TILE : ld_acc, to_slot ? TILE : k - row0, to_slot ? TILE : k - col0,
              to_slot || overwrite, wave, lane);
}

// acc tile += partial slots 1 .. chunks - 1 of a tail tile, in chunk order.
// Block (x nmax + i, y): tail tile i of XCD x, rows 16 y .. 16 y + 15.
__global__ __launch_bounds__(256) void syrk_tail_fixup_kernel(const float* __restrict__ partial, int nt,
                                                              TailPlan plan, float* __restrict__ acc,
                                                              int64_t ld_acc, int64_t k) {
  const int total = nt * (nt + 1) / 2, per = (total + SYRK_XCDS - 1) / SYRK_XCDS;
  const int xcd = blockIdx.x / plan.nmax, i = blockIdx.x - xcd * plan.nmax;
  if (i >= min(per, total - xcd * per) - plan.j1) return;
  int ti, tj;
  upper_tile_for_block(xcd * per + plan.j1 + i, nt, true, ti, tj);
  const int64_t row0 = (int64_t)ti * syrk3::TILE, col0 = (int64_t)tj * syrk3::TILE;
  const int c = threadIdx.x;
  if (col0 + c >= k) return;
  const float* slots = partial + (int64_t)blockIdx.x * (plan.chunks - 1) * (syrk3::TILE * syrk3::TILE);
  for (int rr = 0; rr < 16; ++rr) {
    const int row = blockIdx.y * 16 + rr;
    if (row0 + row >= k) break;
    float* p = acc + (row0 + row) * ld_acc + col0 + c;
    float sum = *p;
    for (int s = 0; s < plan.chunks - 1; ++s) sum += slots[(int64_t)s * (syrk3::TILE * syrk3::TILE) + row * syrk3::TILE + c];
    *p = sum;
  }
}

// The tail split pays when an XCD's last round of tiles leaves CUs idle.
// Rounds are priced in whole-tile times: the tail's chunked rounds cost
// ceil(nmax chunks / cus_x) / chunks, plus 0.01 a chunk for the partial
// slots and the fix-up pass; chunks of fewer than 4 steps are not taken, and
// the split is used only below 0.85 of the one plain tail round.
static TailPlan plan_tail(int ntiles, int cus, int64_t n) {
  TailPlan p{0, 0, 1};
  if (cus < SYRK_XCDS || cus % SYRK_XCDS) return p;
  const int cx = cus / SYRK_XCDS, per = (ntiles + SYRK_XCDS - 1) / SYRK_XCDS;
  const int j1 = per / cx * cx, nmax = per - j1;
  const int64_t steps = (n + syrk3::BK - 1) / syrk3::BK;
  if (nmax == 0) return p;
  double best = 0.85;
  for (int c = 2; c <= 16 && steps >= 4 * c; ++c) {
    const double cost = (double)((nmax * c + cx - 1) / cx) / c + 0.01 * (c - 1);
    if (cost < best) {
      best = cost;
      p = TailPlan{j1, nmax, c};
    }
  }
  return p;
}

// CUs of the device a stream runs on (the current device for the null
// stream), so the grid plan matches where the launch goes.
static int device_cus(hipStream_t st = nullptr) {
  int dev = 0, cus = 0;
  if (st ? hipStreamGetDevice(st, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

static int64_t tail_slot_bytes(const TailPlan& p) {
  return p.chunks > 1 ? (int64_t)SYRK_XCDS * p.nmax * (p.chunks - 1) * syrk3::TILE * syrk3::TILE * 4 : 0;
}

static hipError_t launch_syrk256_dma(const void* x, int64_t ld, int64_t n, int64_t k, float* acc,
                                     int64_t ld_acc, int overwrite, hipStream_t st, void* workspace = nullptr,
                                     int64_t ws_bytes = 0) {
  const int nt = (int)((k + syrk3::TILE - 1) / syrk3::TILE);
  const int ntiles = nt * (nt + 1) / 2;
  const uint32_t nbytes = (uint32_t)(n * ld * 2);
  const int per = (ntiles + SYRK_XCDS - 1) / SYRK_XCDS;
  TailPlan plan{0, 0, 1};
  if (workspace) {
    plan = plan_tail(ntiles, device_cus(st), n);
    if (tail_slot_bytes(plan) > ws_bytes) plan = TailPlan{0, 0, 1};
  }
  const int blocks = SYRK_XCDS * (plan.chunks > 1 ? plan.j1 + plan.nmax * plan.chunks : per);
  syrk256_dma_kernel<<<dim3(blocks), dim3(512), 0, st>>>((const uint16_t*)x, ld, n, k, acc, ld_acc, nt, overwrite,
                                                          nbytes, (float*)workspace, plan);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || plan.chunks <= 1) return e;
  syrk_tail_fixup_kernel<<<dim3(SYRK_XCDS * plan.nmax, syrk3::TILE / 16), dim3(256), 0, st>>>(
      (const float*)workspace, nt, plan, acc, ld_acc, k);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Weighted grouped bf16 SYRK with direct loads (rows of each group
// contiguous, no row index).  Same 256 x 256 tiles, waves and transposed
// reads as syrk256_dma_kernel; X rows go from HBM straight into LDS
// (global_load_lds_dwordx4: 64-bit addresses, so any row count), 16 tokens a
// step through a six-stage ring, and the row weights of a step ride along
// into LDS (wave 0, 16 lanes x 4 bytes).  The weight goes on the A side:
// once a stage has landed, the workgroup rewrites its A slab in place as the
// bf16 high part of w x and writes the bf16 residual to a third slab
// (w x = hi + lo to 16 significant bits), so each product is
// (a_hi + a_lo) b, two MFMAs, with the B slab exact.  That conversion runs a
// step ahead of the MFMAs, in the same barrier interval, so the VALU work
// overlaps the matrix cores.  A diagonal tile loads one slab and keeps it as
// B, writing hi and lo to the other two.  Rows past the group's end load the
// group's last row and convert to zeros.
#ifndef KQ_SYRK4_BK
#define KQ_SYRK4_BK 16
#endif
namespace syrk4 {
constexpr int TILE = 256;
constexpr int BK = KQ_SYRK4_BK;   // tokens per step
constexpr int ROW = TILE * 2;     // bytes per token row
constexpr int SLAB = BK * ROW;
constexpr int STAGE = 3 * SLAB;   // raw / hi, B (or hi), lo
constexpr int NS = 147456 / STAGE;  // ring stages (144 KiB): loads run NS - 3 steps ahead of their conversion
constexpr int LPW = BK / 16;      // load instructions per wave and slab (two token rows each)
static_assert(BK == 16 || BK == 32, "steps of 16 or 32 tokens");
}  // namespace syrk4

__shared__ __attribute__((aligned(16))) unsigned char syrk4_lds[syrk4::NS * syrk4::STAGE];
__shared__ __attribute__((aligned(16))) float syrk4_w[syrk4::NS][syrk4::BK];

__device__ __forceinline__ void global_load_to_lds16(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_addr), "v"(src)
               : "memory", "m0");
}

__device__ __forceinline__ void global_load_to_lds4(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(lds_addr), "v"(src)
               : "memory", "m0");
}

// wait until this wave has at most n (< 16) direct loads in flight, then barrier
__device__ __forceinline__ void syrk4_wait(int n) {
  asm volatile("" ::: "memory");  // the barrier builtin alone does not order LDS accesses
  switch (n) {
#define KQ_WAIT_CASE(c) \
  case c: __builtin_amdgcn_s_waitcnt(waitcnt_vm(c)); break;
    KQ_WAIT_CASE(0) KQ_WAIT_CASE(1) KQ_WAIT_CASE(2) KQ_WAIT_CASE(3) KQ_WAIT_CASE(4) KQ_WAIT_CASE(5)
    KQ_WAIT_CASE(6) KQ_WAIT_CASE(7) KQ_WAIT_CASE(8) KQ_WAIT_CASE(9) KQ_WAIT_CASE(10) KQ_WAIT_CASE(11)
    KQ_WAIT_CASE(12) KQ_WAIT_CASE(13) KQ_WAIT_CASE(14)
#undef KQ_WAIT_CASE
    default: __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); break;
  }
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Persistent: `gridDim.x` workgroups walk the items (group rank, tile) in
// snake order (round q gives item q G + b to workgroup b, reversed on odd
// rounds).  Ranks order the groups by row count, largest first (ties by
// index), computed once per workgroup in LDS for up to LPT_MAX_GROUPS groups
// (natural order beyond); every item's result is independent of the order.
__shared__ int syrk4_rank_order[LPT_MAX_GROUPS];
__shared__ int syrk4_rank_size[LPT_MAX_GROUPS];

__global__ __launch_bounds__(512, 1) void syrk256w_dma_kernel(
    const uint16_t* __restrict__ x, int64_t ld, int64_t k, const float* __restrict__ w, float* __restrict__ acc,
    int nt, const int64_t* __restrict__ offsets, int groups, int square_w) {
  using namespace syrk4;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool lpt = groups <= LPT_MAX_GROUPS;
  if (lpt) {
    for (int g = tid; g < groups; g += 512) {
      const int64_t ng = offsets[g + 1] - offsets[g];
      syrk4_rank_size[g] = ng < 0x7fffffff ? (int)ng : 0x7fffffff;
    }
    __syncthreads();
    for (int g = tid; g < groups; g += 512) {
      const int ng = syrk4_rank_size[g];
      int rank = 0;
      for (int h = 0; h < groups; ++h) {
        const int nh = syrk4_rank_size[h];
        rank += (nh > ng || (nh == ng && h < g)) ? 1 : 0;
      }
      syrk4_rank_order[rank] = g;
    }
    __syncthreads();
  }
  const int ntiles = nt * (nt + 1) / 2;
  const int64_t items = (int64_t)ntiles * groups;
  const int grid = gridDim.x;
  const uint32_t lds0 = lds_offset_of(syrk4_lds), wl0 = lds_offset_of(syrk4_w);
  // loads: instruction q of wave w moves token rows 2 (LPW w + q) + lane / 32;
  // lane % 32 is the LDS slot, holding global chunk slot ^ 4 (row % 4) of the
  // row's 256 features
  const int drow = 2 * LPW * wave + (lane >> 5);
  static_assert(LPW <= 2, "two load instructions per wave at most");
  const int dchunk[2] = {(lane & 31) ^ (4 * (drow & 3)), (lane & 31) ^ (4 * ((drow + 2) & 3))};
  // conversion: chunk c = tid + 512 u -> token row c / 32, LDS slot c % 32
  // (the layout is kept, so the swizzle does not matter)
  const int cr = tid >> 5;
  const int coff = cr * ROW + (tid & 31) * 16;
  // transposed reads (as syrk256_dma_kernel, 16-token steps)
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
  const int g16 = lane >> 4, s16 = lane & 15;
  const int trow = 8 * (g16 >> 1) + (s16 >> 2);
  const int xorv = 4 * (s16 >> 2);
  int offa[2], offb[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int f = wm + i * 32 + 16 * (g16 & 1) + 4 * (s16 & 3);
    offa[i] = trow * ROW + (((f >> 3) ^ xorv) << 4) + (f & 7) * 2;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = wn + j * 32 + 16 * (g16 & 1) + 4 * (s16 & 3);
    offb[j] = trow * ROW + (((f >> 3) ^ xorv) << 4) + (f & 7) * 2;
  }

  for (int64_t q = 0;; ++q) {
    const int64_t item = q * grid + ((q & 1) ? grid - 1 - blockIdx.x : blockIdx.x);
    if (item >= items) break;
    const int rank = (int)(item / ntiles);
    const int64_t g = lpt ? syrk4_rank_order[rank] : rank;
    int ti, tj;
    upper_tile_for_block((int)(item - (int64_t)rank * ntiles), nt, true, ti, tj);
    const bool share = ti == tj;
    const int64_t row0 = (int64_t)ti * TILE, col0 = (int64_t)tj * TILE;
    const int64_t list0 = offsets[g];
    const int n = (int)(offsets[g + 1] - list0);
    const int per_step = LPW * (share ? 1 : 2) + (wave == 0 ? 1 : 0);

    float16_t accv[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) accv[i][j][r] = 0.0f;

    const int steps = (n + BK - 1) / BK;
    if (steps > 0) {
      // a chunk past feature k (edge tiles) reads feature 0 instead: such
      // features only reach accumulator rows / columns past k, never stored
      const float* wg = w + list0;
      auto issue = [&](int stage, int t0) {
#pragma unroll
        for (int q = 0; q < LPW; ++q) {
          const int64_t fa = row0 + dchunk[q] * 8, fb = col0 + dchunk[q] * 8;
          const uint16_t* xa = x + list0 * ld + (fa < k ? fa : 0);
          const uint16_t* xb = x + list0 * ld + (fb < k ? fb : 0);
          const int pos = t0 + drow + 2 * q < n ? t0 + drow + 2 * q : n - 1;
          const int64_t roff = (int64_t)pos * ld;
          const uint32_t dst = lds0 + (uint32_t)(STAGE * stage + (LPW * wave + q) * 1024);
          global_load_to_lds16(xa + roff, dst);  // A (raw) slab
          if (!share) global_load_to_lds16(xb + roff, dst + SLAB);
        }
        if (wave == 0 && lane < BK) {
          const int wp = t0 + lane < n ? t0 + lane : n - 1;
          global_load_to_lds4(wg + wp, wl0 + (uint32_t)(stage * BK * 4));
        }
      };
      // rows past the end get weight 0: finite rows then convert to zeros
      auto convert = [&](int stage, int t0) {
        unsigned char* st = syrk4_lds + STAGE * stage;
#pragma unroll
        for (int u = 0; u < BK / 16; ++u) {
          const int off = coff + u * 16 * ROW, row = cr + 16 * u;
          const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(st + off);
          float wt = syrk4_w[stage][row];
          if (square_w) wt *= wt;
          if (t0 + row >= n) wt = 0.0f;
          u32x4_t hi, lo;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint32_t h, l;
            split_bf16_pair(raw[e], wt, h, l);
            hi[e] = h;
            lo[e] = l;
          }
          // non-diagonal: hi replaces the raw A slab; diagonal: the raw slab stays (as B)
          *reinterpret_cast<u32x4_t*>(st + (share ? SLAB : 0) + off) = hi;
          *reinterpret_cast<u32x4_t*>(st + 2 * SLAB + off) = lo;
        }
      };
      const int hi_slab = share ? SLAB : 0, b_slab = share ? 0 : SLAB;

      // Step s: wait for step s + 1's loads (three later steps may still be
      // in flight) and barrier (step s's conversion is complete; every wave
      // is done with step s - 1's stage), issue the loads of step s + NS - 1
      // into that stage, convert step s + 1, then run step s's MFMAs.  Steps
      // past the end load the last row again (never converted or used),
      // which keeps the per-step count of outstanding loads fixed.
#pragma unroll
      for (int st = 0; st < NS - 1; ++st) issue(st, st * BK);
      syrk4_wait(per_step * (NS - 2));  // step 0 has landed
      convert(0, 0);
      int stage = 0;
      for (int s = 0; s < steps; ++s) {
        const int next = stage == NS - 1 ? 0 : stage + 1;
        const int prev = stage == 0 ? NS - 1 : stage - 1;
        syrk4_wait(per_step * (NS - 3));
        issue(prev, (s + NS - 1) * BK);
        const unsigned char* base = syrk4_lds + STAGE * stage;
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
          const int ko = kk * 16 * ROW;
          bf16x8_t fh[2], fl[2], fb[4];
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const s16x4_t h0 = lds_read_tr16(base + hi_slab, ko + offa[i]);
            const s16x4_t h1 = lds_read_tr16(base + hi_slab, ko + offa[i] + 4 * ROW);
            fh[i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7));
            const s16x4_t l0 = lds_read_tr16(base + 2 * SLAB, ko + offa[i]);
            const s16x4_t l1 = lds_read_tr16(base + 2 * SLAB, ko + offa[i] + 4 * ROW);
            fl[i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7));
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const s16x4_t b0 = lds_read_tr16(base + b_slab, ko + offb[j]);
            const s16x4_t b1 = lds_read_tr16(base + b_slab, ko + offb[j] + 4 * ROW);
            fb[j] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7));
          }
          // (the last step converts the stage loaded past the end: unused, harmless)
          if (kk == 0) convert(next, (s + 1) * BK);
          // the eight high-part products, then the eight residual ones: the two
          // updates of an accumulator are eight MFMAs apart, not back to back
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              accv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh[i], fb[j], accv[i][j], 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              accv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fl[i], fb[j], accv[i][j], 0, 0, 0);
        }
        stage = next;
      }
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // the loads issued past the end have landed
      __syncthreads();                            // every wave is done with the ring
    }
    syrk3_store(accv, acc + g * k * k + row0 * k + col0, k, k - row0, k - col0, true, wave, lane);
  }
}

static hipError_t launch_syrk256w_dma(const void* x, int64_t ld, int64_t k, const float* w, float* acc,
                                      const int64_t* offsets, int groups, int square_w, hipStream_t st) {
  const int nt = (int)((k + syrk4::TILE - 1) / syrk4::TILE);
  const int64_t items = (int64_t)(nt * (nt + 1) / 2) * groups;
  int cus = device_cus(st);
  if (cus <= 0) cus = 256;
  const int grid = (int)(items < cus ? items : cus);
  syrk256w_dma_kernel<<<dim3(grid), dim3(512), 0, st>>>((const uint16_t*)x, ld, k, w, acc, nt, offsets, groups,
                                                          square_w);
  return hipGetLastError();
}

template <bool WEIGHTED, bool GROUPED>
static hipError_t launch_syrk256(const void* x, int64_t ld, int64_t n, int64_t k, const float* w,
                                 float* acc, int64_t ld_acc, int overwrite, hipStream_t st,
                                 const int64_t* offsets = nullptr, const int32_t* index = nullptr,
                                 int groups = 1, int square_w = 0) {
  const int nt = (int)((k + syrk2::TILE - 1) / syrk2::TILE);
  const int ntiles = nt * (nt + 1) / 2;
  const int blocks = GROUPED ? ntiles : SYRK_XCDS * ((ntiles + SYRK_XCDS - 1) / SYRK_XCDS);
  const size_t lds = 2 * (size_t)syrk2::stage_bytes<WEIGHTED>();
  auto kern = syrk256_kernel<WEIGHTED, GROUPED>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  kern<<<dim3(blocks, groups), dim3(syrk2::THREADS), lds, st>>>(
      (const uint16_t*)x, ld, n, k, w, acc, ld_acc, nt, overwrite, offsets, index, k * ld_acc, square_w);
  return hipGetLastError();
}

// out = sym(acc) * inv.  The computed region is tile(i) <= tile(j)
// (128-wide tiles; inside a diagonal tile both halves exist).  One workgroup
// per pair of 64 x 64 blocks (bi <= bj) and its mirror (bj, bi): it reads the
// upper block acc[bi][bj] once (coalesced rows into LDS), writes it scaled,
// and writes its transpose into the mirror block; for a pair inside a
// diagonal tile it also reads acc[bj][bi] and writes the average of the two
// halves, (acc[i][j] inv + acc[j][i] inv) / 2 (kquant's (H + H^T) / 2), each
// product and the sum rounded on its own, with the diagonal acc[i][i] inv.
constexpr int FIN_B = 64;
template <bool FULL>
__device__ __forceinline__ void finalize_pair_impl(const float* __restrict__ a, int64_t lda, int64_t k,
                                                   float inv, float* __restrict__ o, int64_t ldo, int64_t bi,
                                                   int64_t bj, float (*t)[FIN_B][FIN_B + 1]) {
#pragma clang fp contract(off)
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t i0 = bi * FIN_B, j0 = bj * FIN_B;
  const bool two = i0 / syrk::TILE == j0 / syrk::TILE && bi != bj;  // both halves of a diagonal tile
  // t[0][r][c] = acc[i0 + r][j0 + c]; t[1][r][c] = acc[j0 + r][i0 + c]; all
  // of a thread's loads are issued before the first LDS store
  constexpr int R = FIN_B / 4;
  float u[R];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int64_t i = i0 + ty + 4 * q, j = j0 + tx;
    u[q] = FULL || (i < k && j < k) ? a[i * lda + j] : 0.0f;
  }
  if (two) {
    float l[R];
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const int64_t p = j0 + ty + 4 * q, c = i0 + tx;
      l[q] = FULL || (p < k && c < k) ? a[p * lda + c] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < R; ++q) t[1][ty + 4 * q][tx] = l[q];
  }
#pragma unroll
  for (int q = 0; q < R; ++q) t[0][ty + 4 * q][tx] = u[q];
  __syncthreads();
  // block (bi, bj): element (i0 + r, j0 + tx)
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int r = ty + 4 * q;
    const float up = t[0][r][tx] * inv;
    float v = up;
    if (bi == bj) {
      if (r != tx) v = (up + t[0][tx][r] * inv) * 0.5f;
    } else if (two) {
      v = (up + t[1][tx][r] * inv) * 0.5f;
    }
    if (FULL || (i0 + r < k && j0 + tx < k)) o[(i0 + r) * ldo + j0 + tx] = v;
  }
  if (bi == bj) return;
  // mirror block (bj, bi): element (j0 + r, i0 + tx) from acc[i0 + tx][j0 + r]
  // (averaged with acc[j0 + r][i0 + tx] inside a diagonal tile)
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int r = ty + 4 * q;
    const float up = t[0][tx][r] * inv;
    const float v = two ? (up + t[1][r][tx] * inv) * 0.5f : up;
    if (FULL || (j0 + r < k && i0 + tx < k)) o[(j0 + r) * ldo + i0 + tx] = v;
  }
}

__device__ __forceinline__ void finalize_pair(const float* __restrict__ a, int64_t lda, int64_t k, float inv,
                                              float* __restrict__ o, int64_t ldo, int64_t bi, int64_t bj,
                                              float (*t)[FIN_B][FIN_B + 1]) {
  if ((bj + 1) * FIN_B <= k)  // bi <= bj: the whole pair is inside the matrix
    finalize_pair_impl<true>(a, lda, k, inv, o, ldo, bi, bj, t);
  else
    finalize_pair_impl<false>(a, lda, k, inv, o, ldo, bi, bj, t);
}

// block pair b of the upper triangle of nb x nb blocks -> (bi <= bj)
__device__ __forceinline__ void finalize_pair_of(int64_t b, int64_t& bi, int64_t& bj) {
  int64_t c = (int64_t)((sqrt(8.0 * (double)b + 1.0) - 1.0) * 0.5);
  while (c * (c + 1) / 2 > b) --c;
  while ((c + 1) * (c + 2) / 2 <= b) ++c;
  bj = c;
  bi = b - c * (c + 1) / 2;
}

__global__ __launch_bounds__(256) void syrk_finalize_kernel(
    const float* __restrict__ acc, int64_t ld_acc, int64_t k, float inv_denom,
    float* __restrict__ out, int64_t ld_out) {
  __shared__ float t[2][FIN_B][FIN_B + 1];
  int64_t bi, bj;
  finalize_pair_of(blockIdx.x, bi, bj);
  finalize_pair(acc, ld_acc, k, inv_denom, out, ld_out, bi, bj, t);
}

// diag += damp * mean(diag).  One workgroup: reduce the diagonal, then
// update it.
__global__ __launch_bounds__(1024) void syrk_damp_kernel(float* __restrict__ out, int64_t ld_out,
                                                         int64_t k, float damp) {
  __shared__ float partial[1024];
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < k; i += 1024) s += out[i * ld_out + i];
  partial[threadIdx.x] = s;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) partial[threadIdx.x] += partial[threadIdx.x + w];
    __syncthreads();
  }
  const float add = damp * (partial[0] / (float)k);
  for (int64_t i = threadIdx.x; i < k; i += 1024) out[i * ld_out + i] += add;
}

// out = sym(lerp(A, B, alpha)) with A = a, or a_scale * I when a is null.
// torch.lerp: start + w*(end-start) for w < 0.5, else end - (end-start)*(1-w).
__device__ __forceinline__ float lerp_torch(float s, float e, float w) {
  return w < 0.5f ? s + w * (e - s) : e - (e - s) * (1.0f - w);
}
__global__ __launch_bounds__(256) void sym_lerp_kernel(const float* __restrict__ a, float a_scale,
                                                       const float* __restrict__ b, int64_t k,
                                                       float alpha, float* __restrict__ out) {
  const int64_t i = blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= k) return;
  const float aij = a ? a[i * k + j] : (i == j ? a_scale : 0.0f);
  const float aji = a ? a[j * k + i] : (i == j ? a_scale : 0.0f);
  const float x = lerp_torch(aij, b[i * k + j], alpha);
  const float y = lerp_torch(aji, b[j * k + i], alpha);
  out[i * k + j] = (x + y) * 0.5f;
}

// Partial f64 sums of the diagonal and of all squares, one per workgroup.
__global__ __launch_bounds__(256) void cov_stats_partial_kernel(const float* __restrict__ h,
                                                                int64_t k, double* __restrict__ ws) {
  __shared__ double s_tr[256], s_sq[256];
  double tr = 0.0, sq = 0.0;
  const int64_t total = k * k;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const double v = (double)h[e];
    sq += v * v;
    if (e / k == e % k) tr += v;
  }
  s_tr[threadIdx.x] = tr;
  s_sq[threadIdx.x] = sq;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) {
      s_tr[threadIdx.x] += s_tr[threadIdx.x + w];
      s_sq[threadIdx.x] += s_sq[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    ws[2 * blockIdx.x] = s_tr[0];
    ws[2 * blockIdx.x + 1] = s_sq[0];
  }
}

__global__ __launch_bounds__(256) void cov_stats_final_kernel(const double* __restrict__ ws, int nparts,
                                                              double* __restrict__ out) {
  __shared__ double s_tr[256], s_sq[256];
  double tr = 0.0, sq = 0.0;
  for (int p = threadIdx.x; p < nparts; p += 256) {
    tr += ws[2 * p];
    sq += ws[2 * p + 1];
  }
  s_tr[threadIdx.x] = tr;
  s_sq[threadIdx.x] = sq;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) {
      s_tr[threadIdx.x] += s_tr[threadIdx.x + w];
      s_sq[threadIdx.x] += s_sq[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[0] = s_tr[0];
    out[1] = s_sq[0];
  }
}

// Grouped finalize: out[g] = sym(acc[g]) / denominators[g] (zeros when the
// group has no weight), blockIdx.y = group.
__global__ __launch_bounds__(256) void syrk_finalize_grouped_kernel(
    const float* __restrict__ acc, int64_t k, const double* __restrict__ denominators,
    float* __restrict__ out) {
  __shared__ float t[2][FIN_B][FIN_B + 1];
  const int64_t g = blockIdx.y;
  const double d = denominators[g];
  const float inv = d > 0.0 ? (float)(1.0 / d) : 0.0f;
  int64_t bi, bj;
  finalize_pair_of(blockIdx.x, bi, bj);
  finalize_pair(acc + g * k * k, k, k, inv, out + g * k * k, k, bi, bj, t);
}

// Per-group f64 sums of the row weights (of their fp32 squares with
// square_w; of 1 per row without weights): one workgroup per group, a fixed
// reduction tree, so the result is deterministic.
__global__ __launch_bounds__(256) void segment_weight_sum_kernel(const float* __restrict__ w,
                                                                 const int64_t* __restrict__ offsets,
                                                                 int square_w, double* __restrict__ out) {
  __shared__ double part[256];
  const int64_t g = blockIdx.x;
  const int64_t p0 = offsets[g], p1 = offsets[g + 1];
  double s = 0.0;
  for (int64_t p = p0 + threadIdx.x; p < p1; p += 256) {
    float v = w ? w[p] : 1.0f;
    if (square_w == 1) v = v * v;  // fp32 square, then f64 sum
    const double d = (double)v;
    s += square_w == 2 ? d * d : d;  // f64 square
  }
  part[threadIdx.x] = s;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if ((int)threadIdx.x < h) part[threadIdx.x] += part[threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[g] = part[0];
}

// Sums behind covariance_comparison (kquant/candidate_hessian.py:219-258), in
// f64 over fp32 [k, k] matrices R (reference) and C (candidate): per block
// {sum (C-R)^2 with C-R formed in fp32, sum R^2, tr R, tr C, sum diag R^2,
// sum diag C^2, sum diag R*C, max |C - C^T|}.
constexpr int CMP_PARTS = 256;
constexpr int CMP_FIELDS = 8;
__global__ __launch_bounds__(256) void cov_compare_partial_kernel(const float* __restrict__ r,
                                                                  const float* __restrict__ c, int64_t k,
                                                                  double* __restrict__ ws) {
  __shared__ double red[CMP_FIELDS][256];
  double f[CMP_FIELDS] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int64_t total = k * k;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)CMP_PARTS * 256) {
    const int64_t i = e / k, j = e - i * k;
    const float rv = r[e], cv = c[e];
    const double d = (double)(cv - rv);
    f[0] += d * d;
    f[1] += (double)rv * rv;
    if (i == j) {
      f[2] += rv;
      f[3] += cv;
      f[4] += (double)rv * rv;
      f[5] += (double)cv * cv;
      f[6] += (double)rv * cv;
    }
    f[7] = fmax(f[7], (double)fabsf(cv - c[j * k + i]));
  }
  const int t = threadIdx.x;
  for (int q = 0; q < CMP_FIELDS; ++q) red[q][t] = f[q];
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (t < w) {
      for (int q = 0; q < 7; ++q) red[q][t] += red[q][t + w];
      red[7][t] = fmax(red[7][t], red[7][t + w]);
    }
    __syncthreads();
  }
  if (t < CMP_FIELDS) ws[blockIdx.x * CMP_FIELDS + t] = red[t][0];
}

__global__ void cov_compare_final_kernel(const double* __restrict__ ws, double* __restrict__ out) {
  if (threadIdx.x != 0) return;
  double f[CMP_FIELDS] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int b = 0; b < CMP_PARTS; ++b) {
    for (int q = 0; q < 7; ++q) f[q] += ws[b * CMP_FIELDS + q];
    f[7] = fmax(f[7], ws[b * CMP_FIELDS + 7]);
  }
  for (int q = 0; q < CMP_FIELDS; ++q) out[q] = f[q];
}

}  // namespace kq

using namespace kq;

extern "C" int kq_sym_lerp(const float* a, float a_scale, const float* b, int64_t k, float alpha,
                           float* out, void* stream) {
  if (k <= 0 || b == nullptr || out == nullptr)
    return kq_fail(KQ_ERR_INVALID, "kq_sym_lerp: bad arguments (k=%lld)", (long long)k);
  if (out == b || (a != nullptr && out == a))
    return kq_fail(KQ_ERR_INVALID, "kq_sym_lerp: out must not alias the inputs");
  sym_lerp_kernel<<<dim3((unsigned)((k + 255) / 256), (unsigned)k), 256, 0, (hipStream_t)stream>>>(
      a, a_scale, b, k, alpha, out);
  return kq_check_launch(hipGetLastError(), "kq_sym_lerp");
}

extern "C" int kq_cov_stats(const float* h, int64_t k, double* workspace, double* out,
                            void* stream) {
  if (k <= 0) return kq_fail(KQ_ERR_INVALID, "kq_cov_stats: k must be positive");
  hipStream_t st = (hipStream_t)stream;
  cov_stats_partial_kernel<<<KQ_COV_STATS_PARTS, 256, 0, st>>>(h, k, workspace);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return kq_check_launch(e, "kq_cov_stats");
  cov_stats_final_kernel<<<1, 256, 0, st>>>(workspace, KQ_COV_STATS_PARTS, out);
  return kq_check_launch(hipGetLastError(), "kq_cov_stats");
}

template <int IN, bool SPLIT, bool WEIGHTED, bool GROUPED>
static hipError_t launch_syrk(const void* x, int64_t ld, int64_t n, int64_t k, const float* w,
                              float* acc, int64_t ld_acc, int overwrite, hipStream_t st,
                              const int64_t* offsets = nullptr, const int32_t* index = nullptr,
                              int groups = 1, int square_w = 0) {
  const int nt = (int)((k + syrk::TILE - 1) / syrk::TILE);
  const int ntiles = nt * (nt + 1) / 2;
  const int nslab = SPLIT ? 4 : 2;
  const size_t lds = (size_t)2 * nslab * syrk::SLAB_BYTES;
  auto kern = syrk_upper_kernel<IN, SPLIT, WEIGHTED, GROUPED>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  kern<<<dim3(ntiles, groups), dim3(256), lds, st>>>(x, ld, n, k, w, acc, ld_acc, nt, overwrite, offsets,
                                                     index, k * ld_acc, square_w);
  return hipGetLastError();
}

// The direct-load kernel serves unweighted bf16 rows whose byte range fits
// the buffer descriptor's 32-bit offsets.
static bool dma_syrk(int in_dtype, const void* weights, int64_t n, int64_t ld) {
  return in_dtype == KQ_DT_BF16 && !weights && n * ld * 2 < ((int64_t)1 << 32) - 4096;
}

static int syrk_accumulate(int in_dtype, const void* x, int64_t ld, int64_t n, int64_t k, const float* weights,
                           float* acc, int64_t ld_acc, uint32_t flags, void* workspace, int64_t ws_bytes,
                           void* stream);

extern "C" int64_t kq_syrk_accumulate_workspace_size(int in_dtype, int64_t n, int64_t k, int weighted) {
  if (n < 0 || k <= 0) return -1;
  // rows assumed dense (ld == k); a call with a wider ld whose rows pass the
  // 4 GiB range of the direct loads takes the path without a workspace
  if (!dma_syrk(in_dtype, weighted ? (const void*)1 : nullptr, n, k)) return 0;
  const int nt = (int)((k + syrk3::TILE - 1) / syrk3::TILE);
  return tail_slot_bytes(plan_tail(nt * (nt + 1) / 2, device_cus(), n));
}

extern "C" int kq_syrk_accumulate_ws(int in_dtype, const void* x, int64_t ld, int64_t n, int64_t k,
                                     const float* weights, float* acc, int64_t ld_acc, uint32_t flags,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  if (workspace && (workspace_bytes < 0 || kq_misaligned(workspace, 256)))
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_accumulate_ws: workspace must be 256-byte aligned");
  return syrk_accumulate(in_dtype, x, ld, n, k, weights, acc, ld_acc, flags, workspace, workspace_bytes, stream);
}

extern "C" int kq_syrk_accumulate(int in_dtype, const void* x, int64_t ld, int64_t n, int64_t k,
                                  const float* weights, float* acc, int64_t ld_acc, uint32_t flags,
                                  void* stream) {
  return syrk_accumulate(in_dtype, x, ld, n, k, weights, acc, ld_acc, flags, nullptr, 0, stream);
}

static int syrk_accumulate(int in_dtype, const void* x, int64_t ld, int64_t n, int64_t k, const float* weights,
                           float* acc, int64_t ld_acc, uint32_t flags, void* workspace, int64_t ws_bytes,
                           void* stream) {
  if (in_dtype < KQ_DT_BF16 || in_dtype > KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_accumulate: unknown input dtype %d", in_dtype);
  if (n < 0 || k <= 0 || k % 8 != 0 || ld < k || ld % 8 != 0 || ld_acc < k)
    return kq_fail(KQ_ERR_INVALID,
                   "kq_syrk_accumulate: need k > 0, k %% 8 == 0, ld >= k, ld %% 8 == 0, ld_acc >= k "
                   "(n=%lld k=%lld ld=%lld ld_acc=%lld)",
                   (long long)n, (long long)k, (long long)ld, (long long)ld_acc);
  if (kq_misaligned(x, 16))
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_accumulate: rows must be 16-byte aligned");
  if (k > (int64_t)1 << 20)
    return kq_fail(KQ_ERR_LIMIT, "kq_syrk_accumulate: k=%lld exceeds 2^20", (long long)k);
  const int overwrite = (flags & KQ_SYRK_OVERWRITE) ? 1 : 0;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  const bool weighted = weights != nullptr;
  if (in_dtype == KQ_DT_BF16) {
    if (weighted)
      e = launch_syrk256<true, false>(x, ld, n, k, weights, acc, ld_acc, overwrite, st);
    else if (dma_syrk(in_dtype, weights, n, ld))
      e = launch_syrk256_dma(x, ld, n, k, acc, ld_acc, overwrite, st, workspace, ws_bytes);
    else
      e = launch_syrk256<false, false>(x, ld, n, k, weights, acc, ld_acc, overwrite, st);
  } else if (in_dtype == KQ_DT_F16) {
    e = weighted ? launch_syrk<1, true, true, false>(x, ld, n, k, weights, acc, ld_acc, overwrite, st)
                 : launch_syrk<1, true, false, false>(x, ld, n, k, weights, acc, ld_acc, overwrite, st);
  } else {
    e = weighted ? launch_syrk<2, true, true, false>(x, ld, n, k, weights, acc, ld_acc, overwrite, st)
                 : launch_syrk<2, true, false, false>(x, ld, n, k, weights, acc, ld_acc, overwrite, st);
  }
  return kq_check_launch(e, "kq_syrk_accumulate");
}

extern "C" int kq_syrk_finalize(const float* acc, int64_t ld_acc, int64_t k, double denominator,
                                float damp, float* out, int64_t ld_out, void* stream) {
  if (k <= 0 || ld_acc < k || ld_out < k)
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_finalize: bad sizes (k=%lld)", (long long)k);
  if (!(denominator > 0.0))
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_finalize: denominator must be positive");
  if (k > (int64_t)1 << 20)
    return kq_fail(KQ_ERR_LIMIT, "kq_syrk_finalize: k=%lld exceeds 2^20", (long long)k);
  if (acc == out && ld_acc != ld_out)
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_finalize: in-place needs ld_acc == ld_out");
  if (acc == out)
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_finalize: acc and out must not alias");
  hipStream_t st = (hipStream_t)stream;
  const float inv = (float)(1.0 / denominator);
  const int64_t nb = (k + FIN_B - 1) / FIN_B;
  syrk_finalize_kernel<<<(unsigned)(nb * (nb + 1) / 2), 256, 0, st>>>(acc, ld_acc, k, inv, out, ld_out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return kq_check_launch(e, "kq_syrk_finalize");
  if (damp != 0.0f) {
    syrk_damp_kernel<<<1, 1024, 0, st>>>(out, ld_out, k, damp);
    e = hipGetLastError();
  }
  return kq_check_launch(e, "kq_syrk_finalize");
}

extern "C" int kq_syrk_grouped(int in_dtype, const void* x, int64_t ld, const int64_t* offsets,
                               int groups, const int32_t* row_index, const float* weights, int64_t k,
                               float* acc, uint32_t flags, void* stream) {
  if (in_dtype < KQ_DT_BF16 || in_dtype > KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_grouped: unknown input dtype %d", in_dtype);
  if (groups < 1 || groups > 65535 || k <= 0 || k % 8 != 0 || ld < k || ld % 8 != 0 || !offsets)
    return kq_fail(KQ_ERR_INVALID,
                   "kq_syrk_grouped: need 1 <= groups <= 65535, k %% 8 == 0, ld >= k, ld %% 8 == 0 "
                   "(groups=%d k=%lld ld=%lld)", groups, (long long)k, (long long)ld);
  if (kq_misaligned(x, 16) || kq_misaligned(offsets, 8) || kq_misaligned(row_index, 4) ||
      kq_misaligned(weights, 4))
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_grouped: misaligned rows, offsets, index or weights");
  if (k > 16384) return kq_fail(KQ_ERR_LIMIT, "kq_syrk_grouped: k=%lld exceeds 16384", (long long)k);
  const int sq = (flags & KQ_SYRK_SQUARE_WEIGHTS) ? 1 : 0;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  const bool weighted = weights != nullptr;
  if (in_dtype == KQ_DT_BF16)
    e = weighted && !row_index
            ? launch_syrk256w_dma(x, ld, k, weights, acc, offsets, groups, sq, st)
        : weighted ? launch_syrk256<true, true>(x, ld, 0, k, weights, acc, k, 1, st, offsets, row_index, groups, sq)
                 : launch_syrk256<false, true>(x, ld, 0, k, weights, acc, k, 1, st, offsets, row_index, groups, sq);
  else if (in_dtype == KQ_DT_F16)
    e = weighted ? launch_syrk<1, true, true, true>(x, ld, 0, k, weights, acc, k, 1, st, offsets, row_index, groups, sq)
                 : launch_syrk<1, true, false, true>(x, ld, 0, k, weights, acc, k, 1, st, offsets, row_index, groups, sq);
  else
    e = weighted ? launch_syrk<2, true, true, true>(x, ld, 0, k, weights, acc, k, 1, st, offsets, row_index, groups, sq)
                 : launch_syrk<2, true, false, true>(x, ld, 0, k, weights, acc, k, 1, st, offsets, row_index, groups, sq);
  return kq_check_launch(e, "kq_syrk_grouped");
}

extern "C" int kq_segment_weight_sums(const float* weights, const int64_t* offsets, int groups,
                                      uint32_t flags, double* out, void* stream) {
  if (groups < 1 || !offsets || !out || kq_misaligned(offsets, 8) || kq_misaligned(out, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_segment_weight_sums: bad arguments");
  const int mode = (flags & KQ_SUM_SQUARE_F64) ? 2 : (flags & KQ_SYRK_SQUARE_WEIGHTS) ? 1 : 0;
  segment_weight_sum_kernel<<<groups, 256, 0, (hipStream_t)stream>>>(weights, offsets, mode, out);
  return kq_check_launch(hipGetLastError(), "kq_segment_weight_sums");
}

extern "C" int kq_syrk_finalize_grouped(const float* acc, int64_t k, int groups,
                                        const double* denominators, float* out, void* stream) {
  if (k <= 0 || groups < 1 || groups > 65535 || !denominators)
    return kq_fail(KQ_ERR_INVALID, "kq_syrk_finalize_grouped: bad sizes (k=%lld groups=%d)",
                   (long long)k, groups);
  if (acc == out) return kq_fail(KQ_ERR_INVALID, "kq_syrk_finalize_grouped: acc and out must not alias");
  if (k > 65535) return kq_fail(KQ_ERR_LIMIT, "kq_syrk_finalize_grouped: k too large");
  hipStream_t st = (hipStream_t)stream;
  const int64_t nb = (k + FIN_B - 1) / FIN_B;
  syrk_finalize_grouped_kernel<<<dim3((unsigned)(nb * (nb + 1) / 2), (unsigned)groups), 256, 0, st>>>(
      acc, k, denominators, out);
  return kq_check_launch(hipGetLastError(), "kq_syrk_finalize_grouped");
}

extern "C" int kq_covariance_comparison_sums(const float* reference, const float* candidate, int64_t k,
                                             double* workspace, double* out, void* stream) {
  if (k <= 0 || !reference || !candidate || kq_misaligned(workspace, 8) || kq_misaligned(out, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_covariance_comparison_sums: bad arguments");
  hipStream_t st = (hipStream_t)stream;
  cov_compare_partial_kernel<<<CMP_PARTS, 256, 0, st>>>(reference, candidate, k, workspace);
  cov_compare_final_kernel<<<1, 64, 0, st>>>(workspace, out);
  return kq_check_launch(hipGetLastError(), "kq_covariance_comparison_sums");
}
