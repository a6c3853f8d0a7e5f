// Hessian finalize of the trellis encoder on MI355X
// (kquant/exl3_encoder_backend.py:316-386 block_ldl, :1588-1663
// finalize_capture_H): diagonal regularization, sign flips with a blockwise
// Hadamard rotation, a batched blocked Cholesky and the block LDL built on it.
//
//  * regularize: H *= 1/count (fp32 reciprocal, as torch divides a tensor by
//    a host scalar), then diag += sigma * mean(diag) with the mean summed in
//    f64; the regularized diagonal and its mean are returned.
//  * rotation: B S_r X S_c B with B = blockdiag(Had_128 / sqrt(128)), the
//    Sylvester Hadamard of kquant/exl3_reference.py:195-212.  B is block
//    diagonal, so every 128x128 tile of X transforms on its own: one
//    workgroup per tile, a fast Walsh-Hadamard transform along the rows and /
//    or columns in LDS (adds only), then one scale (1/128 exactly for both
//    sides, fl(1/sqrt(128)) for one).
//  * Cholesky (lower, fp32): blocked over 64-column panels grouped into
//    super-panels (four panels for batches of 8 and more, else one), all
//    matrices of a batch per launch.  Within a super-panel one launch per
//    panel brings its block column up to date with the super-panel's earlier
//    panels and computes the panel below the diagonal as A21 inv(L11)^T;
//    diagonal blocks are factored and inverted by one wave in registers, by
//    the workgroup that completes them.  One update A22 -= L21 L21^T over
//    the super-panel's columns then covers the trailing matrix.  Products on
//    v_mfma_f32_16x16x4f32 from LDS.  A failing pivot (<= 0 or NaN) records
//    the leading-minor order in info (LAPACK's convention) and the
//    factorization continues with pivot 1, so every launch still completes.
//  * block LDL: every b x b diagonal block DL_i of L is inverted, each block
//    column multiplied by its inverse and the diagonal blocks set to I.
#include "kq_dma.h"
#include "kq_hadamard.h"
#include "kq_internal.h"

namespace kq {
namespace ldl {

using kq::had::fwht_lines;
using kq::had::fwht128;
using kq::had::HAD;
using kq::had::HLD;

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int NB = 64;     // Cholesky panel
constexpr int LD = 68;     // padded LDS row: lane (i, k) of an MFMA read hits bank 4 i + k
constexpr int MAX_B = 64;  // block LDL block size limit

// ------------------------------------------------------------ regularize --
__global__ __launch_bounds__(256) void diag_mean_kernel(const float* __restrict__ h, int64_t k, int64_t ld,
                                                        float inv, float* __restrict__ mean_out) {
  __shared__ double part[256];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < k; i += 256) s += (double)(h[i * ld + i] * inv);
  part[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) mean_out[0] = (float)(part[0] / (double)k);
}

__global__ __launch_bounds__(256) void regularize_kernel(float* __restrict__ h, int64_t k, int64_t ld, float inv,
                                                         float sigma, const float* __restrict__ mean,
                                                         float* __restrict__ diag_out) {
  const int64_t i = blockIdx.y, j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= k) return;
  float v = h[i * ld + j];
  if (inv != 1.f) v *= inv;
  if (i == j) {
    v += sigma * mean[0];
    if (diag_out) diag_out[i] = v;
  }
  h[i * ld + j] = v;
}

// --------------------------------------------------------------- rotation --
// sides: bit 0 = left (B X: each column of a tile transformed), bit 1 = right
// (X B: each row).  Row / column scales (or none) apply before the transforms.
__global__ __launch_bounds__(1024) void hadamard_kernel(float* __restrict__ x, int64_t rows, int64_t cols,
                                                        int64_t ld, int64_t stride, int sides,
                                                        const float* __restrict__ rs,
                                                        const float* __restrict__ cs, float post, int vec) {
  // one 128 x 128 block per workgroup: 16-byte loads (vec: ld and the block
  // 16-byte aligned) or single ones at ragged edges, both scales at load,
  // then 8 independent lines per wave per direction with the wave-level
  // transform, and the post scale at store
  __shared__ float t[HAD][HLD];
  float* X = x + (int64_t)blockIdx.z * stride;
  const int64_t r0 = (int64_t)blockIdx.y * HAD, c0 = (int64_t)blockIdx.x * HAD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool full = vec && r0 + HAD <= rows && c0 + HAD <= cols;
  if (full) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int i = tid + 1024 * it, r = i >> 5, c = (i & 31) * 4;
      float4 v = *reinterpret_cast<const float4*>(X + (r0 + r) * ld + c0 + c);
      if (rs) {
        const float s = rs[r0 + r];
        v.x *= s; v.y *= s; v.z *= s; v.w *= s;
      }
      if (cs) {
        const float4 s = *reinterpret_cast<const float4*>(cs + c0 + c);
        v.x *= s.x; v.y *= s.y; v.z *= s.z; v.w *= s.w;
      }
      t[r][c] = v.x; t[r][c + 1] = v.y; t[r][c + 2] = v.z; t[r][c + 3] = v.w;
    }
  } else {
    for (int i = tid; i < HAD * HAD; i += 1024) {
      const int r = i >> 7, c = i & (HAD - 1);
      float v = 0.f;
      if (r0 + r < rows && c0 + c < cols) {
        v = X[(r0 + r) * ld + c0 + c];
        if (rs) v *= rs[r0 + r];
        if (cs) v *= cs[c0 + c];
      }
      t[r][c] = v;
    }
  }
  __syncthreads();
  if (sides & 2) {  // every row
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = wave + 16 * i;
      float v0 = t[r][lane], v1 = t[r][lane + 64];
      fwht128(v0, v1, lane);
      t[r][lane] = v0;
      t[r][lane + 64] = v1;
    }
    __syncthreads();
  }
  if (sides & 1) {  // every column
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = wave + 16 * i;
      float v0 = t[lane][c], v1 = t[lane + 64][c];
      fwht128(v0, v1, lane);
      t[lane][c] = v0;
      t[lane + 64][c] = v1;
    }
    __syncthreads();
  }
  if (full) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int i = tid + 1024 * it, r = i >> 5, c = (i & 31) * 4;
      const float4 v = {t[r][c] * post, t[r][c + 1] * post, t[r][c + 2] * post, t[r][c + 3] * post};
      *reinterpret_cast<float4*>(X + (r0 + r) * ld + c0 + c) = v;
    }
  } else {
    for (int i = tid; i < HAD * HAD; i += 1024) {
      const int r = i >> 7, c = i & (HAD - 1);
      if (r0 + r < rows && c0 + c < cols) X[(r0 + r) * ld + c0 + c] = t[r][c] * post;
    }
  }
}

// --------------------------------------------------------------- Cholesky --
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// The workgroup's 256 threads (4 waves) factor the 64 x 64 block a (LDS;
// rows past the matrix padded with the identity) into L, written back to a
// with zeros above the diagonal, and write inv(L) to xi.  By 16-column
// panels, right-looking; per panel:
//  * wave 0 factors the 16 x 16 diagonal block: lane r holds row r, column
//    c is broadcast from lane c with readlane, and each step takes the
//    pivot's reciprocal square root (hardware v_rsq: within an ulp or two,
//    far inside the factorization's own rounding), scales the column by it
//    and updates the trailing columns with one FMA per entry; then lane j
//    solves column j of the block's inverse X by forward substitution, the
//    rows of L broadcast the same way;
//  * the rows below take L21 = A21 X^T and the trailing lower tiles
//    A22 -= L21 L21^T, both on v_mfma_f32_16x16x4f32, a 16 x 16 tile per
//    wave.
// The off-diagonal blocks of inv(L) follow by block rows i = 1, 2, 3:
// X[i][j] = -X[i][i] (sum over k = j .. i - 1 of L[i][k] X[k][j]) on the
// MFMAs, one block per wave; rows 1 and 2 on waves 1 .. i while wave 0
// factors the next diagonal block, row 3 after the last one.  Returns (uniformly) the first failing
// column + 1, or 0; a failing pivot is replaced by 1.  Ends with a barrier:
// a and xi are complete for every thread.
__device__ __forceinline__ int factor64_wg(float (*a)[LD], float (*xi)[LD]) {
  constexpr int PB = 16;  // panel width
  __shared__ float tb[3][PB][PB + 1];
  __shared__ float dg[2][PB];  // L[c][c] and 1 / L[c][c] of the current diagonal block
  __shared__ int s_bad;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lk = lane >> 4;  // v_mfma_f32_16x16x4f32 operand position
  // block (i, j) of inv(L), j < i, on the calling wave: X[i][j] = -X[i][i] T with
  // T = sum over k = j .. i - 1 of L[i][k] X[k][j]
  auto inv_block = [&](int i, int j) {
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int k = j; k < i; ++k) {
#pragma unroll
      for (int u = 0; u < PB; u += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[PB * i + li][PB * k + u + lk], xi[PB * k + u + lk][PB * j + li],
                                                   acc, 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) tb[j][4 * lk + q][li] = acc[q];
    // one wave's LDS accesses complete in order: the T it stored is read back below
    f32x4_t x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < PB; u += 4)
      x = __builtin_amdgcn_mfma_f32_16x16x4f32(xi[PB * i + li][PB * i + u + lk], tb[j][u + lk][li], x, 0, 0, 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) xi[PB * i + 4 * lk + q][PB * j + li] = -x[q];
  };
  if (tid == 0) s_bad = 0;
  // zeros above the diagonal blocks of xi (the blocks themselves are written whole)
  for (int e = tid; e < NB * NB; e += 256) {
    const int rr = e / NB, cc = e % NB;
    if ((cc >> 4) > (rr >> 4)) xi[rr][cc] = 0.f;
  }
  __syncthreads();
  for (int p = 0; p < NB / PB; ++p) {
    const int c0 = PB * p;
    if (wave == 0) {
      float v[PB];
#pragma unroll
      for (int c = 0; c < PB; ++c) v[c] = a[c0 + li][c0 + c];
      int bad = 0;
#pragma unroll
      for (int c = 0; c < PB; ++c) {
        float d = readlane_f(v[c], c);
        if (!(d > 0.f)) {
          if (bad == 0) bad = c0 + c + 1;
          d = 1.f;
        }
        const float rs = __builtin_amdgcn_rsqf(d);  // 1 / L[c][c]
        dg[0][c] = d * rs;                          // L[c][c] (every lane stores the same value)
        dg[1][c] = rs;
        v[c] *= rs;  // L[r][c] for r > c (row c's diagonal is in dg)
#pragma unroll
        for (int q = c + 1; q < PB; ++q) v[q] = fmaf(-v[c], readlane_f(v[c], q), v[q]);
      }
      if (lane < PB) {
        const float dv = dg[0][li];
#pragma unroll
        for (int c = 0; c < PB; ++c) a[c0 + li][c0 + c] = c < li ? v[c] : (c == li ? dv : 0.f);
      }
      // column li of the block's inverse: x[i] = (delta - sum_{k<i} L[i][k] x[k]) / L[i][i]
      float x[PB];
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        float acc = i == li ? 1.f : 0.f;
#pragma unroll
        for (int k = 0; k < i; ++k) acc = fmaf(-readlane_f(v[k], i), x[k], acc);
        x[i] = acc * dg[1][i];
      }
      if (lane < PB) {
#pragma unroll
        for (int i = 0; i < PB; ++i) xi[c0 + i][c0 + li] = x[i];
      }
      if (lane == 0 && bad != 0 && s_bad == 0) s_bad = bad;
    } else if (p >= 2 && wave < p) {
      // meanwhile block row p - 1 of inv(L): its L blocks and X[p - 1][p - 1] are done
      inv_block(p - 1, wave - 1);
    }
    __syncthreads();
    // the panel below: L21 = A21 X^T, row tile w (rows c0 + 16 (1 + w) ..) on wave w
    const int nt = NB / PB - 1 - p;
    f32x4_t l21 = {0.f, 0.f, 0.f, 0.f};
    if (wave < nt) {
      const int r0 = c0 + PB * (1 + wave);
#pragma unroll
      for (int k = 0; k < PB; k += 4)
        l21 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r0 + li][c0 + k + lk], xi[c0 + li][c0 + k + lk], l21, 0, 0,
                                                   0);
    }
    __syncthreads();  // every wave has read A21
    if (wave < nt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) a[c0 + PB * (1 + wave) + 4 * lk + j][c0 + li] = l21[j];
    }
    __syncthreads();
    // trailing lower tiles (ti >= tj) -= L21[ti] L21[tj]^T
    for (int t = wave; t < nt * (nt + 1) / 2; t += 4) {
      int ti = 0;
      while ((ti + 1) * (ti + 2) / 2 <= t) ++ti;
      const int tj = t - ti * (ti + 1) / 2;
      const int r0 = c0 + PB * (1 + ti), q0 = c0 + PB * (1 + tj);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < PB; k += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r0 + li][c0 + k + lk], a[q0 + li][c0 + k + lk], acc, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) a[r0 + 4 * lk + j][q0 + li] -= acc[j];
    }
    __syncthreads();
  }
  // zeros above the diagonal of L (the diagonal blocks' upper parts are zero already)
  for (int e = tid; e < NB * NB; e += 256) {
    const int rr = e / NB, cc = e % NB;
    if ((cc >> 4) > (rr >> 4)) a[rr][cc] = 0.f;
  }
  // the last block row of inv(L)
  if (wave < NB / PB - 1) inv_block(NB / PB - 1, wave);
  __syncthreads();
  return s_bad;
}

// Stores of factor64_wg's results by all 256 threads.  AGENT: inv(L) goes
// out as agent-scope atomic stores (written through the XCD's L2), for
// workgroups of the same launch on other XCDs.
template <bool AGENT = false>
__device__ __forceinline__ void store_diag_wg(float (*a)[LD], float (*xi)[LD], float* L, int64_t ldl, int64_t c0,
                                              int nb, float* W, int bad, int* info) {
  for (int i = threadIdx.x; i < NB * NB; i += 256) {
    const int r = i / NB, c = i % NB;
    if (r < nb && c < nb) L[(c0 + r) * ldl + c0 + c] = a[r][c];
    if (AGENT) __hip_atomic_store(W + i, xi[r][c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else W[i] = xi[r][c];
  }
  if (threadIdx.x == 0 && bad != 0 && *info == 0) *info = (int)(c0 + bad);
}

// L = tril(A) (upper part zero); info = 0.  a and l may be the same buffer.
__global__ __launch_bounds__(256) void chol_init_kernel(const float* a, int64_t lda, int64_t sa, float* l,
                                                        int64_t ldl, int64_t sl, int64_t n, int* __restrict__ info,
                                                        int* __restrict__ diag_done) {
  const int64_t b = blockIdx.z, i = blockIdx.y, j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i == 0 && j == 0) {
    info[b] = 0;
    diag_done[b] = -1;
  }
  if (j >= n) return;
  const float v = j <= i ? a[b * sa + i * lda + j] : 0.f;
  l[b * sl + i * ldl + j] = v;
}

// inv(L11) of panel p lives in slot p % 2 of the matrix's two winv slots
// (winv + (2 b + p % 2) 64 x 64): a launch reads one slot while its
// diagonal-factoring workgroup writes the other.
//
// Factor the diagonal block of panel 0 (one workgroup per matrix; the later
// panels' diagonal blocks are factored by the launch that finishes them),
// writing L11 back (zeros above its diagonal) and inv(L11) to slot 0.
__global__ __launch_bounds__(256) void chol_diag_kernel(float* __restrict__ l, int64_t n, int64_t ldl, int64_t sl,
                                                        float* __restrict__ winv, int* __restrict__ info) {
  __shared__ float a[NB][LD];
  __shared__ float xi[NB][LD];
  const int64_t b = blockIdx.x;
  float* L = l + b * sl;
  const int nb = (int)(n < NB ? n : NB);
  for (int i = threadIdx.x; i < NB * NB; i += 256) {
    const int r = i / NB, c = i % NB;
    a[r][c] = (r < nb && c < nb) ? (c <= r ? L[r * ldl + c] : 0.f) : (r == c ? 1.f : 0.f);
  }
  __syncthreads();
  const int bad = factor64_wg(a, xi);
  store_diag_wg(a, xi, L, ldl, 0, nb, winv + b * 2 * NB * NB, bad, info + b);
}

// acc (this wave's 32x32 of a 64x64 tile, as 2x2 16x16 blocks) += X Y^T over
// k < NB, X and Y row-major in LDS.  v_mfma_f32_16x16x4f32: lane l gives
// A[l % 16][l / 16] and B[l / 16][l % 16]; D block rows 4 (l / 16) + j,
// column l % 16.
__device__ __forceinline__ void mm_nt(const float (*X)[LD], const float (*Y)[LD], f32x4_t acc[2][2]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rb = 32 * (wave >> 1), cb = 32 * (wave & 1);
  const int li = lane & 15, lk = lane >> 4;
#pragma unroll 4
  for (int k = 0; k < NB; k += 4) {
    const float a0 = X[rb + li][k + lk], a1 = X[rb + 16 + li][k + lk];
    const float b0 = Y[cb + li][k + lk], b1 = Y[cb + 16 + li][k + lk];
    acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
    acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
    acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
    acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
  }
}

// Load rows [r0, r0 + 64) x cols [c0, c0 + 64) of M (zero past n): 16-byte
// loads when the tile's columns are all in range and rows 16-byte aligned.
__device__ __forceinline__ void load_tile(float (*T)[LD], const float* M, int64_t ld, int64_t n, int64_t r0,
                                          int64_t c0) {
  if (c0 + NB <= n && ld % 4 == 0 && (reinterpret_cast<uintptr_t>(M) & 15) == 0) {
    for (int i = threadIdx.x; i < NB * NB / 4; i += 256) {
      const int r = i / (NB / 4), c = 4 * (i % (NB / 4));
      f32x4_t v = {0.f, 0.f, 0.f, 0.f};
      if (r0 + r < n) v = *reinterpret_cast<const f32x4_t*>(M + (r0 + r) * ld + c0 + c);
      T[r][c] = v[0];
      T[r][c + 1] = v[1];
      T[r][c + 2] = v[2];
      T[r][c + 3] = v[3];
    }
    return;
  }
  for (int i = threadIdx.x; i < NB * NB; i += 256) {
    const int r = i / NB, c = i % NB;
    T[r][c] = (r0 + r < n && c0 + c < n) ? M[(r0 + r) * ld + c0 + c] : 0.f;
  }
}

// The lane's (row, column) in a 64 x 64 tile for acc[bi][bj][q] of mm_nt.
__device__ __forceinline__ void mm_pos(int bi, int bj, int q, int& r, int& c) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  r = 32 * (wave >> 1) + 16 * bi + 4 * (lane >> 4) + q;
  c = 32 * (wave & 1) + 16 * bj + (lane & 15);
}

// Panel p of the super-panel [s0, s1), row block i = p + 1 + blockIdx.x:
// A[i, p] -= sum over q in [s0, p) of L[i, q] L[p, q]^T (the updates of the
// super-panel's earlier panels, left-looking), then L[i, p] = A[i, p]
// inv(L[p, p])^T.  The workgroup of row block p + 1, when that is still in
// the super-panel, then brings the diagonal block (p + 1, p + 1) up to date
// with panels s0 .. p and factors it.
__global__ __launch_bounds__(256) void chol_panel_kernel(float* __restrict__ l, int64_t n, int64_t ldl, int64_t sl,
                                                         int p, int s0, int s1, float* __restrict__ winv,
                                                         int* __restrict__ info) {
  __shared__ float av[NB][LD];
  __shared__ float xi[NB][LD];
  __shared__ float xj[NB][LD];
  const int64_t b = blockIdx.y;
  float* L = l + b * sl;
  const int64_t r0 = (int64_t)(p + 1 + blockIdx.x) * NB, c0 = (int64_t)p * NB;
  f32x4_t acc[2][2] = {};
  for (int q = s0; q < p; ++q) {
    if (q > s0) __syncthreads();
    load_tile(xi, L, ldl, n, r0, (int64_t)q * NB);
    load_tile(xj, L, ldl, n, c0, (int64_t)q * NB);
    __syncthreads();
    mm_nt(xi, xj, acc);
  }
  load_tile(av, L, ldl, n, r0, c0);
  const float* W = winv + (b * 2 + (p & 1)) * NB * NB;
  __syncthreads();  // every wave is done with xi / xj; av is loaded
  for (int i = threadIdx.x; i < NB * NB; i += 256) xi[i / NB][i % NB] = W[i];
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int r, c;
        mm_pos(bi, bj, q, r, c);
        av[r][c] -= acc[bi][bj][q];
      }
  __syncthreads();
  f32x4_t lp[2][2] = {};
  mm_nt(av, xi, lp);
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int r, c;
        mm_pos(bi, bj, q, r, c);
        if (r0 + r < n && c0 + c < n) L[(r0 + r) * ldl + c0 + c] = lp[bi][bj][q];
      }
  if (blockIdx.x != 0 || p + 1 >= s1) return;
  // diagonal block p + 1: A[p + 1, p + 1] -= sum over q in [s0, p] of
  // L[p + 1, q] L[p + 1, q]^T, where L[p + 1, p] is this workgroup's lp
  __syncthreads();  // every wave is done reading av / xi
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int r, c;
        mm_pos(bi, bj, q, r, c);
        av[r][c] = lp[bi][bj][q];  // rows past n are zero (their A rows are)
      }
  __syncthreads();
  f32x4_t dg[2][2] = {};
  mm_nt(av, av, dg);
  for (int q = s0; q < p; ++q) {
    __syncthreads();
    load_tile(xi, L, ldl, n, r0, (int64_t)q * NB);
    __syncthreads();
    mm_nt(xi, xi, dg);
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int r, c;
        mm_pos(bi, bj, q, r, c);
        xi[r][c] = (r0 + r < n && r0 + c < n) ? L[(r0 + r) * ldl + r0 + c] - dg[bi][bj][q] : (r == c ? 1.f : 0.f);
      }
  __syncthreads();
  const int bad = factor64_wg(xi, xj);
  const int nb = (int)(n - r0 < NB ? n - r0 : NB);
  store_diag_wg(xi, xj, L, ldl, r0, nb, winv + (b * 2 + ((p + 1) & 1)) * NB * NB, bad, info + b);
}

// Trailing update A[bi, bj] -= sum over panels q in [q0, q1) of
// L[bi, q] L[bj, q]^T over the lower tiles bi >= bj >= b0 (blockIdx.x
// enumerates them row by row; the panels' products are summed in registers,
// so A is read and written once).  The workgroup of tile (b0, b0) then
// factors it as panel b0's diagonal block.
// DMA (n and ldl multiples of 64 and 4, l 16-byte aligned): the panel
// tiles of two panels in flight at once, by direct loads into a two-slot LDS
// ring (32 KiB a slot: the two 64 x 64 tiles, 256-byte rows with 16-byte
// chunk c of row r at chunk c ^ (r % 16)), read as 128-bit fragments: lane
// (i, k) of a 16-wide k block reads floats 4k .. 4k + 3 of its row, and
// MFMA e of the block takes the lane's float e, so a 16 x 16 x 4 product
// sums k values k0 + 4 lk + e (any order of k sums the same products).  Two
// workgroups per CU; the other form keeps four with padded tiles loaded
// through registers.
namespace dup {
constexpr int SLOT = 2 * NB * NB * 4;  // bytes: xi and xj
constexpr int LOADS = 8;               // direct loads per wave per slot
}  // namespace dup

template <bool DMA>
__global__ __launch_bounds__(256, DMA ? 2 : 4) void chol_update_kernel(float* __restrict__ l, int64_t n, int64_t ldl,
                                                                     int64_t sl, int b0, int q0, int q1,
                                                                     float* __restrict__ winv, int* __restrict__ info,
                                                                     int* __restrict__ diag_done, int column_only) {
  __shared__ __attribute__((aligned(16))) float ring[DMA ? 2 * dup::SLOT / 4 : 2 * NB * LD];
  static_assert(2 * NB * LD * 4 <= (DMA ? 2 * dup::SLOT : 2 * NB * LD * 4), "padded tiles alias the ring");
  float (*xi)[LD] = reinterpret_cast<float (*)[LD]>(ring);
  float (*xj)[LD] = reinterpret_cast<float (*)[LD]>(ring + NB * LD);
  const int64_t b = blockIdx.y;
  float* L = l + b * sl;
  const int64_t t = blockIdx.x;
  // tile t: (i, j) of the trailing lower triangle, or (t, 0) of its first
  // block column only
  int64_t i = t, j = 0;
  if (!column_only) {
    i = (int64_t)((sqrt(8.0 * (double)t + 1.0) - 1.0) * 0.5);
    while ((i + 1) * (i + 2) / 2 <= t) ++i;
    while (i * (i + 1) / 2 > t) --i;
    j = t - i * (i + 1) / 2;
  }
  const int64_t ri = (int64_t)(b0 + i) * NB, rj = (int64_t)(b0 + j) * NB;
  // this lane's A entries, loaded first: their latency hides behind the products
  float av[2][2][4];
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int lr, lc;
        mm_pos(bi, bj, q, lr, lc);
        const int64_t r = ri + lr, c = rj + lc;
        av[bi][bj][q] = r < n && c < n ? L[r * ldl + c] : 0.f;
      }
  f32x4_t acc[2][2] = {};
  if constexpr (DMA) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t lds0 = dma::lds_offset_of(ring);
    // the rows of tiles xi and xj (zero past n: out-of-range offsets)
    const dma::i32x4_t rs_i = dma::make_rsrc(L + ri * ldl, (uint32_t)((n - ri < NB ? n - ri : NB) * ldl * 4));
    const dma::i32x4_t rs_j = dma::make_rsrc(L + rj * ldl, (uint32_t)((n - rj < NB ? n - rj : NB) * ldl * 4));
    // instruction u of this wave: tile u / 4, rows 4 g .. 4 g + 3 with
    // g = 4 (u % 4) + wave; lane: row 4 g + lane / 16, LDS chunk lane % 16
    auto issue = [&](int q, int slot) {
#pragma unroll
      for (int u = 0; u < dup::LOADS; ++u) {
        const int g = 4 * (u % 4) + wave, row = 4 * g + (lane >> 4);
        const int c = (lane & 15) ^ (row & 15);
        const uint32_t off = (uint32_t)(row * ldl * 4 + q * NB * 4 + c * 16);
        dma::load_to_lds16(u < 4 ? rs_i : rs_j, off,
                           lds0 + (uint32_t)(slot * dup::SLOT + (u / 4) * NB * NB * 4 + g * 1024));
      }
    };
    issue(q0, 0);
    if (q0 + 1 < q1) issue(q0 + 1, 1);
    const int li = lane & 15, lk = lane >> 4;
    const int rb = 32 * (wave >> 1), cb = 32 * (wave & 1);
    for (int q = q0; q < q1; ++q) {
      const int slot = (q - q0) & 1;
      // this wave's loads of slot q have landed (q + 1's may be in flight), then everyone's
      if (q + 1 < q1) __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(dup::LOADS));
      else __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
      __syncthreads();
      const unsigned char* X = reinterpret_cast<const unsigned char*>(ring) + slot * dup::SLOT;
      const unsigned char* Y = X + NB * NB * 4;
#pragma unroll
      for (int k0 = 0; k0 < NB; k0 += 16) {
        const int cl = k0 / 4 + lk;  // logical chunk
        const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(X + (rb + li) * 256 + ((cl ^ li) * 16));
        const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(X + (rb + 16 + li) * 256 + ((cl ^ li) * 16));
        const f32x4_t b0v = *reinterpret_cast<const f32x4_t*>(Y + (cb + li) * 256 + ((cl ^ li) * 16));
        const f32x4_t b1v = *reinterpret_cast<const f32x4_t*>(Y + (cb + 16 + li) * 256 + ((cl ^ li) * 16));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[e], b0v[e], acc[0][0], 0, 0, 0);
          acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[e], b1v[e], acc[0][1], 0, 0, 0);
          acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[e], b0v[e], acc[1][0], 0, 0, 0);
          acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[e], b1v[e], acc[1][1], 0, 0, 0);
        }
      }
      if (q + 2 < q1) {
        __syncthreads();  // every wave is done reading the slot
        issue(q + 2, slot);
      }
    }
  } else {
    for (int q = q0; q < q1; ++q) {
      if (q > q0) __syncthreads();  // every wave is done reading the previous panel's tiles
      load_tile(xi, L, ldl, n, ri, (int64_t)q * NB);
      load_tile(xj, L, ldl, n, rj, (int64_t)q * NB);
      __syncthreads();
      mm_nt(xi, xj, acc);
    }
  }
  const bool next_diag = t == 0;  // tile (b0, b0): panel b0's diagonal block
  const bool panel = diag_done != nullptr && j == 0 && i > 0;  // fused: a tile of panel b0 below it
  if (next_diag || panel) __syncthreads();  // every wave is done reading the tiles xi / xj alias
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int lr, lc;
        mm_pos(bi, bj, q, lr, lc);
        const int64_t r = ri + lr, c = rj + lc;
        if (r < n && c < n) {
          const float v = av[bi][bj][q] - acc[bi][bj][q];
          if (next_diag || panel) xi[lr][lc] = v;
          else L[r * ldl + c] = v;
        } else if (next_diag) {
          xi[lr][lc] = lr == lc ? 1.f : 0.f;
        } else if (panel) {
          xi[lr][lc] = 0.f;
        }
      }
  float* W = winv + (b * 2 + (b0 & 1)) * NB * NB;
  if (next_diag) {
    __syncthreads();
    const int bad = factor64_wg(xi, xj);
    const int nb = (int)(n - ri < NB ? n - ri : NB);
    if (diag_done) {
      // inv(L[b0][b0]) written through to where every XCD reads it, then the count
      store_diag_wg<true>(xi, xj, L, ldl, ri, nb, W, bad, info + b);
      __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
      __syncthreads();
      if (threadIdx.x == 0) __hip_atomic_store(diag_done + b, b0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      store_diag_wg(xi, xj, L, ldl, ri, nb, W, bad, info + b);
    }
    return;
  }
  if (!panel) return;
  // L[b0 + i][b0] = A[b0 + i][b0] inv(L[b0][b0])^T once tile (b0, b0) of this
  // launch is factored.  That workgroup (the launch's first) waits for nothing
  // and precedes this one in every XCD's dispatch order, so the wait ends;
  // it is bounded all the same (info = -1 if it ever ran out).
  __shared__ int s_ok;
  if (threadIdx.x == 0) {
    int ok = 0;
    for (int it = 0; it < (1 << 22); ++it) {
      if (__hip_atomic_load(diag_done + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == b0) {
        ok = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (!ok) __hip_atomic_store(info + b, -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_ok = ok;
  }
  __syncthreads();
  // agent-scope loads read past the L2s, which may hold this slot's older contents
  for (int e = threadIdx.x; e < NB * NB; e += 256)
    xj[e / NB][e % NB] = __hip_atomic_load(W + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  f32x4_t lp[2][2] = {};
  mm_nt(xi, xj, lp);
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int lr, lc;
        mm_pos(bi, bj, q, lr, lc);
        if (ri + lr < n && rj + lc < n) L[(ri + lr) * ldl + rj + lc] = lp[bi][bj][q];
      }
  (void)s_ok;
}

// -------------------------------------------------------------- block LDL --
// inv of every b x b diagonal block (lower triangular) into winv [batch][n / b][b][b].
__global__ __launch_bounds__(64) void ldl_inv_kernel(const float* __restrict__ l, int64_t ldl, int64_t sl,
                                                     int64_t n, int bs, float* __restrict__ winv) {
  __shared__ float a[MAX_B][MAX_B + 1];
  __shared__ float xi[MAX_B][MAX_B + 1];
  const int64_t b = blockIdx.y, blk = blockIdx.x;
  const float* L = l + b * sl + blk * bs * ldl + blk * bs;
  for (int i = threadIdx.x; i < bs * bs; i += 64) a[i / bs][i % bs] = L[(int64_t)(i / bs) * ldl + i % bs];
  __syncthreads();
  if ((int)threadIdx.x < bs) {
    const int j = threadIdx.x;
    for (int i = 0; i < j; ++i) xi[i][j] = 0.f;
    xi[j][j] = 1.f / a[j][j];
    for (int i = j + 1; i < bs; ++i) {
      float acc = 0.f;
      for (int k = j; k < i; ++k) acc += a[i][k] * xi[k][j];
      xi[i][j] = -acc / a[i][i];
    }
  }
  __syncthreads();
  float* W = winv + (b * (n / bs) + blk) * bs * bs;
  for (int i = threadIdx.x; i < bs * bs; i += 64) W[i] = xi[i / bs][i % bs];
}

// Column block cb: rows below it times inv(DL_cb); its diagonal block set to
// I (its diagonal to 0 with zero_diag); rows above it are zero and stay so.
template <int BS>
__global__ __launch_bounds__(256) void ldl_apply_kernel(float* __restrict__ l, int64_t ldl, int64_t sl, int64_t n,
                                                        const float* __restrict__ winv, int zero_diag) {
  constexpr int bs = BS;
  __shared__ float iv[BS * BS];
  const int64_t b = blockIdx.z, cb = blockIdx.y;
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const float* W = winv + (b * (n / bs) + cb) * bs * bs;
  for (int i = threadIdx.x; i < bs * bs; i += 256) iv[i] = W[i];
  __syncthreads();
  const int64_t c0 = cb * bs;
  if (r >= n || r < c0) return;
  float* row = l + b * sl + r * ldl + c0;
  if (r < c0 + bs) {
    for (int c = 0; c < bs; ++c) row[c] = (c0 + c == r && !zero_diag) ? 1.f : 0.f;
    return;
  }
  float v[BS];
#pragma unroll
  for (int k = 0; k < BS; ++k) v[k] = row[k];
#pragma unroll
  for (int c = 0; c < BS; ++c) {
    float acc = 0.f;
#pragma unroll
    for (int k = c; k < BS; ++k) acc += v[k] * iv[k * BS + c];
    row[c] = acc;
  }
}

}  // namespace ldl
}  // namespace kq

using namespace kq::ldl;

extern "C" int kq_h_regularize(float* h, int64_t k, int64_t ld, double count, float sigma_reg, float* diag,
                               float* diag_mean, void* stream) {
  if (k <= 0 || k > 65535 || ld < k)
    return kq_fail(KQ_ERR_INVALID, "kq_h_regularize: need 0 < k <= 65535 and ld >= k");
  if (!h || !diag_mean) return kq_fail(KQ_ERR_INVALID, "kq_h_regularize: null buffer");
  if (!(count >= 0.0)) return kq_fail(KQ_ERR_INVALID, "kq_h_regularize: count must be >= 0");
  hipStream_t st = (hipStream_t)stream;
  const float inv = count > 0.0 ? 1.f / (float)count : 1.f;
  diag_mean_kernel<<<1, 256, 0, st>>>(h, k, ld, inv, diag_mean);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return kq_check_launch(e, "kq_h_regularize");
  regularize_kernel<<<dim3((unsigned)((k + 255) / 256), (unsigned)k), 256, 0, st>>>(h, k, ld, inv, sigma_reg,
                                                                                   diag_mean, diag);
  return kq_check_launch(hipGetLastError(), "kq_h_regularize");
}

extern "C" int kq_blockwise_hadamard(float* x, int64_t rows, int64_t cols, int64_t ld, int64_t batch,
                                     int64_t stride, int sides, const float* row_scale, const float* col_scale,
                                     void* stream) {
  if (sides < 1 || sides > 3) return kq_fail(KQ_ERR_INVALID, "kq_blockwise_hadamard: sides must be 1, 2 or 3");
  if (rows <= 0 || cols <= 0 || ld < cols || batch <= 0 || (batch > 1 && stride < rows * ld))
    return kq_fail(KQ_ERR_INVALID, "kq_blockwise_hadamard: bad sizes");
  if (((sides & 1) && rows % HAD) || ((sides & 2) && cols % HAD))
    return kq_fail(KQ_ERR_INVALID, "kq_blockwise_hadamard: the transformed dimension must be a multiple of 128");
  if (rows / HAD + 1 > 65535 || batch > 65535)
    return kq_fail(KQ_ERR_LIMIT, "kq_blockwise_hadamard: too many blocks");
  const float post = sides == 3 ? 1.f / 128.f : 0.08838834764831845f;  // 1/128, fl(1/sqrt(128))
  const dim3 grid((unsigned)((cols + HAD - 1) / HAD), (unsigned)((rows + HAD - 1) / HAD), (unsigned)batch);
  const int vec = !kq_misaligned(x, 16) && ld % 4 == 0 && (batch == 1 || stride % 4 == 0) &&
                  !kq_misaligned(col_scale, 16);
  hadamard_kernel<<<grid, 1024, 0, (hipStream_t)stream>>>(x, rows, cols, ld, stride, sides, row_scale, col_scale,
                                                         post, vec);
  return kq_check_launch(hipGetLastError(), "kq_blockwise_hadamard");
}

extern "C" int64_t kq_cholesky_workspace_size(int64_t n, int64_t batch) {
  if (n <= 0 || batch <= 0) return -1;
  // two inv(L11) slots per matrix, then a diagonal-block counter per matrix
  return batch * 2 * NB * NB * (int64_t)sizeof(float) + (batch * (int64_t)sizeof(int) + 255) / 256 * 256;
}

#ifndef KQ_CHOL_R
#define KQ_CHOL_R 2
#endif
extern "C" int kq_cholesky(const float* a, int64_t lda, int64_t stride_a, float* l, int64_t ldl, int64_t stride_l,
                           int64_t n, int64_t batch, int32_t* info, void* workspace, int64_t workspace_bytes,
                           void* stream) {
  if (n <= 0 || n > 65535 || batch <= 0 || batch > 65535 || lda < n || ldl < n)
    return kq_fail(KQ_ERR_INVALID, "kq_cholesky: need 0 < n <= 65535, 0 < batch <= 65535, lda and ldl >= n");
  if (batch > 1 && (stride_a < n * lda || stride_l < n * ldl))
    return kq_fail(KQ_ERR_INVALID, "kq_cholesky: batch strides smaller than one matrix");
  if (!a || !l || !info || !workspace) return kq_fail(KQ_ERR_INVALID, "kq_cholesky: null buffer");
  if (a != l && ((a < l + stride_l * (batch - 1) + n * ldl) && (l < a + stride_a * (batch - 1) + n * lda)))
    return kq_fail(KQ_ERR_INVALID, "kq_cholesky: a and l overlap without being the same buffer");
  if (a == l && (lda != ldl || stride_a != stride_l))
    return kq_fail(KQ_ERR_INVALID, "kq_cholesky: in place needs equal leading dimensions and strides");
  if (workspace_bytes < kq_cholesky_workspace_size(n, batch))
    return kq_fail(KQ_ERR_INVALID, "kq_cholesky: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  float* winv = (float*)workspace;
  int* diag_done = (int*)(winv + batch * 2 * NB * NB);
  chol_init_kernel<<<dim3((unsigned)((n + 255) / 256), (unsigned)n, (unsigned)batch), 256, 0, st>>>(
      a, lda, stride_a, l, ldl, stride_l, n, info, diag_done);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return kq_check_launch(e, "kq_cholesky/init");
  const int m = (int)((n + NB - 1) / NB);
  // the update launches' direct-load form: whole 64-column tiles, 16-byte
  // aligned rows, and a 64-row tile's bytes within one 32-bit range
  const bool dma_ok = n % NB == 0 && ldl % 4 == 0 && (reinterpret_cast<uintptr_t>(l) & 15) == 0 &&
                      (batch == 1 || stride_l % 4 == 0) && (uint64_t)NB * ldl * 4 <= kq::dma::MAX_RANGE;
  chol_diag_kernel<<<(unsigned)batch, 256, 0, st>>>(l, n, ldl, stride_l, winv, info);
  if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_cholesky/diag");
  if (batch < 8) {
    // One launch per panel after the first, in super-panels of R panels:
    // the launch of a super-panel's first panel S applies the previous
    // super-panel's panels to the whole trailing matrix (rank 64 R, so the
    // trailing matrix is read and written once per super-panel), the launch
    // of panel s inside it applies panels S .. s - 1 to block column s only.
    // Each launch then factors diagonal block s (its first workgroup) and,
    // in the workgroups of the tiles below that block, once it is factored,
    // computes panel s itself.
    constexpr int R = KQ_CHOL_R;
    if (m > 1) {
      chol_panel_kernel<<<dim3((unsigned)(m - 1), (unsigned)batch), 256, 0, st>>>(l, n, ldl, stride_l, 0, 0, 1,
                                                                                 winv, info);
      if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_cholesky/panel");
    }
    for (int s = 1; s < m; ++s) {
      const int64_t q = m - s;
      const int S = s / R * R;  // this super-panel's first panel
      const dim3 grid((unsigned)(s == S ? q * (q + 1) / 2 : q), (unsigned)batch);
      const int qa = s == S ? s - R : S, col = s == S ? 0 : 1;
      if (dma_ok) chol_update_kernel<true><<<grid, 256, 0, st>>>(l, n, ldl, stride_l, s, qa, s, winv, info, diag_done, col);
      else chol_update_kernel<false><<<grid, 256, 0, st>>>(l, n, ldl, stride_l, s, qa, s, winv, info, diag_done, col);
      if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_cholesky/update");
    }
    return KQ_OK;
  }
  // Super-panels of four panels: one launch per panel (its block column
  // brought up to date with the super-panel's earlier panels, the panel
  // below its diagonal block, and the next diagonal block factored), then one
  // rank-256 update of everything to the right, so the trailing matrix is
  // read and written once per super-panel (measured on MI355X, 48 matrices
  // of n = 2048: 3.90 ms with four panels, 4.12 with two or eight).
  const int rank = 4;
  for (int s0 = 0; s0 < m; s0 += rank) {
    const int s1 = s0 + rank < m ? s0 + rank : m;
    for (int p = s0; p < s1 && p + 1 < m; ++p) {
      chol_panel_kernel<<<dim3((unsigned)(m - p - 1), (unsigned)batch), 256, 0, st>>>(l, n, ldl, stride_l, p, s0,
                                                                                     s1, winv, info);
      if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_cholesky/panel");
    }
    if (s1 < m) {
      const int64_t q = m - s1;
      const dim3 grid((unsigned)(q * (q + 1) / 2), (unsigned)batch);
      if (dma_ok) chol_update_kernel<true><<<grid, 256, 0, st>>>(l, n, ldl, stride_l, s1, s0, s1, winv, info, nullptr, 0);
      else chol_update_kernel<false><<<grid, 256, 0, st>>>(l, n, ldl, stride_l, s1, s0, s1, winv, info, nullptr, 0);
      if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_cholesky/update");
    }
  }
  return KQ_OK;
}

extern "C" int64_t kq_block_ldl_workspace_size(int64_t n, int b, int64_t batch) {
  if (n <= 0 || b <= 0 || batch <= 0) return -1;
  return batch * n * (int64_t)b * (int64_t)sizeof(float);
}

extern "C" int kq_block_ldl(float* l, int64_t ld, int64_t stride, int64_t n, int b, int64_t batch,
                            uint32_t flags, void* workspace, int64_t workspace_bytes, void* stream) {
  if (flags & ~(uint32_t)KQ_LDL_ZERO_DIAGONAL) return kq_fail(KQ_ERR_INVALID, "kq_block_ldl: unknown flags");
  if (n <= 0 || b <= 0 || b > MAX_B || (b & (b - 1)) != 0 || n % b != 0 || ld < n || batch <= 0 ||
      batch > 65535 || (batch > 1 && stride < n * ld))
    return kq_fail(KQ_ERR_INVALID,
                   "kq_block_ldl: need b a power of two <= %d, n %% b == 0, ld >= n (n=%lld b=%d)", MAX_B,
                   (long long)n, b);
  if (n / b > 65535) return kq_fail(KQ_ERR_LIMIT, "kq_block_ldl: too many blocks");
  if (!l || !workspace) return kq_fail(KQ_ERR_INVALID, "kq_block_ldl: null buffer");
  if (workspace_bytes < kq_block_ldl_workspace_size(n, b, batch))
    return kq_fail(KQ_ERR_INVALID, "kq_block_ldl: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  float* winv = (float*)workspace;
  ldl_inv_kernel<<<dim3((unsigned)(n / b), (unsigned)batch), 64, 0, st>>>(l, ld, stride, n, b, winv);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return kq_check_launch(e, "kq_block_ldl/inv");
  const dim3 grid((unsigned)((n + 255) / 256), (unsigned)(n / b), (unsigned)batch);
  const int zd = (flags & KQ_LDL_ZERO_DIAGONAL) ? 1 : 0;
  switch (b) {
#define KQ_LDL_CASE(B) \
    case B: ldl_apply_kernel<B><<<grid, 256, 0, st>>>(l, ld, stride, n, winv, zd); break;
    KQ_LDL_CASE(1) KQ_LDL_CASE(2) KQ_LDL_CASE(4) KQ_LDL_CASE(8) KQ_LDL_CASE(16) KQ_LDL_CASE(32) KQ_LDL_CASE(64)
#undef KQ_LDL_CASE
  }
  return kq_check_launch(hipGetLastError(), "kq_block_ldl/apply");
}
