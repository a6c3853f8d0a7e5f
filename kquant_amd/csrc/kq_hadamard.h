// The 128-point blockwise Hadamard transform shared by the Hessian rotation
// and the QSRT weight decode: the Sylvester matrix (entries
// (-1)^popcount(i & j), kquant/exl3_reference.py:195-212) applied to every
// row or column of a 128 x 128 fp32 tile in LDS as a fast Walsh-Hadamard
// transform (adds only, unscaled).
#pragma once

#include <hip/hip_runtime.h>

namespace kq {
namespace had {

constexpr int HAD = 128;       // Hadamard block
constexpr int HLD = HAD + 1;   // padded LDS row

// 128-point fast Walsh-Hadamard transform (Sylvester order, unscaled) of
// every row (ROWS) or column of the LDS tile: two threads per line, each
// holding 64 consecutive points in registers; stages 1..32 run in
// registers, stage 64 pairs the two threads (lanes 2l, 2l + 1) by shuffle.
template <bool ROWS>
__device__ __forceinline__ void fwht_lines(float (*t)[HLD]) {
  const int line = threadIdx.x >> 1, half = threadIdx.x & 1;
  float v[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) v[i] = ROWS ? t[line][64 * half + i] : t[64 * half + i][line];
#pragma unroll
  for (int h = 1; h < 64; h <<= 1) {
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      if (i & h) continue;
      const float a = v[i], b = v[i + h];
      v[i] = a + b;
      v[i + h] = a - b;
    }
  }
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const float o = __shfl_xor(v[i], 1);
    v[i] = half ? o - v[i] : v[i] + o;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    if (ROWS) t[line][64 * half + i] = v[i];
    else t[64 * half + i][line] = v[i];
  }
  __syncthreads();
}

// v of lane ^ S for S = 1, 2 (DPP quad permutes) and 4, 8 (bit-mask
// swizzles), which go through no LDS addressing.
template <int S>
__device__ __forceinline__ float lane_xor(float v) {
  const int x = __float_as_int(v);
  if constexpr (S == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
  else if constexpr (S == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
  else return __int_as_float(__builtin_amdgcn_ds_swizzle(x, 0x1F | (S << 10)));
}

// Butterfly across lanes l and l ^ S (S < 16): the lower lane keeps
// v + v', the upper v' - v, as one FMA with the lane's sign (exact products
// by +-1, so the sums round as the plain adds would).
template <int S>
__device__ __forceinline__ void fwht_stage(float& v0, float& v1, int lane) {
  const float s = (lane & S) ? -1.f : 1.f;
  const float p0 = lane_xor<S>(v0), p1 = lane_xor<S>(v1);
  v0 = fmaf(s, v0, p0);
  v1 = fmaf(s, v1, p1);
}

// Butterfly across elements e and e + S for S = 16, 32 with the gfx950 row
// swaps: exchanging the upper rows of v0 with the lower rows of v1 leaves
// every lane holding one (e, e + S) pair, which it combines in place; the
// same exchange restores the layout.
template <int S>
__device__ __forceinline__ void fwht_stage_swap(float& v0, float& v1) {
  const auto r = S == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v0), __float_as_uint(v1), false, false)
                         : __builtin_amdgcn_permlane32_swap(__float_as_uint(v0), __float_as_uint(v1), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  const auto q = S == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(a + b), __float_as_uint(a - b), false, false)
                         : __builtin_amdgcn_permlane32_swap(__float_as_uint(a + b), __float_as_uint(a - b), false, false);
  v0 = __uint_as_float(q[0]);
  v1 = __uint_as_float(q[1]);
}

// 128-point Sylvester transform (unnormalized) of the line held as
// (v0, v1) = elements (lane, lane + 64) of one wave.
__device__ __forceinline__ void fwht128(float& v0, float& v1, int lane) {
  const float a = v0 + v1, b = v0 - v1;
  v0 = a;
  v1 = b;
  fwht_stage<1>(v0, v1, lane);
  fwht_stage<2>(v0, v1, lane);
  fwht_stage<4>(v0, v1, lane);
  fwht_stage<8>(v0, v1, lane);
  fwht_stage_swap<16>(v0, v1);
  fwht_stage_swap<32>(v0, v1);
}

}  // namespace had
}  // namespace kq
