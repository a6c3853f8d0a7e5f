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

// v of lane ^ S: quad permutes (DPP) for 1 and 2, a bit-mask swizzle for 4
// and 8, and the gfx950 row swaps for 16 and 32 (lanes 0-31 receive the
// upper half's values in the second result of permlane32_swap, lanes 32-63
// the lower half's in the first; likewise per 16-lane row pair for
// permlane16_swap) - none of them go through LDS addressing.
template <int S>
__device__ __forceinline__ float lane_xor(float v, int lane) {
  const int x = __float_as_int(v);
  if constexpr (S == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
  else if constexpr (S == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
  else if constexpr (S == 4 || S == 8) return __int_as_float(__builtin_amdgcn_ds_swizzle(x, 0x1F | (S << 10)));
  else if constexpr (S == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
    return __uint_as_float((lane & 16) ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    return __uint_as_float((lane & 32) ? r[0] : r[1]);
  }
}

template <int S>
__device__ __forceinline__ void fwht_stage(float& v0, float& v1, int lane) {
  const float p0 = lane_xor<S>(v0, lane), p1 = lane_xor<S>(v1, lane);
  const bool up = lane & S;
  v0 = up ? p0 - v0 : v0 + p0;
  v1 = up ? p1 - v1 : v1 + p1;
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
  fwht_stage<16>(v0, v1, lane);
  fwht_stage<32>(v0, v1, lane);
}

}  // namespace had
}  // namespace kq
