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

}  // namespace had
}  // namespace kq
