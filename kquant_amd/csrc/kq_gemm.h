// Block-scaled weight GEMM building blocks (bf16 activations x MX weights).
//
// C[m][n] = sum_k A[m][k] * dequant(W)[n][k]: A is bf16 [M, K] (K contiguous),
// W is MXFP8 (E4M3 bytes [N, K]) or MXFP4 (packed nibbles [N, K/2]) with E8M0
// scales [N, K/32].  Both operands are K-major, which is the operand order of
// v_mfma_f32_32x32x16_bf16 (each lane holds 8 consecutive k of one row), so no
// transposes are needed.  Weights stay in their packed form in LDS (half or a
// quarter of the bf16 bytes) and are expanded to bf16 when a lane builds its
// MFMA fragment, with the gfx950 scaled convert instructions:
// E4M3/E2M1 x 2^(s-127) is exact in bf16, so the MFMA sees exactly the
// reference-dequantized weight.
#pragma once

#include "kq_common.h"

namespace kq {
namespace gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// 8 consecutive weights of one row as a bf16 MFMA fragment.
// FMT 0: w holds 8 E4M3 bytes; FMT 1: w.x holds 8 E2M1 nibbles (low first).
template <int FMT>
__device__ __forceinline__ bf16x8_t dequant8(u32x2_t w, uint32_t scale_byte) {
  const float sc = __uint_as_float(scale_byte << 23);
  bf16x2_t p0, p1, p2, p3;
  if (FMT == 0) {
    p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0], sc, false);
    p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0], sc, true);
    p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[1], sc, false);
    p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[1], sc, true);
  } else {
    p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[0], sc, 0);
    p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[0], sc, 1);
    p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[0], sc, 2);
    p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[0], sc, 3);
  }
  bf16x8_t r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

}  // namespace gemm
}  // namespace kq
