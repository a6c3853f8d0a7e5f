// Device-side helpers shared by the kquant_amd kernels (gfx950, wave64).
//
// Numeric contract (restated from the reference, written here from the
// format definitions, not from any vendor math library):
//   E8M0 byte b      -> 2^(b-127); b = 0 is the fp32 subnormal 2^-127 and
//                       b = 255 is +inf, as torch.exp2(b - 127) gives
//                       (kquant/io/mxfp4.py:41-43, kquant/mxfp8.py:79-84).
//   block exponent   -> ceil(log2(max(amax, 1e-30) / qmax)) clamped to
//                       [-127, 128] (kquant/mxfp8.py:41-44), qmax = 448 (E4M3)
//                       or 6 (E2M1).
//   E4M3 / E2M1 cast -> round to nearest, ties to even, sign kept (so -0 and
//                       tiny negatives give the sign-only code).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kq {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  bf16x2_t v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t f32x2_to_f16x2_bits(float lo, float hi) {
  f16x2_t v;
  v[0] = (_Float16)lo;
  v[1] = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// E8M0 byte -> fp32 scale, exactly 2^(b-127) (0 -> subnormal, 255 -> +inf).
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
  uint32_t bits = b == 0u ? 0x00400000u : (b == 255u ? 0x7f800000u : (b << 23));
  return __uint_as_float(bits);
}

// Block exponent e = clamp(ceil(log2(max(amax,1e-30)/qmax)), -127, 128)
// for bf16 and fp16 inputs (FMT 0: qmax = 448, FMT 1: qmax = 6), without the
// division.  q = fl(a/qmax) is always a normal float here (a >= 1e-30), so
// the exact ceil(log2(q)) is its unbiased exponent plus one unless q is a
// power of two; for bf16 and fp16 inputs this equals the rounded torch.log2
// result (their quotients are never within log2-rounding of a power of two
// without being one).  With a = m 2^E (1 <= m < 2) and qmax = t 2^T (448 =
// 1.75 2^8, 6 = 1.5 2^2): q = 2^(E-T) exactly when m = t; q lies strictly
// between 2^(E-T) and 2^(E-T+1) when m > t, and strictly between 2^(E-T-1)
// and 2^(E-T) when m < t, because such an m (at most 11 significant bits, or
// the 1e-30 floor) differs from t by far more than the 2^-24 relative step of
// the rounding.  Hence e = E - T + (m > t); infinity gives 128, and finite
// values stay inside [-127, 128].
template <int FMT>
__device__ __forceinline__ int mx_block_exponent(float amax) {
  const uint32_t bits = __float_as_uint(fmaxf(amax, 1e-30f));  // amax >= 0
  const int expo = (int)(bits >> 23);
  if (expo == 0xff) return 128;  // amax = +inf
  const uint32_t t_frac = FMT == 0 ? 0x600000u : 0x400000u;
  return expo - 127 - (FMT == 0 ? 8 : 2) + ((bits & 0x7fffffu) > t_frac ? 1 : 0);
}

// The block exponent for fp32 inputs, whose quotients can sit a few ulps above
// a power of two: kquant/mxfp8.py:41-43 takes torch.log2 in float32, which
// rounds k + log2(1 + f) down to k when log2(1 + f) is below half an ulp of
// k, so the reference keeps exponent k there and clamps the block's top
// values to qmax.  log2 is evaluated in double and rounded once to float; a
// double result within an ulp of the true value rounds like the correctly
// rounded one, because log2(1 + m 2^-23) is never near an f32 midpoint of k.
__device__ __forceinline__ int mx_block_exponent_f32_log2(float amax, float qmax) {
  const float q = __fdiv_rn(fmaxf(amax, 1e-30f), qmax);
  if (__float_as_uint(q) >= 0x7f800000u) return 128;  // amax = +inf
  int e = (int)ceilf((float)log2((double)q));
  e = e < -127 ? -127 : e;
  e = e > 128 ? 128 : e;
  return e;
}

// 2^-e as an exact fp32 multiplier; e = 128 (only for an infinite amax)
// gives 0 so x * 0 reproduces x / exp2(128) = x / inf (0, or NaN for inf).
__device__ __forceinline__ float mx_inv_scale(int e) {
  int b = 127 - e;  // biased exponent of 2^-e
  uint32_t bits = b >= 1 ? ((uint32_t)b << 23) : (b == 0 ? 0x00400000u : 0u);
  return __uint_as_float(bits);
}

// Software fp32 -> E4M3 (float8_e4m3fn) with round-to-nearest-even.
// |y| > 464 (past the midpoint of 448 and the NaN code) and NaN give 0x7f|sign;
// 464 itself ties to the even code 0x7e (448).
__device__ __forceinline__ uint32_t f32_to_e4m3_rne(float y) {
  uint32_t b = __float_as_uint(y);
  uint32_t sign = (b >> 24) & 0x80u;
  uint32_t a = b & 0x7fffffffu;
  uint32_t code;
  if (a > 0x43e80000u) {
    code = 0x7fu;
  } else if (a >= 0x3c800000u) {  // >= 2^-6: normal E4M3, keep 3 mantissa bits
    code = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - (120u << 3);
  } else {  // subnormal E4M3: multiples of 2^-9, rounded to nearest even
    code = (uint32_t)rintf(__uint_as_float(a) * 512.0f);
  }
  return sign | code;
}

// Software fp32 -> E2M1 code with round-to-nearest-even; |y| <= 6 expected
// (callers clamp first, as the quantization rule does).
__device__ __forceinline__ uint32_t f32_to_e2m1_rne(float y) {
  uint32_t b = __float_as_uint(y);
  uint32_t sign = (b >> 28) & 0x8u;
  uint32_t a = b & 0x7fffffffu;
  uint32_t code;
  if (a >= 0x3f800000u) {  // >= 1.0: normal E2M1, keep 1 mantissa bit
    code = ((a + 0x1fffffu + ((a >> 22) & 1u)) >> 22) - 252u;
  } else {  // 0, 0.5, 1.0
    code = (uint32_t)rintf(__uint_as_float(a) * 2.0f);
  }
  return sign | code;
}

// E2M1 code (0..15) -> fp32 value, codes 8..15 the negated mirror.
__device__ __forceinline__ float e2m1_to_f32(uint32_t c) {
  uint32_t m = c & 7u;
  uint32_t bits = m == 0u ? 0u
                : (m == 1u ? 0x3f000000u
                           : ((((m >> 1) + 126u) << 23) | ((m & 1u) << 22)));
  return __uint_as_float(bits | ((c & 8u) << 28));
}

// E4M3 (float8_e4m3fn) byte -> fp32 value (0x7f / 0xff are NaN).
__device__ __forceinline__ float e4m3_to_f32(uint32_t v) {
  uint32_t sign = (v & 0x80u) << 24;
  uint32_t e = (v >> 3) & 0xfu;
  uint32_t m = v & 7u;
  float mag;
  if ((v & 0x7fu) == 0x7fu) {
    mag = __uint_as_float(0x7fc00000u);
  } else if (e == 0u) {
    mag = (float)m * 0.001953125f;  // m * 2^-9
  } else {
    mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(mag) | sign);
}

// Max over the 4 lanes of a quad (lanes 4j..4j+3) with DPP quad permutes.
__device__ __forceinline__ float quad_max(float v) {
  int x = __float_as_int(v);
  int y = __builtin_amdgcn_mov_dpp(x, 0xb1, 0xf, 0xf, true);  // [1,0,3,2]
  v = fmaxf(v, __int_as_float(y));
  x = __float_as_int(v);
  y = __builtin_amdgcn_mov_dpp(x, 0x4e, 0xf, 0xf, true);      // [2,3,0,1]
  return fmaxf(v, __int_as_float(y));
}

}  // namespace kq
