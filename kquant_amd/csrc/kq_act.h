// Expert activations shared by the fused MoE epilogues and the stand-alone
// activation kernel, computed in fp32:
//   SiTU   beta * tanh(g / beta) * sigmoid(g) * linear_beta * tanh(u / linear_beta)
//          (kquant/tp_simulator.py:83-94)
//   SwiGLU g * sigmoid(g) * u
//
// The epilogues evaluate these for every element of a gate/up tile, so the
// transcendental functions are built on the hardware exp2 / reciprocal
// instructions instead of the general library routines (which cost more than
// the MFMAs of a 128-k step):
//   exp(a)      = 2^h with h = fl(a log2 e); the rounding error of that product
//                 (recovered exactly with two FMAs) multiplies the result by
//                 1 + err ln 2.  Measured: <= 1 ulp past the hardware exp2's own.
//   tanh(y)     |y| < 0.625: y + y^3 P(y^2), P of degree 4, a minimax fit of
//                 (tanh(y) - y) / y^3 in relative error (Lawson iterations on
//                 Chebyshev points), <= 0.72 ulp over every fp32 y in range;
//                 otherwise sign(y) (1 - 2 / (exp(2|y|) + 1)), <= 1.5 ulp
//                 (exactly 1 once exp overflows).
//   sigmoid(x)  = 1 / (1 + exp(-x)), <= 3 ulp.
//   g / beta    = q + (g - q beta) / beta with q = g fl(1/beta): the division
//                 corrected once by FMA (exact whenever 1/beta is, e.g. beta 4).
// The bounds are for correctly rounded exp2 / reciprocal; the GPU tests hold
// the kernels to fp32-level agreement with numpy's float32 functions.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/kquant_amd.h"

namespace kq {

struct ActParams {
  int kind;       // KQ_ACT_SITU or KQ_ACT_SWIGLU
  float beta;     // SiTU gate beta
  float lbeta;    // SiTU linear beta
};

// accurate library sigmoid (router scores, whose ordering must match the oracle's)
__device__ __forceinline__ float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }

__device__ __forceinline__ float exp_act(float a) {
  constexpr float L2E = 1.44269502f;            // fl(log2 e)
  constexpr float L2E_LO = 1.925963033500011e-08f;  // log2 e - L2E
  constexpr float LN2 = 0.693147182f;
  const float h = a * L2E;
  float l = fmaf(a, L2E, -h);
  l = fmaf(a, L2E_LO, l);
  const float e = __builtin_amdgcn_exp2f(h);
  return __builtin_isinf(e) ? e : fmaf(e, l * LN2, e);
}

__device__ __forceinline__ float rcp_act(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float sigmoid_act(float x) { return rcp_act(1.0f + exp_act(-x)); }

__device__ __forceinline__ float tanh_act(float y) {
  const float a = fabsf(y);
  const float z = y * y;
  float p = -0.005704986862838268f;
  p = fmaf(p, z, 0.0206390880048275f);
  p = fmaf(p, z, -0.05373971536755562f);
  p = fmaf(p, z, 0.13331441581249237f);
  p = fmaf(p, z, -0.3333328068256378f);
  const float small = fmaf(y * z, p, y);
  const float big = fmaf(-2.0f, rcp_act(exp_act(2.0f * a) + 1.0f), 1.0f);
  return a < 0.625f ? small : copysignf(big, y);
}

// a / b with r = fl(1 / b): one FMA correction of the product
__device__ __forceinline__ float div_act(float a, float b, float r) {
  const float q = a * r;
  return fmaf(fmaf(-q, b, a), r, q);
}

__device__ __forceinline__ float activate(const ActParams& p, float g, float u) {
  const float sg = sigmoid_act(g);
  if (p.kind == KQ_ACT_SWIGLU) return g * sg * u;
  const float gv = p.beta * tanh_act(div_act(g, p.beta, rcp_act(p.beta))) * sg;
  const float uv = p.lbeta * tanh_act(div_act(u, p.lbeta, rcp_act(p.lbeta)));
  return gv * uv;
}

}  // namespace kq
