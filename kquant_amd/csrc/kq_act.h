// Expert activations shared by the fused MoE epilogues and the stand-alone
// activation kernel, computed in fp32:
//   SiTU   beta * tanh(g / beta) * sigmoid(g) * linear_beta * tanh(u / linear_beta)
//          (kquant/tp_simulator.py:83-94)
//   SwiGLU g * sigmoid(g) * u
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/kquant_amd.h"

namespace kq {

struct ActParams {
  int kind;       // KQ_ACT_SITU or KQ_ACT_SWIGLU
  float beta;     // SiTU gate beta
  float lbeta;    // SiTU linear beta
};

__device__ __forceinline__ float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }

__device__ __forceinline__ float activate(const ActParams& p, float g, float u) {
  if (p.kind == KQ_ACT_SWIGLU) return g * sigmoidf_(g) * u;
  const float gv = p.beta * tanhf(g / p.beta) * sigmoidf_(g);
  const float uv = p.lbeta * tanhf(u / p.lbeta);
  return gv * uv;
}

}  // namespace kq
