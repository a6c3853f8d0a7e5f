// Element-wise and small reduction kernels around the expert linears:
// the expert activation, the deterministic reduction of tensor-parallel
// partials, the comparison metrics of the closures, and the K3 router.
// All are HBM-streaming kernels (or one wave per token for the router).
#include "kq_act.h"
#include "kq_common.h"
#include "kq_internal.h"

namespace kq {
namespace {

__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  if (dt == KQ_DT_F32) return static_cast<const float*>(p)[i];
  const uint32_t h = static_cast<const uint16_t*>(p)[i];
  return dt == KQ_DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

__device__ __forceinline__ void store_from_f32(void* p, int dt, int64_t i, float v) {
  if (dt == KQ_DT_F32) static_cast<float*>(p)[i] = v;
  else if (dt == KQ_DT_BF16) static_cast<__bf16*>(p)[i] = (__bf16)v;
  else static_cast<_Float16*>(p)[i] = (_Float16)v;
}

// out[r, c] = act(gate[r, c], up[r, c]) in fp32, rounded to out's type.
__global__ __launch_bounds__(256) void activation_kernel(ActParams p, int in_dt, const void* gate,
                                                         const void* up, int64_t ld_in, int64_t rows,
                                                         int64_t cols, int out_dt, void* out,
                                                         int64_t ld_out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * cols) return;
  const int64_t r = i / cols, c = i - r * cols;
  const float g = load_as_f32(gate, in_dt, r * ld_in + c);
  const float u = load_as_f32(up, in_dt, r * ld_in + c);
  store_from_f32(out, out_dt, r * ld_out + c, activate(p, g, u));
}

// out[i] = sum over p of partials[p * stride + i], in order p = 0, 1, ...
// (kquant/tp_simulator.py:72-80: stack of fp32 partials, sum, cast).
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ partials,
                                                              int64_t parts, int64_t stride,
                                                              int64_t n, int out_dt, void* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float s = 0.0f;
  for (int64_t q = 0; q < parts; ++q) s += partials[q * stride + i];
  store_from_f32(out, out_dt, i, s);
}

constexpr int METRIC_PARTS = 256;
constexpr int METRIC_FIELDS = 5;  // sum d^2, max |d|, sum r^2, sum a^2, sum r*a

// Per-block partial sums in double over a grid-stride range, in a fixed
// order (deterministic); block b writes fields [b * 5, b * 5 + 5).
__global__ __launch_bounds__(256) void metrics_partial_kernel(int ref_dt, const void* ref, int act_dt,
                                                              const void* act, int64_t n,
                                                              double* __restrict__ partial) {
  __shared__ double red[METRIC_FIELDS][256];
  double s_dd = 0.0, m_d = 0.0, s_rr = 0.0, s_aa = 0.0, s_ra = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)METRIC_PARTS * 256) {
    const float r = load_as_f32(ref, ref_dt, i), a = load_as_f32(act, act_dt, i);
    const double d = (double)(a - r);  // the fp32 difference, as the reference forms it
    s_dd += d * d;
    m_d = fmax(m_d, fabs(d));
    s_rr += (double)r * r;
    s_aa += (double)a * a;
    s_ra += (double)r * a;
  }
  const int t = threadIdx.x;
  red[0][t] = s_dd; red[1][t] = m_d; red[2][t] = s_rr; red[3][t] = s_aa; red[4][t] = s_ra;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (t < w) {
      red[0][t] += red[0][t + w];
      red[1][t] = fmax(red[1][t], red[1][t + w]);
      red[2][t] += red[2][t + w];
      red[3][t] += red[3][t + w];
      red[4][t] += red[4][t + w];
    }
    __syncthreads();
  }
  if (t < METRIC_FIELDS) partial[blockIdx.x * METRIC_FIELDS + t] = red[t][0];
}

__global__ void metrics_final_kernel(const double* __restrict__ partial, double* __restrict__ out) {
  if (threadIdx.x != 0) return;
  double f[METRIC_FIELDS] = {0, 0, 0, 0, 0};
  for (int b = 0; b < METRIC_PARTS; ++b) {
    f[0] += partial[b * METRIC_FIELDS];
    f[1] = fmax(f[1], partial[b * METRIC_FIELDS + 1]);
    f[2] += partial[b * METRIC_FIELDS + 2];
    f[3] += partial[b * METRIC_FIELDS + 3];
    f[4] += partial[b * METRIC_FIELDS + 4];
  }
  for (int j = 0; j < METRIC_FIELDS; ++j) out[j] = f[j];
}

// K3 router (kquant/tp_simulator.py:114-134), one wave per token: scores =
// sigmoid(logits), choose the top-k of scores + bias (descending, ties to the
// lower expert id), weights = the chosen scores normalised to sum 1, times
// the routed scaling factor.
constexpr int TOPK_MAX = 64;
constexpr int EXPERTS_MAX = 1024;
constexpr int TOPK_PER_LANE = EXPERTS_MAX / 64;  // experts per lane, in registers

__global__ __launch_bounds__(256) void kimi_topk_kernel(int logit_dt, const void* logits, int64_t ld,
                                                        const float* __restrict__ bias, int64_t tokens,
                                                        int experts, int topk, float scale,
                                                        float* __restrict__ weights,
                                                        int32_t* __restrict__ ids) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;  // whole waves leave together; the kernel has no barrier
  float key[TOPK_PER_LANE], score[TOPK_PER_LANE];
#pragma unroll
  for (int j = 0; j < TOPK_PER_LANE; ++j) {
    const int e = lane + 64 * j;
    key[j] = -INFINITY;
    score[j] = 0.0f;
    if (e < experts) {
      score[j] = sigmoidf_(load_as_f32(logits, logit_dt, t * ld + e));
      key[j] = score[j] + bias[e];
    }
  }
  int my_id = 0;        // lane k < topk keeps the k-th choice
  float my_score = 0.0f;
  for (int k = 0; k < topk; ++k) {
    float best = -INFINITY, best_s = 0.0f;
    int best_e = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < TOPK_PER_LANE; ++j) {
      const int e = lane + 64 * j;
      if (e < experts && (key[j] > best || (key[j] == best && e < best_e))) {
        best = key[j];
        best_e = e;
        best_s = score[j];
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ob = __shfl_xor(best, o, 64);
      const int oe = __shfl_xor(best_e, o, 64);
      const float os = __shfl_xor(best_s, o, 64);
      if (ob > best || (ob == best && oe < best_e)) {
        best = ob;
        best_e = oe;
        best_s = os;
      }
    }
#pragma unroll
    for (int j = 0; j < TOPK_PER_LANE; ++j)
      if (lane + 64 * j == best_e) key[j] = -INFINITY;
    if (lane == k) {
      my_id = best_e;
      my_score = best_s;
    }
  }
  // sum of the chosen scores in choice order, then normalise and scale
  float total = 0.0f;
  for (int k = 0; k < topk; ++k) total += __shfl(my_score, k, 64);
  if (lane < topk) {
    weights[t * topk + lane] = my_score / total * scale;
    ids[t * topk + lane] = my_id;
  }
}

bool dtype_ok(int dt) { return dt == KQ_DT_BF16 || dt == KQ_DT_F16 || dt == KQ_DT_F32; }

}  // namespace
}  // namespace kq

using namespace kq;

extern "C" int kq_expert_activation(int activation, float beta, float linear_beta, int in_dtype,
                                    const void* gate, const void* up, int64_t ld_in, int64_t rows,
                                    int64_t cols, int out_dtype, void* out, int64_t ld_out,
                                    void* stream) {
  if (activation != KQ_ACT_SITU && activation != KQ_ACT_SWIGLU)
    return kq_fail(KQ_ERR_INVALID, "kq_expert_activation: unknown activation %d", activation);
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype))
    return kq_fail(KQ_ERR_INVALID, "kq_expert_activation: unknown dtype");
  if (rows < 0 || cols < 0 || ld_in < cols || ld_out < cols)
    return kq_fail(KQ_ERR_INVALID, "kq_expert_activation: bad sizes");
  if (rows * cols == 0) return KQ_OK;
  const ActParams p{activation, beta, linear_beta};
  activation_kernel<<<(unsigned)((rows * cols + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      p, in_dtype, gate, up, ld_in, rows, cols, out_dtype, out, ld_out);
  return kq_check_launch(hipGetLastError(), "kq_expert_activation");
}

extern "C" int kq_reduce_partials(const float* partials, int64_t parts, int64_t stride, int64_t n,
                                  int out_dtype, void* out, void* stream) {
  if (parts < 1 || n < 0 || stride < n || !dtype_ok(out_dtype))
    return kq_fail(KQ_ERR_INVALID, "kq_reduce_partials: bad sizes or dtype");
  if (n == 0) return KQ_OK;
  reduce_partials_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      partials, parts, stride, n, out_dtype, out);
  return kq_check_launch(hipGetLastError(), "kq_reduce_partials");
}

extern "C" int kq_comparison_sums(int ref_dtype, const void* reference, int act_dtype,
                                  const void* actual, int64_t n, double* workspace, double* out,
                                  void* stream) {
  if (!dtype_ok(ref_dtype) || !dtype_ok(act_dtype) || n < 0)
    return kq_fail(KQ_ERR_INVALID, "kq_comparison_sums: bad dtype or size");
  if (kq_misaligned(workspace, 8) || kq_misaligned(out, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_comparison_sums: misaligned workspace or out");
  hipStream_t st = (hipStream_t)stream;
  metrics_partial_kernel<<<METRIC_PARTS, 256, 0, st>>>(ref_dtype, reference, act_dtype, actual, n,
                                                       workspace);
  metrics_final_kernel<<<1, 64, 0, st>>>(workspace, out);
  return kq_check_launch(hipGetLastError(), "kq_comparison_sums");
}

extern "C" int kq_kimi_topk(int logit_dtype, const void* logits, int64_t ld, const float* bias,
                            int64_t tokens, int experts, int topk, float routed_scaling_factor,
                            float* weights, int32_t* ids, void* stream) {
  if (!dtype_ok(logit_dtype) || tokens < 0 || experts < 1 || experts > EXPERTS_MAX || topk < 1 ||
      topk > TOPK_MAX || topk > experts || ld < experts)
    return kq_fail(KQ_ERR_INVALID,
                   "kq_kimi_topk: need 1 <= topk <= min(64, experts), experts <= 1024, ld >= experts");
  if (tokens == 0) return KQ_OK;
  kimi_topk_kernel<<<(unsigned)((tokens + 3) / 4), 256, 0, (hipStream_t)stream>>>(
      logit_dtype, logits, ld, bias, tokens, experts, topk, routed_scaling_factor, weights, ids);
  return kq_check_launch(hipGetLastError(), "kq_kimi_topk");
}
