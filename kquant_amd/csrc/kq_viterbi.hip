// SQG trellis quantizer (tail-biting Viterbi over 16-bit states) on MI355X:
// the search of kquant/csrc/qsrt_quantize_tiles_kernel.cuh with the SQG
// E4M3 labels of kquant/csrc/sqg_quantize.cu, bit for bit.
//
// A tile of 256 values is coded as 256 K-bit edges (K = 2, 3, 4); the state
// at a step is the last 16 bits of the edge stream, a node its low 16 - K
// bits, and node o is reached from nodes (o >> K) + k 2^(16-2K), k < 2^K, by
// state (k << (16-K)) | o with label lut[state].  In fp16, as the reference:
// w = fp16(x); d = fp16(label - w); the cost is fp16(d d) on a pass's first
// step (the closing pass forces its start node by +inf on every other
// predecessor), else fp16(fma(d, d, prev)) with one rounding; each node keeps
// the first predecessor with the strictly smallest cost.  A primer pass over
// positions -ctx .. ctx-1 is traced back from the argmin of its incoming cost
// buffer - which, after the buffer swaps, holds the second-to-last step's
// costs - to the node before position 0; the closing pass runs 0 .. 255 from
// that node and its traceback gives every position's state and label.  The
// argmin breaks ties as the reference's shuffle-down reductions do: smallest
// (bitrev5(e % 1024 / 32), bitrev5(e % 32), e / 1024).
//
// MI355X mapping: one 1024-thread workgroup per tile (persistent over the
// tiles), the label table staged once per workgroup into LDS transposed to
// [node pair][predecessor][2] so a thread's labels of all predecessors of a
// node pair are one 8/16/32-byte read, both cost buffers in LDS, and each
// thread evaluating node pairs with packed fp16 arithmetic.  The decisions
// (K bits per node and step, packed as the reference packs them) go to a
// per-workgroup global workspace for the traceback.
//
// The same search runs against the two procedural EXL3 control codebooks of
// kquant/csrc/exl3_compat/quant/codebook.cuh (sqg_quantize.cu:261-330), whose
// label of a state is computed, not looked up (no LDS table then):
//   MCG  (1): x = state * 0xCBAC1FED mod 2^32; x = (x & 0x8fff8fff) ^ 0x3b603b60;
//             label = fp16(lo + hi), lo / hi the fp16 numbers x's two halves encode
//             (codebook.cuh:50-59, 64-79);
//   MUL1 (2): x = state * 0x83DCD12D mod 2^32; h = the fp16 1024 + (sum of x's
//             four bytes); label = fp16(h * fp16(0x1eee) + fp16(0xc931)), one
//             rounding (codebook.cuh:27-47, 80-92).
// The products of successive predecessors differ by C << (16 - K) mod 2^32,
// so each predecessor costs an add, as in qsrt_quantize_tiles_kernel.cuh:131-145.
#include "kq_internal.h"

namespace kq {
namespace viterbi {

constexpr int THREADS = 1024;
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int K> constexpr int edges() { return 65536 >> K; }
template <int K> constexpr int row_bytes() { return K == 2 ? edges<K>() / 4 : edges<K>() / 2; }

// E4M3 (fn) byte -> fp16, exact (labels are finite).
__device__ __forceinline__ _Float16 e4m3_to_f16(uint32_t b) {
  const uint32_t s = (b >> 7) & 1, e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;
  else v = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  return (_Float16)(s ? -v : v);
}

// The labels of predecessor k for nodes 2p and 2p + 1, from a 16-bit
// little-endian pair of E4M3 bytes: each byte's 7 magnitude bits shifted
// left by 7 are the fp16 pattern of its value / 2^8 (E4M3 exponent bias 7
// against fp16's 15; E4M3 subnormals land on fp16 subnormals), the sign bit
// moves to bit 15, and one exact packed multiply by 2^8 finishes.
__device__ __forceinline__ h2_t pair_labels(uint32_t word16) {
  const uint32_t t = (word16 & 0xffu) | ((word16 & 0xff00u) << 8);  // bytes -> [b0, 0, b1, 0]
  const uint32_t bits = ((t & 0x007f007fu) << 7) | ((t & 0x00800080u) << 8);
  h2_t scale;
  scale[0] = (_Float16)256.0f;
  scale[1] = (_Float16)256.0f;
  return __builtin_bit_cast(h2_t, bits) * scale;
}

__device__ __forceinline__ int bitrev5(int v) { return (int)(__builtin_bitreverse32((uint32_t)v) >> 27); }

// codebook ids: 0 = an SQG E4M3 table, 1 = MCG, 2 = MUL1
template <int CB> constexpr uint32_t cb_mult() { return CB == 1 ? 0xCBAC1FEDu : 0x83DCD12Du; }

// procedural labels of states s and s + 1 from their products x0 = s C and
// x1 = x0 + C (mod 2^32)
template <int CB>
__device__ __forceinline__ h2_t procedural_pair(uint32_t x0, uint32_t x1) {
  if constexpr (CB == 1) {
    const uint32_t v0 = (x0 & 0x8fff8fffu) ^ 0x3b603b60u;
    const uint32_t v1 = (x1 & 0x8fff8fffu) ^ 0x3b603b60u;
    const uint32_t lo = (v0 & 0xffffu) | (v1 << 16);
    const uint32_t hi = (v0 >> 16) | (v1 & 0xffff0000u);
    return __builtin_bit_cast(h2_t, lo) + __builtin_bit_cast(h2_t, hi);
  } else {
    // v_sad_u8 against zero: the sum of the four bytes, plus 0x6400 (1024.0)
    const uint32_t s0 = __builtin_amdgcn_sad_u8(x0, 0u, 0x6400u);
    const uint32_t s1 = __builtin_amdgcn_sad_u8(x1, 0u, 0x6400u);
    h2_t k_inv, k_bias;
    k_inv[0] = k_inv[1] = __builtin_bit_cast(_Float16, (uint16_t)0x1eee);   // 1 / 147.7
    k_bias[0] = k_bias[1] = __builtin_bit_cast(_Float16, (uint16_t)0xc931); // -10.38
    return __builtin_elementwise_fma(__builtin_bit_cast(h2_t, (s0 & 0xffffu) | (s1 << 16)), k_inv, k_bias);
  }
}

template <int K, int CB>
__global__ __launch_bounds__(THREADS) void sqg_viterbi_kernel(const float* __restrict__ tiles, int64_t n_tiles,
                                                              const uint8_t* __restrict__ lut, int ctx,
                                                              float* __restrict__ out_tiles,
                                                              int16_t* __restrict__ out_states,
                                                              uint8_t* __restrict__ dec_ws) {
  constexpr int E = edges<K>(), PAIRS = E / 2, PER = PAIRS / THREADS, Q = 1 << K;
  constexpr int KR = 16 - K, PSTEP = 1 << (16 - 2 * K), RB = row_bytes<K>();
  constexpr uint32_t CM = cb_mult<CB>(), CSTEP = CM << KR;
  static_assert(PER >= 1 && PAIRS % THREADS == 0, "node pairs per thread");
  __shared__ __attribute__((aligned(16))) uint8_t lab[CB == 0 ? 65536 : 16];  // [pair][k][2]
  __shared__ __attribute__((aligned(16))) _Float16 cost[2][E];
  __shared__ _Float16 w16[256];
  __shared__ float red_c[THREADS];
  __shared__ int red_i[THREADS];
  __shared__ int sh_edge;
  const int tid = threadIdx.x;
  uint8_t* dec = dec_ws + (int64_t)blockIdx.x * 256 * RB;

  if constexpr (CB == 0) {
    for (int s = tid; s < 65536; s += THREADS) {
      const int k = s >> KR, o = s & (E - 1);
      lab[(o >> 1) * (2 * Q) + 2 * k + (o & 1)] = lut[s];
    }
  }

  int cb = 0;  // cost[cb] = the buffer the next step writes; cost[cb ^ 1] its input
  for (int64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
    __syncthreads();
    if (tid < 256) w16[tid] = (_Float16)tiles[tile * 256 + tid];
    __syncthreads();

    // one pass: `steps` steps starting at position `roll`; decisions kept
    // from step trace_start on; pre_state >= 0 forces the first step's
    // predecessor
    auto pass = [&](int roll, int steps, int pre_state, int trace_start) {
      for (int i = 0; i < steps; ++i) {
        cb ^= 1;  // swap: the last step's output becomes this step's input
        const _Float16* prev = cost[cb ^ 1];
        _Float16* cur = cost[cb];
        const int ri = (i + roll) & 255;
        const _Float16 w = w16[ri];
        h2_t w2;
        w2[0] = w;
        w2[1] = w;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const int p = tid + THREADS * j;  // node pair (2p, 2p + 1)
          const int in0 = (2 * p) >> K;
          uint32_t words[Q / 2];  // two predecessors' label pairs per word
          uint32_t x0 = (uint32_t)(2 * p) * CM;  // product of state (0 << KR) | 2p
          if constexpr (CB != 0) {
          } else if constexpr (K == 2) {
            const u32x2_t v = *reinterpret_cast<const u32x2_t*>(lab + p * 2 * Q);
            words[0] = v[0];
            words[1] = v[1];
          } else if constexpr (K == 3) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(lab + p * 2 * Q);
#pragma unroll
            for (int q = 0; q < 4; ++q) words[q] = v[q];
          } else {
            const u32x4_t v0 = *reinterpret_cast<const u32x4_t*>(lab + p * 2 * Q);
            const u32x4_t v1 = *reinterpret_cast<const u32x4_t*>(lab + p * 2 * Q + 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              words[q] = v0[q];
              words[4 + q] = v1[q];
            }
          }
          h2_t best;
          int k0 = 0, k1 = 0;
#pragma unroll
          for (int k = 0; k < Q; ++k) {
            const int in = in0 + k * PSTEP;
            h2_t label;
            if constexpr (CB == 0) {
              label = pair_labels(words[k >> 1] >> (16 * (k & 1)));
            } else {
              label = procedural_pair<CB>(x0, x0 + CM);
              x0 += CSTEP;
            }
            const h2_t d = label - w2;
            h2_t err;
            if (i == 0) {
              err = d * d;
              if (pre_state >= 0 && in != pre_state) {
                err[0] = (_Float16)__builtin_inff();
                err[1] = (_Float16)__builtin_inff();
              }
            } else {
              const _Float16 c = prev[in];
              h2_t c2;
              c2[0] = c;
              c2[1] = c;
              err = __builtin_elementwise_fma(d, d, c2);
            }
            if (k == 0) {
              best = err;
            } else {
              if (err[0] < best[0]) { best[0] = err[0]; k0 = k; }
              if (err[1] < best[1]) { best[1] = err[1]; k1 = k; }
            }
          }
          *reinterpret_cast<h2_t*>(cur + 2 * p) = best;
          if (i >= trace_start) {
            if constexpr (K == 2) {
              // nodes 4m .. 4m + 3 share a byte: pair p and p + 1 (thread tid + 1)
              const int mine = k0 | (k1 << 2);
              const int next = __shfl_down(mine, 1);
              if ((p & 1) == 0) dec[ri * RB + (p >> 1)] = (uint8_t)(mine | (next << 4));
            } else {
              dec[ri * RB + p] = (uint8_t)(k0 | (k1 << 4));
            }
          }
        }
        __syncthreads();
      }
    };

    auto decision_at = [&](int ri, int edge) -> int {
      if constexpr (K == 2) return (dec[ri * RB + (edge >> 2)] >> ((edge & 3) * 2)) & 3;
      else return (dec[ri * RB + (edge >> 1)] >> ((edge & 1) * 4)) & 15;
    };

    // primer
    pass(256 - ctx, 2 * ctx, -1, ctx);
    {
      // argmin of the incoming buffer (the second-to-last step's costs)
      const _Float16* c = cost[cb ^ 1];
      float bc = __builtin_inff();
      int bi = -1;
      for (int e = tid; e < E; e += THREADS) {
        const float v = (float)c[e];
        if (v < bc) {
          bc = v;
          bi = e;
        }
      }
      red_c[tid] = bc;
      red_i[tid] = bi;
      __syncthreads();
      for (int span = THREADS / 2; span > 0; span >>= 1) {
        if (tid < span) {
          const float ca = red_c[tid], cb2 = red_c[tid + span];
          const int ia = red_i[tid], ib = red_i[tid + span];
          bool take_b;
          if (ib < 0) take_b = false;
          else if (ia < 0) take_b = true;
          else if (cb2 != ca) take_b = cb2 < ca;
          else {
            // equal costs: the reference's reduction order
            const int ta = ia & 1023, tb = ib & 1023;
            const int ka = (bitrev5(ta >> 5) << 5) | bitrev5(ta & 31);
            const int kb = (bitrev5(tb >> 5) << 5) | bitrev5(tb & 31);
            take_b = kb < ka || (kb == ka && (ib >> 10) < (ia >> 10));
          }
          if (take_b) {
            red_c[tid] = cb2;
            red_i[tid] = ib;
          }
        }
        __syncthreads();
      }
    }
    if (tid == 0) {
      int edge = red_i[0] < 0 ? 0 : red_i[0];
      for (int i = 2 * ctx - 1; i >= 0; --i) {
        const int ri = (i + 256 - ctx) & 255;
        edge = (decision_at(ri, edge) << (16 - 2 * K)) | (edge >> K);
        if (ri == 0) break;
      }
      sh_edge = edge;
    }
    __syncthreads();
    const int end_state = sh_edge;
    pass(0, 256, end_state, 0);
    if (tid == 0) {
      int edge = end_state;
      for (int i = 255; i >= 0; --i) {
        const int prev_edge = (decision_at(i, edge) << (16 - 2 * K)) | (edge >> K);
        const int state = ((prev_edge << K) | edge) & 0xffff;
        out_states[tile * 256 + i] = (int16_t)(uint16_t)state;
        if constexpr (CB == 0) {
          const int k = state >> KR, o = state & (E - 1);
          out_tiles[tile * 256 + i] = (float)e4m3_to_f16(lab[(o >> 1) * (2 * Q) + 2 * k + (o & 1)]);
        } else {
          const uint32_t x = (uint32_t)state * CM;
          out_tiles[tile * 256 + i] = (float)procedural_pair<CB>(x, x + CM)[0];
        }
        edge = prev_edge;
      }
    }
  }
}

}  // namespace viterbi
}  // namespace kq

using namespace kq::viterbi;

extern "C" int64_t kq_sqg_quantize_workspace_size(int bits, int workgroups) {
  if (bits < 2 || bits > 4 || workgroups <= 0) return -1;
  const int64_t rb = bits == 2 ? row_bytes<2>() : bits == 3 ? row_bytes<3>() : row_bytes<4>();
  return (int64_t)workgroups * 256 * rb;
}

namespace {

template <int CB>
void launch_viterbi(int bits, unsigned grid, hipStream_t st, const float* tiles, int64_t n_tiles, const uint8_t* lut,
                    int ctx, float* out_tiles, int16_t* out_states, uint8_t* ws) {
  if (bits == 2)
    sqg_viterbi_kernel<2, CB><<<grid, THREADS, 0, st>>>(tiles, n_tiles, lut, ctx, out_tiles, out_states, ws);
  else if (bits == 3)
    sqg_viterbi_kernel<3, CB><<<grid, THREADS, 0, st>>>(tiles, n_tiles, lut, ctx, out_tiles, out_states, ws);
  else
    sqg_viterbi_kernel<4, CB><<<grid, THREADS, 0, st>>>(tiles, n_tiles, lut, ctx, out_tiles, out_states, ws);
}

// shared checks of both entry points; 1 = nothing to do, 0 = launch, <0 = error
int check_search(const char* fn, const char* kname, const float* tiles, int64_t n_tiles, int bits,
                 int tailbite_context, float* out_tiles, int16_t* out_states, void* workspace,
                 int64_t workspace_bytes, int workgroups) {
  if (bits < 2 || bits > 4) return kq_fail(KQ_ERR_INVALID, "%s: %s supports K2--K4", fn, kname);
  if (tailbite_context < 1 || tailbite_context > 128)
    return kq_fail(KQ_ERR_INVALID, "%s: tailbite_context must be in 1..128", fn);
  if (n_tiles < 0 || workgroups <= 0) return kq_fail(KQ_ERR_INVALID, "%s: bad tile or workgroup count", fn);
  if (n_tiles == 0) return 1;
  if (!tiles || !out_tiles || !out_states || !workspace) return kq_fail(KQ_ERR_INVALID, "%s: null buffer", fn);
  if (workspace_bytes < kq_sqg_quantize_workspace_size(bits, workgroups))
    return kq_fail(KQ_ERR_INVALID, "%s: workspace too small", fn);
  return 0;
}

}  // namespace

extern "C" int kq_sqg_quantize_tiles(const float* tiles, int64_t n_tiles, const uint8_t* lut, int bits,
                                     int tailbite_context, float* out_tiles, int16_t* out_states, void* workspace,
                                     int64_t workspace_bytes, int workgroups, void* stream) {
  const char* fn = "kq_sqg_quantize_tiles";
  const int rc = check_search(fn, "SQG validation kernel", tiles, n_tiles, bits, tailbite_context, out_tiles,
                              out_states, workspace, workspace_bytes, workgroups);
  if (rc) return rc > 0 ? KQ_OK : rc;
  if (!lut) return kq_fail(KQ_ERR_INVALID, "%s: null buffer", fn);
  const unsigned grid = (unsigned)(n_tiles < workgroups ? n_tiles : workgroups);
  launch_viterbi<0>(bits, grid, (hipStream_t)stream, tiles, n_tiles, lut, tailbite_context, out_tiles, out_states,
                    (uint8_t*)workspace);
  return kq_check_launch(hipGetLastError(), fn);
}

extern "C" int kq_sqg_quantize_tiles_procedural(const float* tiles, int64_t n_tiles, int bits, int codebook,
                                                int tailbite_context, float* out_tiles, int16_t* out_states,
                                                void* workspace, int64_t workspace_bytes, int workgroups,
                                                void* stream) {
  const char* fn = "kq_sqg_quantize_tiles_procedural";
  if (codebook != 1 && codebook != 2)
    return kq_fail(KQ_ERR_INVALID, "%s: procedural codebook must be 1 (MCG) or 2 (MUL1)", fn);
  const int rc = check_search(fn, "procedural control", tiles, n_tiles, bits, tailbite_context, out_tiles,
                              out_states, workspace, workspace_bytes, workgroups);
  if (rc) return rc > 0 ? KQ_OK : rc;
  const unsigned grid = (unsigned)(n_tiles < workgroups ? n_tiles : workgroups);
  if (codebook == 1)
    launch_viterbi<1>(bits, grid, (hipStream_t)stream, tiles, n_tiles, nullptr, tailbite_context, out_tiles,
                      out_states, (uint8_t*)workspace);
  else
    launch_viterbi<2>(bits, grid, (hipStream_t)stream, tiles, n_tiles, nullptr, tailbite_context, out_tiles,
                      out_states, (uint8_t*)workspace);
  return kq_check_launch(hipGetLastError(), fn);
}
