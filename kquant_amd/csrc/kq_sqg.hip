// SQG E4M3 reconstruction tables: the rank permutations of the L16 trellis
// codewords, the finite-E4M3 normal staircase, its modal 12-bit compression
// (T12), the label gathers and the R44 research table.  Each table has
// 65,536 (or 4,096) entries and one thread per entry; they are built once per
// process, so the only aim is a handful of launches with exact integer and
// rounding behaviour.
#include "kq_common.h"
#include "kq_internal.h"

namespace kq {
namespace {

constexpr int TRANSITIONS = 1 << 16;

__device__ __forceinline__ uint32_t reverse_low_bits(uint32_t v, int bits) {
  return __brev(v) >> (32 - bits);
}

// Bijective xorshift/multiply mixer modulo 2^width (kquant/sqg_e4m3.py:38-60).
__device__ __forceinline__ uint32_t mix_width(uint32_t v, int width, uint32_t ma, uint32_t mb,
                                              int sa, int sb, int sc) {
  const uint32_t mask = (1u << width) - 1u;
  const int lim = width - 1;
  uint32_t r = v & mask;
  r ^= r >> min(max(sa, 1), lim);
  r = (r * (ma | 1u)) & mask;
  r ^= r >> min(max(sb, 1), lim);
  r = (r * (mb | 1u)) & mask;
  r ^= r >> min(max(sc, 1), lim);
  return r & mask;
}

// Pre-projection SQG rank (kquant/sqg_e4m3.py:408-438, same mixers as :96-115).
__device__ __forceinline__ uint32_t mix_rank(uint32_t t, int bits) {
  const int width = 16 - bits;
  const uint32_t branch_mask = (1u << bits) - 1u;
  const uint32_t history = t >> bits, branch = t & branch_mask;
  const uint32_t phase = mix_width(history, width, 0x65AF, 0x16BF, 6, 4, 5);
  const uint32_t syndrome = mix_width(history ^ 0x5105u, width, 0x8693, 0x2A21, 2, 4, 4) & branch_mask;
  const uint32_t stratum = (7u * (reverse_low_bits(branch, bits) ^ syndrome)) & branch_mask;
  return (stratum << width) | phase;
}

// Carry-mixed primary rank (kquant/sqg_e4m3.py:261-285): two triangular
// xorshifts over the history, an odd 32-bit affine multiply, phase from the
// low bits and the branch syndrome from the top bits.
__device__ __forceinline__ uint32_t xor_rank(uint32_t t, int bits) {
  const int width = 16 - bits;
  const uint32_t history_mask = (1u << width) - 1u;
  const uint32_t history = t >> bits, branch = t & ((1u << bits) - 1u);
  uint32_t mixed = history ^ (history >> 11);
  mixed ^= (mixed << 11) & history_mask;
  const uint32_t product = 0x3FA7D929u * mixed + 0xC928FD8Eu;  // mod 2^32
  const uint32_t phase = product & history_mask;
  const uint32_t syndrome = product >> (32 - bits);
  return ((reverse_low_bits(branch, bits) ^ syndrome) << width) | phase;
}

// KIND 0: xor rank; 1: mix rank; 2: K2 eight-stratum rank, the K3 mix rank of
// the codeword whose bit 2 and bit history_bit are swapped
// (kquant/sqg_e4m3.py:356-389).
template <int KIND>
__global__ __launch_bounds__(256) void sqg_rank_kernel(int bits, int history_bit,
                                                       int64_t* __restrict__ ranks) {
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  uint32_t r;
  if (KIND == 0) {
    r = xor_rank(t, bits);
  } else if (KIND == 1) {
    r = mix_rank(t, bits);
  } else {
    const uint32_t swap = ((t >> 2) ^ (t >> history_bit)) & 1u;
    r = mix_rank(t ^ (swap << 2) ^ (swap << history_bit), 3);
  }
  ranks[t] = (int64_t)r;
}

// Standard normal quantile in double precision.  Start: Abramowitz & Stegun
// 26.2.23 on the lower tail (|error| < 4.5e-4); then three Halley steps on
// Phi(x) - q, with the residual taken through erf near the centre and erfc in
// the tail so it keeps full relative accuracy.  Odd symmetry about 1/2 is
// exact because 1 - p is exact for the dyadic probabilities used here.
__device__ double normal_quantile(double p) {
  const bool upper = p > 0.5;
  const double q = upper ? 1.0 - p : p;  // lower-tail probability, exact
  const double t = sqrt(-2.0 * log(q));
  double x = -(t - (2.515517 + t * (0.802853 + t * 0.010328)) /
                       (1.0 + t * (1.432788 + t * (0.189269 + t * 0.001308))));
  const double sqrt_2pi = 2.5066282746310002;
  for (int it = 0; it < 3; ++it) {
    const double e = q > 0.25 ? 0.5 * erf(x * M_SQRT1_2) - (q - 0.5)
                              : 0.5 * erfc(-x * M_SQRT1_2) - q;
    const double u = e * sqrt_2pi * exp(0.5 * x * x);
    x -= u / (1.0 + 0.5 * x * u);
  }
  return upper ? -x : x;
}

// E4M3 byte with one canonical zero (kquant/sqg_e4m3.py:204-208).
__device__ __forceinline__ uint8_t canonical_e4m3(float v) {
  const uint32_t b = f32_to_e4m3_rne(v);
  return (uint8_t)((b & 0x7fu) == 0u ? 0u : b);
}

// Exact finite normal staircase: E4M3(float(1.5 * ndtri((rank + 0.5) / 2^16)))
// (kquant/sqg_e4m3.py:218-230).
__global__ __launch_bounds__(256) void sqg_normal_law_kernel(uint8_t* __restrict__ law) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  const double p = ((double)r + 0.5) / (double)TRANSITIONS;
  law[r] = canonical_e4m3((float)(1.5 * normal_quantile(p)));
}

// Canonical E4M3 bytes of caller-supplied fp32 rank-law values
// (kquant/sqg_e4m3.py:197-209).
__global__ __launch_bounds__(256) void sqg_finite_lut_kernel(const float* __restrict__ values,
                                                             uint8_t* __restrict__ law) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  law[r] = canonical_e4m3(values[r]);
}

__global__ void status_clear_kernel(uint32_t* status) { *status = 0u; }

// status bit 0: a NaN byte; bit 1: a decrease between neighbours
// (kquant/sqg_e4m3.py:209-213).
__global__ __launch_bounds__(256) void sqg_law_check_kernel(const uint8_t* __restrict__ law,
                                                            uint32_t* status) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  const uint32_t b = law[r];
  if ((b & 0x7fu) == 0x7fu) atomicOr(status, 1u);
  if (r + 1 < TRANSITIONS && e4m3_to_f32(law[r + 1]) < e4m3_to_f32(b)) atomicOr(status, 2u);
}

// Modal byte of each block of 16 consecutive ranks, ties to the lower byte
// (kquant/sqg_e4m3.py:243-257).
__global__ __launch_bounds__(256) void sqg_modal_kernel(const uint8_t* __restrict__ law,
                                                        uint8_t* __restrict__ t12) {
  const int blk = blockIdx.x * 256 + threadIdx.x;
  uint32_t v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = law[blk * 16 + i];
  uint32_t best = 0xffffffffu;  // key = (16 - count) << 8 | byte, minimised
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) c += v[j] == v[i];
    best = min(best, ((16u - c) << 8) | v[i]);
  }
  t12[blk] = (uint8_t)best;
}

// out[i] = lut[ranks[i] >> shift]; status bit 0: a NaN label, bit 1: a rank
// outside the table (kquant/sqg_e4m3.py:176-179, :289-291).
__global__ __launch_bounds__(256) void sqg_gather_kernel(const uint8_t* __restrict__ lut,
                                                         int64_t lut_len, int shift,
                                                         const int64_t* __restrict__ ranks,
                                                         int64_t n, uint8_t* __restrict__ out,
                                                         uint32_t* status) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = ranks[i];
  const int64_t j = r >> shift;
  if (r < 0 || j >= lut_len) {
    atomicOr(status, 2u);
    out[i] = 0;
    return;
  }
  const uint32_t b = lut[j];
  if ((b & 0x7fu) == 0x7fu) atomicOr(status, 1u);
  out[i] = (uint8_t)b;
}

// R44 research table (kquant/sqg_e4m3.py:75-127): clipped midpoint
// probability of the mix rank, a degree-4/4 rational inverse normal in
// a^2 (a = 2p - 1), times 1.5, rounded to float then E4M3.  Every product and
// sum is a separately rounded double operation, as in the reference's
// element-wise tensor arithmetic (no fused multiply-add).
__global__ __launch_bounds__(256) void sqg_r44_kernel(int bits, uint8_t* __restrict__ out,
                                                      uint32_t* status) {
  // Coefficients of the reference's R44 compander (kquant/sqg_e4m3.py:31-32).
  const double P[5] = {1.25667142, 2.87422731, -9.02398882, 5.36810336, -0.46703015};
  const double Q[5] = {1.0, 2.07630930, -8.08332684, 6.32135736, -1.31208298};
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  const uint32_t rank = mix_rank(t, bits);
  const double clip = 1.0 / 2048.0;
  double p = ((double)rank + 0.5) / (double)TRANSITIONS;
  p = fmin(fmax(p, clip), 1.0 - clip);
  const double a = __dadd_rn(__dmul_rn(2.0, p), -1.0);
  const double x = __dmul_rn(a, a);
  double num = P[4], den = Q[4];
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    num = __dadd_rn(__dmul_rn(num, x), P[i]);
    den = __dadd_rn(__dmul_rn(den, x), Q[i]);
  }
  const double g = __ddiv_rn(__dmul_rn(a, num), den);
  const float v = (float)__dmul_rn(1.5, g);
  if (!isfinite(v)) atomicOr(status, 1u);
  out[t] = (uint8_t)f32_to_e4m3_rne(v);
}

constexpr unsigned GRID = TRANSITIONS / 256;

int bad_bits(const char* who, int bits) {
  return kq_fail(KQ_ERR_INVALID, "%s: SQG supports integer K2, K3, or K4 (got %d)", who, bits);
}

}  // namespace
}  // namespace kq

using namespace kq;

extern "C" int kq_sqg_rank_permutation(int kind, int bits, int history_bit, int64_t* ranks,
                                       void* stream) {
  hipStream_t st = (hipStream_t)stream;
  if (kind == KQ_SQG_RANK_K2_OCTILE) {
    if (history_bit < 2 || history_bit > 15)
      return kq_fail(KQ_ERR_INVALID,
                     "kq_sqg_rank_permutation: K2 eight-stratum history bit must be in [2, 15]");
    sqg_rank_kernel<2><<<GRID, 256, 0, st>>>(2, history_bit, ranks);
    return kq_check_launch(hipGetLastError(), "kq_sqg_rank_permutation");
  }
  if (bits < 2 || bits > 4) return bad_bits("kq_sqg_rank_permutation", bits);
  if (kind == KQ_SQG_RANK_XOR)
    sqg_rank_kernel<0><<<GRID, 256, 0, st>>>(bits, 0, ranks);
  else if (kind == KQ_SQG_RANK_MIX)
    sqg_rank_kernel<1><<<GRID, 256, 0, st>>>(bits, 0, ranks);
  else
    return kq_fail(KQ_ERR_INVALID, "kq_sqg_rank_permutation: unknown kind %d", kind);
  return kq_check_launch(hipGetLastError(), "kq_sqg_rank_permutation");
}

extern "C" int kq_sqg_normal_rank_law(uint8_t* law, void* stream) {
  sqg_normal_law_kernel<<<GRID, 256, 0, (hipStream_t)stream>>>(law);
  return kq_check_launch(hipGetLastError(), "kq_sqg_normal_rank_law");
}

extern "C" int kq_sqg_finite_rank_lut(const float* values, uint8_t* law, void* stream) {
  if (kq_misaligned(values, 4))
    return kq_fail(KQ_ERR_INVALID, "kq_sqg_finite_rank_lut: values must be 4-byte aligned");
  sqg_finite_lut_kernel<<<GRID, 256, 0, (hipStream_t)stream>>>(values, law);
  return kq_check_launch(hipGetLastError(), "kq_sqg_finite_rank_lut");
}

extern "C" int kq_sqg_check_rank_law(const uint8_t* law, uint32_t* status, void* stream) {
  if (!status || kq_misaligned(status, 4))
    return kq_fail(KQ_ERR_INVALID, "kq_sqg_check_rank_law: status must be a 4-byte aligned word");
  hipStream_t st = (hipStream_t)stream;
  status_clear_kernel<<<1, 1, 0, st>>>(status);
  sqg_law_check_kernel<<<GRID, 256, 0, st>>>(law, status);
  return kq_check_launch(hipGetLastError(), "kq_sqg_check_rank_law");
}

extern "C" int kq_sqg_modal_compress(const uint8_t* law, uint8_t* t12, void* stream) {
  sqg_modal_kernel<<<(TRANSITIONS / 16) / 256, 256, 0, (hipStream_t)stream>>>(law, t12);
  return kq_check_launch(hipGetLastError(), "kq_sqg_modal_compress");
}

extern "C" int kq_sqg_gather(const uint8_t* lut, int64_t lut_len, int shift, const int64_t* ranks,
                             int64_t n, uint8_t* out, uint32_t* status, void* stream) {
  if (lut_len < 1 || n < 0 || shift < 0 || shift > 16)
    return kq_fail(KQ_ERR_INVALID, "kq_sqg_gather: bad sizes (lut_len=%lld n=%lld shift=%d)",
                   (long long)lut_len, (long long)n, shift);
  if (!status || kq_misaligned(status, 4) || kq_misaligned(ranks, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_sqg_gather: misaligned ranks or status");
  hipStream_t st = (hipStream_t)stream;
  status_clear_kernel<<<1, 1, 0, st>>>(status);
  if (n > 0)
    sqg_gather_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(lut, lut_len, shift, ranks, n,
                                                                    out, status);
  return kq_check_launch(hipGetLastError(), "kq_sqg_gather");
}

extern "C" int kq_sqg_r44_bytes(int bits, uint8_t* out, uint32_t* status, void* stream) {
  if (bits < 2 || bits > 4) return bad_bits("kq_sqg_r44_bytes", bits);
  if (!status || kq_misaligned(status, 4))
    return kq_fail(KQ_ERR_INVALID, "kq_sqg_r44_bytes: status must be a 4-byte aligned word");
  hipStream_t st = (hipStream_t)stream;
  status_clear_kernel<<<1, 1, 0, st>>>(status);
  sqg_r44_kernel<<<GRID, 256, 0, st>>>(bits, out, status);
  return kq_check_launch(hipGetLastError(), "kq_sqg_r44_bytes");
}
