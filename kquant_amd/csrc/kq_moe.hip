// Routed MoE expert forward with MXFP4 weights (W4A16).
//
// Semantics: scripts/closure_exl3_layer.py:557-598 (_reference_rank, tp = 1):
// for every (token, slot) pair routed to expert e,
//   gate = x W1_e^T, up = x W3_e^T (w13 rows [0, I) gate, [I, 2I) up),
//   a = act(gate, up) (SiTU kquant/tp_simulator.py:83-94, or SwiGLU), bf16,
//   partial = a W2_e^T, contribution = route_weight * partial (fp32),
//   out[token] = sum over its slots (fp32).
//
// Pipeline (all on one stream, all buffers in the caller's workspace):
//   1. route_hist / route_scan / route_scatter: deterministic counting sort of
//      the T*topk pairs by expert (stable in pair order), each pair's sorted
//      position, the list of experts with 1..16 pairs ("small") and the
//      (expert, row-tile) list of the others.
//   2. gate/up: small experts on a GEMV-shaped MFMA kernel (16 token slots,
//      weights streamed once with 16-byte loads, K split over 8 waves);
//      large experts on a persistent 256x256-tile grouped GEMM (gathered
//      token rows and packed weights loaded straight into LDS).  Both fuse
//      the activation and write bf16 intermediates in expert-sorted order.
//   3. down: same two shapes over W2; the epilogue writes one fp32 row per
//      pair, in expert-sorted order (row = the pair's sorted position, so
//      the epilogue needs no index or weight loads).
//   4. combine: out[t] = sum over its slots, in slot order, of
//      route_weight * the pair's row (each product rounded to fp32 before
//      the sum, as when the down epilogue applied the weight).
// No atomics touch floating-point data, so results are bitwise reproducible.
#include "kq_dma.h"
#include "kq_gemm.h"
#include "kq_internal.h"
#include "kq_act.h"

#include <mutex>

namespace kq {
namespace moe {

constexpr int SMALL_MAX = 16;        // pairs per expert handled by the GEMV path
constexpr int DECODE_MAX_PAIRS = 256;  // at most this many pairs: decode routing, all GEMV
constexpr int PREP = 256;            // pairs per prep block
constexpr int MAX_EXPERTS = 4096;
constexpr int BM = 256, BN = 256, BK = 64, THREADS = 512;  // large tiles
constexpr int DMA_BM = 128, DMA_BN = 512;  // tiles of the bf16-activation direct-to-LDS grouped GEMM
constexpr int A_ROW = BK * 2 + 16;
constexpr int B_ROW = 36;            // 32 packed bytes + pad
constexpr int A_BYTES = BM * A_ROW;
constexpr int B_BYTES = BN * B_ROW;
constexpr int S_BYTES = BN * 2;
constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;

struct Layout {
  size_t counts, offsets, block_counts, sorted, pos, small_list, large_tiles, meta, act, y;
  size_t xq, xs, aq, as;  // MX-quantized tokens / intermediates (activation-quantized modes)
  size_t rank_of, routed, s13, s2;  // routed-expert ranks and expanded scale slots (X4T scales)
  size_t total;
  int64_t pairs, nblk, max_small, max_large, max_list, max_routed;
};

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static Layout make_layout(int64_t tokens, int topk, int experts, int64_t hidden, int64_t inter,
                          bool x4t = false) {
  Layout L;
  L.pairs = tokens * topk;
  // experts on the grouped GEMM (more than SMALL_MAX pairs; none when decoding)
  L.max_routed = L.pairs <= DECODE_MAX_PAIRS ? 0
               : L.pairs / (SMALL_MAX + 1) < experts ? L.pairs / (SMALL_MAX + 1) : experts;
  L.nblk = (L.pairs + PREP - 1) / PREP;
  L.max_small = L.pairs < experts ? L.pairs : experts;
  L.max_large = L.pairs / (SMALL_MAX + 1) + L.pairs / DMA_BM + 1;
  // GEMV list entries: one per small expert, or (decode) one per 16 pairs of
  // every routed expert, at most experts + pairs / 16
  L.max_list = L.pairs <= DECODE_MAX_PAIRS ? L.max_small + L.pairs / SMALL_MAX + 1 : L.max_small;
  const int64_t list_cap = L.max_list > experts ? L.max_list : experts;
  size_t o = 0;
  L.counts = o;       o = align256(o + sizeof(int) * experts);
  L.offsets = o;      o = align256(o + sizeof(int) * (experts + 1));
  L.block_counts = o; o = align256(o + sizeof(int) * (size_t)L.nblk * experts);
  L.sorted = o;       o = align256(o + sizeof(int) * (size_t)L.pairs);
  L.pos = o;          o = align256(o + sizeof(int) * (size_t)L.pairs);
  L.small_list = o;   o = align256(o + sizeof(int) * 3 * (size_t)list_cap);
  L.large_tiles = o;  o = align256(o + sizeof(int) * 2 * (size_t)L.max_large);
  L.meta = o;         o = align256(o + sizeof(int) * 4);
  L.act = o;          o = align256(o + 2 * (size_t)L.pairs * inter);
  L.y = o;            o = align256(o + 4 * (size_t)L.pairs * hidden);
  L.xq = o;           o = align256(o + (size_t)tokens * hidden);
  L.xs = o;           o = align256(o + (size_t)tokens * hidden / 32);
  L.aq = o;           o = align256(o + (size_t)L.pairs * inter);
  L.as = o;           o = align256(o + (size_t)L.pairs * inter / 32);
  L.rank_of = L.routed = L.s13 = L.s2 = o;
  if (x4t) {  // a scale slot per grouped-GEMM expert: w13 [2I, H/32] and w2 [H, I/32] scale tiles
    L.rank_of = o;    o = align256(o + sizeof(int) * experts);
    L.routed = o;     o = align256(o + sizeof(int) * (size_t)L.max_routed);
    L.s13 = o;        o = align256(o + (size_t)L.max_routed * 2 * inter * (hidden / 32));
    L.s2 = o;         o = align256(o + (size_t)L.max_routed * hidden * (inter / 32));
  }
  L.total = o;
  return L;
}

// ------------------------------------------------------------ activations --
// ------------------------------------------------------------ routing prep --
__global__ __launch_bounds__(PREP) void route_hist_kernel(const int* __restrict__ ids, int64_t pairs,
                                                          int experts, int* __restrict__ block_counts) {
  __shared__ int cnt[MAX_EXPERTS];
  for (int e = threadIdx.x; e < experts; e += PREP) cnt[e] = 0;
  __syncthreads();
  const int64_t p = (int64_t)blockIdx.x * PREP + threadIdx.x;
  if (p < pairs) {
    const int e = ids[p];
    if (e >= 0 && e < experts) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += PREP)
    block_counts[(int64_t)blockIdx.x * experts + e] = cnt[e];
}

// Exclusive scan of v[0..n) (n <= 4 * 1024) in place in LDS by 1024 threads;
// returns the total.
__device__ int block_exclusive_scan(int* v, int n, int* scratch /*[1024]*/) {
  const int t = threadIdx.x;
  int local[4];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t * 4 + i;
    local[i] = idx < n ? v[idx] : 0;
    sum += local[i];
  }
  scratch[t] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int add = t >= off ? scratch[t - off] : 0;
    __syncthreads();
    scratch[t] += add;
    __syncthreads();
  }
  int run = scratch[t] - sum;  // exclusive prefix of this thread's chunk
  const int total = scratch[1023];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = t * 4 + i;
    if (idx < n) v[idx] = run;
    run += local[i];
  }
  __syncthreads();
  return total;
}

// Ranks of the grouped-GEMM experts (count > SMALL_MAX) in ascending expert
// order, for the per-call expansion of compressed scales: rank_of[e] for each
// such e, routed[r] = the expert of rank r, -1 for r in [their number,
// max_routed).
// Called by all 1024 threads after counts[0, experts) are written; tmp is an
// LDS array of `experts` ints that is overwritten and then rebuilt.
__device__ void routed_ranks(const int* counts, int experts, int* rank_of, int* routed, int max_routed,
                             int* tmp, int* scratch) {
  int keep[4];
  for (int i = 0; i < 4; ++i) {
    const int e = threadIdx.x + 1024 * i;
    keep[i] = e < experts ? tmp[e] : 0;
    if (e < experts) tmp[e] = counts[e] > SMALL_MAX ? 1 : 0;
  }
  __syncthreads();
  const int nrouted = block_exclusive_scan(tmp, experts, scratch);
  for (int i = 0; i < 4; ++i) {
    const int e = threadIdx.x + 1024 * i;
    if (e < experts && counts[e] > SMALL_MAX) {
      rank_of[e] = tmp[e];
      if (tmp[e] < max_routed) routed[tmp[e]] = e;
    }
  }
  for (int r = nrouted + (int)threadIdx.x; r < max_routed; r += 1024) routed[r] = -1;
  __syncthreads();
  for (int i = 0; i < 4; ++i) {
    const int e = threadIdx.x + 1024 * i;
    if (e < experts) tmp[e] = keep[i];
  }
  __syncthreads();
}

__global__ __launch_bounds__(1024) void route_scan_kernel(
    int* __restrict__ block_counts, int nblk, int experts, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ small_list, int* __restrict__ large_tiles,
    int* __restrict__ meta, int max_large, int* __restrict__ rank_of, int* __restrict__ routed,
    int max_routed, int bm) {
  __shared__ int s_cnt[MAX_EXPERTS];
  __shared__ int s_small[MAX_EXPERTS];
  __shared__ int s_tiles[MAX_EXPERTS];
  __shared__ int scratch[1024];
  for (int e = threadIdx.x; e < experts; e += 1024) {
    // column scan of this expert's per-block counts, 16 independent loads at
    // a time so their latencies overlap
    int s = 0;
    for (int b0 = 0; b0 < nblk; b0 += 16) {
      int c[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        c[i] = b0 + i < nblk ? block_counts[(int64_t)(b0 + i) * experts + e] : 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (b0 + i < nblk) block_counts[(int64_t)(b0 + i) * experts + e] = s;
        s += c[i];
      }
    }
    counts[e] = s;
    s_cnt[e] = s;
    s_small[e] = (s >= 1 && s <= SMALL_MAX) ? 1 : 0;
    s_tiles[e] = s > SMALL_MAX ? (s + bm - 1) / bm : 0;
  }
  __syncthreads();
  if (rank_of) routed_ranks(counts, experts, rank_of, routed, max_routed, s_small, scratch);
  const int npairs = block_exclusive_scan(s_cnt, experts, scratch);
  const int nsmall = block_exclusive_scan(s_small, experts, scratch);
  const int ntiles = block_exclusive_scan(s_tiles, experts, scratch);
  for (int e = threadIdx.x; e < experts; e += 1024) {
    offsets[e] = s_cnt[e];
    const int n = counts[e];
    if (n >= 1 && n <= SMALL_MAX) {
      small_list[3 * s_small[e]] = e;
      small_list[3 * s_small[e] + 1] = s_cnt[e];
      small_list[3 * s_small[e] + 2] = n;
    }
    if (n > SMALL_MAX) {
      const int nt = (n + bm - 1) / bm;
      for (int t = 0; t < nt; ++t) {
        const int slot = s_tiles[e] + t;
        if (slot < max_large) {
          large_tiles[2 * slot] = e;
          large_tiles[2 * slot + 1] = t * bm;
        }
      }
    }
  }
  for (int i = nsmall + (int)threadIdx.x; i < experts; i += 1024) small_list[3 * i] = -1;
  if (threadIdx.x == 0) {
    offsets[experts] = npairs;
    meta[0] = nsmall;
    meta[1] = ntiles < max_large ? ntiles : max_large;
    meta[2] = npairs;
  }
}

__global__ __launch_bounds__(PREP) void route_scatter_kernel(
    const int* __restrict__ ids, int64_t pairs, int experts, const int* __restrict__ offsets,
    const int* __restrict__ block_counts, int* __restrict__ sorted, int* __restrict__ pos) {
  __shared__ int ex[PREP];
  const int64_t p = (int64_t)blockIdx.x * PREP + threadIdx.x;
  int e = p < pairs ? ids[p] : -1;
  if (e < 0 || e >= experts) e = -1;
  ex[threadIdx.x] = e;
  __syncthreads();
  if (e >= 0) {
    int rank = 0;
    for (int j = 0; j < (int)threadIdx.x; ++j) rank += ex[j] == e ? 1 : 0;
    const int at = offsets[e] + block_counts[(int64_t)blockIdx.x * experts + e] + rank;
    sorted[at] = (int)p;
    if (pos) pos[p] = at;
  }
}

// Whole routing prep in one workgroup for up to PREP_ONE pairs: histogram,
// scans and the stable scatter (rank = earlier pairs with the same expert).
constexpr int PREP_ONE = 1024;
__global__ __launch_bounds__(1024) void route_prep_one_kernel(
    const int* __restrict__ ids, int pairs, int experts, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ sorted, int* __restrict__ small_list,
    int* __restrict__ large_tiles, int* __restrict__ meta, int max_large, int* __restrict__ rank_of,
    int* __restrict__ routed, int max_routed, int bm, int* __restrict__ pos) {
  __shared__ int s_cnt[MAX_EXPERTS];
  __shared__ int s_small[MAX_EXPERTS];
  __shared__ int s_tiles[MAX_EXPERTS];
  __shared__ int s_ids[PREP_ONE];
  __shared__ int scratch[1024];
  const int t = threadIdx.x;
  for (int e = t; e < experts; e += 1024) s_cnt[e] = 0;
  int my = -1;
  if (t < pairs) {
    my = ids[t];
    if (my < 0 || my >= experts) my = -1;
  }
  s_ids[t] = my;
  __syncthreads();
  if (my >= 0) atomicAdd(&s_cnt[my], 1);
  __syncthreads();
  for (int e = t; e < experts; e += 1024) {
    const int c = s_cnt[e];
    counts[e] = c;
    s_small[e] = (c >= 1 && c <= SMALL_MAX) ? 1 : 0;
    s_tiles[e] = c > SMALL_MAX ? (c + bm - 1) / bm : 0;
  }
  __syncthreads();
  if (rank_of) routed_ranks(counts, experts, rank_of, routed, max_routed, s_small, scratch);
  const int npairs = block_exclusive_scan(s_cnt, experts, scratch);
  const int nsmall = block_exclusive_scan(s_small, experts, scratch);
  const int ntiles = block_exclusive_scan(s_tiles, experts, scratch);
  for (int e = t; e < experts; e += 1024) {
    offsets[e] = s_cnt[e];
    const int c = counts[e];
    if (c >= 1 && c <= SMALL_MAX) {
      small_list[3 * s_small[e]] = e;
      small_list[3 * s_small[e] + 1] = s_cnt[e];
      small_list[3 * s_small[e] + 2] = c;
    }
    if (c > SMALL_MAX) {
      const int nt = (c + bm - 1) / bm;
      for (int k = 0; k < nt; ++k) {
        const int slot = s_tiles[e] + k;
        if (slot < max_large) {
          large_tiles[2 * slot] = e;
          large_tiles[2 * slot + 1] = k * bm;
        }
      }
    }
  }
  if (my >= 0) {
    int rank = 0;
    for (int j = 0; j < t; ++j) rank += s_ids[j] == my ? 1 : 0;
    sorted[s_cnt[my] + rank] = t;
    if (pos) pos[t] = s_cnt[my] + rank;
  }
  for (int i = nsmall + t; i < experts; i += 1024) small_list[3 * i] = -1;
  if (t == 0) {
    offsets[experts] = npairs;
    meta[0] = nsmall;
    meta[1] = ntiles < max_large ? ntiles : max_large;
    meta[2] = npairs;
  }
}

// Routing for a few pairs (decode): one workgroup, one pair per thread, no
// per-expert work.  The pairs are sorted stably by expert, and every routed
// expert, whatever its count, is listed in ascending expert order as entries
// (expert, first sorted position, count <= 16), one per 16 of its pairs.
__global__ __launch_bounds__(DECODE_MAX_PAIRS) void route_decode_kernel(
    const int* __restrict__ ids, int pairs, int experts, int* __restrict__ sorted,
    int* __restrict__ small_list, int max_list, int* __restrict__ meta, int* __restrict__ pos) {
  // ids past `pairs` are -1 and the loops run over whole groups of four
  // (one 16-byte LDS read each), so no read waits on the previous one
  __shared__ __attribute__((aligned(16))) int s_id[DECODE_MAX_PAIRS];
  __shared__ __attribute__((aligned(16))) int s_first[DECODE_MAX_PAIRS];  // expert at its first pair, else -1
  __shared__ __attribute__((aligned(16))) int s_nent[DECODE_MAX_PAIRS];   // list entries of that expert
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  const int t = threadIdx.x;
  const int pairs4 = (pairs + 3) & ~3;
  int my = t < pairs ? ids[t] : -1;
  if (my < 0 || my >= experts) my = -1;
  s_id[t] = my;
  __syncthreads();
  int rank = 0, below = 0, cnt = 0;
#pragma unroll 4
  for (int j4 = 0; j4 < pairs4; j4 += 4) {
    const i32x4 v4 = *reinterpret_cast<const i32x4*>(s_id + j4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = v4[i];
      rank += (j4 + i < t && v == my) ? 1 : 0;
      below += (v >= 0 && v < my) ? 1 : 0;
      cnt += v == my ? 1 : 0;
    }
  }
  const bool first = my >= 0 && rank == 0;
  const int nent = (cnt + SMALL_MAX - 1) / SMALL_MAX;
  s_first[t] = first ? my : -1;
  s_nent[t] = first ? nent : 0;
  __syncthreads();
  int e0 = 0, nlist = 0;
#pragma unroll 4
  for (int j4 = 0; j4 < pairs4; j4 += 4) {
    const i32x4 v4 = *reinterpret_cast<const i32x4*>(s_first + j4);
    const i32x4 n4 = *reinterpret_cast<const i32x4*>(s_nent + j4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      nlist += n4[i];
      e0 += (v4[i] >= 0 && v4[i] < my) ? n4[i] : 0;
    }
  }
  if (my >= 0) {
    sorted[below + rank] = t;
    pos[t] = below + rank;
  }
  if (first) {
    for (int q = 0; q < nent; ++q) {
      small_list[3 * (e0 + q)] = my;
      small_list[3 * (e0 + q) + 1] = below + SMALL_MAX * q;
      small_list[3 * (e0 + q) + 2] = cnt - SMALL_MAX * q < SMALL_MAX ? cnt - SMALL_MAX * q : SMALL_MAX;
    }
  }
  for (int i = nlist + t; i < max_list; i += DECODE_MAX_PAIRS) small_list[3 * i] = -1;
  if (t == 0) {
    meta[0] = nlist;
    meta[1] = 0;
  }
}

using gemm::bf16x8_t;
using gemm::u32x2_t;
using gemm::u32x4_t;
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ------------------------------------------- fused X4T scales (GEMV path) --
// With X4T-coded scales the GEMV workgroup decodes the scales of its own row
// blocks into LDS before its K loop: no separate launch and no dense scale
// traffic.  Planes: w1 and w3 (gate and up rows) for gate/up, w2 for down.
struct X4TGemv {
  const uint8_t* fixed[2];    // [experts][tiles][16 (1 + ceil(cols / 8))]
  const uint32_t* exc[2];     // matrix-local position | value << 24
  const uint32_t* idx[2];     // [experts * tiles + 1] first exception per tile
  int64_t tiles;              // 16-row tiles per matrix
  int cols;                   // scale columns, K / 32 (<= 255)
};

// Registers carried from the prologue's loads to its LDS work.
struct X4TPending {
  u32x4_t piece[2];
  uint32_t xr;
};

// LDS use of the fused decode for nrb row blocks: decoded scale tiles
// [nrb][nchunk][64], the staged fixed tiles, the exception ranges.
static inline size_t x4t_gemv_lds(int nrb, int64_t nchunk, int cols) {
  return (size_t)nrb * nchunk * 64 + (size_t)nrb * 16 * (1 + (cols + 7) / 8) + 8 * (size_t)nrb;
}

// Row block q of the workgroup (q = row group of waves * NB + block b): its
// plane (1 = up rows of w13) and its tile in that plane.
template <bool GATEUP, int NB, int NBP>
__device__ __forceinline__ int64_t x4t_rb_tile(int q, int64_t tile0, bool& up) {
  const int b = q % NB;
  up = GATEUP && b >= NBP;
  return tile0 + (q / NB) * NBP + (up ? b - NBP : b);
}

// LDS barrier without waiting for outstanding global loads: this wave's LDS
// accesses complete, then s_barrier; compiler memory clobbers on both sides.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// First half: the loads of the row blocks' fixed tiles and exception ranges
// (issued before the weight prefetch, so waiting for them leaves it in flight).
template <bool GATEUP, int NB, int NBP, int NRB, int T>
__device__ __forceinline__ void x4t_issue(const X4TGemv& xg, int e, int64_t tile0, X4TPending& pd) {
  const int tp = 1 + ((xg.cols + 7) >> 3);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = threadIdx.x + u * T;
    if (i < NRB * tp) {
      const int q = i / tp, pc = i - q * tp;
      bool up;
      const int64_t t = x4t_rb_tile<GATEUP, NB, NBP>(q, tile0, up);
      const uint8_t* f = up ? xg.fixed[1] : xg.fixed[0];
      pd.piece[u] = *reinterpret_cast<const u32x4_t*>(f + ((int64_t)e * xg.tiles + t) * (16 * tp) + 16 * pc);
    }
  }
  if (threadIdx.x < 2 * NRB) {
    bool up;
    const int64_t t = x4t_rb_tile<GATEUP, NB, NBP>((int)threadIdx.x >> 1, tile0, up);
    const uint32_t* ix = up ? xg.idx[1] : xg.idx[0];
    pd.xr = ix[(int64_t)e * xg.tiles + t + (threadIdx.x & 1)];
  }
}

// Second half: decode into sl[(q * nchunk + chunk) * 64 + l] (the scale-tile
// layout: byte l = scale[16 tile + l % 16][4 chunk + l / 16]) and patch the
// exceptions; ends with a barrier after which every wave may read sl.
template <bool GATEUP, int NB, int NBP, int NRB, int T>
__device__ __forceinline__ void x4t_finish(const X4TGemv& xg, int e, int64_t tile0, int nchunk,
                                           const X4TPending& pd, uint8_t* lds) {
  constexpr int U = 4;
  const int tid = threadIdx.x;
  const int cols = xg.cols, sb = (cols + 7) >> 3, tp = 1 + sb, span = 16 * cols;
  uint8_t* sl = lds;
  uint8_t* fl = lds + (size_t)NRB * nchunk * 64;
  uint32_t* xl = reinterpret_cast<uint32_t*>(fl + NRB * 16 * tp);
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if (tid + u * T < NRB * tp) *reinterpret_cast<u32x4_t*>(fl + 16 * (tid + u * T)) = pd.piece[u];
  if (tid < 2 * NRB) xl[tid] = pd.xr;
  lds_barrier();
  int lo[NRB], pre[NRB + 1];
  pre[0] = 0;
#pragma unroll
  for (int q = 0; q < NRB; ++q) {
    lo[q] = (int)xl[2 * q];
    const int hi = (int)xl[2 * q + 1];
    pre[q + 1] = pre[q] + (hi > lo[q] ? hi - lo[q] : 0);
  }
  const int total = pre[NRB];
  uint32_t wv[U];
  int qv[U];
  auto fetch = [&](int base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = base + tid + u * T;
      qv[u] = -1;
      int src = 0;
#pragma unroll
      for (int q = 0; q < NRB; ++q)
        if (k >= pre[q] && k < pre[q + 1]) {
          qv[u] = q;
          src = lo[q] + (k - pre[q]);
        }
      if (qv[u] >= 0) {
        const bool up = GATEUP && (qv[u] % NB) >= NBP;
        wv[u] = (up ? xg.exc[1] : xg.exc[0])[src];
      }
    }
  };
  fetch(0);
#pragma unroll
  for (int q = 0; q < NRB; ++q) {
    const uint8_t* f = fl + q * 16 * tp;
    for (int j = tid; j < nchunk * 16; j += T) {
      const int w = j & 15, r0 = 4 * (w & 3), c = 4 * (j >> 4) + (w >> 2);
      const uint32_t base4 = *reinterpret_cast<const uint32_t*>(f + r0);
      const uint8_t* sel = f + 16 + r0 * sb + (c >> 3);
      uint32_t v = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v |= (((base4 >> (8 * i)) + ((sel[i * sb] >> (c & 7)) & 1)) & 0xffu) << (8 * i);
      *reinterpret_cast<uint32_t*>(sl + (q * nchunk + (j >> 4)) * 64 + 4 * w) = v;
    }
  }
  lds_barrier();
  for (int base = 0; base < total; base += U * T) {
    if (base > 0) fetch(base);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (qv[u] < 0) continue;
      bool up;
      const int64_t t = x4t_rb_tile<GATEUP, NB, NBP>(qv[u], tile0, up);
      const uint32_t off = (wv[u] & 0xffffffu) - (uint32_t)(t * span);  // wraps past the tile when outside
      if (off >= (uint32_t)span) continue;
      const int r = (int)off / cols, c = (int)off - r * cols;
      sl[(qv[u] * nchunk + (c >> 2)) * 64 + (c & 3) * 16 + r] = (uint8_t)(wv[u] >> 24);
    }
  }
  lds_barrier();
}

// ------------------------------------------------- GEMV-shaped small path --
// One workgroup: up to 16 pairs of one expert (a list entry (expert, first
// sorted position, count)).  Its S * RW waves form RW row
// groups of S waves; the S waves of a group split K, and each holds NBP
// 16-row blocks per projection (GATEUP: gate rows c and up rows I + c), so a
// workgroup covers CH = RW * 16 * NBP output channels.  Weights stream from
// the kq_mx_tile_weights layout with one 16-byte non-temporal load per lane
// per 1 KiB tile: lane (r, g) of a tile holds weight row r, k 32 g .. 32 g + 31
// of the 128-k chunk, and its own E8M0 byte.  They are expanded to bf16 in
// registers (gfx950 scaled converts; E2M1 x 2^s is exact in bf16) and fed to
// v_mfma_f32_16x16x32_bf16 with the bf16 activation rows read as they are, so
// every product is exact and the accumulation is fp32.  MFMA t (0..3) of a
// chunk takes k = 32 g + 8 t + [0, 8) from lane half-group g of both
// operands, which puts each lane's 16 weight bytes and its 64 activation bytes
// in one contiguous piece.  Loads run P 128-k steps ahead of the MFMAs through
// a ring of P + 1 register buffers (straight-line code for a compile-time
// step count, so the compiler counts the outstanding loads exactly).
//
// GATEUP: rows of w13, output act -> bf16 intermediates.
// !GATEUP: rows of w2, output partial -> fp32 pair rows (sorted order).
// ROUTE (a decode of at most 64 pairs): no routing launch and no list.  The
// pairs routed to one expert, in pair order, form entries of up to
// SMALL_MAX token slots as in the listed form; workgroup x runs the entry
// that pair x starts (x's rank among its expert's pairs is a multiple of
// SMALL_MAX) and exits otherwise, so every expert's weights are read once.
// Slot m holds the entry's m-th pair, whose intermediate goes to row = pair
// index.  Each MFMA output row depends only on its own A row, so the values
// are those of the listed form.  With X4T-coded scales the workgroup decodes
// its expert's scale tiles as in the listed form.
struct DecodeRouteArgs {
  const int* ids;
  int experts;
  int pairs;  // entries of ids (<= 64)
};

// Pair of token slot m (< SMALL_MAX) of the entry pair x starts among the
// pairs routed to expert e (ids[0 .. pairs)), the entry's slot count in n;
// -1 when x does not start an entry.  Every lane of a wave calls it.
__device__ __forceinline__ int route_entry_slot(const int* __restrict__ ids, int pairs, int x, int e, int m,
                                                int& n) {
  const int lane = threadIdx.x & 63;
  const int ej = lane < pairs ? ids[lane] : -1;
  const uint64_t same = __ballot(ej == e);
  const int rank = __popcll(same & ((1ull << x) - 1));
  if (rank % SMALL_MAX != 0) return -1;
  const int cnt = __popcll(same) - rank;
  n = cnt < SMALL_MAX ? cnt : SMALL_MAX;
  uint64_t mk = same;
  for (int i = rank + (m < n ? m : 0); i > 0; --i) mk &= mk - 1;  // drop the lower set bits
  return (int)__builtin_ctzll(mk);
}

template <bool GATEUP, bool X4T, int NBP, int S, int RW, int P, int STEPS, bool ROUTE = false>
__global__ __launch_bounds__(S * RW * 64) void moe_small_kernel(
    const uint16_t* __restrict__ a, int64_t lda, int topk, const int* __restrict__ sorted,
    const int* __restrict__ small_list, const uint8_t* __restrict__ wt,
    const uint8_t* __restrict__ wst, const int* __restrict__ sslot, X4TGemv xg, int64_t rows_per_expert,
    int64_t K, int64_t inter, ActParams act, const float* __restrict__ route_w,
    uint16_t* __restrict__ act_out, float* __restrict__ y_out, int64_t hidden, DecodeRouteArgs route) {
  constexpr int NB = GATEUP ? 2 * NBP : NBP;      // 16-row blocks per wave
  constexpr int CH = RW * 16 * NBP;               // channels per workgroup
  constexpr int NBUF = P + 1;
  constexpr int T = S * RW * 64, NRB = RW * NB;
  static_assert(NB * 33 <= 128 * S, "fixed tiles of the row blocks: at most two 16-byte loads per thread");
  static_assert(!ROUTE || GATEUP, "per-pair decode: gate/up");
  extern __shared__ __attribute__((aligned(16))) unsigned char x4t_lds[];
  int e, beg, n, spair = 0;
  if constexpr (ROUTE) {
    e = route.ids[blockIdx.x];
    if (e < 0 || e >= route.experts) return;
    spair = route_entry_slot(route.ids, route.pairs, (int)blockIdx.x, e, (int)(threadIdx.x & 15), n);
    if (spair < 0) return;  // uniform: x does not start an entry
    beg = 0;
  } else {
    e = small_list[3 * blockIdx.x];               // -1 past the last entry
    if (e < 0) return;
    beg = small_list[3 * blockIdx.x + 1];
    n = small_list[3 * blockIdx.x + 2];
  }
  X4TPending pd;
  const int64_t tile0 = (int64_t)blockIdx.y * RW * NBP;  // first tile of this workgroup's row blocks
  if constexpr (X4T) x4t_issue<GATEUP, NB, NBP, NRB, T>(xg, e, tile0, pd);
  const int se = sslot ? sslot[e] : e;            // scale slot of the expert
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kpart = wave % S, rgw = wave / S;
  const int m = lane & 15, g = lane >> 4;
  const int64_t c0 = (int64_t)blockIdx.y * CH + rgw * 16 * NBP;  // first channel of this wave

  // weight tiles (kq_mx_tile_weights layout): [expert][row group][chunk][1 KiB]
  const int64_t nchunk = K / 128;
  const int64_t rgs = rows_per_expert / 16;
  const int64_t c_first = kpart * nchunk / S;     // this wave's 128-k chunks
  const int steps = (int)((kpart + 1) * nchunk / S - c_first);
  const uint8_t* wtile[NB];
  const uint8_t* stile[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int64_t rg = GATEUP ? (b < NBP ? c0 / 16 + b : inter / 16 + c0 / 16 + (b - NBP)) : c0 / 16 + b;
    const int64_t t0 = ((int64_t)e * rgs + rg) * nchunk + c_first;
    wtile[b] = wt + t0 * 1024 + 16 * lane;
    stile[b] = wst + (((int64_t)se * rgs + rg) * nchunk + c_first) * 64 + lane;
  }
  struct WBuf {
    u32x4_t w[NB];
    uint32_t ws[NB];
  };
  struct ABuf {
    u32x4_t v[4];
  };
  auto load_w = [&](int s, WBuf& B) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      B.w[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wtile[b] + (int64_t)s * 1024));
      if constexpr (!X4T) B.ws[b] = stile[b][(int64_t)s * 64];
    }
  };
  // Issue the first weight loads before the dependent token-index loads.
  WBuf wb[NBUF];
  ABuf ab[NBUF];
  if constexpr (STEPS > 0) {
#pragma unroll
    for (int s = 0; s < P && s < STEPS; ++s) load_w(s, wb[s]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // A row of this lane's token slot.  Slots past n re-read slot 0 (always
  // valid, n >= 1): MFMA output row m depends only on A row m and rows >= n
  // are never stored, so the duplicate needs no masking, and the loads stay
  // unconditional so the compiler keeps them in flight across steps.
  const int mslot = m < n ? m : 0;
  const int apair = ROUTE ? spair : sorted[beg + mslot];
  const int64_t arow = GATEUP ? (int64_t)(apair / topk) : (int64_t)(beg + mslot);
  const uint16_t* ap = a + arow * lda + 32 * g;
  auto load_a = [&](int s, ABuf& B) {
    const int64_t c = c_first + s;                // 128-k chunk
#pragma unroll
    for (int t = 0; t < 4; ++t) B.v[t] = *reinterpret_cast<const u32x4_t*>(ap + 128 * c + 8 * t);
  };
  f32x4_t acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // X4T: this wave's decoded scale bytes, sl[((rgw * NB + b) * nchunk + c_first + s) * 64 + lane]
  const uint8_t* xs = x4t_lds + ((int64_t)rgw * NB * nchunk + c_first) * 64 + lane;
  auto compute = [&](const WBuf& W, const ABuf& A, int s) {
    uint32_t ws[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ws[b] = X4T ? (uint32_t)xs[((int64_t)b * nchunk + s) * 64] : W.ws[b];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const bf16x8_t fa = __builtin_bit_cast(bf16x8_t, A.v[t]);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const bf16x8_t fb = gemm::dequant8<1>(u32x2_t{W.w[b][t], 0u}, ws[b]);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, fb, acc[b], 0, 0, 0);
      }
    }
  };
  if constexpr (STEPS > 0) {
#pragma unroll
    for (int s = 0; s < P && s < STEPS; ++s) load_a(s, ab[s]);
    if constexpr (X4T) x4t_finish<GATEUP, NB, NBP, NRB, T>(xg, e, tile0, (int)nchunk, pd, x4t_lds);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      if (s + P < STEPS) {
        load_w(s + P, wb[(s + P) % NBUF]);
        load_a(s + P, ab[(s + P) % NBUF]);
      }
      __builtin_amdgcn_sched_barrier(0);
      compute(wb[s % NBUF], ab[s % NBUF], s);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    // Runtime step count: two alternating buffers; loads are never
    // predicated (past the last step they re-read it, in bounds).
    const int last = steps - 1;
    load_w(0, wb[0]);
    load_a(0, ab[0]);
    if constexpr (X4T) x4t_finish<GATEUP, NB, NBP, NRB, T>(xg, e, tile0, (int)nchunk, pd, x4t_lds);
    for (int s = 0; s < steps; s += 2) {
      const int s1 = s + 1 < last ? s + 1 : last, s2 = s + 2 < last ? s + 2 : last;
      load_w(s1, wb[1]);
      load_a(s1, ab[1]);
      __builtin_amdgcn_sched_barrier(0);
      compute(wb[0], ab[0], s);
      __builtin_amdgcn_sched_barrier(0);
      load_w(s2, wb[0]);
      load_a(s2, ab[0]);
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < steps) compute(wb[1], ab[1], s + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // D layout (16x16): lane holds rows (token slots) 4*(lane/16) + j, column lane % 16.
  // ROUTE: output row of slot 4 g + j = that slot's pair (lane 4 g + j holds it)
  int orow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) orow[j] = ROUTE ? __shfl(spair, 4 * g + j) : beg + 4 * g + j;
  auto store = [&](int u, f32x4_t x0, f32x4_t x1) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int slot = 4 * g + j;
      if (slot >= n) continue;
      const int64_t ch = c0 + 16 * u + m;
      if (GATEUP) {
        const float v = activate(act, x0[j], x1[j]);
        reinterpret_cast<__bf16*>(act_out)[(int64_t)orow[j] * inter + ch] = (__bf16)v;
      } else {
        y_out[(int64_t)(beg + slot) * hidden + ch] = x0[j];
      }
    }
  };
  if constexpr (S == 1) {
#pragma unroll
    for (int u = 0; u < NBP; ++u) store(u, acc[u], GATEUP ? acc[u + NBP] : acc[u]);
  } else {
    // sum the S partial products of each block through LDS (in k order);
    // wave kpart of a row group finishes blocks kpart, kpart + S, ...
    __shared__ f32x4_t red[S * RW][NB][64];
#pragma unroll
    for (int b = 0; b < NB; ++b) red[wave][b][lane] = acc[b];
    __syncthreads();
    for (int u = kpart; u < NBP; u += S) {
      f32x4_t x0 = red[rgw * S][u][lane], x1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 1; p < S; ++p) x0 += red[rgw * S + p][u][lane];
      if (GATEUP) {
        x1 = red[rgw * S][u + NBP][lane];
#pragma unroll
        for (int p = 1; p < S; ++p) x1 += red[rgw * S + p][u + NBP][lane];
      }
      store(u, x0, x1);
    }
  }

}

// ------------------------------------ activation-quantized GEMV (W4A8/W4A4) --
// Same workgroup shape, weight stream and epilogues as moe_small_kernel, for
// activations MX-quantized beforehand (AF = 0: E4M3 bytes [rows, K]; AF = 4:
// E2M1 packed [rows, K/2]; E8M0 scales [rows, K/32]).  Both operands go into
// v_mfma_scale_f32_16x16x128_f8f6f4 as they are: lane (m, g) of a 128-k chunk
// supplies A = E2M1 k 32g .. 32g + 31 (16 bytes) or E4M3 k 16g .. 16g + 15 and
// 64 + 16g .. + 15 (2 x 16 bytes) of token slot m, the weights of row m of the
// tile and block g, and the scales of (slot m, block g) and (row m, block g).
typedef int i32x8_t __attribute__((ext_vector_type(8)));

template <bool GATEUP, bool X4T, int AF, int NBP, int S, int RW, int P, int STEPS>
__global__ __launch_bounds__(S * RW * 64) void moe_small_mx_kernel(
    const uint8_t* __restrict__ aq, const uint8_t* __restrict__ as, int topk,
    const int* __restrict__ sorted, const int* __restrict__ small_list,
    const uint8_t* __restrict__ wt, const uint8_t* __restrict__ wst, const int* __restrict__ sslot,
    X4TGemv xg, int64_t rows_per_expert, int64_t K, int64_t inter, ActParams act,
    const float* __restrict__ route_w, uint16_t* __restrict__ act_out, float* __restrict__ y_out,
    int64_t hidden) {
  constexpr int NB = GATEUP ? 2 * NBP : NBP;
  constexpr int CH = RW * 16 * NBP;
  constexpr int NBUF = P + 1;
  constexpr int ABYTES = AF == 4 ? 64 : 128;      // A bytes per row per 128-k chunk
  constexpr int T = S * RW * 64, NRB = RW * NB;
  static_assert(NB * 33 <= 128 * S, "fixed tiles of the row blocks: at most two 16-byte loads per thread");
  extern __shared__ __attribute__((aligned(16))) unsigned char x4t_lds[];
  const int e = small_list[3 * blockIdx.x];
  if (e < 0) return;
  X4TPending pd;
  const int64_t tile0 = (int64_t)blockIdx.y * RW * NBP;
  if constexpr (X4T) x4t_issue<GATEUP, NB, NBP, NRB, T>(xg, e, tile0, pd);
  const int beg = small_list[3 * blockIdx.x + 1];
  const int n = small_list[3 * blockIdx.x + 2];
  const int se = sslot ? sslot[e] : e;            // scale slot of the expert
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kpart = wave % S, rgw = wave / S;
  const int m = lane & 15, g = lane >> 4;
  const int64_t c0 = (int64_t)blockIdx.y * CH + rgw * 16 * NBP;
  const int64_t nchunk = K / 128;
  const int64_t rgs = rows_per_expert / 16;
  const int64_t c_first = kpart * nchunk / S;
  const int steps = (int)((kpart + 1) * nchunk / S - c_first);
  const uint8_t* wtile[NB];
  const uint8_t* stile[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int64_t rg = GATEUP ? (b < NBP ? c0 / 16 + b : inter / 16 + c0 / 16 + (b - NBP)) : c0 / 16 + b;
    const int64_t t0 = ((int64_t)e * rgs + rg) * nchunk + c_first;
    wtile[b] = wt + t0 * 1024 + 16 * lane;
    stile[b] = wst + (((int64_t)se * rgs + rg) * nchunk + c_first) * 64 + lane;
  }
  struct WBuf {
    u32x4_t w[NB];
    uint32_t ws[NB];
  };
  struct ABuf {
    u32x4_t v[AF == 4 ? 1 : 2];
    uint32_t s;
  };
  auto load_w = [&](int s, WBuf& B) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      B.w[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wtile[b] + (int64_t)s * 1024));
      if constexpr (!X4T) B.ws[b] = stile[b][(int64_t)s * 64];
    }
  };
  WBuf wb[NBUF];
  ABuf ab[NBUF];
  if constexpr (STEPS > 0) {
#pragma unroll
    for (int s = 0; s < P && s < STEPS; ++s) load_w(s, wb[s]);
  }
  __builtin_amdgcn_sched_barrier(0);
  const int mslot = m < n ? m : 0;
  const int apair = sorted[beg + mslot];
  const int64_t arow = GATEUP ? (int64_t)(apair / topk) : (int64_t)(beg + mslot);
  const uint8_t* ap = aq + arow * (AF == 4 ? K / 2 : K);
  const uint8_t* sp = as + arow * (K / 32);
  auto load_a = [&](int s, ABuf& B) {
    const int64_t c = c_first + s;
    if (AF == 4) {
      B.v[0] = *reinterpret_cast<const u32x4_t*>(ap + ABYTES * c + 16 * g);
    } else {
      B.v[0] = *reinterpret_cast<const u32x4_t*>(ap + ABYTES * c + 16 * g);
      B.v[AF == 4 ? 0 : 1] = *reinterpret_cast<const u32x4_t*>(ap + ABYTES * c + 64 + 16 * g);
    }
    B.s = sp[4 * c + g];
  };
  f32x4_t acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint8_t* xs = x4t_lds + ((int64_t)rgw * NB * nchunk + c_first) * 64 + lane;
  auto compute = [&](const WBuf& W, const ABuf& A, int s) {
    i32x8_t a8;
    if (AF == 4) {
      a8 = i32x8_t{(int)A.v[0][0], (int)A.v[0][1], (int)A.v[0][2], (int)A.v[0][3], 0, 0, 0, 0};
    } else {
      const int h = AF == 4 ? 0 : 1;
      a8 = i32x8_t{(int)A.v[0][0], (int)A.v[0][1], (int)A.v[0][2], (int)A.v[0][3],
                   (int)A.v[h][0], (int)A.v[h][1], (int)A.v[h][2], (int)A.v[h][3]};
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const i32x8_t w8 = i32x8_t{(int)W.w[b][0], (int)W.w[b][1], (int)W.w[b][2], (int)W.w[b][3], 0, 0, 0, 0};
      const int wsb = X4T ? (int)xs[((int64_t)b * nchunk + s) * 64] : (int)W.ws[b];
      acc[b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, w8, acc[b], AF, 4, 0, (int)A.s, 0, wsb);
    }
  };
  if constexpr (STEPS > 0) {
#pragma unroll
    for (int s = 0; s < P && s < STEPS; ++s) load_a(s, ab[s]);
    if constexpr (X4T) x4t_finish<GATEUP, NB, NBP, NRB, T>(xg, e, tile0, (int)nchunk, pd, x4t_lds);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      if (s + P < STEPS) {
        load_w(s + P, wb[(s + P) % NBUF]);
        load_a(s + P, ab[(s + P) % NBUF]);
      }
      __builtin_amdgcn_sched_barrier(0);
      compute(wb[s % NBUF], ab[s % NBUF], s);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    const int last = steps - 1;
    load_w(0, wb[0]);
    load_a(0, ab[0]);
    if constexpr (X4T) x4t_finish<GATEUP, NB, NBP, NRB, T>(xg, e, tile0, (int)nchunk, pd, x4t_lds);
    for (int s = 0; s < steps; s += 2) {
      const int s1 = s + 1 < last ? s + 1 : last, s2 = s + 2 < last ? s + 2 : last;
      load_w(s1, wb[1]);
      load_a(s1, ab[1]);
      __builtin_amdgcn_sched_barrier(0);
      compute(wb[0], ab[0], s);
      __builtin_amdgcn_sched_barrier(0);
      load_w(s2, wb[0]);
      load_a(s2, ab[0]);
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < steps) compute(wb[1], ab[1], s + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  auto store = [&](int u, f32x4_t x0, f32x4_t x1) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int slot = 4 * g + j;
      if (slot >= n) continue;
      const int64_t ch = c0 + 16 * u + m;
      if (GATEUP) {
        const float v = activate(act, x0[j], x1[j]);
        reinterpret_cast<__bf16*>(act_out)[(int64_t)(beg + slot) * inter + ch] = (__bf16)v;
      } else {
        y_out[(int64_t)(beg + slot) * hidden + ch] = x0[j];
      }
    }
  };
  if constexpr (S == 1) {
#pragma unroll
    for (int u = 0; u < NBP; ++u) store(u, acc[u], GATEUP ? acc[u + NBP] : acc[u]);
  } else {
    __shared__ f32x4_t red[S * RW][NB][64];
#pragma unroll
    for (int b = 0; b < NB; ++b) red[wave][b][lane] = acc[b];
    __syncthreads();
    for (int u = kpart; u < NBP; u += S) {
      f32x4_t x0 = red[rgw * S][u][lane], x1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 1; p < S; ++p) x0 += red[rgw * S + p][u][lane];
      if (GATEUP) {
        x1 = red[rgw * S][u + NBP][lane];
#pragma unroll
        for (int p = 1; p < S; ++p) x1 += red[rgw * S + p][u + NBP][lane];
      }
      store(u, x0, x1);
    }
  }
}

// ------------------------------------------------ grouped GEMM large path --
// Tile (expert, 256 sorted pair rows) x 256 weight rows, 8 waves of 64 x 128,
// K step 64.  GATEUP: the 256 weight rows are 128 gate rows c0.. and the 128
// matching up rows, so each wave holds gate (blocks 0,1) and up (blocks 2,3)
// of the same channels and applies the activation in registers.
template <bool GATEUP>
__global__ __launch_bounds__(512, 1) void moe_large_kernel(
    const uint16_t* __restrict__ a, int64_t lda, int topk, const int* __restrict__ offsets,
    const int* __restrict__ sorted, const int* __restrict__ tiles, const int* __restrict__ meta,
    const uint8_t* __restrict__ wt, const uint8_t* __restrict__ wst, const int* __restrict__ sslot,
    int64_t rows_per_expert, int64_t K, int64_t inter, ActParams act, const float* __restrict__ route_w,
    uint16_t* __restrict__ act_out, float* __restrict__ y_out, int64_t hidden) {
  const int ti = blockIdx.x;
  if (ti >= meta[1]) return;
  const int e = tiles[2 * ti], m0 = tiles[2 * ti + 1];
  const int se = sslot ? sslot[e] : e;  // scale slot of the expert
  const int beg = offsets[e];
  const int n = offsets[e + 1] - beg;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  int* rowsrc = reinterpret_cast<int*>(lds + 2 * STAGE);  // A source row per tile row (-1: none)
  if (tid < BM) {
    const int slot = m0 + tid;
    int src = -1;
    if (slot < n) src = GATEUP ? sorted[beg + slot] / topk : beg + slot;
    rowsrc[tid] = src;
  }
  __syncthreads();

  // weights in the kq_mx_tile_weights layout: [expert][row group][chunk][1 KiB]
  const int64_t nchunk = K / 128, rgs = rows_per_expert / 16;
  const int64_t c0 = (int64_t)blockIdx.y * (GATEUP ? BN / 2 : BN);
  const int64_t nrows = GATEUP ? 2 * inter : hidden;  // weight rows per expert
  auto grow_group = [&](int lrg) -> int64_t {  // global row group of local group lrg (16 per tile)
    if (GATEUP) return lrg < 8 ? c0 / 16 + lrg : inter / 16 + c0 / 16 + (lrg - 8);
    return c0 / 16 + lrg;
  };

  u32x4_t ra[4], rb;
  uint32_t rs = 0;
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + THREADS * i;
      const int row = ch >> 3, col = (ch & 7) * 8;
      const int src = rowsrc[row];
      ra[i] = src >= 0 ? *reinterpret_cast<const u32x4_t*>(a + (int64_t)src * lda + k0 + col)
                       : u32x4_t{0u, 0u, 0u, 0u};
    }
    const int64_t chunk = k0 / 128;
    const int h = (int)((k0 / 64) & 1);  // which half of the 128-k tile this step reads
    {
      // 16 local row groups x 32 lanes x 16 B: one contiguous 512 B half tile each
      const int lrg = tid >> 5, l = h * 32 + (tid & 31);
      const int64_t rg = grow_group(lrg);
      rb = 16 * rg < nrows
               ? *reinterpret_cast<const u32x4_t*>(wt + (((int64_t)e * rgs + rg) * nchunk + chunk) * 1024 + 16 * l)
               : u32x4_t{0u, 0u, 0u, 0u};
    }
    if (tid < BN) {
      // two scale bytes per thread: tile lanes l, l + 1 (rows 2q, 2q + 1 of the group)
      const int lrg = tid >> 4, q = tid & 15, l = h * 32 + 2 * q;
      const int64_t rg = grow_group(lrg);
      rs = 16 * rg < nrows
               ? *reinterpret_cast<const uint16_t*>(wst + (((int64_t)se * rgs + rg) * nchunk + chunk) * 64 + l)
               : 0u;
    }
  };
  auto store = [&](int buf) {
    unsigned char* base = lds + buf * STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + THREADS * i;
      const int row = ch >> 3, col = (ch & 7) * 16;
      *reinterpret_cast<u32x4_t*>(base + row * A_ROW + col) = ra[i];
    }
    {
      const int lrg = tid >> 5, l = tid & 31;  // lane within the half tile
      const int row = 16 * lrg + (l & 15), col = 16 * (l >> 4);
#pragma unroll
      for (int d = 0; d < 4; ++d)
        *reinterpret_cast<uint32_t*>(base + A_BYTES + row * B_ROW + col + 4 * d) = rb[d];
    }
    if (tid < BN) {
      const int lrg = tid >> 4, q = tid & 15;
      const int j = q >> 3;                   // scale block within this step
      unsigned char* sb = base + A_BYTES + B_BYTES;
      sb[(16 * lrg + ((2 * q) & 15)) * 2 + j] = (unsigned char)(rs & 0xffu);
      sb[(16 * lrg + ((2 * q + 1) & 15)) * 2 + j] = (unsigned char)(rs >> 8);
    }
  };

  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  float16_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const int frow = lane & 31, fk = lane >> 5;
  // B row of MFMA column block j for this wave
  auto brow = [&](int j) -> int {
    if (GATEUP) return (j < 2 ? 0 : BN / 2) + wn + (j & 1) * 32 + frow;
    return 2 * wn + j * 32 + frow;
  };

  const int steps = (int)(K / BK);
  load(0);
  store(0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < steps) load((int64_t)(s + 1) * BK);
    const unsigned char* base = lds + buf * STAGE;
    const unsigned char* bb = base + A_BYTES;
    const unsigned char* sb = bb + B_BYTES;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8_t fa[2], fb[4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        fa[i] = *reinterpret_cast<const bf16x8_t*>(base + (wm + i * 32 + frow) * A_ROW + kk * 32 + fk * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = brow(j);
        u32x2_t w;
        w[0] = *reinterpret_cast<const uint32_t*>(bb + r * B_ROW + kk * 8 + fk * 4);
        w[1] = 0u;
        fb[j] = gemm::dequant8<1>(w, sb[r * 2 + (kk >> 1)]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < steps) store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = wm + i * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
      const int slot = m0 + row;
      if (slot >= n) continue;
      if (GATEUP) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float v = activate(act, acc[i][j][r], acc[i][j + 2][r]);
          const int64_t ch = c0 + wn + j * 32 + frow;
          if (ch < inter)
            reinterpret_cast<__bf16*>(act_out)[(int64_t)(beg + slot) * inter + ch] = (__bf16)v;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t h = c0 + 2 * wn + j * 32 + frow;
          if (h < hidden) y_out[(int64_t)(beg + slot) * hidden + h] = acc[i][j][r];
        }
      }
    }
}

// Tile t of the grouped GEMMs -> (row-tile index mt, column tile nt).  The
// row tiles of one expert are consecutive in the tile list, so its tiles
// occupy the range [first * col_tiles, (first + cnt) * col_tiles); inside it
// they are taken in blocks of nblk column tiles x all cnt row tiles, so the
// ~32 workgroups of an XCD that run neighbouring tiles together share a few
// activation row tiles and a few weight tiles in its L2 (instead of one row
// tile against all of the expert's weight tiles).  A permutation within each
// expert's range: results do not depend on it.
template <int TM = BM>
__device__ __forceinline__ void grouped_tile(int t, int col_tiles, int nblk, const int* __restrict__ tiles,
                                             const int* __restrict__ offsets, int& mt, int& nt) {
  const int mt0 = t / col_tiles;
  const int e = tiles[2 * mt0], m0 = tiles[2 * mt0 + 1];
  const int first = mt0 - m0 / TM;
  const int cnt = (offsets[e + 1] - offsets[e] + TM - 1) / TM;
  const int u = t - first * col_tiles;
  const int nb = u / (cnt * nblk), rem = u - nb * cnt * nblk;
  mt = first + rem / nblk;
  nt = nb * nblk + rem % nblk;
}

// ------------------------------------- grouped GEMM, direct-to-LDS loads --
// The bf16-activation grouped GEMM (W4A16), organised around direct HBM ->
// LDS loads:
//  * tiles of 128 gathered token rows x 512 weight rows (gate/up: 256 gate
//    and the matching 256 up channels), 4 waves of 128 x 128 (1 x 4).  The
//    bf16 activations are four fifths of a 256 x 256 tile's operand bytes;
//    this shape moves 33 KiB per 64-k step instead of 41 for the same MFMA
//    work, and four stages fit in LDS, so three steps are in flight.
//  * persistent: one workgroup per CU walks the (row tile, column tile) list
//    (grouped_tile order).  Worker w (the G/8 workers of one XCD are
//    consecutive) takes tiles w, w + G, ...; the 32 workgroups of one XCD
//    therefore work on neighbouring tiles of the same expert at the same
//    time and share operand rows in that XCD's L2.
//  * the ring of LDS stages continues across tile boundaries: the first
//    stages of a workgroup's next tile are in flight while it finishes and
//    stores the current one.
//  * activation rows: 128 bytes of a row per stage, 16-byte chunk c of tile
//    row r stored at slot c ^ ((r / 2) % 8), so the 16 lanes of an MFMA
//    fragment read hit 16 distinct bank groups.  Rows past the expert's count
//    read as zero without touching memory (out-of-range buffer offset).
//  * k order: in a 64-k step, lane half f of MFMA q (0..3) takes
//    k = 32 f + 8 q + [0, 8) on both operands, so a lane's weights for the
//    step are the one 16-byte tile unit (row, block f) -- one 128-bit LDS
//    read, the 16 lanes of a row group reading 256 contiguous bytes -- under
//    the one scale byte of block f.
//  * one wave per SIMD (16 32x32 accumulators in AGPRs, 64 MFMAs per step),
//    issuing in order, so every other instruction of a step has a fixed
//    place between two MFMAs: k16 block 0 (the rest of the stage in flight
//    issued between its MFMAs), the step's one barrier (stage s + 1 landed,
//    slot s in registers everywhere, hence free), then blocks 1-3 with the
//    LDS reads of step s + 1 (at most one per MFMA, each into its registers
//    once their old value is dead; A block 3 from the current slot during
//    the next step's block 0), the first direct loads of stage s + 4 (into
//    slot s) and the expansions.  Each wave loads 4
//    activation blocks, 4 weight row-group pairs and (16 lanes) one scale
//    block per stage; stages are waited for three steps after their first
//    loads.
namespace dma_gemm {
constexpr int NSTAGE = 4;
constexpr int DA_BYTES = DMA_BM * BK * 2;    // 16 KiB, unpadded 128-byte rows
constexpr int DB_BYTES = DMA_BN * BK / 2;    // 16 KiB: 32 row groups x 512 B half tiles
constexpr int DS_BYTES = DMA_BN * BK / 32;   // 1 KiB: 32 row groups x 32 B
constexpr int DSTAGE = DA_BYTES + DB_BYTES + DS_BYTES;
constexpr int LOADS_PER_STAGE = 5;           // per wave: 2 activation, 2 weight, 1 scale
}  // namespace dma_gemm

__shared__ __attribute__((aligned(16))) unsigned char moe_dma_lds[dma_gemm::NSTAGE * dma_gemm::DSTAGE];

template <bool GATEUP>
__global__ __launch_bounds__(256, 1) void moe_large_dma_kernel(
    const uint16_t* __restrict__ a, int64_t lda, uint32_t a_bytes, int topk,
    const int* __restrict__ offsets, const int* __restrict__ sorted, const int* __restrict__ tiles,
    const int* __restrict__ meta, const uint8_t* __restrict__ wt, const uint8_t* __restrict__ wst,
    const int* __restrict__ sslot, int64_t rows_per_expert, int64_t K, int64_t inter, int col_tiles,
    ActParams act, const float* __restrict__ route_w, uint16_t* __restrict__ act_out,
    float* __restrict__ y_out, int64_t hidden) {
  using namespace dma_gemm;
  using dma::i32x4_t;
  constexpr int LOADS = 9, LA = 5;  // direct loads per wave per stage; of them issued in the step after the barrier
  const int G = gridDim.x;
  const int worker = (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8);
  const int total = meta[1] * col_tiles;
  if (worker >= total) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t nchunk = K / 128, rgs = rows_per_expert / 16;
  const int64_t nrows = GATEUP ? 2 * inter : hidden;  // weight rows per expert
  const uint32_t b_bytes = (uint32_t)(rgs * nchunk * 1024), s_bytes = (uint32_t)(rgs * nchunk * 64);
  const int steps = (int)(K / BK);
  const uint32_t lds0 = dma::lds_offset_of(moe_dma_lds);
  int nblk = 8;  // column tiles per block of grouped_tile: the largest divisor <= 8
  while (col_tiles % nblk != 0) --nblk;
  const i32x4_t a_rsrc = dma::make_rsrc(a, a_bytes);

  auto grow_group = [&](int64_t c0, int lrg) -> int64_t {
    if (GATEUP) return lrg < 16 ? c0 / 16 + lrg : inter / 16 + c0 / 16 + (lrg - 16);
    return c0 / 16 + lrg;
  };

  // ---- load side: tile lt, step ls; per-lane byte offsets (invalid -> past the range)
  int lt = worker, ls = 0;
  uint32_t a_off[4], b_off[4], s_off = 0;
  i32x4_t b_rsrc = dma::make_rsrc(wt, 0), s_rsrc = dma::make_rsrc(wst, 0);
  auto set_load_tile = [&]() {
    if (lt >= total) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a_off[q] = a_bytes;
        b_off[q] = b_bytes;
      }
      s_off = s_bytes;
      return;
    }
    int mt, nt;
    grouped_tile<DMA_BM>(lt, col_tiles, nblk, tiles, offsets, mt, nt);
    const int e = tiles[2 * mt], m0 = tiles[2 * mt + 1];
    const int beg = offsets[e], n = offsets[e + 1] - beg;
    const int64_t c0 = (int64_t)nt * (GATEUP ? DMA_BN / 2 : DMA_BN);
    int src[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int slot = m0 + 8 * (4 * q + wave) + (lane >> 3);
      src[q] = GATEUP ? sorted[beg + (slot < n ? slot : n - 1)] : beg + slot;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 8 * (4 * q + wave) + (lane >> 3);
      const int c = (lane & 7) ^ ((row >> 1) & 7);
      const int64_t r = GATEUP ? src[q] / topk : src[q];
      a_off[q] = m0 + row < n ? (uint32_t)(r * lda * 2 + c * 16) : a_bytes;
    }
    b_rsrc = dma::make_rsrc(wt + (int64_t)e * rgs * nchunk * 1024, b_bytes);
    s_rsrc = dma::make_rsrc(wst + (int64_t)(sslot ? sslot[e] : e) * rgs * nchunk * 64, s_bytes);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t rg = grow_group(c0, 2 * (4 * wave + q) + (lane >> 5));
      b_off[q] = 16 * rg < nrows ? (uint32_t)(rg * nchunk * 1024 + (lane & 31) * 16) : b_bytes;
    }
    {
      const int64_t rg = grow_group(c0, 8 * wave + ((lane >> 1) & 7));
      s_off = 16 * rg < nrows ? (uint32_t)(rg * nchunk * 64 + (lane & 1) * 16) : s_bytes;
    }
  };
  // load u of the stage at ls into ring slot `slot`: 0-3 activation blocks,
  // 4-7 weight row-group pairs, 8 the scale block (lanes 0-15)
  auto issue_one = [&](int slot, int u) {
    const uint32_t base = lds0 + (uint32_t)(slot * DSTAGE);
    const uint32_t k0 = (uint32_t)(ls * BK);
    const uint32_t chunk = k0 / 128, h = (k0 / 64) & 1;
    if (u < 4) {
      const uint32_t off = a_off[u] >= a_bytes ? a_bytes : a_off[u] + 2 * k0;
      dma::load_to_lds16(a_rsrc, off, base + (uint32_t)((4 * u + wave) * 1024));
    } else if (u < 8) {
      const int q = u - 4;
      dma::load_to_lds16(b_rsrc, b_off[q] >= b_bytes ? b_bytes : b_off[q] + chunk * 1024 + h * 512,
                         base + (uint32_t)(DA_BYTES + (4 * wave + q) * 1024));
    } else if (lane < 16) {
      dma::load_to_lds16(s_rsrc, s_off >= s_bytes ? s_bytes : s_off + chunk * 64 + h * 32,
                         base + (uint32_t)(DA_BYTES + DB_BYTES + wave * 256));
    }
  };
  int lslot = 0;  // ring slot of the stage at ls
  auto next_stage = [&]() {
    if (++ls == steps) {
      ls = 0;
      lt += G;
      set_load_tile();
    }
    lslot = lslot == NSTAGE - 1 ? 0 : lslot + 1;
  };

  // ---- compute side: per-lane LDS read offsets (fixed for the whole kernel)
  const int wn = wave * 64;
  const int frow = lane & 31, fk = lane >> 5;
  int arow[4], axor[4], boff[4], soff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = i * 32 + frow;
    arow[i] = row * (BK * 2);
    axor[i] = (4 * fk) ^ ((row >> 1) & 7);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = GATEUP ? (j < 2 ? 0 : DMA_BN / 2) + wn + (j & 1) * 32 + frow : 2 * wn + j * 32 + frow;
    boff[j] = DA_BYTES + (r >> 4) * 512 + (fk * 16 + (r & 15)) * 16;
    soff[j] = DA_BYTES + DB_BYTES + (r >> 4) * 32 + fk * 16 + (r & 15);
  }
  // read r of a step: 0-3 weight chunks, 4-7 scale bytes, 8-23 A fragments
  constexpr int NR = 24;
  auto read_one = [&](const unsigned char* st, int r, u32x4_t (&w)[4], uint32_t (&sc)[4], bf16x8_t (&fa)[4][4]) {
    if (r < 4) {
      w[r] = *reinterpret_cast<const u32x4_t*>(st + boff[r]);
    } else if (r < 8) {
      sc[r - 4] = st[soff[r - 4]];
    } else {
      const int e = r - 8, q = e >> 2, i = e & 3;
      fa[q][i] = *reinterpret_cast<const bf16x8_t*>(st + arow[i] + 16 * (q ^ axor[i]));
    }
  };
  auto pinned = [](bf16x8_t v) -> bf16x8_t {
    asm volatile("" : "+v"(v));  // computed where it is placed, not sunk to its first use
    return v;
  };
  auto expand1 = [&](const u32x4_t (&w)[4], int q, int j, const uint32_t (&sc)[4]) -> bf16x8_t {
    return gemm::dequant8<1>(u32x2_t{w[j][q], 0u}, sc[j]);
  };

  u32x4_t wv[4];
  uint32_t sc[4];
  bf16x8_t fa[4][4], fb0[4];
  set_load_tile();
#pragma unroll
  for (int p = 0; p < NSTAGE - 1; ++p) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) issue_one(lslot, u);
    next_stage();
  }
  dma::wait_and_barrier<(NSTAGE - 2) * LOADS>();  // stage 0 landed
#pragma unroll
  for (int r = 0; r < NR; ++r) read_one(moe_dma_lds, r, wv, sc, fa);
#pragma unroll
  for (int u = 0; u < LA; ++u) issue_one(lslot, u);
#pragma unroll
  for (int j = 0; j < 4; ++j) fb0[j] = expand1(wv, 0, j, sc);
  int cslot = 0;
  for (int t = worker; t < total; t += G) {
    int mt, nt;
    grouped_tile<DMA_BM>(t, col_tiles, nblk, tiles, offsets, mt, nt);
    const int e = tiles[2 * mt], m0 = tiles[2 * mt + 1];
    const int beg = offsets[e], n = offsets[e + 1] - beg;
    const int64_t c0 = (int64_t)nt * (GATEUP ? DMA_BN / 2 : DMA_BN);

    float16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    for (int s = 0; s < steps; ++s) {
      const unsigned char* cst = moe_dma_lds + cslot * DSTAGE;
      bf16x8_t fb1[4], fb2[4], fb3[4];
      // k16 block 0; the rest of the stage in flight; expansion of block 1
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[0][m >> 2], fb0[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
        if (!(m & 1) && m / 2 < LOADS - LA) issue_one(lslot, LA + m / 2);
        if ((m & 1) && m / 2 < 4) fb1[m / 2] = pinned(expand1(wv, 1, m / 2, sc));
        if ((m & 1) && m >= 9) read_one(cst, 20 + (m - 9) / 2, wv, sc, fa);  // A block 3
        __builtin_amdgcn_sched_barrier(0);
      }
      next_stage();
      // stage s + 1 landed; every wave has every fragment of slot s in registers
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): no read of slot s is still in flight
      dma::wait_and_barrier<(NSTAGE - 2) * LOADS>();
      __builtin_amdgcn_sched_barrier(0);
      const int nslot = cslot == NSTAGE - 1 ? 0 : cslot + 1;
      const unsigned char* nst = moe_dma_lds + nslot * DSTAGE;
      // reads of step s + 1 in place, each once its register is dead (A block 3
      // is read from this slot during the next step's block 0)
      auto slot_work = [&](int m) {
        if (m < 8 && !(m & 1)) read_one(nst, 8 + m / 2, wv, sc, fa);
        if (m >= 16 && m < 24 && !(m & 1)) read_one(nst, 12 + (m - 16) / 2, wv, sc, fa);
        if (m >= 24 && m < 32) read_one(nst, m - 24, wv, sc, fa);
        if (m >= 36 && m < 40) read_one(nst, 16 + (m - 36), wv, sc, fa);
        if (m < 8 && (m & 1)) fb2[m / 2] = pinned(expand1(wv, 2, m / 2, sc));
        if (m >= 16 && m < 24 && (m & 1)) fb3[(m - 16) / 2] = pinned(expand1(wv, 3, (m - 16) / 2, sc));
        if (m >= 32 && !(m & 1) && (m - 32) / 2 < LA) issue_one(lslot, (m - 32) / 2);
        if (m >= 44) fb0[m - 44] = pinned(expand1(wv, 0, m - 44, sc));
      };
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[1][m >> 2], fb1[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
        slot_work(m);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[2][m >> 2], fb2[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
        slot_work(16 + m);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[3][m >> 2], fb3[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
        slot_work(32 + m);
        __builtin_amdgcn_sched_barrier(0);
      }
      cslot = nslot;
    }

#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = i * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
        const int slot = m0 + row;
        if (slot >= n) continue;
        if (GATEUP) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float v = activate(act, acc[i][j][r], acc[i][j + 2][r]);
            const int64_t ch = c0 + wn + j * 32 + frow;
            reinterpret_cast<__bf16*>(act_out)[(int64_t)(beg + slot) * inter + ch] = (__bf16)v;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t h = c0 + 2 * wn + j * 32 + frow;
            y_out[(int64_t)(beg + slot) * hidden + h] = acc[i][j][r];
          }
        }
      }
  }
  __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));  // no load may land after the workgroup ends
}

// ------------------------- grouped GEMM, activation-quantized (W4A8/W4A4) --
// moe_large_dma_kernel's tiles, waves, persistent order and epilogues, with
// MX-quantized activations (AF = 0 E4M3, 4 E2M1) and one
// v_mfma_scale_f32_16x16x128_f8f6f4 per 16x16 block and 128-k step: a wave's
// 64 x 128 output is 4 x 8 blocks.  Per stage (128 k) in LDS: A in the weight
// tiles' order -- per 16-row group, [16-byte chunk][row][16 B] (4 chunks of
// E2M1, 8 of E4M3) --, A scales (one dword per row: its four blocks), the row
// groups' 1 KiB weight tiles and their 64-byte scale tiles, all by direct
// loads.  Lane (m, g) of a block reads A chunk g (E2M1) or chunks g and 4 + g
// (E4M3) of row m, the weight unit (g, m) of its row group and the two scale
// bytes; the 16 lanes of every 128-bit read cover 256 contiguous bytes.
namespace mx_gemm {
constexpr int BKQ = 128;
template <int AF> constexpr int a_row() { return AF == 4 ? 64 : 128; }   // A bytes per row per stage
template <int AF> constexpr int a_bytes() { return BM * a_row<AF>(); }
constexpr int AS_BYTES = BM * 4;
constexpr int W_BYTES = 16 * 1024;
constexpr int WS_BYTES = 16 * 64;
template <int AF> constexpr int stage() { return a_bytes<AF>() + AS_BYTES + W_BYTES + WS_BYTES; }
template <int AF> constexpr int nstage() { return AF == 4 ? 4 : 3; }
template <int AF> constexpr int loads() { return (AF == 4 ? 2 : 4) + 1 + 2 + 1; }  // per wave per stage
}  // namespace mx_gemm

__shared__ __attribute__((aligned(16))) unsigned char moe_mx_lds[3 * mx_gemm::stage<0>()];
static_assert(4 * mx_gemm::stage<4>() <= 3 * mx_gemm::stage<0>(), "LDS ring size");

template <bool GATEUP, int AF>
__global__ __launch_bounds__(512, 1) void moe_large_mx_kernel(
    const uint8_t* __restrict__ aq, const uint8_t* __restrict__ as, uint32_t aq_bytes,
    uint32_t as_bytes, int topk, const int* __restrict__ offsets, const int* __restrict__ sorted,
    const int* __restrict__ tiles, const int* __restrict__ meta, const uint8_t* __restrict__ wt,
    const uint8_t* __restrict__ wst, const int* __restrict__ sslot, int64_t rows_per_expert, int64_t K,
    int64_t inter, int col_tiles, ActParams act, const float* __restrict__ route_w,
    uint16_t* __restrict__ act_out, float* __restrict__ y_out, int64_t hidden) {
  using namespace mx_gemm;
  using dma::i32x4_t;
  constexpr int AROW = a_row<AF>(), ABYTES = a_bytes<AF>(), STAGE = stage<AF>();
  constexpr int NST = nstage<AF>(), LOADS = loads<AF>();
  constexpr int AQ = AF == 4 ? 2 : 4;  // A direct loads per wave per stage
  const int G = gridDim.x;
  const int worker = (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8);
  const int total = meta[1] * col_tiles;
  if (worker >= total) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t nchunk = K / 128, rgs = rows_per_expert / 16;
  const int64_t nrows = GATEUP ? 2 * inter : hidden;
  const int64_t arow_bytes = AF == 4 ? K / 2 : K, asrow = K / 32;
  const uint32_t b_bytes = (uint32_t)(rgs * nchunk * 1024), s_bytes = (uint32_t)(rgs * nchunk * 64);
  const int steps = (int)(K / BKQ);
  const uint32_t lds0 = dma::lds_offset_of(moe_mx_lds);
  const int nblk = col_tiles % 8 == 0 ? 8 : col_tiles % 4 == 0 ? 4 : 1;
  const i32x4_t a_rsrc = dma::make_rsrc(aq, aq_bytes);
  const i32x4_t as_rsrc = dma::make_rsrc(as, as_bytes);
  auto grow_group = [&](int64_t c0, int lrg) -> int64_t {
    if (GATEUP) return lrg < 8 ? c0 / 16 + lrg : inter / 16 + c0 / 16 + (lrg - 8);
    return c0 / 16 + lrg;
  };

  // ---- load side
  int lt = worker, ls = 0;
  uint32_t a_off[AQ], as_off, b_off[2], bs_off = 0;
  i32x4_t b_rsrc = dma::make_rsrc(wt, 0), s_rsrc = dma::make_rsrc(wst, 0);
  auto set_load_tile = [&]() {
    if (lt >= total) {
#pragma unroll
      for (int q = 0; q < AQ; ++q) a_off[q] = aq_bytes;
      as_off = as_bytes;
      b_off[0] = b_off[1] = b_bytes;
      bs_off = s_bytes;
      return;
    }
    int mt, nt;
    grouped_tile(lt, col_tiles, nblk, tiles, offsets, mt, nt);
    const int e = tiles[2 * mt], m0 = tiles[2 * mt + 1];
    const int beg = offsets[e], n = offsets[e + 1] - beg;
    const int64_t c0 = (int64_t)nt * (GATEUP ? BN / 2 : BN);
    // rows of this lane's A loads (all lookups issued before the first use)
    // A load q of wave w: 1 KiB = 16 rows x 4 chunks, row group (8q + w) (E2M1)
    // or (8q + w) / 2 with chunks 4 ((8q + w) % 2) .. + 3 (E4M3); lane l:
    // row 16 rg + l % 16, chunk l / 16 (+ 4 for the second half)
    int src[AQ + 1];
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int t = 8 * q + wave;
      const int row = 16 * (AF == 4 ? t : t >> 1) + (lane & 15);
      const int slot = m0 + row;
      src[q] = GATEUP ? sorted[beg + (slot < n ? slot : n - 1)] : beg + slot;
    }
    {
      const int slot = m0 + 32 * wave + (lane & 31);
      src[AQ] = GATEUP ? sorted[beg + (slot < n ? slot : n - 1)] : beg + slot;
    }
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int t = 8 * q + wave;
      const int row = 16 * (AF == 4 ? t : t >> 1) + (lane & 15);
      const int ch = (lane >> 4) + (AF == 4 ? 0 : 4 * (t & 1));
      const int64_t r = GATEUP ? src[q] / topk : src[q];
      a_off[q] = m0 + row < n ? (uint32_t)(r * arow_bytes + ch * 16) : aq_bytes;
    }
    {
      const int row = 32 * wave + (lane & 31);
      const int64_t r = GATEUP ? src[AQ] / topk : src[AQ];
      as_off = m0 + row < n ? (uint32_t)(r * asrow) : as_bytes;
    }
    b_rsrc = dma::make_rsrc(wt + (int64_t)e * rgs * nchunk * 1024, b_bytes);
    s_rsrc = dma::make_rsrc(wst + (int64_t)(sslot ? sslot[e] : e) * rgs * nchunk * 64, s_bytes);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int64_t rg = grow_group(c0, 2 * wave + q);
      b_off[q] = 16 * rg < nrows ? (uint32_t)(rg * nchunk * 1024 + lane * 16) : b_bytes;
    }
    {
      const int64_t rg = grow_group(c0, 2 * wave + ((lane >> 2) & 1));
      bs_off = 16 * rg < nrows ? (uint32_t)(rg * nchunk * 64 + (lane & 3) * 16) : s_bytes;
    }
  };
  auto issue = [&](int slot) {
    const uint32_t base = lds0 + (uint32_t)(slot * STAGE);
    const uint32_t chunk = (uint32_t)ls;  // one 128-k chunk per step
#pragma unroll
    for (int q = 0; q < AQ; ++q)
      dma::load_to_lds16(a_rsrc, a_off[q] >= aq_bytes ? aq_bytes : a_off[q] + chunk * AROW,
                         base + (uint32_t)((8 * q + wave) * 1024));
    if (lane < 32)
      dma::load_to_lds4(as_rsrc, as_off >= as_bytes ? as_bytes : as_off + chunk * 4,
                        base + (uint32_t)(ABYTES + wave * 128));
#pragma unroll
    for (int q = 0; q < 2; ++q)
      dma::load_to_lds16(b_rsrc, b_off[q] >= b_bytes ? b_bytes : b_off[q] + chunk * 1024,
                         base + (uint32_t)(ABYTES + AS_BYTES + (2 * wave + q) * 1024));
    if (lane < 8)
      dma::load_to_lds16(s_rsrc, bs_off >= s_bytes ? s_bytes : bs_off + chunk * 64,
                         base + (uint32_t)(ABYTES + AS_BYTES + W_BYTES + wave * 128));
  };
  auto advance = [&]() {
    if (++ls == steps) {
      ls = 0;
      lt += G;
      set_load_tile();
    }
  };

  // ---- compute side
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int fm = lane & 15, fg = lane >> 4;
  int aoff[4][AF == 4 ? 1 : 2], asoff[4], boff[8], bsoff[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = wm + 16 * i + fm;
    const int rgb = (r >> 4) * 16 * AROW;  // this row group's A block
    aoff[i][0] = rgb + (fg * 16 + fm) * 16;
    if (AF != 4) aoff[i][AF == 4 ? 0 : 1] = rgb + ((4 + fg) * 16 + fm) * 16;
    asoff[i] = ABYTES + r * 4 + fg;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int rr = GATEUP ? (j < 4 ? 0 : BN / 2) + wn + 16 * (j & 3) + fm : 2 * wn + 16 * j + fm;
    boff[j] = ABYTES + AS_BYTES + (rr >> 4) * 1024 + (fg * 16 + (rr & 15)) * 16;
    bsoff[j] = ABYTES + AS_BYTES + W_BYTES + (rr >> 4) * 64 + fg * 16 + (rr & 15);
  }

  set_load_tile();
#pragma unroll
  for (int p = 0; p < NST - 1; ++p) {
    issue(p);
    advance();
  }
  int cslot = 0;
  for (int t = worker; t < total; t += G) {
    int mt, nt;
    grouped_tile(t, col_tiles, nblk, tiles, offsets, mt, nt);
    const int e = tiles[2 * mt], m0 = tiles[2 * mt + 1];
    const int beg = offsets[e], n = offsets[e + 1] - beg;
    const int64_t c0 = (int64_t)nt * (GATEUP ? BN / 2 : BN);
    const bool active = m0 + wm < n;
    f32x4_t acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int s = 0; s < steps; ++s) {
      dma::wait_and_barrier<(NST - 2) * LOADS>();
      issue(cslot == 0 ? NST - 1 : cslot - 1);
      advance();
      if (active) {
        const unsigned char* st = moe_mx_lds + cslot * STAGE;
        i32x8_t a8[4];
        uint32_t sa[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4_t v0 = *reinterpret_cast<const u32x4_t*>(st + aoff[i][0]);
          if (AF == 4) {
            a8[i] = i32x8_t{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3], 0, 0, 0, 0};
          } else {
            const u32x4_t v1 = *reinterpret_cast<const u32x4_t*>(st + aoff[i][AF == 4 ? 0 : 1]);
            a8[i] = i32x8_t{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3],
                            (int)v1[0], (int)v1[1], (int)v1[2], (int)v1[3]};
          }
          sa[i] = st[asoff[i]];
        }
        // all of the step's weight reads are issued before the first MFMA, so
        // their LDS latency is paid once per step, not once per column block
        u32x4_t wv[8];
        int sb[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          wv[j] = *reinterpret_cast<const u32x4_t*>(st + boff[j]);
          sb[j] = st[bsoff[j]];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const i32x8_t b8 = i32x8_t{(int)wv[j][0], (int)wv[j][1], (int)wv[j][2], (int)wv[j][3], 0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8[i], b8, acc[i][j], AF, 4, 0,
                                                                         (int)sa[i], 0, sb[j]);
        }
      }
      cslot = cslot == NST - 1 ? 0 : cslot + 1;
    }

    if (active) {
      // D layout (16x16): lane holds rows 4 fg + r, column fm of its block
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int slot = m0 + wm + 16 * i + 4 * fg + r;
          if (slot >= n) continue;
          if (GATEUP) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float v = activate(act, acc[i][j][r], acc[i][j + 4][r]);
              const int64_t ch = c0 + wn + 16 * j + fm;
              reinterpret_cast<__bf16*>(act_out)[(int64_t)(beg + slot) * inter + ch] = (__bf16)v;
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const int64_t h = c0 + 2 * wn + 16 * j + fm;
              y_out[(int64_t)(beg + slot) * hidden + h] = acc[i][j][r];
            }
          }
        }
    }
  }
  __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));  // no load may land after the workgroup ends
}

// -------------- grouped GEMM, MXFP4 activations (W4A4), whole-line stages --
// moe_large_mx_kernel<*, 4> with two LDS stages of 256 k (two MFMA steps
// each, double buffered) instead of four of 128 k: every direct load of a
// gathered E2M1 row then fetches its whole 128-byte line for the stage (8
// rows x 128 B per instruction), and a row's scales for the stage are one 8-
// byte pair of dwords; with 128-k stages each row fetched half a line and a
// 4-byte scale dword per step, which made the loads issue about 2.4x the
// line requests their bytes need (the bound of these kernels: with their
// MFMAs switched off they kept 80 % of their time).  Same tiles, waves, tile
// order, MFMA sequence and epilogues, so the result is bitwise that of
// moe_large_mx_kernel<*, 4>.  Per stage in LDS: A [row][8 chunks of 16 B],
// chunk c of row r at slot c ^ ((r / 2) % 8); the A scale bytes [row][8];
// the weight tiles [half][row group][1 KiB] and their scale tiles [row
// group][half][64 B].  Needs K % 256 == 0.
namespace mx4_gemm {
constexpr int SK = 256;                      // k per stage
constexpr int AS_OFF = BM * 128;             // A: 256 rows x 128 B
constexpr int W_OFF = AS_OFF + BM * 8;       // A scales: 8 bytes per row
constexpr int WS_OFF = W_OFF + 2 * 16 * 1024;
constexpr int STAGE4 = WS_OFF + 16 * 128;
constexpr int LOADS = 4 + 1 + 4 + 1;         // direct loads per wave per stage
}  // namespace mx4_gemm

__shared__ __attribute__((aligned(16))) unsigned char moe_mx4_lds[2 * mx4_gemm::STAGE4];

template <bool GATEUP>
__global__ __launch_bounds__(512, 1) void moe_large_mx4_kernel(
    const uint8_t* __restrict__ aq, const uint8_t* __restrict__ as, uint32_t aq_bytes,
    uint32_t as_bytes, int topk, const int* __restrict__ offsets, const int* __restrict__ sorted,
    const int* __restrict__ tiles, const int* __restrict__ meta, const uint8_t* __restrict__ wt,
    const uint8_t* __restrict__ wst, const int* __restrict__ sslot, int64_t rows_per_expert, int64_t K,
    int64_t inter, int col_tiles, ActParams act, const float* __restrict__ route_w,
    uint16_t* __restrict__ act_out, float* __restrict__ y_out, int64_t hidden) {
  using namespace mx4_gemm;
  using dma::i32x4_t;
  const int G = gridDim.x;
  const int worker = (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8);
  const int total = meta[1] * col_tiles;
  if (worker >= total) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t nchunk = K / 128, rgs = rows_per_expert / 16;
  const int64_t nrows = GATEUP ? 2 * inter : hidden;
  const int64_t arow_bytes = K / 2, asrow = K / 32;
  const uint32_t b_bytes = (uint32_t)(rgs * nchunk * 1024), s_bytes = (uint32_t)(rgs * nchunk * 64);
  const int stages = (int)(K / SK);
  const uint32_t lds0 = dma::lds_offset_of(moe_mx4_lds);
  const int nblk = col_tiles % 8 == 0 ? 8 : col_tiles % 4 == 0 ? 4 : 1;
  const i32x4_t a_rsrc = dma::make_rsrc(aq, aq_bytes);
  const i32x4_t as_rsrc = dma::make_rsrc(as, as_bytes);
  auto grow_group = [&](int64_t c0, int lrg) -> int64_t {
    if (GATEUP) return lrg < 8 ? c0 / 16 + lrg : inter / 16 + c0 / 16 + (lrg - 8);
    return c0 / 16 + lrg;
  };

  // ---- load side.  A load q (0..3) of wave w: the 8-row piece w + 8 q,
  // lane l: row 8 (w + 8 q) + l / 8, slot l % 8, i.e. logical chunk
  // (l % 8) ^ ((row / 2) % 8).  A scales: lane l: row 32 w + l / 2, dword
  // l % 2 of its 8 bytes.  W load q: tile 4 w + q of [half][row group].  W
  // scales (lanes 0..15): row group 2 w + l / 8, 16-byte piece l % 8 of its
  // two 64-byte scale tiles.
  int lt = worker, ls = 0;
  uint32_t a_off[4], as_off = 0, b_off[4], bs_off = 0;
  i32x4_t b_rsrc = dma::make_rsrc(wt, 0), s_rsrc = dma::make_rsrc(wst, 0);
  auto set_load_tile = [&]() {
    if (lt >= total) {
#pragma unroll
      for (int q = 0; q < 4; ++q) a_off[q] = aq_bytes, b_off[q] = b_bytes;
      as_off = as_bytes;
      bs_off = s_bytes;
      return;
    }
    int mt, nt;
    grouped_tile(lt, col_tiles, nblk, tiles, offsets, mt, nt);
    const int e = tiles[2 * mt], m0 = tiles[2 * mt + 1];
    const int beg = offsets[e], n = offsets[e + 1] - beg;
    const int64_t c0 = (int64_t)nt * (GATEUP ? BN / 2 : BN);
    int src[5];  // every row lookup issued before the first use
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int slot = m0 + 8 * (wave + 8 * q) + (lane >> 3);
      src[q] = GATEUP ? sorted[beg + (slot < n ? slot : n - 1)] : beg + slot;
    }
    {
      const int slot = m0 + 32 * wave + (lane >> 1);
      src[4] = GATEUP ? sorted[beg + (slot < n ? slot : n - 1)] : beg + slot;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 8 * (wave + 8 * q) + (lane >> 3);
      const int ch = (lane & 7) ^ ((row >> 1) & 7);
      const int64_t r = GATEUP ? src[q] / topk : src[q];
      a_off[q] = m0 + row < n ? (uint32_t)(r * arow_bytes + ch * 16) : aq_bytes;
    }
    {
      const int row = 32 * wave + (lane >> 1);
      const int64_t r = GATEUP ? src[4] / topk : src[4];
      as_off = m0 + row < n ? (uint32_t)(r * asrow + 4 * (lane & 1)) : as_bytes;
    }
    b_rsrc = dma::make_rsrc(wt + (int64_t)e * rgs * nchunk * 1024, b_bytes);
    s_rsrc = dma::make_rsrc(wst + (int64_t)(sslot ? sslot[e] : e) * rgs * nchunk * 64, s_bytes);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int tile = 4 * wave + q, half = tile >> 4;
      const int64_t rg = grow_group(c0, tile & 15);
      b_off[q] = 16 * rg < nrows ? (uint32_t)((rg * nchunk + half) * 1024 + lane * 16) : b_bytes;
    }
    {
      const int64_t rg = grow_group(c0, 2 * wave + ((lane >> 3) & 1));
      bs_off = 16 * rg < nrows ? (uint32_t)(rg * nchunk * 64 + (lane & 7) * 16) : s_bytes;
    }
  };
  auto issue = [&](int slot) {
    const uint32_t base = lds0 + (uint32_t)(slot * STAGE4);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dma::load_to_lds16(a_rsrc, a_off[q] >= aq_bytes ? aq_bytes : a_off[q] + (uint32_t)ls * 128u,
                         base + (uint32_t)((wave + 8 * q) * 1024));
    dma::load_to_lds4(as_rsrc, as_off >= as_bytes ? as_bytes : as_off + (uint32_t)ls * 8u,
                      base + (uint32_t)(AS_OFF + wave * 256));
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dma::load_to_lds16(b_rsrc, b_off[q] >= b_bytes ? b_bytes : b_off[q] + (uint32_t)ls * 2048u,
                         base + (uint32_t)(W_OFF + (4 * wave + q) * 1024));
    if (lane < 16)
      dma::load_to_lds16(s_rsrc, bs_off >= s_bytes ? s_bytes : bs_off + (uint32_t)ls * 128u,
                         base + (uint32_t)(WS_OFF + wave * 256));
  };
  auto advance = [&]() {
    if (++ls == stages) {
      ls = 0;
      lt += G;
      set_load_tile();
    }
  };

  // ---- compute side (offsets of half 0; half h adds 64 h to the A chunk
  // position, 4 h to the scale byte, 16 KiB / 64 B on the weight side)
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int fm = lane & 15, fg = lane >> 4;
  int aoff[2][4], asoff[4], boff[8], bsoff[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = wm + 16 * i + fm, sw = (r >> 1) & 7;
    aoff[0][i] = r * 128 + 16 * (fg ^ sw);
    aoff[1][i] = r * 128 + 16 * ((4 + fg) ^ sw);
    asoff[i] = AS_OFF + 8 * r + fg;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int rr = GATEUP ? (j < 4 ? 0 : BN / 2) + wn + 16 * (j & 3) + fm : 2 * wn + 16 * j + fm;
    boff[j] = W_OFF + (rr >> 4) * 1024 + (fg * 16 + (rr & 15)) * 16;
    bsoff[j] = WS_OFF + (rr >> 4) * 128 + fg * 16 + (rr & 15);
  }

  set_load_tile();
  issue(0);
  advance();
  int cslot = 0;
  for (int t = worker; t < total; t += G) {
    int mt, nt;
    grouped_tile(t, col_tiles, nblk, tiles, offsets, mt, nt);
    const int e = tiles[2 * mt], m0 = tiles[2 * mt + 1];
    const int beg = offsets[e], n = offsets[e + 1] - beg;
    const int64_t c0 = (int64_t)nt * (GATEUP ? BN / 2 : BN);
    const bool active = m0 + wm < n;
    f32x4_t acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int s = 0; s < stages; ++s) {
      // stage s landed (the only one in flight) and every wave is done with
      // the other slot, which now takes the next stage
      dma::wait_and_barrier<0>();
      issue(cslot ^ 1);
      advance();
      if (active) {
        const unsigned char* st = moe_mx4_lds + cslot * STAGE4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          i32x8_t a8[4];
          uint32_t sa[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32x4_t v0 = *reinterpret_cast<const u32x4_t*>(st + aoff[h][i]);
            a8[i] = i32x8_t{(int)v0[0], (int)v0[1], (int)v0[2], (int)v0[3], 0, 0, 0, 0};
            sa[i] = st[asoff[i] + 4 * h];
          }
          u32x4_t wv[8];
          int sb[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            wv[j] = *reinterpret_cast<const u32x4_t*>(st + boff[j] + h * 16384);
            sb[j] = st[bsoff[j] + h * 64];
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const i32x8_t b8 = i32x8_t{(int)wv[j][0], (int)wv[j][1], (int)wv[j][2], (int)wv[j][3], 0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8[i], b8, acc[i][j], 4, 4, 0,
                                                                           (int)sa[i], 0, sb[j]);
          }
        }
      }
      cslot ^= 1;
    }

    if (active) {
      // D layout (16x16): lane holds rows 4 fg + r, column fm of its block
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int slot = m0 + wm + 16 * i + 4 * fg + r;
          if (slot >= n) continue;
          if (GATEUP) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float v = activate(act, acc[i][j][r], acc[i][j + 4][r]);
              const int64_t ch = c0 + wn + 16 * j + fm;
              reinterpret_cast<__bf16*>(act_out)[(int64_t)(beg + slot) * inter + ch] = (__bf16)v;
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const int64_t h = c0 + 2 * wn + 16 * j + fm;
              y_out[(int64_t)(beg + slot) * hidden + h] = acc[i][j][r];
            }
          }
        }
    }
  }
  __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));  // no load may land after the workgroup ends
}

// ---------------------------------------------------------------- combine --
template <int OUT>
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y,
                                                          const int* __restrict__ pos,
                                                          const float* __restrict__ route_w,
                                                          const int* __restrict__ ids, int topk,
                                                          int experts, int64_t hidden,
                                                          void* __restrict__ out) {
#pragma clang fp contract(off)
  const int64_t t = blockIdx.y;
  const int64_t h4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (h4 >= hidden) return;
  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < topk; ++k) {
    const int e = ids[t * topk + k];
    if (e < 0 || e >= experts) continue;
    // route weight x the pair's row (each product rounded), summed in slot order
    const float rw = route_w[t * topk + k];
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(y + (int64_t)pos[t * topk + k] * hidden + h4);
    s += f32x4_t{rw * v[0], rw * v[1], rw * v[2], rw * v[3]};
  }
  if (OUT == 2) {
    *reinterpret_cast<f32x4_t*>(static_cast<float*>(out) + t * hidden + h4) = s;
  } else {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 o = {f32x2_to_bf16x2_bits(s[0], s[1]), f32x2_to_bf16x2_bits(s[2], s[3])};
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + t * hidden + h4) = o;
  }
}

// Expert-sorted pair list -> int64 offsets, token rows and gathered weights.
__global__ __launch_bounds__(256) void route_rows_kernel(const int* __restrict__ offsets32, int experts,
                                                         const int* __restrict__ sorted, int topk,
                                                         const float* __restrict__ pair_w,
                                                         int64_t* __restrict__ offsets, int32_t* __restrict__ rows,
                                                         int32_t* __restrict__ pairs_out,
                                                         float* __restrict__ w_out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i <= experts) offsets[i] = offsets32[i];
  const int total = offsets32[experts];
  if (i >= total) return;
  const int pair = sorted[i];
  rows[i] = pair / topk;
  if (pairs_out) pairs_out[i] = pair;
  if (w_out) w_out[i] = pair_w[pair];
}

// ------------------------------- decode down projection with the combine --
// For at most DD_PAIRS pairs (one decode token at top-8): workgroup b owns
// the 16 NBP output channels from 16 NBP b of every token and runs every
// pair on them: wave w takes pair w / 2 (intermediate row w / 2, as the
// per-pair gate/up GEMV wrote it) and K half w % 2 (the split, chunk order
// and MFMA order of moe_small_kernel's down shape with S = 2), the halves
// are summed in LDS in the same order and scaled by the route weight into
// the pair's row of an LDS buffer, and each token's pairs are then summed in
// slot order as moe_combine_kernel sums them.  Same operations in the same
// order, so the output is bitwise that of the routing, down GEMV and
// combine launches it replaces -- without the fp32 pair rows in HBM.
// X4T: the w2 scales stay X4T-coded; the two waves of a pair each decode
// one of its two 16-row scale tiles into LDS (scale-tile layout, exceptions
// patched after the fixed bytes) while their first weight loads are in
// flight, so the K loop reads each lane's scale byte from LDS -- the bytes of
// the dense-scale form, hence the same output bit for bit.
constexpr int DD_PAIRS = 8;
constexpr int DD_X4T_COLS = 128;  // w2 scale columns (I / 32) the fused X4T decode stages
constexpr int DD_X4T_TP = 1 + DD_X4T_COLS / 8;  // 16-byte pieces of a fixed tile at most

template <int NBP, int P, int STEPS, int OUT, bool X4T = false>
__global__ __launch_bounds__(DD_PAIRS * 2 * 64) void moe_decode_down_kernel(
    const uint16_t* __restrict__ act, int64_t inter, const int* __restrict__ ids, int topk, int experts,
    int tokens, const uint8_t* __restrict__ wt, const uint8_t* __restrict__ wst, int64_t hidden,
    const float* __restrict__ route_w, void* __restrict__ out, X4TGemv xg) {
  constexpr int CH = 16 * NBP, NBUF = P < STEPS ? P + 1 : STEPS;
  static_assert(STEPS > 0, "compile-time K steps");
  static_assert(!X4T || NBP == 2, "X4T: one 16-row scale tile per wave of a pair");
  __shared__ f32x4_t red[2 * DD_PAIRS][NBP][64];
  __shared__ float ybuf[DD_PAIRS][CH];
  // X4T: decoded scale tiles [pair][row block][chunk][64] and each wave's staged fixed tile
  __shared__ __attribute__((aligned(16))) uint8_t xsl[X4T ? DD_PAIRS * 2 * (DD_X4T_COLS / 4) * 64 : 16];
  __shared__ __attribute__((aligned(16))) uint8_t xfl[X4T ? 2 * DD_PAIRS * 16 * DD_X4T_TP : 16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, g = lane >> 4;
  const int pair = wave >> 1, kpart = wave & 1;   // pair = intermediate row
  const int pairs = tokens * topk;
  const int pe = pair < pairs ? ids[pair] : -1;
  const bool valid = pe >= 0 && pe < experts;
  const int64_t c0 = (int64_t)blockIdx.x * CH;
  const int64_t nchunk = inter / 128, rgs = hidden / 16;
  const int64_t c_first = kpart * nchunk / 2;
  f32x4_t acc[NBP];
#pragma unroll
  for (int b = 0; b < NBP; ++b) acc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // X4T: this wave decodes tile c0 / 16 + kpart of its pair's expert; the
  // fixed tile and the tile's exception range are loaded before the weights
  u32x4_t xpiece = {0u, 0u, 0u, 0u};
  uint32_t xr[2] = {0u, 0u};
  const int64_t xt = c0 / 16 + kpart;
  const int tp = X4T ? 1 + ((xg.cols + 7) >> 3) : 1;
  if (X4T && valid) {
    if (lane < tp)
      xpiece = *reinterpret_cast<const u32x4_t*>(xg.fixed[0] + ((int64_t)pe * xg.tiles + xt) * (16 * tp) + 16 * lane);
    xr[0] = xg.idx[0][(int64_t)pe * xg.tiles + xt];
    xr[1] = xg.idx[0][(int64_t)pe * xg.tiles + xt + 1];
  }
  auto x4t_decode = [&]() {
    const int cols = xg.cols, sb = (cols + 7) >> 3, span = 16 * cols;
    uint8_t* fl = xfl + wave * 16 * DD_X4T_TP;
    uint8_t* sl = xsl + (pair * 2 + kpart) * (DD_X4T_COLS / 4) * 64;
    if (lane < tp) *reinterpret_cast<u32x4_t*>(fl + 16 * lane) = xpiece;
    // one wave's LDS accesses complete in order: the staged bytes are read
    // below, and the exception bytes overwrite the fixed ones
    const int lo = (int)xr[0], hi = (int)xr[1];
    const uint32_t w0 = lo + lane < hi ? xg.exc[0][lo + lane] : 0u;
    for (int c = lane; c < cols; c += 64) {  // column c of the tile: base(row) + selector bit (row, c)
      uint32_t v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 4 * i + r;
          const uint32_t bit = (fl[16 + row * sb + (c >> 3)] >> (c & 7)) & 1u;
          v[i] |= ((fl[row] + bit) & 0xffu) << (8 * r);
        }
      }
      *reinterpret_cast<u32x4_t*>(sl + (c >> 2) * 64 + (c & 3) * 16) = u32x4_t{v[0], v[1], v[2], v[3]};
    }
    for (int k = lo + lane; k < hi; k += 64) {
      const uint32_t w = k == lo + lane ? w0 : xg.exc[0][k];
      const uint32_t off = (w & 0xffffffu) - (uint32_t)(xt * span);  // wraps past the tile when outside
      if (off < (uint32_t)span) {
        const int r = (int)off / cols, c = (int)off - r * cols;
        sl[(c >> 2) * 64 + (c & 3) * 16 + r] = (uint8_t)(w >> 24);
      }
    }
  };
  // this wave's K half of its pair's intermediate row, staged in LDS once:
  // every lane group of the MFMA A operand reads the same row, so the K
  // loop reads A as LDS broadcasts and only weight loads are in flight
  __shared__ __attribute__((aligned(16))) uint16_t arow[2 * DD_PAIRS][STEPS * 128];
  if (valid) {
    const int e = pe;
    constexpr int APIECES = STEPS * 16, APL = (APIECES + 63) / 64;  // 16-byte pieces of a K half
    const u32x4_t* asrc = reinterpret_cast<const u32x4_t*>(act + (int64_t)pair * inter + c_first * 128);
    u32x4_t apc[APL];
#pragma unroll
    for (int i = 0; i < APL; ++i)
      if (lane + 64 * i < APIECES) apc[i] = asrc[lane + 64 * i];
    const uint8_t* wtile[NBP];
    const uint8_t* stile[NBP];
#pragma unroll
    for (int b = 0; b < NBP; ++b) {
      const int64_t rg = c0 / 16 + b;
      const int64_t t0 = ((int64_t)e * rgs + rg) * nchunk + c_first;
      wtile[b] = wt + t0 * 1024 + 16 * lane;
      stile[b] = X4T ? nullptr : wst + t0 * 64 + lane;
    }
    struct WBuf {
      u32x4_t w[NBP];
      uint32_t ws[NBP];
    };
    auto load_w = [&](int s, WBuf& B) {
#pragma unroll
      for (int b = 0; b < NBP; ++b) {
        B.w[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wtile[b] + (int64_t)s * 1024));
        if (!X4T) B.ws[b] = stile[b][(int64_t)s * 64];
      }
    };
    WBuf wb[NBUF];
#pragma unroll
    for (int s = 0; s < P && s < STEPS; ++s) load_w(s, wb[s]);
    __builtin_amdgcn_sched_barrier(0);
    if (X4T) x4t_decode();
    // one wave's LDS accesses complete in order: its K loop reads what it staged here
    u32x4_t* al = reinterpret_cast<u32x4_t*>(&arow[wave][0]);
#pragma unroll
    for (int i = 0; i < APL; ++i)
      if (lane + 64 * i < APIECES) al[lane + 64 * i] = apc[i];
    __builtin_amdgcn_sched_barrier(0);
    // X4T: this pair's decoded tiles; row block b is tile c0 / 16 + b
    const uint8_t* xs = xsl + pair * 2 * (DD_X4T_COLS / 4) * 64 + c_first * 64 + lane;
    // every token slot (lane group) reads the pair's row; only slot 0 is stored
    auto compute = [&](const WBuf& W, int s) {
      uint32_t ws[NBP];
#pragma unroll
      for (int b = 0; b < NBP; ++b) ws[b] = X4T ? (uint32_t)xs[(b * (DD_X4T_COLS / 4) + s) * 64] : W.ws[b];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16x8_t fa = __builtin_bit_cast(bf16x8_t, al[16 * s + 4 * g + t]);
#pragma unroll
        for (int b = 0; b < NBP; ++b) {
          const bf16x8_t fb = gemm::dequant8<1>(u32x2_t{W.w[b][t], 0u}, ws[b]);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, fb, acc[b], 0, 0, 0);
        }
      }
    };
    // X4T: both tiles of every pair decoded before any wave reads them
    if (X4T) lds_barrier();
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      if (s + P < STEPS) load_w(s + P, wb[(s + P) % NBUF]);
      __builtin_amdgcn_sched_barrier(0);
      compute(wb[s % NBUF], s);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else if (X4T) {
    lds_barrier();  // invalid pairs cross the decode barrier with the others
  }
#pragma unroll
  for (int b = 0; b < NBP; ++b) red[wave][b][lane] = acc[b];
  __syncthreads();
  if (valid && kpart == 0 && g == 0) {  // slot 0: D rows 4 (lane / 16) + j, j = 0
#pragma unroll
    for (int b = 0; b < NBP; ++b) {
      f32x4_t x0 = red[wave][b][lane];
      x0 += red[wave + 1][b][lane];
      ybuf[pair][16 * b + m] = route_w[pair] * x0[0];
    }
  }
  __syncthreads();
  // combine: two adjacent channels per thread, each token's slots in order
  for (int o = threadIdx.x; o < tokens * (CH / 2); o += blockDim.x) {
    const int t = o / (CH / 2), c = 2 * (o % (CH / 2));
    float s0 = 0.f, s1 = 0.f;
    for (int k = 0; k < topk; ++k) {
      const int e = ids[t * topk + k];
      if (e < 0 || e >= experts) continue;
      s0 += ybuf[t * topk + k][c];
      s1 += ybuf[t * topk + k][c + 1];
    }
    if (OUT == 2) {
      float* op = static_cast<float*>(out) + (int64_t)t * hidden + c0 + c;
      op[0] = s0;
      op[1] = s1;
    } else {
      *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(out) + (int64_t)t * hidden + c0 + c) =
          f32x2_to_bf16x2_bits(s0, s1);
    }
  }
}

// ------------------------ decode down projection with the combine, 9-32 pairs --
// For a decode of up to DW_PAIRS pairs (dense scales, intermediate 1024 or
// 2048): workgroup b owns output channels 32 b .. 32 b + 31 of every token.
// The pairs routed to one expert form entries of up to SMALL_MAX token slots
// exactly as the per-pair gate/up GEMV groups them; the work units are
// (entry, K half), unit u = 2 entry + half, and wave w runs units w, w + 16,
// ... back to back with the weight prefetch running across unit boundaries.
// A unit is the listed down GEMV's work for that entry, half and channel
// block: the same chunk order and MFMA order, the intermediates of every
// pair staged in LDS once and read as the MFMA A operand.  The two halves of
// a pair meet in LDS and are summed in the GEMV's order, scaled by the route
// weight and summed over each token's slots in the combine's order, so the
// output is bitwise that of the routing, listed down GEMV and combine
// launches this one kernel replaces.
// X4T: the w2 scales stay X4T-coded.  A unit's wave decodes the scale bytes
// of its K half of the two 16-row scale tiles into its own LDS region in the
// dense tiles' per-step order (row bases and selector bits, then the tiles'
// exceptions in that half); the fixed bytes and the first 64 exception words
// of the next unit are loaded at its setup, while the current unit runs, and
// the region is rewritten after the current unit's last read of it (one
// wave's LDS accesses complete in order).  The bytes are those of the dense
// scale tiles, so the output is bitwise that of the dense-scale form.
constexpr int DW_PAIRS = 32;
#ifndef KQ_DW_P
#define KQ_DW_P 2
#endif

template <int STEPS, int OUT, bool X4T = false>
__global__ __launch_bounds__(1024) void moe_decode_down_wide_kernel(
    const uint16_t* __restrict__ act, int64_t inter, const int* __restrict__ ids, int topk, int experts,
    int tokens, const uint8_t* __restrict__ wt, const uint8_t* __restrict__ wst, int64_t hidden,
    const float* __restrict__ route_w, void* __restrict__ out, X4TGemv xg) {
#pragma clang fp contract(off)
  constexpr int NBP = 2, CH = 16 * NBP, NBUF = 4, P = KQ_DW_P;
  constexpr int KH = STEPS * 128;                  // k per half
  constexpr int AROW = 2 * KH + 8;                 // bf16 per staged row: both halves + 16 B of pad
  // X4T: scale columns of a K half (cols = inter / 32 = 8 STEPS in all) and
  // each wave's decoded bytes [b][s][64]
  constexpr int XHC = 4 * STEPS, XREG = NBP * STEPS * 64;
  static_assert(STEPS % NBUF == 0, "ring slot of step s is s % NBUF in every unit");
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[DW_PAIRS][AROW];
  __shared__ float yh[DW_PAIRS][2][CH];            // each pair's two K-half partials
  __shared__ float ybuf[DW_PAIRS][CH];             // route weight x (half 0 + half 1)
  __shared__ __attribute__((aligned(16))) uint8_t xsl[X4T ? 16 * XREG : 16];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m = lane & 15, g = lane >> 4;
  const int pairs = tokens * topk;
  const int64_t c0 = (int64_t)blockIdx.x * CH;
  const int64_t nchunk = inter / 128, rgs = hidden / 16;

  // entries: lane j < pairs holds pair j's expert (-1 if invalid) and its
  // rank among the pairs of that expert; pair j starts an entry when the rank
  // is a multiple of SMALL_MAX
  int ej = lane < pairs ? ids[lane] : -1;
  if (ej >= experts) ej = -1;
  int rank = 0;
  for (int i = 0; i < pairs; ++i) {
    const int ei = __shfl(ej, i);
    rank += (i < lane && ei == ej) ? 1 : 0;
  }
  const uint64_t starts = __ballot(ej >= 0 && rank % SMALL_MAX == 0);
  const int units = 2 * __popcll(starts);

  // stage every pair's intermediate row (rows = pair index, as the gate/up
  // GEMV wrote them) with direct loads: 1 KiB of a row per instruction,
  // instruction q = wave + 16 i moving KiB q % CPR of row q / CPR; they are
  // issued before the weight prefetch and waited for after it
  constexpr int CPR = 2 * KH * 2 / 1024;           // KiB per row
  const dma::i32x4_t a_rsrc = dma::make_rsrc(act, (uint32_t)(pairs * inter * 2));
  const uint32_t a_lds0 = dma::lds_offset_of(a_lds);
  int staged = 0;                                  // this wave's direct loads
  for (int q = wave; q < pairs * CPR; q += 16) {
    const int pr = q / CPR, kb = q - pr * CPR;
    dma::load_to_lds16(a_rsrc, (uint32_t)(pr * inter * 2 + kb * 1024 + 16 * lane),
                       a_lds0 + (uint32_t)(pr * AROW * 2 + kb * 1024));
    ++staged;
  }

  // unit u: entry u / 2 starts at the (u / 2)-th set bit of `starts`; its
  // expert, slot count and this lane's slot pair (slot m; slot 0 past n)
  struct Unit {
    const uint8_t* w[NBP];
    const uint8_t* s[NBP];
    int half, n, spair;
    // X4T, lanes 0..31 = (tile b = lane / 16, row lane % 16): the row base
    // and the selector bytes of the half's columns; every lane: one of the
    // first 64 exception words of both tiles, and the tiles' exception range
    uint32_t xbase, xb[XHC / 8], xexc;
    int xlo, xhi;
  };
  const int64_t xt0 = c0 / 16;  // X4T: the workgroup's first scale tile
  auto setup = [&](int u, Unit& U) {
    uint64_t st = starts;
    for (int i = u >> 1; i > 0; --i) st &= st - 1;
    const int x = (int)__builtin_ctzll(st);
    const int e = __shfl(ej, x);
    const uint64_t same = __ballot(ej == e);
    const int r0 = __popcll(same & ((1ull << x) - 1));
    const int cnt = __popcll(same) - r0;
    U.n = cnt < SMALL_MAX ? cnt : SMALL_MAX;
    uint64_t mk = same;
    for (int i = r0 + (m < U.n ? m : 0); i > 0; --i) mk &= mk - 1;
    U.spair = (int)__builtin_ctzll(mk);
    U.half = u & 1;
#pragma unroll
    for (int b = 0; b < NBP; ++b) {
      const int64_t t0 = ((int64_t)e * rgs + c0 / 16 + b) * nchunk + U.half * STEPS;
      U.w[b] = wt + t0 * 1024 + 16 * lane;
      U.s[b] = X4T ? nullptr : wst + t0 * 64 + lane;
    }
    if constexpr (X4T) {
      // the exception range of tiles xt0 and xt0 + 1 (one range: they are
      // consecutive), then the fixed bytes; the words themselves are loaded
      // by x4t_fetch once the range has landed
      const int64_t ti = (int64_t)e * xg.tiles + xt0;
      U.xlo = (int)xg.idx[0][ti];  // (kept in vector registers: a scalar copy would wait for the load here)
      U.xhi = (int)xg.idx[0][ti + 2];
      // (lanes 32..63 load what lanes 0..31 load: every lane issues the
      // same loads, so the waits for them are counted exactly)
      const uint8_t* pc = xg.fixed[0] + (ti + ((lane >> 4) & 1)) * (16 * (1 + XHC / 4));
      U.xbase = pc[lane & 15];
      // selector bytes of row lane % 16, columns XHC half .. XHC half + XHC - 1
      const uint8_t* bm = pc + 16 + (lane & 15) * (XHC / 4) + U.half * (XHC / 8);
#pragma unroll
      for (int i = 0; i < XHC / 8; ++i) U.xb[i] = bm[i];
    }
  };
  // (lanes past the range read a valid word they do not use, so that the
  // load is issued by every lane)
  auto x4t_fetch = [&](Unit& U) {
    const uint32_t* src = U.xlo + lane < U.xhi ? xg.exc[0] + U.xlo + lane : xg.idx[0];
    U.xexc = *src;
  };
  // X4T: decode unit U's bytes into this wave's region (after the wave's
  // last read of the previous unit's bytes)
  auto x4t_write = [&](const Unit& U) {
    uint8_t* sl = xsl + wave * XREG;
    if (lane < 32) {
      const int b = lane >> 4, row = lane & 15;
#pragma unroll
      for (int j = 0; j < XHC; ++j) {  // column XHC half + j: base + selector bit
        const uint32_t bit = (U.xb[j >> 3] >> (j & 7)) & 1u;
        sl[(b * STEPS + (j >> 2)) * 64 + (j & 3) * 16 + row] = (uint8_t)(U.xbase + bit);
      }
    }
    auto patch = [&](uint32_t w) {
      const int cols = 8 * STEPS, span = 16 * cols;
      const uint32_t off = (w & 0xffffffu) - (uint32_t)(xt0 * span);  // wraps past the tiles when outside
      if (off < 2u * span) {
        const int b = off >= (uint32_t)span ? 1 : 0, o = (int)off - b * span;
        const int r = o / cols, j = o - r * cols - U.half * XHC;
        if (j >= 0 && j < XHC) sl[(b * STEPS + (j >> 2)) * 64 + (j & 3) * 16 + r] = (uint8_t)(w >> 24);
      }
    };
    if (U.xlo + lane < U.xhi) patch(U.xexc);
    // more than 64 exceptions: the rest loaded here (its waits also wait for
    // the weight prefetch in flight)
    for (int k = U.xlo + 64 + lane; k < U.xhi; k += 64) patch(xg.exc[0][k]);
  };
  struct WBuf {
    u32x4_t w[NBP];
    uint32_t ws[NBP];
  };
  auto load_w = [&](const Unit& U, int s, WBuf& B) {
#pragma unroll
    for (int b = 0; b < NBP; ++b) {
      B.w[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(U.w[b] + (int64_t)s * 1024));
      if constexpr (!X4T) B.ws[b] = U.s[b][(int64_t)s * 64];
    }
  };
  WBuf wb[NBUF];
  Unit cur, nxt;
  int u = wave;
  if (u < units) {
    setup(u, cur);
#pragma unroll
    for (int s = 0; s < P; ++s) load_w(cur, s, wb[s]);
    if constexpr (X4T) x4t_fetch(cur);
  }
  // the staged rows have landed once only the (younger) weight prefetch is in
  // flight: 2 P loads per block (with X4T scales one per block, and the
  // exception word), or none without a unit
  if (u < units) __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(X4T ? NBP * P + 1 : 2 * NBP * P));
  else __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
  (void)staged;
  if constexpr (X4T)
    if (u < units) x4t_write(cur);
  lds_barrier();  // every wave's rows are staged
  while (u < units) {
    const int un = u + 16;
    // the next unit; after the wave's last, this one again with its weight
    // pointers on the first 2 KiB of the weights (cached by every wave that
    // reads them): every unit issues the same loads, so the waits for them
    // are counted exactly (with a conditional prefetch the compiler waits for
    // all loads in flight at the last steps)
    setup(un < units ? un : u, nxt);
    if (un >= units) {
#pragma unroll
      for (int b = 0; b < NBP; ++b) {
        nxt.w[b] = wt + 16 * lane;
        nxt.s[b] = X4T ? nullptr : wst + lane;
      }
    }
    f32x4_t acc[NBP];
#pragma unroll
    for (int b = 0; b < NBP; ++b) acc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const u32x4_t* arow = reinterpret_cast<const u32x4_t*>(&a_lds[cur.spair][cur.half * KH]);
    const uint8_t* xs = xsl + wave * XREG + lane;  // X4T: this unit's decoded bytes
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      if (s + P < STEPS) load_w(cur, s + P, wb[(s + P) % NBUF]);
      else load_w(nxt, s + P - STEPS, wb[(s + P) % NBUF]);
      // X4T: the next unit's first exception words, once its range has landed
      if (X4T && s == STEPS / 2) x4t_fetch(nxt);
      __builtin_amdgcn_sched_barrier(0);
      const WBuf& W = wb[s % NBUF];
      uint32_t ws[NBP];
#pragma unroll
      for (int b = 0; b < NBP; ++b) ws[b] = X4T ? (uint32_t)xs[(b * STEPS + s) * 64] : W.ws[b];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16x8_t fa = __builtin_bit_cast(bf16x8_t, arow[16 * s + 4 * g + t]);
#pragma unroll
        for (int b = 0; b < NBP; ++b) {
          const bf16x8_t fb = gemm::dequant8<1>(u32x2_t{W.w[b][t], 0u}, ws[b]);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, fb, acc[b], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (X4T)
      if (un < units) x4t_write(nxt);
    // D layout: lane holds rows (slots) 4 g + j, column m
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int slot = 4 * g + j;
      const int pr = __shfl(cur.spair, slot);
      if (slot < cur.n) {
#pragma unroll
        for (int b = 0; b < NBP; ++b) yh[pr][cur.half][16 * b + m] = acc[b][j];
      }
    }
    u = un;
    cur = nxt;
  }
  lds_barrier();
  for (int o = threadIdx.x; o < pairs * CH; o += 1024) {
    const int pr = o / CH, c = o - pr * CH;
    if (pr < pairs) {
      const int e = ids[pr];
      if (e >= 0 && e < experts) ybuf[pr][c] = route_w[pr] * (yh[pr][0][c] + yh[pr][1][c]);
    }
  }
  lds_barrier();
  // combine: two adjacent channels per thread, each token's slots in order
  for (int o = threadIdx.x; o < tokens * (CH / 2); o += 1024) {
    const int t = o / (CH / 2), c = 2 * (o % (CH / 2));
    float s0 = 0.f, s1 = 0.f;
    for (int k = 0; k < topk; ++k) {
      const int e = ids[t * topk + k];
      if (e < 0 || e >= experts) continue;
      s0 += ybuf[t * topk + k][c];
      s1 += ybuf[t * topk + k][c + 1];
    }
    if (OUT == 2) {
      float* op = static_cast<float*>(out) + (int64_t)t * hidden + c0 + c;
      op[0] = s0;
      op[1] = s1;
    } else {
      *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(out) + (int64_t)t * hidden + c0 + c) =
          f32x2_to_bf16x2_bits(s0, s1);
    }
  }
}

}  // namespace moe
}  // namespace kq

using namespace kq;
using namespace kq::moe;

// GEMV launch shapes (channels per workgroup = RW * 16 * NBP), measured on
// the decode batches of 1, 4 and 16 tokens (hidden 7168, intermediate 2048):
// K split over 4 waves for gate/up (14 steps of 128 each) and over 2 for down
// (8 steps) streams better than shorter per-wave runs; prefetch depth 2-3 and
// one or two row groups per workgroup are within 1 % of each other.
#ifndef KQ_GU_NBP
#define KQ_GU_NBP 2
#define KQ_GU_S 4
#define KQ_GU_RW 1
#define KQ_GU_P 2
#endif
#ifndef KQ_DD_P
#define KQ_DD_P 2
#endif
#ifndef KQ_DN_NBP
#define KQ_DN_NBP 4
#define KQ_DN_S 2
#define KQ_DN_RW 1
#define KQ_DN_P 2
#endif

// x4t: the instantiation decoding X4T scales in its prologue, with that
// decode's dynamic LDS.
// route: one workgroup per decode pair, no list (dense scales, gate/up shape)
template <bool GATEUP, int NBP, int S, int RW, int P, typename... Args>
static hipError_t launch_small(bool x4t, int64_t experts_max, int64_t channels, int64_t K, int cols,
                               hipStream_t st, const DecodeRouteArgs* route, Args... args) {
  constexpr int CH = RW * 16 * NBP, NB = GATEUP ? 2 * NBP : NBP;
  const dim3 grid((unsigned)experts_max, (unsigned)(channels / CH));
  const int64_t nchunk = K / 128;
  const int64_t steps = nchunk % S == 0 ? nchunk / S : 0;
  const size_t shm = x4t ? x4t_gemv_lds(RW * NB, nchunk, cols) : 0;
  const DecodeRouteArgs none{nullptr, 0, 0};
  constexpr bool CAN_ROUTE = GATEUP;
  if (route && !CAN_ROUTE) return hipErrorInvalidValue;
  switch (steps) {
#define KQ_SMALL_CASE(N)                                                                                      \
    case N:                                                                                                   \
      if (x4t && route) moe_small_kernel<GATEUP, true, NBP, S, RW, P, N, CAN_ROUTE>                           \
          <<<grid, S * RW * 64, shm, st>>>(args..., *route);                                                  \
      else if (x4t) moe_small_kernel<GATEUP, true, NBP, S, RW, P, N><<<grid, S * RW * 64, shm, st>>>(args..., none); \
      else if (route) moe_small_kernel<GATEUP, false, NBP, S, RW, P, N, CAN_ROUTE>                            \
          <<<grid, S * RW * 64, 0, st>>>(args..., *route);                                                    \
      else moe_small_kernel<GATEUP, false, NBP, S, RW, P, N><<<grid, S * RW * 64, 0, st>>>(args..., none);    \
      break;
    KQ_SMALL_CASE(2) KQ_SMALL_CASE(4) KQ_SMALL_CASE(7) KQ_SMALL_CASE(8) KQ_SMALL_CASE(14)
    KQ_SMALL_CASE(16) KQ_SMALL_CASE(28)
#undef KQ_SMALL_CASE
    default:
      if (x4t && route)
        moe_small_kernel<GATEUP, true, NBP, S, RW, P, 0, CAN_ROUTE><<<grid, S * RW * 64, shm, st>>>(args..., *route);
      else if (x4t) moe_small_kernel<GATEUP, true, NBP, S, RW, P, 0><<<grid, S * RW * 64, shm, st>>>(args..., none);
      else if (route)
        moe_small_kernel<GATEUP, false, NBP, S, RW, P, 0, CAN_ROUTE><<<grid, S * RW * 64, 0, st>>>(args..., *route);
      else moe_small_kernel<GATEUP, false, NBP, S, RW, P, 0><<<grid, S * RW * 64, 0, st>>>(args..., none);
  }
  return hipGetLastError();
}

template <bool GATEUP, int AF, int NBP, int S, int RW, int P, typename... Args>
static hipError_t launch_small_mx(bool x4t, int64_t experts_max, int64_t channels, int64_t K, int cols,
                                  hipStream_t st, Args... args) {
  constexpr int CH = RW * 16 * NBP, NB = GATEUP ? 2 * NBP : NBP;
  const dim3 grid((unsigned)experts_max, (unsigned)(channels / CH));
  const int64_t nchunk = K / 128;
  const int64_t steps = nchunk % S == 0 ? nchunk / S : 0;
  const size_t shm = x4t ? x4t_gemv_lds(RW * NB, nchunk, cols) : 0;
  switch (steps) {
#define KQ_SMALL_MX_CASE(N)                                                                                \
    case N:                                                                                                \
      if (x4t) moe_small_mx_kernel<GATEUP, true, AF, NBP, S, RW, P, N><<<grid, S * RW * 64, shm, st>>>(args...); \
      else moe_small_mx_kernel<GATEUP, false, AF, NBP, S, RW, P, N><<<grid, S * RW * 64, 0, st>>>(args...);       \
      break;
    KQ_SMALL_MX_CASE(2) KQ_SMALL_MX_CASE(4) KQ_SMALL_MX_CASE(7) KQ_SMALL_MX_CASE(8) KQ_SMALL_MX_CASE(14)
    KQ_SMALL_MX_CASE(16)
#undef KQ_SMALL_MX_CASE
    default:
      if (x4t) moe_small_mx_kernel<GATEUP, true, AF, NBP, S, RW, P, 0><<<grid, S * RW * 64, shm, st>>>(args...);
      else moe_small_mx_kernel<GATEUP, false, AF, NBP, S, RW, P, 0><<<grid, S * RW * 64, 0, st>>>(args...);
  }
  return hipGetLastError();
}

// The GEMV kernels' X4T planes from the expansion's plane descriptors:
// w1 / w3 for gate/up, w2 for down (or nothing without X4T scales).
static X4TGemv x4t_gemv(const X4TExpandArgs* xa, bool gateup) {
  X4TGemv g{};
  if (!xa) return g;
  const X4TPlane& p0 = gateup ? xa->p[0] : xa->p[2];
  const X4TPlane& p1 = gateup ? xa->p[1] : xa->p[2];
  g.fixed[0] = p0.fixed;
  g.fixed[1] = p1.fixed;
  g.exc[0] = p0.exceptions;
  g.exc[1] = p1.exceptions;
  g.idx[0] = p0.tile_index;
  g.idx[1] = p1.tile_index;
  g.tiles = p0.tiles;
  g.cols = p0.cols;
  return g;
}

// Activation-quantized forward (W4A8 / W4A4): the same routing and combine,
// tokens and intermediates MX-quantized (kq_mx_quantize's rule) before each
// projection, both GEMM shapes on the block-scaled MFMA.
template <int AF>
static int moe_forward_mx(const Layout& L, unsigned char* w, const ActParams& ap, const void* x,
                          int64_t ldx, int64_t tokens, int64_t hidden, const float* route_weights,
                          int topk, int64_t inter, const uint8_t* w13_t, const uint8_t* w13_st,
                          const uint8_t* w2_t, const uint8_t* w2_st, const int* sslot,
                          const X4TExpandArgs* xa, bool decode, int grid_dma, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  const int fmt = AF == 4 ? KQ_FMT_MXFP4_E2M1 : KQ_FMT_MXFP8_E4M3;
  const int* offsets = (const int*)(w + L.offsets);
  const int* sorted = (const int*)(w + L.sorted);
  const int* small_list = (const int*)(w + L.small_list);
  const int* large_tiles = (const int*)(w + L.large_tiles);
  const int* meta = (const int*)(w + L.meta);
  uint16_t* act = (uint16_t*)(w + L.act);
  float* y = (float*)(w + L.y);
  uint8_t *xq = w + L.xq, *xs = w + L.xs, *aq = w + L.aq, *as = w + L.as;
  const bool any_large = !decode && L.pairs > SMALL_MAX;
  hipError_t e;
  int rc = kq_mx_quantize(fmt, KQ_DT_BF16, x, ldx, tokens, hidden, xq, xs, 0, stream);
  if (rc != KQ_OK) return rc;
  const int* gslot = xa ? nullptr : sslot;  // the GEMVs decode X4T scales themselves
  e = launch_small_mx<true, AF, KQ_GU_NBP, KQ_GU_S, KQ_GU_RW, KQ_GU_P>(
      xa != nullptr, L.max_list, inter, hidden, (int)(hidden / 32), st, (const uint8_t*)xq,
      (const uint8_t*)xs, topk, sorted, small_list, w13_t, w13_st, gslot, x4t_gemv(xa, true), 2 * inter,
      hidden, inter, ap, route_weights, act, y, hidden);
  if (e != hipSuccess) return kq_check_launch(e, "kq_moe_forward/gateup_small");
  const int64_t abytes = AF == 4 ? hidden / 2 : hidden;
  // E2M1 activations with K a multiple of 256 take the whole-line kernel
  const bool lines = AF == 4 && hidden % mx4_gemm::SK == 0 && inter % mx4_gemm::SK == 0;
  if (any_large && lines) {
    moe_large_mx4_kernel<true><<<grid_dma, THREADS, 0, st>>>(
        xq, xs, (uint32_t)(tokens * abytes), (uint32_t)(tokens * hidden / 32), topk, offsets, sorted,
        large_tiles, meta, w13_t, w13_st, sslot, 2 * inter, hidden, inter, (int)(inter / (BN / 2)), ap,
        route_weights, act, y, hidden);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/gateup_large");
  } else if (any_large) {
    moe_large_mx_kernel<true, AF><<<grid_dma, THREADS, 0, st>>>(
        xq, xs, (uint32_t)(tokens * abytes), (uint32_t)(tokens * hidden / 32), topk, offsets, sorted,
        large_tiles, meta, w13_t, w13_st, sslot, 2 * inter, hidden, inter, (int)(inter / (BN / 2)), ap,
        route_weights, act, y, hidden);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/gateup_large");
  }
  rc = kq_mx_quantize(fmt, KQ_DT_BF16, act, inter, L.pairs, inter, aq, as, 0, stream);
  if (rc != KQ_OK) return rc;
  e = launch_small_mx<false, AF, KQ_DN_NBP, KQ_DN_S, KQ_DN_RW, KQ_DN_P>(
      xa != nullptr, L.max_list, hidden, inter, (int)(inter / 32), st, (const uint8_t*)aq,
      (const uint8_t*)as, topk, sorted, small_list, w2_t, w2_st, gslot, x4t_gemv(xa, false), hidden, inter,
      inter, ap, route_weights, act, y, hidden);
  if (e != hipSuccess) return kq_check_launch(e, "kq_moe_forward/down_small");
  if (any_large && lines) {
    moe_large_mx4_kernel<false><<<grid_dma, THREADS, 0, st>>>(
        aq, as, (uint32_t)(L.pairs * inter / 2), (uint32_t)(L.pairs * inter / 32), topk, offsets, sorted,
        large_tiles, meta, w2_t, w2_st, sslot, hidden, inter, inter, (int)(hidden / BN), ap, route_weights, act,
        y, hidden);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/down_large");
  } else if (any_large) {
    const int64_t ibytes = AF == 4 ? inter / 2 : inter;
    moe_large_mx_kernel<false, AF><<<grid_dma, THREADS, 0, st>>>(
        aq, as, (uint32_t)(L.pairs * ibytes), (uint32_t)(L.pairs * inter / 32), topk, offsets, sorted,
        large_tiles, meta, w2_t, w2_st, sslot, hidden, inter, inter, (int)(hidden / BN), ap, route_weights, act,
        y, hidden);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/down_large");
  }
  return KQ_OK;
}

extern "C" int64_t kq_moe_workspace_size(int64_t tokens, int topk, int experts, int64_t hidden,
                                         int64_t inter) {
  if (tokens < 0 || topk <= 0 || experts <= 0 || hidden <= 0 || inter <= 0) return -1;
  return (int64_t)make_layout(tokens, topk, experts, hidden, inter).total;
}

// The forward behind both entry points.  With xa non-null the scales come
// from X4T planes: the routing also ranks the routed experts, one launch
// expands their scales into workspace slots (xa's output fields are filled
// here) and the GEMMs read each expert's scales from its slot.
static int moe_forward_impl(const char* fn, int activation, float act_beta, float act_linear_beta,
                            const void* x, int64_t ldx, int64_t tokens, int64_t hidden,
                            const int32_t* route_ids, const float* route_weights, int topk, int experts,
                            int64_t inter, const uint8_t* w13_t, const uint8_t* w13_st,
                            const uint8_t* w2_t, const uint8_t* w2_st, X4TExpandArgs* xa, int out_dtype,
                            void* out, void* workspace, int64_t workspace_bytes, uint32_t flags,
                            void* stream) {
  if (flags & ~(uint32_t)(KQ_MOE_REGISTER_STAGED | KQ_MOE_ACT_MXFP8 | KQ_MOE_ACT_MXFP4))
    return kq_fail(KQ_ERR_INVALID, "%s: unknown flags 0x%x", fn, flags);
  const int act_fmt = (flags & KQ_MOE_ACT_MXFP4) ? 4 : (flags & KQ_MOE_ACT_MXFP8) ? 0 : -1;
  if ((flags & KQ_MOE_ACT_MXFP4) && (flags & KQ_MOE_ACT_MXFP8))
    return kq_fail(KQ_ERR_INVALID, "%s: KQ_MOE_ACT_MXFP8 and KQ_MOE_ACT_MXFP4 exclude each other", fn);
  if (act_fmt >= 0 && (flags & KQ_MOE_REGISTER_STAGED))
    return kq_fail(KQ_ERR_INVALID, "%s: the activation-quantized modes have no register-staged kernel", fn);
  if (activation != KQ_ACT_SITU && activation != KQ_ACT_SWIGLU)
    return kq_fail(KQ_ERR_INVALID, "%s: unknown activation %d", fn, activation);
  if (out_dtype != KQ_DT_BF16 && out_dtype != KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "%s: output dtype must be bf16 or f32", fn);
  if (tokens < 0 || topk <= 0 || topk > 64 || experts <= 0 || experts > MAX_EXPERTS)
    return kq_fail(KQ_ERR_INVALID, "%s: need tokens >= 0, 1 <= topk <= 64, 1 <= experts <= %d", fn,
                   MAX_EXPERTS);
  // A decode batch with bf16 activations runs only the GEMV kernels, whose K
  // and channel blocks need multiples of 128 / 64: there an intermediate size
  // that is a multiple of 256 (a tensor-parallel shard, e.g. 256 channels per
  // rank at hidden 3584) is accepted too.
  const bool gemv_only = act_fmt < 0 && tokens * topk <= DECODE_MAX_PAIRS;
  if (hidden <= 0 || inter <= 0 || hidden % 512 != 0 || inter % (gemv_only ? 256 : 512) != 0)
    return kq_fail(KQ_ERR_INVALID,
                   "%s: hidden and intermediate sizes must be multiples of 512, the intermediate size of a "
                   "bf16-activation decode batch a multiple of 256 (hidden=%lld inter=%lld)",
                   fn, (long long)hidden, (long long)inter);
  if (ldx < hidden || ldx % 8 != 0)
    return kq_fail(KQ_ERR_INVALID, "%s: ldx must be >= hidden and a multiple of 8", fn);
  if (kq_misaligned(x, 16) || kq_misaligned(w13_t, 16) || kq_misaligned(w2_t, 16) ||
      kq_misaligned(w13_st, 2) || kq_misaligned(w2_st, 2) || kq_misaligned(workspace, 256) ||
      kq_misaligned(out, 16))
    return kq_fail(KQ_ERR_INVALID, "%s: misaligned buffer", fn);
  if (tokens * topk > INT32_MAX / 2)
    return kq_fail(KQ_ERR_LIMIT, "%s: too many routed pairs", fn);
  const Layout L = make_layout(tokens, topk, experts, hidden, inter, xa != nullptr);
  if (workspace_bytes < (int64_t)L.total)
    return kq_fail(KQ_ERR_INVALID, "%s: workspace of %lld bytes < required %lld", fn,
                   (long long)workspace_bytes, (long long)L.total);
  if (tokens == 0) return KQ_OK;
  hipStream_t st = (hipStream_t)stream;
  unsigned char* w = (unsigned char*)workspace;
  int* counts = (int*)(w + L.counts);
  int* offsets = (int*)(w + L.offsets);
  int* block_counts = (int*)(w + L.block_counts);
  int* sorted = (int*)(w + L.sorted);
  int* pos = (int*)(w + L.pos);  // sorted position of every routed pair: its row of y
  int* small_list = (int*)(w + L.small_list);
  int* large_tiles = (int*)(w + L.large_tiles);
  int* meta = (int*)(w + L.meta);
  uint16_t* act = (uint16_t*)(w + L.act);
  float* y = (float*)(w + L.y);
  const ActParams ap{activation, act_beta, act_linear_beta};
  int* rank_of = xa ? (int*)(w + L.rank_of) : nullptr;
  int* routed = xa ? (int*)(w + L.routed) : nullptr;
  const int max_routed = (int)L.max_routed;
  hipError_t e;
  // Decode: few pairs.  Every routed expert takes the GEMV path (in entries
  // of up to 16 pairs) and the grouped GEMM is not launched.
  const bool decode = L.pairs <= DECODE_MAX_PAIRS;
  // bf16 activations: the direct-to-LDS grouped GEMM (128-row tiles) unless a
  // buffer exceeds one 32-bit buffer range; the register-staged and the
  // activation-quantized kernels take 256-row tiles
  const uint64_t x_bytes = (uint64_t)tokens * ldx * 2, act_bytes = (uint64_t)L.pairs * inter * 2;
  const bool dma_path = act_fmt < 0 && !(flags & KQ_MOE_REGISTER_STAGED) && x_bytes <= dma::MAX_RANGE &&
                        act_bytes <= dma::MAX_RANGE && (uint64_t)(2 * inter) * hidden / 2 <= dma::MAX_RANGE;
  const int tile_rows = dma_path ? DMA_BM : BM;

  // A decode of at most DD_PAIRS pairs with dense scales and bf16
  // activations needs no routing launch: one gate/up workgroup per pair, and
  // the down projection with the combine in one launch.
  // decodes of at most DD_PAIRS pairs: per-pair gate/up + moe_decode_down_kernel;
  // up to DW_PAIRS pairs: per-pair gate/up + moe_decode_down_wide_kernel
  const bool dd = L.pairs <= DD_PAIRS && (inter == 512 || inter == 1024 || inter == 2048 || inter == 4096) &&
                  (!xa || inter / 32 <= DD_X4T_COLS);
  const bool dw = !dd && L.pairs <= DW_PAIRS && (inter == 1024 || inter == 2048) && tokens <= 64;
  const bool route_in_gemv = decode && act_fmt < 0 && hidden % 32 == 0 && (dd || dw);
  const DecodeRouteArgs dra{route_ids, experts, (int)L.pairs};
  if (decode && !route_in_gemv) {
    route_decode_kernel<<<1, DECODE_MAX_PAIRS, 0, st>>>(route_ids, (int)L.pairs, experts, sorted,
                                                         small_list, (int)L.max_list, meta, pos);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/route");
  } else if (decode) {
  } else if (L.pairs <= PREP_ONE) {
    route_prep_one_kernel<<<1, 1024, 0, st>>>(route_ids, (int)L.pairs, experts, counts, offsets,
                                               sorted, small_list, large_tiles, meta, (int)L.max_large,
                                               rank_of, routed, max_routed, tile_rows, pos);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/prep");
  } else {
    route_hist_kernel<<<(unsigned)L.nblk, PREP, 0, st>>>(route_ids, L.pairs, experts, block_counts);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/hist");
    route_scan_kernel<<<1, 1024, 0, st>>>(block_counts, (int)L.nblk, experts, counts, offsets,
                                          small_list, large_tiles, meta, (int)L.max_large, rank_of,
                                          routed, max_routed, tile_rows);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/scan");
    route_scatter_kernel<<<(unsigned)L.nblk, PREP, 0, st>>>(route_ids, L.pairs, experts, offsets,
                                                            block_counts, sorted, pos);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/scatter");
  }

  if (xa) {
    xa->p[0].out = xa->p[1].out = w + L.s13;
    xa->p[2].out = w + L.s2;
    if ((e = x4t_expand_routed(*xa, routed, max_routed, st)) != hipSuccess)
      return kq_check_launch(e, "kq_moe_forward_x4t/expand");
    w13_st = w + L.s13;
    w2_st = w + L.s2;
  }
  const int* sslot = rank_of;                // grouped-GEMM experts' scale slots
  const int* gslot = nullptr;                // the GEMVs read dense scales or decode X4T ones

  auto combine = [&]() -> int {
    const dim3 cgrid((unsigned)((hidden / 4 + 255) / 256), (unsigned)tokens);
    if (out_dtype == KQ_DT_F32)
      moe_combine_kernel<2><<<cgrid, 256, 0, st>>>(y, pos, route_weights, route_ids, topk, experts, hidden, out);
    else
      moe_combine_kernel<0><<<cgrid, 256, 0, st>>>(y, pos, route_weights, route_ids, topk, experts, hidden, out);
    return kq_check_launch(hipGetLastError(), "kq_moe_forward/combine");
  };

  if (act_fmt >= 0) {
    if ((uint64_t)tokens * hidden > dma::MAX_RANGE || (uint64_t)L.pairs * inter > dma::MAX_RANGE ||
        (uint64_t)(2 * inter) * hidden / 2 > dma::MAX_RANGE)
      return kq_fail(KQ_ERR_LIMIT, "%s: activation-quantized operands exceed 4 GiB", fn);
    int grid_mx = 8;
    if (!decode && L.pairs > SMALL_MAX) {
      int dev = 0, cus = 0;
      if ((e = hipGetDevice(&dev)) == hipSuccess)
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      if (e != hipSuccess) return kq_check_launch(e, "kq_moe_forward/device");
      grid_mx = cus / 8 * 8 > 0 ? cus / 8 * 8 : 8;
    }
    const int rc = act_fmt == 4
        ? moe_forward_mx<4>(L, w, ap, x, ldx, tokens, hidden, route_weights, topk, inter, w13_t, w13_st,
                            w2_t, w2_st, sslot, xa, decode, grid_mx, stream)
        : moe_forward_mx<0>(L, w, ap, x, ldx, tokens, hidden, route_weights, topk, inter, w13_t, w13_st,
                            w2_t, w2_st, sslot, xa, decode, grid_mx, stream);
    if (rc != KQ_OK) return rc;
    return combine();
  }

  const uint16_t* xb = (const uint16_t*)x;
  // gate/up
  {
    e = launch_small<true, KQ_GU_NBP, KQ_GU_S, KQ_GU_RW, KQ_GU_P>(
        xa != nullptr, route_in_gemv ? L.pairs : L.max_list, inter, hidden, (int)(hidden / 32), st,
        route_in_gemv ? &dra : nullptr, xb,
        ldx, topk, (const int*)sorted,
        (const int*)small_list, w13_t, w13_st, gslot, x4t_gemv(xa, true), 2 * inter, hidden, inter, ap,
        route_weights, act, y, hidden);
    if (e != hipSuccess) return kq_check_launch(e, "kq_moe_forward/gateup_small");
  }
  const size_t lds = 2 * (size_t)STAGE + BM * sizeof(int);
  const bool any_large = !decode && L.pairs > SMALL_MAX;
  int grid_dma = 0;
  if (any_large && dma_path) {
    int dev = 0, cus = 0;
    if ((e = hipGetDevice(&dev)) == hipSuccess)
      e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return kq_check_launch(e, "kq_moe_forward/device");
    grid_dma = cus / 8 * 8 > 0 ? cus / 8 * 8 : 8;
    const int col_tiles = (int)(inter / (DMA_BN / 2));
    moe_large_dma_kernel<true><<<grid_dma, 256, 0, st>>>(
        xb, ldx, (uint32_t)x_bytes, topk, offsets, sorted, large_tiles, meta, w13_t, w13_st, sslot,
        2 * inter, hidden, inter, col_tiles, ap, route_weights, act, y, hidden);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/gateup_large");
  } else if (any_large) {
    e = hipFuncSetAttribute((const void*)moe_large_kernel<true>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void*)moe_large_kernel<false>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return kq_check_launch(e, "kq_moe_forward/attr");
    moe_large_kernel<true><<<dim3((unsigned)L.max_large, (unsigned)(inter / (BN / 2))), THREADS, lds, st>>>(
        xb, ldx, topk, offsets, sorted, large_tiles, meta, w13_t, w13_st, sslot, 2 * inter, hidden,
        inter, ap, route_weights, act, y, hidden);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/gateup_large");
  }
  // down
  if (route_in_gemv && dw) {
    const dim3 grid((unsigned)(hidden / 32));
    const bool f32 = out_dtype == KQ_DT_F32;
    const X4TGemv xg2 = x4t_gemv(xa, false);
#define KQ_DW_LAUNCH(NS, OUTC, X)                                                                              \
    moe_decode_down_wide_kernel<NS, OUTC, X><<<grid, 1024, 0, st>>>((const uint16_t*)act, inter, route_ids,     \
                                                                    topk, experts, (int)tokens, w2_t, w2_st,     \
                                                                    hidden, route_weights, out, xg2)
#define KQ_DW_CASE(NS, X) \
    if (f32) KQ_DW_LAUNCH(NS, 2, X); else KQ_DW_LAUNCH(NS, 0, X);
    if (inter == 1024) {
      if (xa) { KQ_DW_CASE(4, true) } else { KQ_DW_CASE(4, false) }
    } else {
      if (xa) { KQ_DW_CASE(8, true) } else { KQ_DW_CASE(8, false) }
    }
#undef KQ_DW_CASE
#undef KQ_DW_LAUNCH
    return kq_check_launch(hipGetLastError(), "kq_moe_forward/decode_down_wide");
  }
  if (route_in_gemv) {
    const int64_t steps = inter / 128 / 2;
    const dim3 grid((unsigned)(hidden / 32));
    const bool f32 = out_dtype == KQ_DT_F32;
    const X4TGemv xg2 = x4t_gemv(xa, false);
#define KQ_DD_LAUNCH(NS, OUTC, X)                                                                             \
    moe_decode_down_kernel<2, KQ_DD_P, NS, OUTC, X><<<grid, DD_PAIRS * 2 * 64, 0, st>>>(                            \
        (const uint16_t*)act, inter, route_ids, topk, experts, (int)tokens, w2_t, w2_st, hidden, route_weights, \
        out, xg2)
#define KQ_DD_CASE(NS)                                                                                        \
    if (steps == NS) {                                                                                        \
      if (xa) {                                                                                               \
        if (f32) KQ_DD_LAUNCH(NS, 2, true); else KQ_DD_LAUNCH(NS, 0, true);                                   \
      } else {                                                                                                \
        if (f32) KQ_DD_LAUNCH(NS, 2, false); else KQ_DD_LAUNCH(NS, 0, false);                                 \
      }                                                                                                       \
      return kq_check_launch(hipGetLastError(), "kq_moe_forward/decode_down");                               \
    }
    KQ_DD_CASE(2) KQ_DD_CASE(4) KQ_DD_CASE(8) KQ_DD_CASE(16)
#undef KQ_DD_CASE
#undef KQ_DD_LAUNCH
    return kq_fail(KQ_ERR_INVALID, "%s: decode down shape", fn);
  }
  {
    e = launch_small<false, KQ_DN_NBP, KQ_DN_S, KQ_DN_RW, KQ_DN_P>(
        xa != nullptr, L.max_list, hidden, inter, (int)(inter / 32), st, nullptr, (const uint16_t*)act, inter, topk,
        (const int*)sorted, (const int*)small_list, w2_t, w2_st, gslot, x4t_gemv(xa, false), hidden, inter,
        inter, ap, route_weights, act, y, hidden);
    if (e != hipSuccess) return kq_check_launch(e, "kq_moe_forward/down_small");
  }
  if (any_large && dma_path) {
    const int col_tiles = (int)(hidden / DMA_BN);
    moe_large_dma_kernel<false><<<grid_dma, 256, 0, st>>>(
        act, inter, (uint32_t)act_bytes, topk, offsets, sorted, large_tiles, meta, w2_t, w2_st, sslot,
        hidden, inter, inter, col_tiles, ap, route_weights, act, y, hidden);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/down_large");
  } else if (any_large) {
    moe_large_kernel<false><<<dim3((unsigned)L.max_large, (unsigned)((hidden + BN - 1) / BN)), THREADS, lds, st>>>(
        act, inter, topk, offsets, sorted, large_tiles, meta, w2_t, w2_st, sslot, hidden, inter, inter,
        ap, route_weights, act, y, hidden);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_moe_forward/down_large");
  }
  return combine();
}

extern "C" int kq_moe_forward(int activation, float act_beta, float act_linear_beta,
                              const void* x, int64_t ldx, int64_t tokens, int64_t hidden,
                              const int32_t* route_ids, const float* route_weights, int topk,
                              int experts, int64_t inter, const uint8_t* w13_t,
                              const uint8_t* w13_st, const uint8_t* w2_t,
                              const uint8_t* w2_st, int out_dtype, void* out,
                              void* workspace, int64_t workspace_bytes, uint32_t flags,
                              void* stream) {
  if (!w13_st || !w2_st) return kq_fail(KQ_ERR_INVALID, "kq_moe_forward: null scale tiles");
  return moe_forward_impl("kq_moe_forward", activation, act_beta, act_linear_beta, x, ldx, tokens, hidden,
                          route_ids, route_weights, topk, experts, inter, w13_t, w13_st, w2_t, w2_st,
                          nullptr, out_dtype, out, workspace, workspace_bytes, flags, stream);
}

extern "C" int64_t kq_moe_x4t_workspace_size(int64_t tokens, int topk, int experts, int64_t hidden,
                                             int64_t inter) {
  if (tokens < 0 || topk <= 0 || experts <= 0 || hidden <= 0 || inter <= 0) return -1;
  return (int64_t)make_layout(tokens, topk, experts, hidden, inter, true).total;
}

extern "C" int kq_moe_forward_x4t(int activation, float act_beta, float act_linear_beta,
                                  const void* x, int64_t ldx, int64_t tokens, int64_t hidden,
                                  const int32_t* route_ids, const float* route_weights, int topk,
                                  int experts, int64_t inter, const uint8_t* w13_t, const uint8_t* w2_t,
                                  const uint8_t* w1_fixed, const uint32_t* w1_exceptions,
                                  const uint32_t* w1_tile_index, const uint8_t* w3_fixed,
                                  const uint32_t* w3_exceptions, const uint32_t* w3_tile_index,
                                  const uint8_t* w2_fixed, const uint32_t* w2_exceptions,
                                  const uint32_t* w2_tile_index, int out_dtype, void* out,
                                  void* workspace, int64_t workspace_bytes, uint32_t flags,
                                  void* stream) {
  const char* fn = "kq_moe_forward_x4t";
  if (hidden <= 0 || inter <= 0 || hidden % 512 != 0 || inter % 256 != 0)
    return kq_fail(KQ_ERR_INVALID, "%s: hidden and intermediate sizes must be multiples of 512 / 256", fn);
  // X4T planes: w1 / w3 [inter, hidden / 32], w2 [hidden, inter / 32]; at most
  // 255 columns and 2^24 positions per matrix
  if (hidden / 32 > 255 || inter / 32 > 255 || inter * (hidden / 32) > (1 << 24) - 1 ||
      hidden * (inter / 32) > (1 << 24) - 1)
    return kq_fail(KQ_ERR_LIMIT, "%s: scale planes beyond the X4T geometry (hidden=%lld inter=%lld)", fn,
                   (long long)hidden, (long long)inter);
  const void* planes[9] = {w1_fixed, w1_exceptions, w1_tile_index, w3_fixed, w3_exceptions,
                           w3_tile_index, w2_fixed, w2_exceptions, w2_tile_index};
  for (int i = 0; i < 9; ++i) {
    if (!planes[i]) return kq_fail(KQ_ERR_INVALID, "%s: null X4T component", fn);
    if (i % 3 != 0 && kq_misaligned(planes[i], 4))
      return kq_fail(KQ_ERR_INVALID, "%s: misaligned X4T exceptions or tile index", fn);
  }
  X4TExpandArgs xa{};
  xa.n = 3;
  xa.p[0] = X4TPlane{w1_fixed, w1_exceptions, w1_tile_index, nullptr, inter / 16, 2 * inter / 16, 0,
                     (int)(hidden / 32)};
  xa.p[1] = X4TPlane{w3_fixed, w3_exceptions, w3_tile_index, nullptr, inter / 16, 2 * inter / 16,
                     inter / 16, (int)(hidden / 32)};
  xa.p[2] = X4TPlane{w2_fixed, w2_exceptions, w2_tile_index, nullptr, hidden / 16, hidden / 16, 0,
                     (int)(inter / 32)};
  return moe_forward_impl(fn, activation, act_beta, act_linear_beta, x, ldx, tokens, hidden, route_ids,
                          route_weights, topk, experts, inter, w13_t, nullptr, w2_t, nullptr, &xa,
                          out_dtype, out, workspace, workspace_bytes, flags, stream);
}

// ------------------------------------------------- allocation-free forward --
// kq_moe_forward with its workspace in this library's own device array, for
// callers that cannot allocate (code under HIP graph capture, serving loops).
// Each GPU holds one copy of the array, at its own address, until the process
// ends.  The forward writes every workspace entry before reading it (routing
// lists, intermediates, pair rows), so the previous call's contents need no
// clearing; calls that overlap on one GPU share the array and race.
static __device__ __align__(256) unsigned char scratch[KQ_MOE_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[SCRATCH_DEVICES];  // device address of `scratch`, per device
}  // namespace

// The address of `scratch` on the device that owns `stream` (the current
// device for the null stream), looked up once per device with that device
// current.
static int scratch_for_stream(const char* fn, void* stream, void** out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice((hipStream_t)stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return kq_check_launch(e, fn);
  if (dev < 0 || dev >= SCRATCH_DEVICES) return kq_fail(KQ_ERR_LIMIT, "%s: device %d out of range", fn, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return kq_check_launch(e, fn);
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return kq_check_launch(e, fn);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return kq_check_launch(e, fn);
    if (!p || kq_misaligned(p, 256)) return kq_fail(KQ_ERR_HIP, "%s: bad scratch address", fn);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KQ_OK;
}

extern "C" int kq_moe_forward_noalloc(int activation, float act_beta, float act_linear_beta,
                                      const void* x, int64_t ldx, int64_t tokens, int64_t hidden,
                                      const int32_t* route_ids, const float* route_weights, int topk,
                                      int experts, int64_t inter, const uint8_t* w13_t,
                                      const uint8_t* w13_st, const uint8_t* w2_t, const uint8_t* w2_st,
                                      int out_dtype, void* out, uint32_t flags, void* stream) {
  const char* fn = "kq_moe_forward_noalloc";
  if (!w13_st || !w2_st) return kq_fail(KQ_ERR_INVALID, "%s: null scale tiles", fn);
  // sizes the forward itself accepts are priced here; the others reach its
  // own argument checks below
  if (tokens >= 0 && topk > 0 && topk <= 64 && experts > 0 && experts <= MAX_EXPERTS && hidden > 0 &&
      inter > 0 && hidden <= (1 << 20) && inter <= (1 << 20) && tokens <= INT32_MAX / 2 / topk) {
    const int64_t need = (int64_t)make_layout(tokens, topk, experts, hidden, inter).total;
    if (need > KQ_MOE_NOALLOC_SCRATCH_BYTES)
      return kq_fail(KQ_ERR_LIMIT,
                     "%s: %lld tokens x top-%d need %lld bytes of workspace, more than the %lld-byte "
                     "scratch array; use kq_moe_forward with a caller workspace", fn, (long long)tokens,
                     topk, (long long)need, (long long)KQ_MOE_NOALLOC_SCRATCH_BYTES);
  }
  void* ws = nullptr;
  const int rc = scratch_for_stream(fn, stream, &ws);
  if (rc != KQ_OK) return rc;
  return moe_forward_impl(fn, activation, act_beta, act_linear_beta, x, ldx, tokens, hidden, route_ids,
                          route_weights, topk, experts, inter, w13_t, w13_st, w2_t, w2_st, nullptr,
                          out_dtype, out, ws, KQ_MOE_NOALLOC_SCRATCH_BYTES, flags, stream);
}

// Routing sort alone (for per-expert calibration statistics): the pairs
// (t, s) of route_ids [tokens, topk] grouped by expert, stable in pair order.
static size_t route_sort_layout(int64_t pairs, int experts, size_t* parts) {
  const int64_t nblk = (pairs + PREP - 1) / PREP;
  const int64_t max_large = pairs / (SMALL_MAX + 1) + pairs / BM + 1;
  size_t o = 0;
  parts[0] = o; o = align256(o + sizeof(int) * experts);                 // counts
  parts[1] = o; o = align256(o + sizeof(int) * (experts + 1));           // offsets32
  parts[2] = o; o = align256(o + sizeof(int) * (size_t)nblk * experts);  // block counts
  parts[3] = o; o = align256(o + sizeof(int) * (size_t)pairs);           // sorted pairs
  parts[4] = o; o = align256(o + sizeof(int) * 3 * experts);             // small list
  parts[5] = o; o = align256(o + sizeof(int) * 2 * (size_t)max_large);   // large tiles
  parts[6] = o; o = align256(o + sizeof(int) * 4);                       // meta
  return o;
}

extern "C" int64_t kq_route_sort_workspace_size(int64_t tokens, int topk, int experts) {
  if (tokens < 0 || topk <= 0 || experts <= 0) return -1;
  size_t parts[7];
  return (int64_t)route_sort_layout(tokens * topk, experts, parts);
}

extern "C" int kq_route_sort(const int32_t* route_ids, int64_t tokens, int topk, int experts,
                             const float* pair_weights, int64_t* offsets, int32_t* rows,
                             int32_t* sorted_pairs, float* sorted_weights, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  if (tokens < 0 || topk <= 0 || topk > 64 || experts <= 0 || experts > MAX_EXPERTS)
    return kq_fail(KQ_ERR_INVALID, "kq_route_sort: need 1 <= topk <= 64, 1 <= experts <= %d",
                   MAX_EXPERTS);
  if (tokens * topk > INT32_MAX / 2) return kq_fail(KQ_ERR_LIMIT, "kq_route_sort: too many pairs");
  if (sorted_weights && !pair_weights)
    return kq_fail(KQ_ERR_INVALID, "kq_route_sort: sorted_weights needs pair_weights");
  size_t parts[7];
  const int64_t pairs = tokens * topk;
  const size_t need = route_sort_layout(pairs, experts, parts);
  if (workspace_bytes < (int64_t)need || kq_misaligned(workspace, 256))
    return kq_fail(KQ_ERR_INVALID, "kq_route_sort: workspace needs %lld bytes, 256-byte aligned",
                   (long long)need);
  if (kq_misaligned(offsets, 8)) return kq_fail(KQ_ERR_INVALID, "kq_route_sort: misaligned offsets");
  hipStream_t st = (hipStream_t)stream;
  unsigned char* w = (unsigned char*)workspace;
  int* counts = (int*)(w + parts[0]);
  int* off32 = (int*)(w + parts[1]);
  int* block_counts = (int*)(w + parts[2]);
  int* sorted = (int*)(w + parts[3]);
  int* small_list = (int*)(w + parts[4]);
  int* large_tiles = (int*)(w + parts[5]);
  int* meta = (int*)(w + parts[6]);
  const int64_t nblk = (pairs + PREP - 1) / PREP;
  const int max_large = (int)(pairs / (SMALL_MAX + 1) + pairs / BM + 1);
  hipError_t e;
  if (pairs <= PREP_ONE) {
    route_prep_one_kernel<<<1, 1024, 0, st>>>(route_ids, (int)pairs, experts, counts, off32, sorted,
                                               small_list, large_tiles, meta, max_large, nullptr, nullptr, 0,
                                               BM, nullptr);
  } else {
    route_hist_kernel<<<(unsigned)nblk, PREP, 0, st>>>(route_ids, pairs, experts, block_counts);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_route_sort");
    route_scan_kernel<<<1, 1024, 0, st>>>(block_counts, (int)nblk, experts, counts, off32, small_list,
                                          large_tiles, meta, max_large, nullptr, nullptr, 0, BM);
    if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_route_sort");
    route_scatter_kernel<<<(unsigned)nblk, PREP, 0, st>>>(route_ids, pairs, experts, off32,
                                                          block_counts, sorted, nullptr);
  }
  if ((e = hipGetLastError()) != hipSuccess) return kq_check_launch(e, "kq_route_sort");
  const int64_t n = pairs > experts + 1 ? pairs : experts + 1;
  route_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(off32, experts, sorted, topk, pair_weights,
                                                                 offsets, rows, sorted_pairs, sorted_weights);
  return kq_check_launch(hipGetLastError(), "kq_route_sort");
}
