// Lossless E8M0 scale-plane codecs: X4T (per-row adjacent pair, fixed
// selector stream, sorted uint32 exceptions) and KQSC (row-palette tiles,
// versions 1 and 2).  A scale plane is 1/32 of its weight matrix, so these
// are small integer kernels whose cost is a handful of dispatches.
//
// Work mapping shared by every kernel: one workgroup per tile, one wave per
// row (columns <= 255, so lane l owns columns l, l+64, l+128, l+192), a
// wave-private 256-bin LDS histogram per row, and ballots to rank positions,
// which yields the row-major order both formats use for selector bits and
// exception lists.  Variable-length outputs use three passes: measure (one
// count per tile), an exclusive scan, and emit at the scanned offsets.
#include "kq_common.h"
#include "kq_internal.h"

namespace kq {
namespace {

constexpr int SP_THREADS = 256;
constexpr int SP_WAVES = SP_THREADS / 64;
constexpr int X4T_ROWS = 16;
constexpr uint32_t X4T_POS_MASK = (1u << 24) - 1;

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ uint64_t lanes_below(int lane) { return (1ull << lane) - 1ull; }

// Columns lane + 64k of one row, -1 where the row has ended.
__device__ __forceinline__ void load_row(const uint8_t* __restrict__ row, int cols, int lane,
                                         int v[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = lane + 64 * k;
    v[k] = c < cols ? (int)row[c] : -1;
  }
}

// Row histogram into a wave-private 256-bin array.  Called by every thread of
// the block with the same trip count (the barriers are block-wide).
__device__ __forceinline__ void row_histogram(unsigned* h, const int v[4], int lane) {
#pragma unroll
  for (int k = 0; k < 4; ++k) h[lane + 64 * k] = 0u;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (v[k] >= 0) atomicAdd(&h[v[k]], 1u);
  __syncthreads();
}

// X4T base: argmax over b in [0, 254] of h[b] + h[b+1], lowest b on ties
// (kquant/x4t.py:71-83).
__device__ __forceinline__ int adjacent_base(const unsigned* h, int lane) {
  int key = -1;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int b = lane * 4 + k;
    if (b < 255) key = max(key, (int)((h[b] + h[b + 1]) << 8) | (255 - b));
  }
  return 255 - (wave_max_i(key) & 255);
}

// KQSC palette: most frequent value, then the next most frequent, ties to the
// lower value; a constant row repeats its value (mxfp4_scale_codec.py:19-24).
__device__ __forceinline__ void row_palette(const unsigned* h, int lane, int& first, int& second) {
  int key = -1;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int b = lane + 64 * k;
    const unsigned c = h[b];
    if (c) key = max(key, (int)(c << 8) | (255 - b));
  }
  first = 255 - (wave_max_i(key) & 255);
  int key2 = -1;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int b = lane + 64 * k;
    const unsigned c = h[b];
    if (c && b != first) key2 = max(key2, (int)(c << 8) | (255 - b));
  }
  key2 = wave_max_i(key2);
  second = key2 < 0 ? first : 255 - (key2 & 255);
}

// Selector byte j (columns 8j..8j+7) out of the four 64-column ballots.
__device__ __forceinline__ uint8_t ballot_byte(const uint64_t m[4], int j) {
  const uint64_t w = j < 8 ? m[0] : j < 16 ? m[1] : j < 24 ? m[2] : m[3];
  return (uint8_t)(w >> (8 * (j & 7)));
}

// ---------------------------------------------------------------- scan --
// In-place exclusive prefix sum of data[0, n), total stored at data[n].
__global__ __launch_bounds__(1024) void exclusive_scan_kernel(int64_t* __restrict__ data,
                                                              int64_t n) {
  __shared__ int64_t wsum[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t carry = 0;
  for (int64_t base = 0; base < n; base += 4096) {
    int64_t v[4], s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t idx = base + threadIdx.x * 4 + j;
      v[j] = idx < n ? data[idx] : 0;
      s += v[j];
    }
    int64_t x = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int64_t before = carry + (x - s), chunk = 0;
    for (int w = 0; w < 16; ++w) {
      const int64_t t = wsum[w];
      if (w < wave) before += t;
      chunk += t;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t idx = base + threadIdx.x * 4 + j;
      if (idx < n) data[idx] = before;
      before += v[j];
    }
    carry += chunk;
    __syncthreads();
  }
  if (threadIdx.x == 0) data[n] = carry;
}

// ----------------------------------------------------------------- X4T --
// Fixed stream of one 16-row tile: 16 base bytes, then 16 rows of sb
// selector bytes (bit = value is base + 1).  tile_counts[tile] = number of
// values outside their row's pair (kquant/x4t.py:90-130).
__global__ __launch_bounds__(SP_THREADS) void x4t_analyze_kernel(
    const uint8_t* __restrict__ scale, int cols, int sb, uint8_t* __restrict__ fixed,
    int64_t* __restrict__ tile_counts) {
  __shared__ unsigned hist[SP_WAVES][256];
  __shared__ unsigned row_exc[X4T_ROWS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t tile = blockIdx.x;
  uint8_t* f = fixed + tile * (int64_t)(X4T_ROWS * (1 + sb));
  for (int it = 0; it < X4T_ROWS / SP_WAVES; ++it) {
    const int i = it * SP_WAVES + wave;
    int v[4];
    load_row(scale + (tile * X4T_ROWS + i) * cols, cols, lane, v);
    row_histogram(hist[wave], v, lane);
    const int base = adjacent_base(hist[wave], lane);
    uint64_t hi[4];
    unsigned n_exc = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      hi[k] = __ballot(v[k] == base + 1);
      n_exc += __popcll(__ballot(v[k] >= 0 && v[k] != base && v[k] != base + 1));
    }
    if (lane == 0) {
      f[i] = (uint8_t)base;
      row_exc[i] = n_exc;
    }
    if (lane < sb) f[X4T_ROWS + i * sb + lane] = ballot_byte(hi, lane);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t s = 0;
    for (int i = 0; i < X4T_ROWS; ++i) s += row_exc[i];
    tile_counts[tile] = s;
  }
}

// Exception words pos | value << 24 in row-major order, written at the
// scanned tile offsets; positions are local to each matrix.
__global__ __launch_bounds__(SP_THREADS) void x4t_emit_kernel(
    const uint8_t* __restrict__ scale, int cols, int sb, int64_t tiles_per_mat,
    const uint8_t* __restrict__ fixed, const int64_t* __restrict__ tile_offsets,
    uint32_t* __restrict__ exceptions) {
  __shared__ unsigned row_exc[X4T_ROWS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t tile = blockIdx.x;
  const int64_t local_row0 = (tile % tiles_per_mat) * X4T_ROWS;
  const uint8_t* f = fixed + tile * (int64_t)(X4T_ROWS * (1 + sb));
  int v[X4T_ROWS / SP_WAVES][4];
  uint64_t ex[X4T_ROWS / SP_WAVES][4];
#pragma unroll
  for (int it = 0; it < X4T_ROWS / SP_WAVES; ++it) {
    const int i = it * SP_WAVES + wave;
    load_row(scale + (tile * X4T_ROWS + i) * cols, cols, lane, v[it]);
    const int base = f[i];
    unsigned n = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int x = v[it][k];
      ex[it][k] = __ballot(x >= 0 && x != base && x != base + 1);
      n += __popcll(ex[it][k]);
    }
    if (lane == 0) row_exc[i] = n;
  }
  __syncthreads();
  const int64_t tile_base = tile_offsets[tile];
#pragma unroll
  for (int it = 0; it < X4T_ROWS / SP_WAVES; ++it) {
    const int i = it * SP_WAVES + wave;
    int64_t o = tile_base;
    for (int r = 0; r < i; ++r) o += row_exc[r];
    const uint32_t pos0 = (uint32_t)((local_row0 + i) * cols);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if ((ex[it][k] >> lane) & 1ull) {
        const int64_t rank = __popcll(ex[it][k] & lanes_below(lane));
        exceptions[o + rank] = (pos0 + lane + 64 * k) | ((uint32_t)v[it][k] << 24);
      }
      o += __popcll(ex[it][k]);
    }
  }
}

// Index of the first exception in [lo, hi) whose position is >= key, or hi.
// Block-cooperative: each round samples 256 evenly spaced entries, so a
// sorted list needs ceil(log256(n)) dependent load rounds.  On unsorted input
// it still returns an index in [lo, hi].
__device__ int64_t block_lower_bound(const uint32_t* __restrict__ exc, int64_t lo, int64_t hi,
                                     uint32_t key) {
  while (hi - lo > SP_THREADS) {
    const int64_t step = (hi - lo + SP_THREADS - 1) / SP_THREADS;
    const int64_t idx = lo + (int64_t)threadIdx.x * step;
    const int below = idx < hi && (exc[idx] & X4T_POS_MASK) < key;
    const int64_t cnt = __syncthreads_count(below);
    const int64_t nlo = cnt == 0 ? lo : lo + (cnt - 1) * step + 1;
    const int64_t nhi = min(hi, lo + cnt * step);
    lo = nlo;
    hi = max(nhi, nlo);
  }
  const int64_t idx = lo + threadIdx.x;
  const int below = idx < hi && (exc[idx] & X4T_POS_MASK) < key;
  return lo + __syncthreads_count(below);
}

// Dense plane of one tile: base + selector bit per position (uint8 wrap, as
// kquant/x4t.py:497-501), then the tile's exceptions found by a cooperative
// binary search (kquant/x4t.py:504-516), staged in LDS and stored row-major.
__global__ __launch_bounds__(SP_THREADS) void x4t_decode_kernel(
    const uint8_t* __restrict__ fixed, const uint32_t* __restrict__ exceptions, int64_t n_exc,
    const int64_t* __restrict__ exc_offsets, int64_t tiles_per_mat, int cols, int sb,
    uint8_t* __restrict__ out) {
  __shared__ uint8_t buf[X4T_ROWS * 256];
  const int64_t tile = blockIdx.x;
  const int64_t m = tile / tiles_per_mat;
  const uint8_t* f = fixed + tile * (int64_t)(X4T_ROWS * (1 + sb));
  const int span = X4T_ROWS * cols;
  for (int p = threadIdx.x; p < span; p += SP_THREADS) {
    const int i = p / cols, c = p - i * cols;
    buf[p] = (uint8_t)(f[i] + ((f[X4T_ROWS + i * sb + (c >> 3)] >> (c & 7)) & 1));
  }
  int64_t e0 = 0, e1 = n_exc;
  if (exc_offsets) {
    e0 = min(max(exc_offsets[m], (int64_t)0), n_exc);
    e1 = min(max(exc_offsets[m + 1], e0), n_exc);
  }
  const uint32_t lo_pos = (uint32_t)((tile % tiles_per_mat) * span);
  const int64_t a = block_lower_bound(exceptions, e0, e1, lo_pos);
  const int64_t b = block_lower_bound(exceptions, a, e1, lo_pos + (uint32_t)span);
  // block_lower_bound ends in a barrier, so the dense fill above is visible.
  for (int64_t e = a + threadIdx.x; e < b; e += SP_THREADS) {
    const uint32_t w = exceptions[e];
    const uint32_t pos = w & X4T_POS_MASK;
    if (pos >= lo_pos && pos < lo_pos + (uint32_t)span) buf[pos - lo_pos] = (uint8_t)(w >> 24);
  }
  __syncthreads();
  uint8_t* o = out + tile * (int64_t)span;
  for (int p = threadIdx.x; p < span; p += SP_THREADS) o[p] = buf[p];
}

// Per-tile exception index of X4T matrices: index[m * tiles + t] = first
// exception of matrix m at or after tile t's first position (a lower bound
// over the matrix's sorted exception range), index[mats * tiles] = n_exc.
// Built once per weight set, it lets a runtime expansion find a tile's
// exceptions without any search.
__global__ __launch_bounds__(256) void x4t_tile_index_kernel(
    const uint32_t* __restrict__ exc, int64_t n_exc, const int64_t* __restrict__ exc_offsets,
    int64_t mats, int64_t tiles_per_mat, int cols, uint32_t* __restrict__ index) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x, total = mats * tiles_per_mat;
  if (g > total) return;
  if (g == total) {
    index[total] = (uint32_t)n_exc;
    return;
  }
  const int64_t m = g / tiles_per_mat, t = g - m * tiles_per_mat;
  int64_t lo = 0, hi = n_exc;
  if (exc_offsets) {
    lo = min(max(exc_offsets[m], (int64_t)0), n_exc);
    hi = min(max(exc_offsets[m + 1], lo), n_exc);
  }
  const uint32_t key = (uint32_t)(t * X4T_ROWS * cols);
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if ((exc[mid] & X4T_POS_MASK) < key) lo = mid + 1;
    else hi = mid;
  }
  index[g] = (uint32_t)lo;
}

// Runtime expansion of routed experts' X4T scales (one launch, no search, no
// allocation).  Block (r, y) takes X4T_EXPAND_TILES consecutive 16-row tiles
// of one plane (y runs over every plane's tile groups in turn) of matrix
// routed[r] (nothing when -1): their fixed bytes (contiguous) are staged in
// LDS with 16-byte loads, decoded - base + selector bit - straight into the
// kq_mx_tile_weights scale layout in LDS (64-byte tiles [row group][cols / 4],
// byte l = scale[16 rg + l % 16][4 c + l / 16]), patched with the group's
// exceptions (one contiguous range of the sorted stream, from the precomputed
// tile index) and copied to slot r of the plane's output with 16-byte stores.
constexpr int X4T_EXPAND_TILES = 8;
constexpr int X4T_MAX_PIECES = X4T_EXPAND_TILES * 33;  // 16-byte pieces of 8 fixed tiles, cols <= 255

__global__ __launch_bounds__(SP_THREADS) void x4t_expand_tiled_kernel(X4TExpandArgs a,
                                                                       const int* __restrict__ routed) {
  constexpr int G = X4T_EXPAND_TILES, U = 4;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int e = routed[blockIdx.x];
  if (e < 0) return;
  int64_t grp = blockIdx.y;
  int pi = 0;
  if (grp >= a.p[0].tiles / G) {
    grp -= a.p[0].tiles / G;
    pi = 1;
    if (a.n > 2 && grp >= a.p[1].tiles / G) {
      grp -= a.p[1].tiles / G;
      pi = 2;
    }
  }
  const X4TPlane P = pi == 0 ? a.p[0] : pi == 1 ? a.p[1] : a.p[2];
  __shared__ __attribute__((aligned(16))) uint8_t buf[G * X4T_ROWS * 256];
  __shared__ __attribute__((aligned(16))) uint8_t fl[X4T_MAX_PIECES * 16];
  const int tid = threadIdx.x;
  const int cols = P.cols, sb = (cols + 7) >> 3, tp = 1 + sb, span = X4T_ROWS * cols, nchunk = cols >> 2;
  const int64_t t0 = grp * G, ti0 = (int64_t)e * P.tiles + t0;
  const uint8_t* fsrc = P.fixed + ti0 * (16 * tp);
  u32x4 pc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if (tid + u * SP_THREADS < G * tp) pc[u] = *reinterpret_cast<const u32x4*>(fsrc + 16 * (tid + u * SP_THREADS));
  const uint32_t lo = P.tile_index[ti0], hi = P.tile_index[ti0 + G];
  const int total = hi > lo ? (int)(hi - lo) : 0;
  uint32_t wv[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (tid + u * SP_THREADS < total) wv[u] = P.exceptions[lo + tid + u * SP_THREADS];
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if (tid + u * SP_THREADS < G * tp) *reinterpret_cast<u32x4*>(fl + 16 * (tid + u * SP_THREADS)) = pc[u];
  __syncthreads();
  // dword j of a tile: chunk j / 16, bytes l = 4 (j % 16) .. + 3, i.e. rows
  // 4 (j % 4) .. + 3 of column 4 (j / 16) + (j % 16) / 4
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint8_t* f = fl + g * 16 * tp;
    for (int j = tid; j < nchunk * 16; j += SP_THREADS) {
      const int w = j & 15, r0 = 4 * (w & 3), c = 4 * (j >> 4) + (w >> 2);
      const uint32_t base4 = *reinterpret_cast<const uint32_t*>(f + r0);
      const uint8_t* sel = f + X4T_ROWS + r0 * sb + (c >> 3);
      uint32_t v = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v |= (((base4 >> (8 * i)) + ((sel[i * sb] >> (c & 7)) & 1)) & 0xffu) << (8 * i);
      *reinterpret_cast<uint32_t*>(buf + (g * nchunk + (j >> 4)) * 64 + 4 * w) = v;
    }
  }
  __syncthreads();
  const uint32_t pos0 = (uint32_t)(t0 * span);
  for (int base = 0; base < total; base += U * SP_THREADS) {
    if (base > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (base + tid + u * SP_THREADS < total) wv[u] = P.exceptions[lo + base + tid + u * SP_THREADS];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + tid + u * SP_THREADS >= total) continue;
      const uint32_t off = (wv[u] & X4T_POS_MASK) - pos0;  // wraps past the group when outside it
      if (off >= (uint32_t)(G * span)) continue;
      const int g = (int)off / span, rem = (int)off - g * span;
      const int r = rem / cols, c = rem - r * cols;
      buf[(g * nchunk + (c >> 2)) * 64 + (c & 3) * 16 + r] = (uint8_t)(wv[u] >> 24);
    }
  }
  __syncthreads();
  u32x4* dst = reinterpret_cast<u32x4*>(P.out + (((int64_t)blockIdx.x * P.out_rgs + P.out_rg0 + t0) * nchunk) * 64);
  for (int i = tid; i < G * span / 16; i += SP_THREADS) dst[i] = reinterpret_cast<const u32x4*>(buf)[i];
}

// status: {selector padding, first bad position index, first redundant value
// index, non-canonical}.
__global__ void x4t_status_init_kernel(uint32_t* status) {
  status[0] = 0u;
  status[1] = 0xffffffffu;
  status[2] = 0xffffffffu;
  status[3] = 0u;
}

// Validation of a decoded single-matrix plane (kquant/x4t.py:501-523).
// Blocks [0, tiles) re-derive each row's canonical base from the decoded
// values and check selector padding; the remaining blocks check one
// exception per thread: strictly increasing positions in range, values off
// the adjacent pair, and a zero selector bit under every exception (what the
// reference's re-encode comparison requires of the fixed stream).
__global__ __launch_bounds__(SP_THREADS) void x4t_check_kernel(
    const uint8_t* __restrict__ fixed, const uint32_t* __restrict__ exceptions, int64_t n_exc,
    int64_t tiles, int cols, int sb, const uint8_t* __restrict__ out, uint32_t* status) {
  __shared__ unsigned hist[SP_WAVES][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tile_bytes = X4T_ROWS * (1 + sb);
  if ((int64_t)blockIdx.x < tiles) {
    const int64_t tile = blockIdx.x;
    const uint8_t* f = fixed + tile * (int64_t)tile_bytes;
    for (int it = 0; it < X4T_ROWS / SP_WAVES; ++it) {
      const int i = it * SP_WAVES + wave;
      int v[4];
      load_row(out + (tile * X4T_ROWS + i) * cols, cols, lane, v);
      row_histogram(hist[wave], v, lane);
      const int base = adjacent_base(hist[wave], lane);
      if (lane == 0) {
        if (base != f[i]) atomicOr(&status[3], 1u);
        if ((cols & 7) && (f[X4T_ROWS + i * sb + sb - 1] >> (cols & 7))) atomicOr(&status[0], 1u);
      }
    }
    return;
  }
  const int64_t e = ((int64_t)blockIdx.x - tiles) * SP_THREADS + threadIdx.x;
  if (e >= n_exc) return;
  const uint32_t w = exceptions[e];
  const int64_t pos = w & X4T_POS_MASK;
  const int64_t prev = e > 0 ? (int64_t)(exceptions[e - 1] & X4T_POS_MASK) : -1;
  if (pos >= tiles * X4T_ROWS * cols || pos <= prev) {
    atomicMin(&status[1], (uint32_t)e);
    return;
  }
  const int64_t row = pos / cols;
  const int c = (int)(pos - row * cols);
  const uint8_t* f = fixed + (row / X4T_ROWS) * tile_bytes;
  const int i = (int)(row % X4T_ROWS);
  const int base = f[i];
  const int value = (int)(w >> 24);
  if (value == base || value == base + 1) {
    atomicMin(&status[2], (uint32_t)e);
    return;
  }
  if ((f[X4T_ROWS + i * sb + (c >> 3)] >> (c & 7)) & 1) atomicOr(&status[3], 1u);
}

// ---------------------------------------------------------------- KQSC --
constexpr int KQSC_MAX_TILE_ROWS = 255;

__device__ __forceinline__ bool adjacent_pair(int first, int second) {
  return second - first == 1 || first - second == 1;
}

// Per row: first | second << 8 | exceptions << 16; per tile: body bytes.
// Body sizes follow kquant/mxfp4_scale_codec.py:43-69 (v1) and :235-275 (v2).
template <int VERSION>
__global__ __launch_bounds__(SP_THREADS) void kqsc_measure_kernel(
    const uint8_t* __restrict__ scale, int64_t rows, int cols, int tile_rows, int sb,
    uint32_t* __restrict__ row_meta, int64_t* __restrict__ tile_sizes) {
  __shared__ unsigned hist[SP_WAVES][256];
  __shared__ int acc[3];  // exceptions, explicit palettes, extended counts
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t tile = blockIdx.x;
  const int64_t r0 = tile * tile_rows;
  const int rc = (int)min((int64_t)tile_rows, rows - r0);
  if (threadIdx.x < 3) acc[threadIdx.x] = 0;
  for (int it = 0; it < (rc + SP_WAVES - 1) / SP_WAVES; ++it) {
    const int i = it * SP_WAVES + wave;
    const bool active = i < rc;
    int v[4] = {-1, -1, -1, -1};
    if (active) load_row(scale + (r0 + i) * cols, cols, lane, v);
    row_histogram(hist[wave], v, lane);
    if (active) {
      int first, second;
      row_palette(hist[wave], lane, first, second);
      unsigned n = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        n += __popcll(__ballot(v[k] >= 0 && v[k] != first && v[k] != second));
      if (lane == 0) {
        row_meta[r0 + i] = (uint32_t)first | ((uint32_t)second << 8) | (n << 16);
        atomicAdd(&acc[0], (int)n);
        atomicAdd(&acc[1], adjacent_pair(first, second) ? 0 : 1);
        atomicAdd(&acc[2], n >= 3 ? 1 : 0);
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t fb = (rc + 7) / 8, cb = (2 * rc + 7) / 8;
    tile_sizes[tile] = VERSION == 1
                           ? (int64_t)rc * (3 + sb) + 2 * (int64_t)acc[0]
                           : rc + 2 * fb + cb + acc[1] + acc[2] + (int64_t)rc * sb + 2 * (int64_t)acc[0];
  }
}

// Packed per-row quantities for tile-local prefix sums: exceptions in bits
// 0..31, explicit palettes in 32..47, extended counts in 48..63.
__device__ __forceinline__ int64_t pack_row_counts(int64_t n_exc, int64_t expl, int64_t ext) {
  return n_exc | (expl << 32) | (ext << 48);
}

// Exclusive prefix of q over rows [0, rc) into pre[0..rc] (pre[rc] = total),
// by wave 0 with four rows per lane.  Caller synchronises afterwards.
__device__ __forceinline__ void tile_row_scan(int64_t q[4], int lane, int rc, int64_t* pre) {
  int64_t s = q[0] + q[1] + q[2] + q[3];
  int64_t x = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  int64_t before = x - s;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = lane * 4 + j;
    if (r <= rc) pre[r] = before;
    before += q[j];
  }
}

__device__ __forceinline__ void put_u32(uint8_t* p, uint32_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
  p[2] = (uint8_t)(v >> 16);
  p[3] = (uint8_t)(v >> 24);
}

__device__ __forceinline__ uint32_t get_u32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Header <4sBBH I H H>, the uint32 offset table and each tile body
// (kquant/mxfp4_scale_codec.py:71-85 and :276-292).
template <int VERSION>
__global__ __launch_bounds__(SP_THREADS) void kqsc_emit_kernel(
    const uint8_t* __restrict__ scale, int64_t rows, int cols, int tile_rows, int sb,
    int64_t tiles, const uint32_t* __restrict__ row_meta, const int64_t* __restrict__ offsets,
    uint8_t* __restrict__ payload) {
  __shared__ uint32_t meta[KQSC_MAX_TILE_ROWS + 1];
  __shared__ int64_t pre[KQSC_MAX_TILE_ROWS + 2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t tile = blockIdx.x;
  const int64_t r0 = tile * tile_rows;
  const int rc = (int)min((int64_t)tile_rows, rows - r0);
  const int64_t start = 16 + 4 * (tiles + 1);
  uint8_t* body = payload + start + offsets[tile];
  if (tile == 0 && threadIdx.x == 0) {
    payload[0] = 'K'; payload[1] = 'Q'; payload[2] = 'S'; payload[3] = 'C';
    payload[4] = (uint8_t)VERSION;
    payload[5] = (uint8_t)tile_rows;
    payload[6] = 0; payload[7] = 0;
    put_u32(payload + 8, (uint32_t)rows);
    payload[12] = (uint8_t)cols; payload[13] = 0;
    payload[14] = 0; payload[15] = 0;
  }
  if (threadIdx.x == 0) {
    put_u32(payload + 16 + 4 * tile, (uint32_t)offsets[tile]);
    if (tile == tiles - 1) put_u32(payload + 16 + 4 * tiles, (uint32_t)offsets[tiles]);
  }
  if ((int)threadIdx.x < rc) meta[threadIdx.x] = row_meta[r0 + threadIdx.x];
  __syncthreads();
  if (wave == 0) {
    int64_t q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = lane * 4 + j;
      q[j] = 0;
      if (r < rc) {
        const uint32_t m = meta[r];
        const int first = m & 255, second = (m >> 8) & 255, n = (int)(m >> 16);
        q[j] = pack_row_counts(n, adjacent_pair(first, second) ? 0 : 1, n >= 3 ? 1 : 0);
      }
    }
    tile_row_scan(q, lane, rc, pre);
  }
  __syncthreads();
  const int fb = (rc + 7) >> 3, cb = (2 * rc + 7) >> 3;
  const int64_t total = pre[rc];
  const int n_expl = (int)((total >> 32) & 0xffff);
  const int n_ext = (int)(total >> 48);
  int sel0;
  if (VERSION == 1) {
    if ((int)threadIdx.x < rc) {
      const uint32_t m = meta[threadIdx.x];
      body[threadIdx.x] = (uint8_t)m;
      body[rc + threadIdx.x] = (uint8_t)(m >> 8);
      body[2 * rc + threadIdx.x] = (uint8_t)(m >> 16);
    }
    sel0 = 3 * rc;
  } else {
    const int meta0 = rc + 2 * fb + cb;
    const int t = threadIdx.x;
    if (t < rc) {
      const uint32_t m = meta[t];
      const int first = m & 255, second = (m >> 8) & 255, n = (int)(m >> 16);
      body[t] = (uint8_t)first;
      if (!adjacent_pair(first, second)) body[meta0 + ((pre[t] >> 32) & 0xffff)] = (uint8_t)second;
      if (n >= 3) body[meta0 + n_expl + (pre[t] >> 48)] = (uint8_t)n;
    }
    if (t < fb) {
      unsigned dir = 0, expl = 0;
      for (int j = 0; j < 8; ++j) {
        const int r = 8 * t + j;
        if (r >= rc) break;
        const uint32_t m = meta[r];
        const int first = m & 255, second = (m >> 8) & 255;
        if (adjacent_pair(first, second)) dir |= (unsigned)(second > first) << j;
        else expl |= 1u << j;
      }
      body[rc + t] = (uint8_t)dir;
      body[rc + fb + t] = (uint8_t)expl;
    }
    if (t < cb) {
      unsigned codes = 0;
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * t + j;
        if (r >= rc) break;
        codes |= (unsigned)min((int)(meta[r] >> 16), 3) << (2 * j);
      }
      body[rc + 2 * fb + t] = (uint8_t)codes;
    }
    sel0 = meta0 + n_expl + n_ext;
  }
  const int exc0 = sel0 + rc * sb;
  for (int i = wave; i < rc; i += SP_WAVES) {
    const uint32_t m = meta[i];
    const int first = m & 255, second = (m >> 8) & 255;
    int v[4];
    load_row(scale + (r0 + i) * cols, cols, lane, v);
    uint64_t hi[4], ex[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      hi[k] = __ballot(second != first && v[k] == second);
      ex[k] = __ballot(v[k] >= 0 && v[k] != first && v[k] != second);
    }
    if (lane < sb) body[sel0 + i * sb + lane] = ballot_byte(hi, lane);
    int64_t o = pre[i] & 0xffffffff;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if ((ex[k] >> lane) & 1ull) {
        const int64_t at = exc0 + 2 * (o + __popcll(ex[k] & lanes_below(lane)));
        body[at] = (uint8_t)(lane + 64 * k);
        body[at + 1] = (uint8_t)v[k];
      }
      o += __popcll(ex[k]);
    }
  }
}

// Error keys of the decoders, in the order the reference raises them.
// Tile-level codes come first; row-level keys are 8 + row * 1024 + sub with
// sub 0 palette escape, 1 adjacent range, 2 selector padding, 3 + 2e bad
// position of exception e, 4 + 2e redundant value of exception e.
enum {
  KQSC_E_TRUNC_FIXED = 0,    // v1 fixed fields / v2 row fields truncated
  KQSC_E_PAD_DIR = 1,        // v2
  KQSC_E_PAD_EXPL = 2,       // v2
  KQSC_E_PAD_CODES = 3,      // v2
  KQSC_E_TRUNC_ESCAPES = 4,  // v2
  KQSC_E_COUNT_ESCAPE = 5,   // v2
  KQSC_E_COUNTS_LEN = 6,
  KQSC_E_OFFSETS = 7,
  KQSC_E_ROW = 8,
};

__global__ void status_fill_kernel(unsigned long long* status) { *status = ~0ull; }

// Decode and validate one tile (kquant/mxfp4_scale_codec.py:116-160 for v1,
// :318-424 for v2).  The header and offset table were checked by the caller;
// body ranges are still clamped to the payload.
template <int VERSION>
__global__ __launch_bounds__(SP_THREADS) void kqsc_decode_kernel(
    const uint8_t* __restrict__ payload, int64_t payload_bytes, int64_t rows, int cols,
    int tile_rows, int sb, int64_t tiles, uint8_t* __restrict__ out,
    unsigned long long* status) {
  __shared__ int64_t pre[KQSC_MAX_TILE_ROWS + 2];
  __shared__ int16_t second_of[KQSC_MAX_TILE_ROWS + 1];
  __shared__ uint8_t cnt_of[KQSC_MAX_TILE_ROWS + 1];
  __shared__ unsigned first_idx[SP_WAVES][256];
  __shared__ uint8_t rowbuf[SP_WAVES][256];
  __shared__ int tile_err;
  __shared__ int row_err;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = threadIdx.x;
  const int64_t tile = blockIdx.x;
  const int64_t r0 = tile * tile_rows;
  const int rc = (int)min((int64_t)tile_rows, rows - r0);
  const int64_t start = 16 + 4 * (tiles + 1);
  const int64_t oa = get_u32(payload + 16 + 4 * tile);
  const int64_t ob = get_u32(payload + 16 + 4 * (tile + 1));
  const uint8_t* body = payload + start + oa;
  const int64_t len = ob - oa;
  if (t == 0) {
    tile_err = (ob < oa || start + ob > payload_bytes) ? KQSC_E_OFFSETS : 0x7fffffff;
    row_err = 0x7fffffff;
  }
  __syncthreads();
  if (tile_err != 0x7fffffff) {
    if (t == 0) atomicMin(status, ((unsigned long long)tile << 20) | (unsigned)tile_err);
    return;
  }
  const int fb = (rc + 7) >> 3, cb = (2 * rc + 7) >> 3;
  int sel0;
  // ---- tile-level fields and checks
  if (VERSION == 1) {
    if (len < (int64_t)rc * (3 + sb)) {
      if (t == 0) atomicMin(status, ((unsigned long long)tile << 20) | KQSC_E_TRUNC_FIXED);
      return;
    }
    if (wave == 0) {
      int64_t q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = lane * 4 + j;
        q[j] = r < rc ? body[2 * rc + r] : 0;
      }
      tile_row_scan(q, lane, rc, pre);
    }
    if (t < rc) {
      second_of[t] = body[rc + t];
      cnt_of[t] = body[2 * rc + t];
    }
    __syncthreads();
    sel0 = 3 * rc;
    if (len != sel0 + (int64_t)rc * sb + 2 * pre[rc]) {
      if (t == 0) atomicMin(status, ((unsigned long long)tile << 20) | KQSC_E_COUNTS_LEN);
      return;
    }
  } else {
    const int meta0 = rc + 2 * fb + cb;
    if (len < meta0) {
      if (t == 0) atomicMin(status, ((unsigned long long)tile << 20) | KQSC_E_TRUNC_FIXED);
      return;
    }
    const int used = 2 * rc;
    int code = 0x7fffffff;
    if ((rc & 7) && (body[rc + fb - 1] >> (rc & 7))) code = KQSC_E_PAD_DIR;
    else if ((rc & 7) && (body[rc + 2 * fb - 1] >> (rc & 7))) code = KQSC_E_PAD_EXPL;
    else if ((used & 7) && (body[rc + 2 * fb + cb - 1] >> (used & 7))) code = KQSC_E_PAD_CODES;
    if (code != 0x7fffffff) {
      if (t == 0) atomicMin(status, ((unsigned long long)tile << 20) | (unsigned)code);
      return;
    }
    // explicit palettes and extended counts, in row order
    if (wave == 0) {
      int64_t q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = lane * 4 + j;
        q[j] = 0;
        if (r < rc) {
          const int expl = (body[rc + fb + (r >> 3)] >> (r & 7)) & 1;
          const int c = (body[rc + 2 * fb + (r >> 2)] >> (2 * (r & 3))) & 3;
          q[j] = pack_row_counts(0, expl, c == 3 ? 1 : 0);
        }
      }
      tile_row_scan(q, lane, rc, pre);
    }
    __syncthreads();
    const int64_t tot = pre[rc];
    const int n_expl = (int)((tot >> 32) & 0xffff), n_ext = (int)(tot >> 48);
    sel0 = meta0 + n_expl + n_ext;
    if (len < sel0 + (int64_t)rc * sb) {
      if (t == 0) atomicMin(status, ((unsigned long long)tile << 20) | KQSC_E_TRUNC_ESCAPES);
      return;
    }
    int n = 0;
    bool bad_escape = false;
    if (t < rc) {
      const int first = body[t];
      const int expl = (body[rc + fb + (t >> 3)] >> (t & 7)) & 1;
      const int dir = (body[rc + (t >> 3)] >> (t & 7)) & 1;
      const int c = (body[rc + 2 * fb + (t >> 2)] >> (2 * (t & 3))) & 3;
      if (c < 3) {
        n = c;
      } else {
        n = body[meta0 + n_expl + (pre[t] >> 48)];
        bad_escape = n < 3;
      }
      second_of[t] = (int16_t)(expl ? (int)body[meta0 + ((pre[t] >> 32) & 0xffff)]
                                    : first + (dir ? 1 : -1));
      cnt_of[t] = (uint8_t)n;
    }
    if (__syncthreads_or(bad_escape)) {
      if (t == 0) atomicMin(status, ((unsigned long long)tile << 20) | KQSC_E_COUNT_ESCAPE);
      return;
    }
    if (wave == 0) {
      int64_t q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = lane * 4 + j;
        q[j] = r < rc ? cnt_of[r] : 0;
      }
      tile_row_scan(q, lane, rc, pre);
    }
    __syncthreads();
    if (len != sel0 + (int64_t)rc * sb + 2 * pre[rc]) {
      if (t == 0) atomicMin(status, ((unsigned long long)tile << 20) | KQSC_E_COUNTS_LEN);
      return;
    }
  }
  // ---- rows: palette checks, selector expansion, exceptions
  const int exc0 = sel0 + rc * sb;
  for (int it = 0; it < (rc + SP_WAVES - 1) / SP_WAVES; ++it) {
    const int i = it * SP_WAVES + wave;
    const bool active = i < rc;
    int first = 0, second = 0, n = 0;
    int key = 0x7fffffff;
    if (active) {
      first = body[i];
      second = second_of[i];
      n = cnt_of[i];
      if (VERSION == 2) {
        const int expl = (body[rc + fb + (i >> 3)] >> (i & 7)) & 1;
        if (expl && adjacent_pair(first, second)) key = 0;
        else if (!expl && (second < 0 || second > 255)) key = 1;
      }
      if (key == 0x7fffffff && (cols & 7) && (body[sel0 + i * sb + sb - 1] >> (cols & 7))) key = 2;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      first_idx[wave][lane + 64 * k] = 0xffffffffu;
      const int c = lane + 64 * k;
      if (active && c < cols)
        rowbuf[wave][c] = (uint8_t)(((body[sel0 + i * sb + (c >> 3)] >> (c & 7)) & 1) ? second : first);
    }
    __syncthreads();
    const int64_t e_base = exc0 + 2 * (active ? pre[i] : 0);
    int pos[4], val[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = lane + 64 * k;
      pos[k] = -1;
      val[k] = 0;
      if (active && e < n) {
        pos[k] = body[e_base + 2 * e];
        val[k] = body[e_base + 2 * e + 1];
        if (pos[k] < cols) atomicMin(&first_idx[wave][pos[k]], (unsigned)e);
      }
    }
    __syncthreads();
    int ekey = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = lane + 64 * k;
      if (pos[k] < 0) continue;
      const bool bad_pos = pos[k] >= cols || first_idx[wave][pos[k]] < (unsigned)e;
      if (bad_pos) ekey = min(ekey, 3 + 2 * e);
      else if (val[k] == first || val[k] == second) ekey = min(ekey, 4 + 2 * e);
      if (pos[k] < cols) rowbuf[wave][pos[k]] = (uint8_t)val[k];
    }
    ekey = wave_min_i(ekey);
    if (active && lane == 0) {
      key = min(key, ekey);
      if (key != 0x7fffffff) atomicMin(&row_err, i * 1024 + key);
    }
    __syncthreads();
    if (active) {
      uint8_t* o = out + (r0 + i) * cols;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int c = lane + 64 * k;
        if (c < cols) o[c] = rowbuf[wave][c];
      }
    }
    __syncthreads();
  }
  if (t == 0 && row_err != 0x7fffffff)
    atomicMin(status, ((unsigned long long)tile << 20) | (unsigned)(KQSC_E_ROW + row_err));
}

// Per-tile accounting of a version-2 payload (kquant/mxfp4_scale_codec.py:427-499):
// {palette escapes, count escapes, exceptions}.  Body slices follow Python
// slice semantics, so a short or inverted range reads as a shorter body.
__global__ __launch_bounds__(SP_THREADS) void kqsc_stats_kernel(
    const uint8_t* __restrict__ payload, int64_t payload_bytes, int64_t rows, int cols,
    int tile_rows, int sb, int64_t tiles, uint32_t* __restrict__ tile_stats,
    unsigned long long* status) {
  const int64_t tile = (int64_t)blockIdx.x * SP_THREADS + threadIdx.x;
  if (tile >= tiles) return;
  const int rc = (int)min((int64_t)tile_rows, rows - tile * tile_rows);
  const int64_t start = 16 + 4 * (tiles + 1);
  const int64_t s = min(start + (int64_t)get_u32(payload + 16 + 4 * tile), payload_bytes);
  const int64_t e = min(start + (int64_t)get_u32(payload + 16 + 4 * (tile + 1)), payload_bytes);
  const int64_t len = max(e - s, (int64_t)0);
  const uint8_t* body = payload + s;
  const int fb = (rc + 7) >> 3, cb = (2 * rc + 7) >> 3;
  int code = -1;
  int pe = 0, ce = 0;
  int64_t eb = 0;
  if (len < rc + 2 * fb) {
    code = 0;
  } else if ((rc & 7) && (body[rc + 2 * fb - 1] >> (rc & 7))) {
    code = 1;
  } else if (len < rc + 2 * fb + cb) {
    code = 2;
  } else if (((2 * rc) & 7) && (body[rc + 2 * fb + cb - 1] >> ((2 * rc) & 7))) {
    code = 3;
  } else {
    for (int j = 0; j < fb; ++j) pe += __popc(body[rc + fb + j]);
    for (int r = 0; r < rc; ++r) ce += ((body[rc + 2 * fb + (r >> 2)] >> (2 * (r & 3))) & 3) == 3;
    eb = len - (rc + 2 * fb + cb + pe + ce + (int64_t)rc * sb);
    if (eb < 0 || (eb & 1)) code = 4;
  }
  if (code >= 0) {
    atomicMin(status, ((unsigned long long)tile << 20) | (unsigned)code);
    return;
  }
  tile_stats[3 * tile] = (uint32_t)pe;
  tile_stats[3 * tile + 1] = (uint32_t)ce;
  tile_stats[3 * tile + 2] = (uint32_t)(eb / 2);
}

int launch_scan(int64_t* data, int64_t n, hipStream_t st) {
  exclusive_scan_kernel<<<1, 1024, 0, st>>>(data, n);
  return kq_check_launch(hipGetLastError(), "exclusive scan");
}

}  // namespace
}  // namespace kq

using namespace kq;

static int x4t_geometry(const char* who, int64_t mats, int64_t rows, int64_t cols) {
  if (mats < 1 || rows <= 0 || rows % X4T_ROWS != 0)
    return kq_fail(KQ_ERR_INVALID, "%s: X4T scale rows must be a nonzero multiple of 16", who);
  if (cols < 1 || cols > 255)
    return kq_fail(KQ_ERR_INVALID, "%s: X4T scale columns must lie in 1..255", who);
  if (rows * cols > (int64_t)X4T_POS_MASK)
    return kq_fail(KQ_ERR_INVALID, "%s: X4T logical scale plane exceeds its 24-bit position field",
                   who);
  if (mats * (rows / X4T_ROWS) > 0x7fffffff)
    return kq_fail(KQ_ERR_LIMIT, "%s: too many tiles", who);
  return KQ_OK;
}

extern "C" int kq_x4t_analyze(const uint8_t* scale, int64_t mats, int64_t rows, int64_t cols,
                              uint8_t* fixed, int64_t* tile_offsets, void* stream) {
  if (int rc = x4t_geometry("kq_x4t_analyze", mats, rows, cols)) return rc;
  if (kq_misaligned(tile_offsets, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_analyze: tile_offsets must be 8-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const int64_t tiles = mats * (rows / X4T_ROWS);
  const int sb = (int)((cols + 7) / 8);
  x4t_analyze_kernel<<<(unsigned)tiles, SP_THREADS, 0, st>>>(scale, (int)cols, sb, fixed,
                                                             tile_offsets);
  if (int rc = kq_check_launch(hipGetLastError(), "kq_x4t_analyze")) return rc;
  return launch_scan(tile_offsets, tiles, st);
}

extern "C" int kq_x4t_emit_exceptions(const uint8_t* scale, int64_t mats, int64_t rows,
                                      int64_t cols, const uint8_t* fixed,
                                      const int64_t* tile_offsets, uint32_t* exceptions,
                                      void* stream) {
  if (int rc = x4t_geometry("kq_x4t_emit_exceptions", mats, rows, cols)) return rc;
  if (kq_misaligned(tile_offsets, 8) || kq_misaligned(exceptions, 4))
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_emit_exceptions: misaligned offsets or exceptions");
  const int64_t tiles = mats * (rows / X4T_ROWS);
  x4t_emit_kernel<<<(unsigned)tiles, SP_THREADS, 0, (hipStream_t)stream>>>(
      scale, (int)cols, (int)((cols + 7) / 8), rows / X4T_ROWS, fixed, tile_offsets, exceptions);
  return kq_check_launch(hipGetLastError(), "kq_x4t_emit_exceptions");
}

extern "C" int kq_x4t_decode(const uint8_t* fixed, const uint32_t* exceptions, int64_t n_exceptions,
                             const int64_t* exception_offsets, int64_t mats, int64_t rows,
                             int64_t cols, uint8_t* out, uint32_t* status, void* stream) {
  if (int rc = x4t_geometry("kq_x4t_decode", mats, rows, cols)) return rc;
  if (n_exceptions < 0 || n_exceptions > 0xffffffffLL)
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_decode: bad exception count %lld",
                   (long long)n_exceptions);
  if (mats > 1 && !exception_offsets)
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_decode: several matrices need exception_offsets");
  if (status && (mats != 1 || exception_offsets))
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_decode: validation takes one matrix and no offsets");
  if (kq_misaligned(exceptions, 4) || kq_misaligned(exception_offsets, 8) ||
      kq_misaligned(status, 4))
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_decode: misaligned buffers");
  hipStream_t st = (hipStream_t)stream;
  const int64_t tiles = mats * (rows / X4T_ROWS);
  const int sb = (int)((cols + 7) / 8);
  x4t_decode_kernel<<<(unsigned)tiles, SP_THREADS, 0, st>>>(
      fixed, exceptions, n_exceptions, exception_offsets, rows / X4T_ROWS, (int)cols, sb, out);
  if (int rc = kq_check_launch(hipGetLastError(), "kq_x4t_decode")) return rc;
  if (!status) return KQ_OK;
  x4t_status_init_kernel<<<1, 1, 0, st>>>(status);
  if (int rc = kq_check_launch(hipGetLastError(), "kq_x4t_decode")) return rc;
  const int64_t blocks = tiles + (n_exceptions + SP_THREADS - 1) / SP_THREADS;
  x4t_check_kernel<<<(unsigned)blocks, SP_THREADS, 0, st>>>(fixed, exceptions, n_exceptions, tiles,
                                                            (int)cols, sb, out, status);
  return kq_check_launch(hipGetLastError(), "kq_x4t_decode");
}

static int kqsc_geometry(const char* who, int version, int64_t rows, int64_t cols, int tile_rows,
                         int64_t* tiles) {
  if (version != 1 && version != 2)
    return kq_fail(KQ_ERR_INVALID, "%s: unsupported version %d", who, version);
  if (rows <= 0 || rows > 0xffffffffLL || cols < 1 || cols > 255)
    return kq_fail(KQ_ERR_INVALID,
                   "%s: scale dimensions must be nonzero and columns must fit uint8", who);
  if (tile_rows < 1 || tile_rows > KQSC_MAX_TILE_ROWS)
    return kq_fail(KQ_ERR_INVALID, "%s: tile_rows must fit uint8", who);
  *tiles = (rows + tile_rows - 1) / tile_rows;
  if (*tiles > 0x7fffffff) return kq_fail(KQ_ERR_LIMIT, "%s: too many tiles", who);
  return KQ_OK;
}

extern "C" int kq_x4t_tile_index(const uint32_t* exceptions, int64_t n_exceptions,
                                 const int64_t* exception_offsets, int64_t mats, int64_t rows,
                                 int64_t cols, uint32_t* index, void* stream) {
  if (int rc = x4t_geometry("kq_x4t_tile_index", mats, rows, cols)) return rc;
  if (n_exceptions < 0 || n_exceptions > 0xffffffffLL)
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_tile_index: bad exception count %lld", (long long)n_exceptions);
  if (mats > 1 && !exception_offsets)
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_tile_index: several matrices need exception_offsets");
  if (kq_misaligned(exceptions, 4) || kq_misaligned(exception_offsets, 8) || kq_misaligned(index, 4))
    return kq_fail(KQ_ERR_INVALID, "kq_x4t_tile_index: misaligned buffers");
  const int64_t total = mats * (rows / X4T_ROWS) + 1;
  x4t_tile_index_kernel<<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      exceptions, n_exceptions, exception_offsets, mats, rows / X4T_ROWS, (int)cols, index);
  return kq_check_launch(hipGetLastError(), "kq_x4t_tile_index");
}

namespace kq {
hipError_t x4t_expand_routed(const X4TExpandArgs& args, const int* routed, int max_routed, hipStream_t st) {
  int64_t groups = 0;
  for (int i = 0; i < args.n; ++i) {
    if (args.p[i].tiles % X4T_EXPAND_TILES != 0 || args.p[i].cols % 4 != 0 || args.p[i].cols > 255)
      return hipErrorInvalidValue;
    groups += args.p[i].tiles / X4T_EXPAND_TILES;
  }
  if (max_routed <= 0 || groups == 0) return hipSuccess;
  x4t_expand_tiled_kernel<<<dim3((unsigned)max_routed, (unsigned)groups), SP_THREADS, 0, st>>>(args, routed);
  return hipGetLastError();
}
}  // namespace kq

extern "C" int kq_kqsc_measure(int version, const uint8_t* scale, int64_t rows, int64_t cols,
                               int tile_rows, uint32_t* row_meta, int64_t* tile_offsets,
                               void* stream) {
  int64_t tiles;
  if (int rc = kqsc_geometry("kq_kqsc_measure", version, rows, cols, tile_rows, &tiles)) return rc;
  if (kq_misaligned(row_meta, 4) || kq_misaligned(tile_offsets, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_kqsc_measure: misaligned buffers");
  hipStream_t st = (hipStream_t)stream;
  const int sb = (int)((cols + 7) / 8);
  if (version == 1)
    kqsc_measure_kernel<1><<<(unsigned)tiles, SP_THREADS, 0, st>>>(scale, rows, (int)cols, tile_rows,
                                                                  sb, row_meta, tile_offsets);
  else
    kqsc_measure_kernel<2><<<(unsigned)tiles, SP_THREADS, 0, st>>>(scale, rows, (int)cols, tile_rows,
                                                                  sb, row_meta, tile_offsets);
  if (int rc = kq_check_launch(hipGetLastError(), "kq_kqsc_measure")) return rc;
  return launch_scan(tile_offsets, tiles, st);
}

extern "C" int kq_kqsc_emit(int version, const uint8_t* scale, int64_t rows, int64_t cols,
                            int tile_rows, const uint32_t* row_meta, const int64_t* tile_offsets,
                            uint8_t* payload, void* stream) {
  int64_t tiles;
  if (int rc = kqsc_geometry("kq_kqsc_emit", version, rows, cols, tile_rows, &tiles)) return rc;
  if (kq_misaligned(row_meta, 4) || kq_misaligned(tile_offsets, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_kqsc_emit: misaligned buffers");
  hipStream_t st = (hipStream_t)stream;
  const int sb = (int)((cols + 7) / 8);
  if (version == 1)
    kqsc_emit_kernel<1><<<(unsigned)tiles, SP_THREADS, 0, st>>>(scale, rows, (int)cols, tile_rows, sb,
                                                               tiles, row_meta, tile_offsets, payload);
  else
    kqsc_emit_kernel<2><<<(unsigned)tiles, SP_THREADS, 0, st>>>(scale, rows, (int)cols, tile_rows, sb,
                                                               tiles, row_meta, tile_offsets, payload);
  return kq_check_launch(hipGetLastError(), "kq_kqsc_emit");
}

extern "C" int kq_kqsc_decode(int version, const uint8_t* payload, int64_t payload_bytes,
                              int64_t rows, int64_t cols, int tile_rows, uint8_t* out,
                              uint64_t* status, void* stream) {
  int64_t tiles;
  if (int rc = kqsc_geometry("kq_kqsc_decode", version, rows, cols, tile_rows, &tiles)) return rc;
  if (!status || kq_misaligned(status, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_kqsc_decode: status must be an 8-byte aligned word");
  if (payload_bytes < 16 + 4 * (tiles + 1))
    return kq_fail(KQ_ERR_INVALID, "kq_kqsc_decode: payload is truncated in its offset table");
  hipStream_t st = (hipStream_t)stream;
  unsigned long long* s = reinterpret_cast<unsigned long long*>(status);
  status_fill_kernel<<<1, 1, 0, st>>>(s);
  if (int rc = kq_check_launch(hipGetLastError(), "kq_kqsc_decode")) return rc;
  const int sb = (int)((cols + 7) / 8);
  if (version == 1)
    kqsc_decode_kernel<1><<<(unsigned)tiles, SP_THREADS, 0, st>>>(
        payload, payload_bytes, rows, (int)cols, tile_rows, sb, tiles, out, s);
  else
    kqsc_decode_kernel<2><<<(unsigned)tiles, SP_THREADS, 0, st>>>(
        payload, payload_bytes, rows, (int)cols, tile_rows, sb, tiles, out, s);
  return kq_check_launch(hipGetLastError(), "kq_kqsc_decode");
}

extern "C" int kq_kqsc_stats(const uint8_t* payload, int64_t payload_bytes, int64_t rows,
                             int64_t cols, int tile_rows, uint32_t* tile_stats, uint64_t* status,
                             void* stream) {
  int64_t tiles;
  if (int rc = kqsc_geometry("kq_kqsc_stats", 2, rows, cols, tile_rows, &tiles)) return rc;
  if (!status || kq_misaligned(status, 8) || kq_misaligned(tile_stats, 4))
    return kq_fail(KQ_ERR_INVALID, "kq_kqsc_stats: misaligned buffers");
  if (payload_bytes < 16 + 4 * (tiles + 1))
    return kq_fail(KQ_ERR_INVALID, "kq_kqsc_stats: payload is truncated in its offset table");
  hipStream_t st = (hipStream_t)stream;
  unsigned long long* s = reinterpret_cast<unsigned long long*>(status);
  status_fill_kernel<<<1, 1, 0, st>>>(s);
  if (int rc = kq_check_launch(hipGetLastError(), "kq_kqsc_stats")) return rc;
  kqsc_stats_kernel<<<(unsigned)((tiles + SP_THREADS - 1) / SP_THREADS), SP_THREADS, 0, st>>>(
      payload, payload_bytes, rows, (int)cols, tile_rows, (int)((cols + 7) / 8), tiles, tile_stats, s);
  return kq_check_launch(hipGetLastError(), "kq_kqsc_stats");
}
