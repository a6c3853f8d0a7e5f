// QSRT trellis bitstream and weight decode on MI355X.
//
// Bitstream (kquant/qsrt.py:811-857): a 16x16 tile stores its 256 K-bit edge
// symbols (K = 2, 3, 4) as 16 spans of 16 symbols, each span K uint16 words
// written MSB first, then every pair of adjacent words exchanged.  Undoing
// the exchange leaves one contiguous MSB-first stream of 256 K bits, so the
// 16-bit trellis state at position i - the low 16 bits of
// (previous << K) | edge_i, cyclic in the tile (kquant/exl3_reference.py:
// 37-61) - is simply the 16 stream bits ending at symbol i, read cyclically.
//
// Weight decode (kquant/exl3_reference.py:110-192, 270-295): state ->
// E4M3 label of the tile's rate -> fp32, placed at row-major position
// perm[i] of the tile (the tensor-core element order of :88-108), tiles to
// [K, N]; then diag(suh) B_K W B_N diag(svh) with B the blockwise 128-point
// Hadamard.  A payload holds 128-channel records along the rate axis, each at
// its own rate (kquant/qsrt.py:974-1018), so a 128 x 128 output block is one
// record: one workgroup decodes its 64 tiles into LDS, transforms both sides
// there and writes the block.
#include "kq_act.h"
#include "kq_dma.h"
#include "kq_hadamard.h"
#include "kq_internal.h"

namespace kq {
namespace qsrt {

using had::fwht_lines;
using had::fwht128;
using had::HAD;
using had::HLD;

constexpr int TILE = 16;
constexpr int RECORD_TILES = 8;  // 128 channels per record
constexpr int MAX_RECORDS = 1024;

// Per-record rates, passed by value as a kernel argument (no device copy).
struct RecordRates {
  uint8_t bits[MAX_RECORDS];
};

// E4M3 (fn) byte -> fp32, exact for every finite code (labels are finite).
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t s = (b >> 7) & 1, e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;  // m * 2^-9
  else v = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  return s ? -v : v;
}

// Row-major position in the tile of trellis element t (tensor-core order).
__device__ __forceinline__ int tc_position(int t) {
  const int thread = t >> 3, j = t & 7;
  const int row0 = (thread & 3) * 2;
  const int rsel = j & 3;
  const int row = row0 + (rsel & 1) + ((rsel >> 1) << 3);
  const int col = (thread >> 2) + ((j >> 2) << 3);
  return row * TILE + col;
}

// ------------------------------------------------------------- bitstream --
// One thread per stored word: bits 16 w' .. 16 w' + 15 of the tile stream,
// written at word w' ^ 1.
__global__ __launch_bounds__(256) void pack_kernel(const int16_t* __restrict__ sym, int64_t tiles, int bits,
                                                   int16_t* __restrict__ packed) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int words = TILE * bits;
  if (g >= tiles * words) return;
  const int64_t tile = g / words;
  const int w = (int)(g - tile * words);
  const int16_t* s = sym + tile * 256;
  const uint32_t mask = (1u << bits) - 1;
  uint32_t word = 0;
  for (int b = 0; b < 16; ++b) {
    const int bit = 16 * w + b, j = bit / bits, within = bit - j * bits;
    word |= (((uint32_t)(uint16_t)s[j] & mask) >> (bits - 1 - within) & 1u) << (15 - b);
  }
  packed[tile * words + (w ^ 1)] = (int16_t)word;
}

// One thread per symbol: the K-bit edge (states == 0) or the 16-bit state
// ending at it (states != 0).
__global__ __launch_bounds__(256) void unpack_kernel(const int16_t* __restrict__ packed, int64_t tiles, int bits,
                                                     int states, int16_t* __restrict__ out) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= tiles * 256) return;
  const int64_t tile = g >> 8;
  const int i = (int)(g & 255);
  const int words = TILE * bits, nbits = 256 * bits;
  const uint16_t* p = reinterpret_cast<const uint16_t*>(packed) + tile * words;
  const int width = states ? 16 : bits;
  const int q0 = ((i + 1) * bits - width + nbits) % nbits;  // first stream bit of the window
  const int w = q0 >> 4, o = q0 & 15;
  const uint32_t hi = p[w ^ 1], lo = p[((w + 1) % words) ^ 1];
  const uint32_t window = ((hi << 16) | lo) << o;  // window bits at the top
  out[g] = (int16_t)(window >> (32 - width));
}

// -------------------------------------------------------------- decoding --
// Block (nb, kb): output rows 128 kb .. + 127 and columns 128 nb .. + 127,
// 8 x 8 trellis tiles; tile u = (local k tile u / 8, local n tile u % 8).
// FROM_STATES: the 16-bit states are given ([k_tiles][n_tiles][256]) with
// per-tile rates along the rate axis (tile_bits); otherwise the block's
// record is read from the packed payload and its states rebuilt.
template <int OUT, bool FROM_STATES>
__global__ __launch_bounds__(256) void decode_kernel(const int16_t* __restrict__ src, int64_t k_tiles,
                                                     int64_t n_tiles, int rate_n, RecordRates rates,
                                                     const uint8_t* __restrict__ tile_bits,
                                                     const uint8_t* __restrict__ labels,
                                                     const float* __restrict__ suh, const float* __restrict__ svh,
                                                     void* __restrict__ out, int64_t ldo, int transposed) {
  __shared__ float t[HAD][HLD];
  __shared__ uint16_t words[64][64];  // each tile's stored words (at most 16 * 4)
  const int tid = threadIdx.x;
  const int64_t kb = blockIdx.y, nb = blockIdx.x;
  const int u = tid >> 2, part = tid & 3;  // this thread: tile u, elements 64 part .. + 63
  const int64_t kt = kb * 8 + (u >> 3), nt = nb * 8 + (u & 7);
  const int lr = (u >> 3) * TILE, lc = (u & 7) * TILE;
  if constexpr (FROM_STATES) {
    const int tb = tile_bits[rate_n ? nt : kt];
    const int bits = tb < 2 ? 2 : tb > 4 ? 4 : tb;  // validated by the caller; clamped to stay in the tables
    const uint8_t* lab = labels + (int64_t)(bits - 2) * 65536;
    const uint16_t* st = reinterpret_cast<const uint16_t*>(src) + (kt * n_tiles + nt) * 256;
#pragma unroll 16
    for (int e = 0; e < 64; ++e) {
      const int i = 64 * part + e;
      const int pos = tc_position(i);
      t[lr + (pos >> 4)][lc + (pos & 15)] = e4m3_to_f32(lab[st[i]]);
    }
  } else {
    const int64_t record = rate_n ? nb : kb;
    const int64_t per_record = (int64_t)RECORD_TILES * (rate_n ? k_tiles : n_tiles);  // tiles per record
    int64_t offset = 0;
    for (int64_t r = 0; r < record; ++r) offset += per_record * TILE * rates.bits[r];
    const int bits = rates.bits[record];
    const int nwords = TILE * bits, nbits = 256 * bits;
    for (int i = tid; i < 64 * nwords; i += 256) {
      const int v = i / nwords, w = i - v * nwords;
      const int64_t vk = kb * 8 + (v >> 3), vn = nb * 8 + (v & 7);
      const int64_t in_record = rate_n ? vk * RECORD_TILES + (vn - nb * 8) : (vk - kb * 8) * n_tiles + vn;
      words[v][w] = reinterpret_cast<const uint16_t*>(src)[offset + in_record * nwords + w];
    }
    __syncthreads();
    const uint8_t* lab = labels + (int64_t)(bits - 2) * 65536;
#pragma unroll 16
    for (int e = 0; e < 64; ++e) {
      const int i = 64 * part + e;
      const int q0 = ((i + 1) * bits - 16 + nbits) % nbits;
      const int w = q0 >> 4, o = q0 & 15;
      const uint32_t hi = words[u][w ^ 1], lo = words[u][((w + 1) % nwords) ^ 1];
      const uint32_t state = ((((hi << 16) | lo) << o) >> 16) & 0xffffu;
      const int pos = tc_position(i);
      t[lr + (pos >> 4)][lc + (pos & 15)] = e4m3_to_f32(lab[state]);
    }
  }
  __syncthreads();
  const bool rotate = suh != nullptr;
  if (rotate) {
    fwht_lines<true>(t);
    fwht_lines<false>(t);
  }
  for (int i = tid; i < HAD * HAD; i += 256) {
    const int r = transposed ? (i & (HAD - 1)) : (i >> 7), c = transposed ? (i >> 7) : (i & (HAD - 1));
    const int64_t row = kb * HAD + r, col = nb * HAD + c;
    float v = t[r][c];
    if (rotate) v = v * (1.f / 128.f) * suh[row] * svh[col];
    const int64_t o = transposed ? col * ldo + row : row * ldo + col;
    if (OUT == 2) reinterpret_cast<float*>(out)[o] = v;
    else if (OUT == 0) reinterpret_cast<__bf16*>(out)[o] = (__bf16)v;
    else reinterpret_cast<_Float16*>(out)[o] = (_Float16)v;
  }
}


// ---------------------------------------------------------- fused linear --
// out[m, n] = sum_k x[m, k] W[k, n] with W the decoded weight, never written
// to memory: the serving use of the decode (scripts/stream_k3_pytorch.py:
// 771-775 decodes, then the expert's linear applies it).  With suh / svh,
// W = diag(suh) B W_reg B diag(svh), so the product is computed as
// (((x o suh) B) W_reg) B o svh: the activation rows are rotated once per
// workgroup, the tiles feed fp32 FMAs straight from the trellis, and the
// 128-column output block is rotated in the epilogue (B is linear, so each
// K chunk's partial block may be rotated before the chunks are summed).
//
// Workgroup (n block nb, K chunk, row group): 16 waves = 8 n tiles x 2 halves
// of every 128-row k block of the chunk (4 k tiles each).  Lane l of a wave
// owns trellis symbols 4l .. 4l + 3 of each tile: one column
// (l >> 3) + 8 (l & 1) and rows r0, r0 + 1, r0 + 8, r0 + 9 with
// r0 = 2 ((l >> 1) & 3) in the tensor-core order, and their four states are
// one window of 16 + 3K stream bits.  Stored dword d of a tile is stream
// bits 32 d .. 32 d + 31, most significant first (the word exchange makes
// it so), so the window comes from two dwords.  The block's 65,536-entry
// label table of the current rate lives in LDS, and the k blocks' trellis
// words stream through a ring of LDS stages filled by direct loads several
// blocks ahead.  The table lookups (one random LDS byte read per weight)
// bound the main loop.
constexpr int LIN_THREADS = 1024;
// 128-row k blocks a workgroup may cover: its rotated activation rows
// (M x 128 per block, fp32) take at most 32 KB of LDS.
constexpr int lin_max_kb(int m) { return 64 / m; }
// k blocks of trellis words in flight per workgroup (8 KB of LDS each)
constexpr int LIN_STAGES = 4;

struct LinRecords {
  uint8_t bits[MAX_RECORDS];
  uint32_t prefix8[MAX_RECORDS / 8 + 1];  // sum of bits[r] over r < 8 i
};

struct LinArgs {
  const void* x;
  int64_t ldx, m;
  const uint32_t* payload;
  const uint8_t* labels;
  const float* suh;
  const float* svh;
  void* out;
  int64_t ldo;
  // when chunks > 1: the partials [chunks][m][N] and, for more than two
  // rows per workgroup, completion counters [row groups][n blocks]; both are
  // zero between calls (a polled partial is never stored as +0.0, see
  // store_partial)
  float* partial;
  int* counters;
  int k_tiles, n_tiles, rate_n, kbw, chunks, x_dtype, out_dtype;
};

// Rate of record r and the sum of the rates of records before it, from the
// kernel-argument table through uniform dword loads (r is uniform).
__device__ __forceinline__ int record_rate(const LinRecords& rec, int r) {
  r = __builtin_amdgcn_readfirstlane(r);
  const uint32_t w = reinterpret_cast<const uint32_t*>(rec.bits)[r >> 2];
  return (int)((w >> (8 * (r & 3))) & 0xffu);
}

__device__ __forceinline__ uint32_t record_rates_before(const LinRecords& rec, int r) {
  r = __builtin_amdgcn_readfirstlane(r);
  const uint32_t* w = reinterpret_cast<const uint32_t*>(rec.bits) + ((r >> 3) << 1);
  const int n = r & 7;  // records r & ~7 .. r - 1 on top of the prefix
  const uint32_t m0 = n >= 4 ? 0xffffffffu : (1u << (8 * n)) - 1u;
  const uint32_t m1 = n <= 4 ? 0u : (1u << (8 * (n - 4))) - 1u;
  // rates are at most 4, so the byte sums of a multiply do not carry
  return rec.prefix8[r >> 3] + (((w[0] & m0) * 0x01010101u) >> 24) + (((w[1] & m1) * 0x01010101u) >> 24);
}


// E4M3 (OCP, fn) byte -> fp32 with the gfx950 conversion instruction (exact:
// every finite E4M3 value is an fp32 value).
__device__ __forceinline__ float e4m3_scaled(uint32_t b) { return __builtin_amdgcn_cvt_f32_fp8((int)b, 0); }

__device__ __forceinline__ float load_x(const void* x, int dtype, int64_t i) {
  if (dtype == KQ_DT_F32) return reinterpret_cast<const float*>(x)[i];
  if (dtype == KQ_DT_F16) return (float)reinterpret_cast<const _Float16*>(x)[i];
  return (float)reinterpret_cast<const __bf16*>(x)[i];
}

// output codes of store_out: KQ_DT_* and, for the regularized weight only,
// its E4M3 label bytes (every value is an E4M3 label, so the conversion
// returns the label byte exactly)
constexpr int OUT_E4M3 = KQ_QSRT_OUT_E4M3;

__device__ __forceinline__ void store_out(void* out, int dtype, int64_t i, float v) {
  if (dtype == KQ_DT_F32) reinterpret_cast<float*>(out)[i] = v;
  else if (dtype == KQ_DT_F16) reinterpret_cast<_Float16*>(out)[i] = (_Float16)v;
  else if (dtype == OUT_E4M3)
    reinterpret_cast<uint8_t*>(out)[i] = (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false) & 0xff);
  else reinterpret_cast<__bf16*>(out)[i] = (__bf16)v;
}

// Stage the label table of rate `bits` into LDS (direct loads; the caller
// waits and crosses a barrier).
__device__ __forceinline__ void stage_labels(const uint8_t* labels, int bits, uint8_t* lut, int wave, int lane) {
  const dma::i32x4_t rs = dma::make_rsrc(labels + (int64_t)(bits - 2) * 65536, 65536);
  const uint32_t base = dma::lds_offset_of(lut);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const uint32_t c = (uint32_t)__builtin_amdgcn_readfirstlane((it * 16 + wave) * 1024);
    dma::load_to_lds16(rs, c + (uint32_t)lane * 16u, base + c);
  }
}

// A wave-uniform pointer held in scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// Wait until this wave's stage loads older than the `younger` most recent
// ones have landed (its direct loads complete in order).
__device__ __forceinline__ void wait_own_stage(int younger) {
  static_assert(LIN_STAGES == 4, "the waits below count up to four younger loads");
  if (younger >= 4) __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(4));
  else if (younger == 3) __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(3));
  else if (younger == 2) __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(2));
  else if (younger == 1) __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(1));
  else __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
}

// This wave's 4 tiles of k block kb - k tiles kb * 8 + half * 4 + i, n tile
// nb * 8 + ntl - into its own 512-byte slot of a ring stage (tile i at byte
// 32 K i): 2 K lanes of 16 bytes per tile, one direct load per wave, so a
// wave waits for its own loads only and the ring needs no barrier.  rec0:
// dword offset of the block's record in the payload.
__device__ __forceinline__ void stage_wave(const uint32_t* payload, int64_t rec0, int bits, int rate_n,
                                           int n_tiles, int nb, int kb, uint32_t* stage, int wave, int lane) {
  const int half = wave >> 3, ntl = wave & 7;
  const int tile_bytes = 32 * bits;
  const int64_t first = rate_n ? (int64_t)kb * 64 + half * 32 + ntl : (int64_t)half * 4 * n_tiles + nb * 8 + ntl;
  const int64_t step = rate_n ? RECORD_TILES : n_tiles;  // tiles from one k tile of the block to the next
  const uint8_t* base = uniform_ptr(reinterpret_cast<const uint8_t*>(payload) + rec0 * 4 + first * tile_bytes);
  const dma::i32x4_t rs = dma::make_rsrc(base, (uint32_t)dma::MAX_RANGE);
  const uint32_t lds =
      (uint32_t)__builtin_amdgcn_readfirstlane((int)(dma::lds_offset_of(stage) + (uint32_t)wave * 512u));
  // i = lane / (2 K) by a multiply: exact for lane < 64 and 2 K in {4, 6, 8}
  const int magic = bits == 2 ? 16385 : bits == 3 ? 10923 : 8193;
  const int i = (lane * magic) >> 16, within = (lane - i * 2 * bits) * 16;
  if (lane < 8 * bits) dma::load_to_lds16(rs, (uint32_t)(i * step * tile_bytes + within), lds);
}

// acc[m] += this lane's part of xs[m][k rows of the block] . W[block, column]
// for one staged k block: the wave's 4 tiles in its slot (k tiles
// half * 4 + i of the block), 4 symbols each.  xs points at row 0, k block
// kbi.
template <int M>
__device__ __forceinline__ void accumulate_block(const uint32_t* slot, int bits, const uint8_t* lut,
                                                 const float* xs, int xs_stride, int half, int lane,
                                                 float (&acc)[M]) {
  const int r0 = 2 * ((lane >> 1) & 3);
  // first stream bit of the window: (4 lane + 1) K - 16, cyclic (lane 0 wraps)
  int sb = (4 * lane + 1) * bits - 16;
  if (sb < 0) sb += 256 * bits;
  const int d0 = sb >> 5, d1 = d0 + 1 == 8 * bits ? 0 : d0 + 1, off = sb & 31, sh = 64 - (16 + 3 * bits);
  uint32_t st[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t* t = slot + i * 8 * bits;
    const uint64_t v = (((uint64_t)t[d0] << 32) | t[d1]) << off;
    const uint32_t win = (uint32_t)(v >> sh);
    st[4 * i + 0] = (win >> (3 * bits)) & 0xffffu;
    st[4 * i + 1] = (win >> (2 * bits)) & 0xffffu;
    st[4 * i + 2] = (win >> bits) & 0xffffu;
    st[4 * i + 3] = win & 0xffffu;
  }
  float w[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) w[e] = e4m3_scaled(lut[st[e]]);
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float* xr = xs + m * xs_stride + (half * 4 + i) * 16 + r0;
      const float2 xa = *reinterpret_cast<const float2*>(xr);
      const float2 xb = *reinterpret_cast<const float2*>(xr + 8);
      acc[m] = fmaf(xa.x, w[4 * i + 0], acc[m]);
      acc[m] = fmaf(xa.y, w[4 * i + 1], acc[m]);
      acc[m] = fmaf(xb.x, w[4 * i + 2], acc[m]);
      acc[m] = fmaf(xb.y, w[4 * i + 3], acc[m]);
    }
  }
  // pin the products here: sunk past the caller's next barrier, they would
  // keep every activation value of the block live across it
#pragma unroll
  for (int m = 0; m < M; ++m) asm volatile("" : "+v"(acc[m]));
}

// Sum the four lanes of a column (lanes differing in bits 1 and 2), then
// lanes with (lane & 6) == 0 hold column (lane >> 3) + 8 (lane & 1).
template <int M>
__device__ __forceinline__ void column_sums(float (&acc)[M]) {
#pragma unroll
  for (int m = 0; m < M; ++m) {
    acc[m] += __shfl_xor(acc[m], 2);
    acc[m] += __shfl_xor(acc[m], 4);
  }
}

// Cross-workgroup partial sums polled by their reader (one or two rows per
// workgroup, where the sum is a few words per thread and its latency is what
// counts): the buffer is zero between calls, a partial is stored with +0.0
// replaced by -0.0, so a word that is still +0.0 has not been stored yet, and
// the reader clears every word after reading.  A relaxed agent-scope atomic
// store is written through the XCD's L2 to the memory-side coherence point
// shared by all XCDs, and a relaxed agent-scope atomic load reads that point,
// so the reader sees a word once its store has been performed there.
// (-0.0 + x == x for every x other than +0.0, so the sums change at most in
// the sign of a zero.)
__device__ __forceinline__ void store_partial(float* p, float v) {
  __hip_atomic_store(p, v == 0.f ? -0.f : v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_partial(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool stored(float v) { return __float_as_uint(v) != 0u; }

// words a thread polls at once (more cost instruction fetches at the tail)
constexpr int POLL_BATCH = 2;
// Upper bound of re-reads of a batch (each one a memory round trip after a
// short sleep: well beyond a second) before the reader gives up and returns
// NaN for the words still missing.
constexpr int POLL_LIMIT = 1 << 20;

// v[u] = p[(ch0 + u * STEP) * stride] for the chunks below `count`, once all
// of them have been stored (NaN for a word still unstored after POLL_LIMIT
// re-reads).
template <int U, int STEP>
__device__ __forceinline__ void poll_partials(const float* p, int64_t stride, int ch0, int count, float (&v)[U]) {
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = ch0 + u * STEP < count ? load_partial(p + (ch0 + u * STEP) * stride) : 1.f;
  for (int it = 0;; ++it) {
    bool ready = true;
#pragma unroll
    for (int u = 0; u < U; ++u) ready &= stored(v[u]);
    if (ready) return;
    if (it == POLL_LIMIT) break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (!stored(v[u])) v[u] = load_partial(p + (ch0 + u * STEP) * stride);
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (!stored(v[u])) v[u] = __builtin_nanf("");
}

typedef float qf32x4_t __attribute__((ext_vector_type(4)));

// Four or more rows: the block's products on v_mfma_f32_16x16x4f32, one
// 16 x 16 output (rows m, columns of the wave's n tile) per wave.  The four
// k values of MFMA j are tile rows 4 kq + j for lane group kq, so lane
// (n, kq) decodes the symbols at rows 4 kq .. 4 kq + 3 of column n -- in
// the tensor-core order symbols b, b + 1, b + 8, b + 9 with b = (n % 8) << 5
// | (kq % 2) << 4 | (n / 8) << 2 | (kq / 2) << 1, two windows of 16 + K
// stream bits -- and reads x[n][4 kq .. 4 kq + 3] of the tile's k as one
// 128-bit fragment (rows n >= M give zeros).  acc: rows 4 kq + r, column n.
template <int M>
__device__ __forceinline__ void accumulate_block_mfma(const uint32_t* slot, int bits, const uint8_t* lut,
                                                      const float* xs, int xs_stride, int half, int lane,
                                                      qf32x4_t& acc) {
  const int n = lane & 15, kq = lane >> 4;
  const int b = ((n & 7) << 5) | ((kq & 1) << 4) | ((n >> 3) << 2) | ((kq >> 1) << 1);
  const int sh = 64 - (16 + bits);
  int d0[2], d1[2], off[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {  // symbols b + 8 p and b + 8 p + 1: the window ending at the second
    int sb = (b + 8 * p + 1) * bits - 16;
    if (sb < 0) sb += 256 * bits;
    d0[p] = sb >> 5;
    d1[p] = d0[p] + 1 == 8 * bits ? 0 : d0[p] + 1;
    off[p] = sb & 31;
  }
  const bool live = n < M;
  const float* xr = xs + (live ? n : 0) * xs_stride + half * 64 + 4 * kq;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t* t = slot + i * 8 * bits;
    float w[4];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const uint64_t v = (((uint64_t)t[d0[p]] << 32) | t[d1[p]]) << off[p];
      const uint32_t win = (uint32_t)(v >> sh);
      w[2 * p] = e4m3_scaled(lut[(win >> bits) & 0xffffu]);
      w[2 * p + 1] = e4m3_scaled(lut[win & 0xffffu]);
    }
    qf32x4_t xa = *reinterpret_cast<const qf32x4_t*>(xr + i * 16);
    if (!live) xa = qf32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[j], w[j], acc, 0, 0, 0);
  }
}

// Stage this wave's tiles of k block kb of the kernel-argument matrix.
__device__ __forceinline__ void stage_block(const LinArgs& a, const LinRecords& rec, int nb, int kb,
                                            uint32_t* stage, int wave, int lane) {
  const int record = a.rate_n ? nb : kb;
  const int64_t record_dw = (int64_t)RECORD_TILES * (a.rate_n ? a.k_tiles : a.n_tiles) * 8;
  stage_wave(a.payload, (int64_t)record_rates_before(rec, record) * record_dw, record_rate(rec, record), a.rate_n,
             a.n_tiles, nb, kb, stage, wave, lane);
}

template <int M, bool ROT>
__global__ __launch_bounds__(LIN_THREADS) void linear_kernel(LinArgs a, LinRecords rec) {
  __shared__ __attribute__((aligned(16))) uint8_t lut[65536];
  __shared__ __attribute__((aligned(16))) uint32_t ring[LIN_STAGES][2048];  // 16 waves x 512 bytes
  // rows padded by 16 bytes: the 128-bit fragment reads of 16 rows hit distinct bank groups
  constexpr int XS = lin_max_kb(M) * 128 + 4;
  constexpr bool MF = M >= 4;  // products on MFMA
  __shared__ __attribute__((aligned(16))) float xs[M][XS];
  __shared__ float yb[2][M][128];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = wave >> 3, ntl = wave & 7;
  const int n_blocks = a.n_tiles >> 3, k_blocks = a.k_tiles >> 3;
  const int nb = (int)(blockIdx.x % (unsigned)n_blocks), chunk = (int)(blockIdx.x / (unsigned)n_blocks);
  const int kb0 = chunk * a.kbw;
  const int kbn = min(a.kbw, k_blocks - kb0);
  const int64_t m0 = (int64_t)blockIdx.y * M;
  const int mc = (int)min((int64_t)M, a.m - m0);
  const int64_t n_cols = (int64_t)a.n_tiles * TILE;

  // labels of the first block's rate, then the first stages of the ring
  int lut_bits = record_rate(rec, a.rate_n ? nb : kb0);
  stage_labels(a.labels, lut_bits, lut, wave, lane);
#pragma unroll
  for (int j = 0; j < LIN_STAGES; ++j)
    if (j < kbn) stage_block(a, rec, nb, kb0 + j, ring[j], wave, lane);

  // rotated activation rows of this chunk: lines (row m, k block kbi)
  for (int line = wave; line < M * kbn; line += 16) {
    const int m = line / kbn, kbi = line - m * kbn;
    float v0 = 0.f, v1 = 0.f;
    if (m < mc) {
      const int64_t k = (int64_t)(kb0 + kbi) * 128 + lane;
      const int64_t row = (m0 + m) * a.ldx;
      v0 = load_x(a.x, a.x_dtype, row + k);
      v1 = load_x(a.x, a.x_dtype, row + k + 64);
      if constexpr (ROT) {
        v0 *= a.suh[k];
        v1 *= a.suh[k + 64];
        fwht128(v0, v1, lane);
      }
    }
    xs[m][kbi * 128 + lane] = v0;
    xs[m][kbi * 128 + lane + 64] = v1;
  }

  // the output scales of this column block, loaded now so the epilogue does
  // not wait on memory
  float sv0 = 1.f, sv1 = 1.f;
  if constexpr (ROT) {
    sv0 = a.svh[(int64_t)nb * 128 + lane] * (1.f / 128.f);
    sv1 = a.svh[(int64_t)nb * 128 + lane + 64] * (1.f / 128.f);
  }
  float acc[MF ? 1 : M];
#pragma unroll
  for (int m = 0; m < (MF ? 1 : M); ++m) acc[m] = 0.f;
  qf32x4_t macc = {0.f, 0.f, 0.f, 0.f};
  // every wave's labels (older than its stage loads) and activation rows
  wait_own_stage(min(LIN_STAGES, kbn));
  __syncthreads();

  for (int kbi = 0; kbi < kbn; ++kbi) {
    const int bits = record_rate(rec, a.rate_n ? nb : kb0 + kbi);
    if (bits != lut_bits) {  // rate along k changed: restage the labels (uniform)
      __syncthreads();
      stage_labels(a.labels, bits, lut, wave, lane);
      __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
      __syncthreads();
      lut_bits = bits;
    }
    // this wave's block kbi has landed once only its younger stages are in flight
    wait_own_stage(min(LIN_STAGES - 1, kbn - 1 - kbi));
    if constexpr (MF)
      accumulate_block_mfma<M>(ring[kbi % LIN_STAGES] + wave * 128, bits, lut, &xs[0][kbi * 128], XS, half, lane,
                               macc);
    else
      accumulate_block<M>(ring[kbi % LIN_STAGES] + wave * 128, bits, lut, &xs[0][kbi * 128], XS, half, lane, acc);
    // the wave has consumed its slot: refill it with block kbi + stages
    if (kbi + LIN_STAGES < kbn)
      stage_block(a, rec, nb, kb0 + kbi + LIN_STAGES, ring[kbi % LIN_STAGES], wave, lane);
  }
  if constexpr (MF) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * (lane >> 4) + r;
      if (m < M) yb[half][m][ntl * 16 + (lane & 15)] = macc[r];
    }
  } else {
    column_sums<M>(acc);
    if ((lane & 6) == 0) {
      const int c = ntl * 16 + (lane >> 3) + 8 * (lane & 1);
#pragma unroll
      for (int m = 0; m < M; ++m) yb[half][m][c] = acc[m];
    }
  }
  __syncthreads();

  // The K chunks of a column block meet in one workgroup, which sums the
  // partials in chunk order.  One or two rows: the workgroup of the last
  // chunk keeps its own partial in LDS and polls the others (it is the last
  // of the block's workgroups in dispatch order, and they wait on nothing, so
  // every one of them runs to its stores).  More rows: the last workgroup to
  // finish, found by a completion counter.
  constexpr bool POLLED = M <= 2;
  const int64_t col0 = (int64_t)nb * 128;
  const bool reader = POLLED && chunk == a.chunks - 1;
  if (wave < mc) {
    const int m = wave;
    float v0 = yb[0][m][lane] + yb[1][m][lane];
    float v1 = yb[0][m][lane + 64] + yb[1][m][lane + 64];
    if constexpr (ROT) {
      fwht128(v0, v1, lane);
      v0 *= sv0;
      v1 *= sv1;
    }
    float* p = a.partial + ((int64_t)chunk * a.m + m0 + m) * n_cols + col0;
    if (a.chunks == 1) {
      store_out(a.out, a.out_dtype, (m0 + m) * a.ldo + col0 + lane, v0);
      store_out(a.out, a.out_dtype, (m0 + m) * a.ldo + col0 + lane + 64, v1);
    } else if (reader) {
      yb[0][m][lane] = v0;  // this thread's own reads above
      yb[0][m][lane + 64] = v1;
    } else if (POLLED) {
      store_partial(p + lane, v0);
      store_partial(p + lane + 64, v1);
    } else {
      __hip_atomic_store(p + lane, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p + lane + 64, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (a.chunks == 1) return;
  constexpr int TPO = LIN_THREADS / (M * 128) > 0 ? LIN_THREADS / (M * 128) : 1;
  const int64_t stride = a.m * n_cols;

  if constexpr (POLLED) {
    if (!reader) return;
    __syncthreads();
    // TPO adjacent threads per output, thread j of them summing chunks j,
    // j + TPO, ... in order (the last chunk from LDS), then a fixed shuffle
    // tree; each word is polled until it has been stored
    const int o = tid / TPO, j = tid % TPO, m = o >> 7, c = o & 127;
    const float* p = a.partial + (m0 + m) * n_cols + col0 + c;
    float sum = 0.f;
    if (m < mc) {
      for (int ch0 = j; ch0 < a.chunks; ch0 += POLL_BATCH * TPO) {
        float v[POLL_BATCH];
        poll_partials<POLL_BATCH, TPO>(p, stride, ch0, a.chunks - 1, v);
#pragma unroll
        for (int u = 0; u < POLL_BATCH; ++u) {
          const int ch = ch0 + u * TPO;
          if (ch < a.chunks - 1) sum += v[u];
          else if (ch == a.chunks - 1) sum += yb[0][m][c];
        }
      }
    }
#pragma unroll
    for (int sft = 1; sft < TPO; sft <<= 1) sum += __shfl_xor(sum, sft);
    if (m >= mc) return;
    if (j == 0) store_out(a.out, a.out_dtype, (m0 + m) * a.ldo + col0 + c, sum);
    // clear the words read (after every load: a wait for a load would also
    // wait for the stores issued before it)
    for (int ch = j; ch < a.chunks - 1; ch += TPO)
      __hip_atomic_store(const_cast<float*>(p) + ch * stride, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    // Every wave waits for its partial stores to complete before the barrier
    // that precedes the counter increment; the last workgroup reads after
    // seeing the count.
    __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
    __syncthreads();
    int* counter = a.counters + (int64_t)blockIdx.y * n_blocks + nb;
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.chunks - 1;
    __syncthreads();
    if (!s_last) return;
    // TPO adjacent threads per output, thread j of them summing chunks j,
    // j + TPO, ... (loads issued together), then a fixed shuffle tree
    for (int o0 = 0; o0 < M * 128; o0 += LIN_THREADS / TPO) {
      const int o = o0 + tid / TPO, j = tid % TPO, m = o >> 7, c = o & 127;
      float sum = 0.f;
      if (m < mc) {
        const float* p = a.partial + (m0 + m) * n_cols + col0 + c;
        int ch = j;
        for (; ch + 3 * TPO < a.chunks; ch += 4 * TPO) {
          float v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = load_partial(p + (ch + u * TPO) * stride);
          sum += v[0];
          sum += v[1];
          sum += v[2];
          sum += v[3];
        }
        for (; ch < a.chunks; ch += TPO) sum += load_partial(p + ch * stride);
      }
#pragma unroll
      for (int sft = 1; sft < TPO; sft <<= 1) sum += __shfl_xor(sum, sft);
      if (j == 0 && m < mc) store_out(a.out, a.out_dtype, (m0 + m) * a.ldo + col0 + c, sum);
    }
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}


// -------------------------------------------------------- fast decode --
// kq_qsrt_decode_weight from a payload on the fused workgroup's machinery:
// the rate's label table in LDS, every wave's 4 tiles of a 128 x 128 block
// streamed through its LDS ring slot, the block's fp32 values in an LDS tile,
// the two 128-point rotations as wave-level transforms over its rows and
// columns, and coalesced stores in either orientation.  A workgroup walks a
// chunk of k blocks of one n block (records along n share one rate).
struct DecArgs {
  const uint32_t* payload;
  const uint8_t* labels;
  const float* suh;
  const float* svh;
  void* out;
  int64_t ldo;
  int k_tiles, n_tiles, rate_n, kbw, transposed, out_dtype;
  // E4M3 output with 4-byte aligned rows: the label bytes go to a byte tile
  // in the output's orientation and leave as 4-byte stores
  int bytes;
};

template <bool ROT>
__global__ __launch_bounds__(LIN_THREADS) void decode_fast_kernel(DecArgs a, LinRecords rec) {
  __shared__ __attribute__((aligned(16))) uint8_t lut[65536];
  constexpr int ST = 3;  // ring stages (the fp32 tile takes the fourth's LDS)
  __shared__ __attribute__((aligned(16))) uint32_t ring[ST][2048];  // 16 waves x 512 bytes
  __shared__ __attribute__((aligned(16))) float t[128][129];
  constexpr int TBL = 132;  // byte tile row (bytes: 33 dwords, rows on distinct banks)
  uint8_t* tb = reinterpret_cast<uint8_t*>(&t[0][0]);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = wave >> 3, ntl = wave & 7;
  const int n_blocks = a.n_tiles >> 3, k_blocks = a.k_tiles >> 3;
  const int nb = (int)(blockIdx.x % (unsigned)n_blocks), chunk = (int)(blockIdx.x / (unsigned)n_blocks);
  const int kb0 = chunk * a.kbw;
  const int kbn = min(a.kbw, k_blocks - kb0);
  const int64_t record_dw_nb = (int64_t)RECORD_TILES * (a.rate_n ? a.k_tiles : a.n_tiles) * 8;

  auto stage = [&](int kb, uint32_t* slot_stage) {
    const int record = a.rate_n ? nb : kb;
    stage_wave(a.payload, (int64_t)record_rates_before(rec, record) * record_dw_nb, record_rate(rec, record),
               a.rate_n, a.n_tiles, nb, kb, slot_stage, wave, lane);
  };
  int lut_bits = record_rate(rec, a.rate_n ? nb : kb0);
  stage_labels(a.labels, lut_bits, lut, wave, lane);
#pragma unroll
  for (int j = 0; j < ST; ++j)
    if (j < kbn) stage(kb0 + j, ring[j]);
  // output scales of this n block's columns (ROT), one pair per lane
  float sv0 = 1.f, sv1 = 1.f;
  if constexpr (ROT) {
    sv0 = a.svh[(int64_t)nb * 128 + lane] * (1.f / 128.f);
    sv1 = a.svh[(int64_t)nb * 128 + lane + 64] * (1.f / 128.f);
  }
  wait_own_stage(min(ST, kbn));  // every wave's labels
  __syncthreads();

  const int r0 = 2 * ((lane >> 1) & 3), col = ntl * 16 + (lane >> 3) + 8 * (lane & 1);
  for (int kbi = 0; kbi < kbn; ++kbi) {
    const int kb = kb0 + kbi;
    const int bits = record_rate(rec, a.rate_n ? nb : kb);
    if (bits != lut_bits) {  // the rate along k changed (uniform): restage the labels
      __syncthreads();
      stage_labels(a.labels, bits, lut, wave, lane);
      __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
      __syncthreads();
      lut_bits = bits;
    }
    wait_own_stage(min(ST - 1, kbn - 1 - kbi));
    {  // this wave's 4 tiles -> the fp32 tile (rows of the k tiles, columns of n tile ntl)
      const uint32_t* slot = ring[kbi % ST] + wave * 128;
      int sb = (4 * lane + 1) * bits - 16;
      if (sb < 0) sb += 256 * bits;
      const int d0 = sb >> 5, d1 = d0 + 1 == 8 * bits ? 0 : d0 + 1, off = sb & 31, sh = 64 - (16 + 3 * bits);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t* w = slot + i * 8 * bits;
        const uint64_t v = (((uint64_t)w[d0] << 32) | w[d1]) << off;
        const uint32_t win = (uint32_t)(v >> sh);
        const int row = (half * 4 + i) * 16 + r0;
        const uint8_t l0 = lut[(win >> (3 * bits)) & 0xffffu], l1 = lut[(win >> (2 * bits)) & 0xffffu];
        const uint8_t l2 = lut[(win >> bits) & 0xffffu], l3 = lut[win & 0xffffu];
        if (!ROT && a.bytes) {  // byte tile [output row][128 + 4]
          const int rs = a.transposed ? 1 : TBL, cs = a.transposed ? TBL : 1;
          tb[row * rs + col * cs] = l0;
          tb[(row + 1) * rs + col * cs] = l1;
          tb[(row + 8) * rs + col * cs] = l2;
          tb[(row + 9) * rs + col * cs] = l3;
        } else {
          t[row][col] = e4m3_scaled(l0);
          t[row + 1][col] = e4m3_scaled(l1);
          t[row + 8][col] = e4m3_scaled(l2);
          t[row + 9][col] = e4m3_scaled(l3);
        }
      }
    }
    if (kbi + ST < kbn) stage(kb + ST, ring[kbi % ST]);
    __syncthreads();
    const int64_t row0 = (int64_t)kb * 128, col0 = (int64_t)nb * 128;
    if constexpr (ROT) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // along the columns of every row: B_N (8 independent rows per wave)
        const int r = wave + 16 * i;
        float v0 = t[r][lane], v1 = t[r][lane + 64];
        fwht128(v0, v1, lane);
        t[r][lane] = v0 * sv0;
        t[r][lane + 64] = v1 * sv1;
      }
      __syncthreads();
      const float su0 = a.suh[row0 + lane], su1 = a.suh[row0 + lane + 64];
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // along the rows of every column: B_K, then suh
        const int c = wave + 16 * i;
        float v0 = t[lane][c], v1 = t[lane + 64][c];
        fwht128(v0, v1, lane);
        v0 *= su0;
        v1 *= su1;
        if (a.transposed) {  // out [N, K]: the column is an output row, stored from registers
          const int64_t o = (col0 + c) * a.ldo + row0;
          store_out(a.out, a.out_dtype, o + lane, v0);
          store_out(a.out, a.out_dtype, o + lane + 64, v1);
        } else {
          t[lane][c] = v0;
          t[lane + 64][c] = v1;
        }
      }
      if (a.transposed) {
        __syncthreads();  // the tile is rewritten by the next block
        continue;
      }
      __syncthreads();
    }
    if (!ROT && a.bytes) {  // 128 output rows of 128 bytes: two per wave pass, 4 bytes a lane
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int orow = 8 * wave + 2 * h + (lane >> 5), ob = 4 * (lane & 31);
        const uint32_t v = *reinterpret_cast<const uint32_t*>(tb + orow * TBL + ob);
        const int64_t o = a.transposed ? (col0 + orow) * a.ldo + row0 + ob : (row0 + orow) * a.ldo + col0 + ob;
        *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.out) + o) = v;
      }
    } else if (a.transposed) {  // out [N, K]: one output row (a column of the block) per wave pass
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = wave + 16 * i;
        const int64_t o = (col0 + c) * a.ldo + row0;
        store_out(a.out, a.out_dtype, o + lane, t[lane][c]);
        store_out(a.out, a.out_dtype, o + lane + 64, t[lane + 64][c]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = wave + 16 * i;
        const int64_t o = (row0 + r) * a.ldo + col0;
        store_out(a.out, a.out_dtype, o + lane, t[r][lane]);
        store_out(a.out, a.out_dtype, o + lane + 64, t[r][lane + 64]);
      }
    }
    __syncthreads();  // the tile is rewritten by the next block
  }
}

// ---------------------------------------------------------------- prefill --
// Row-wise 128-point rotation for the prefill form of the QSRT linear: one
// wave per (row, 128-column block), the block held as (lane, lane + 64), the
// wave-level Sylvester transform, scales applied before (PRE: the input's
// suh) or after it (the output's svh), and a power-of-two post factor.
// Without ROT it converts only.  All 64 lanes of a wave take the same row.
// An input of several planes (element stride `plane`) is their sum.
template <bool PRE, bool ROT>
__global__ __launch_bounds__(256) void rot_rows_kernel(const void* __restrict__ in, int in_dtype, int64_t ldi,
                                                       int64_t rows, const float* __restrict__ scale, float post,
                                                       void* __restrict__ out, int out_dtype, int64_t ldo,
                                                       int planes = 1, int64_t plane = 0) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t c = (int64_t)blockIdx.x * 128 + lane;
  float v0 = load_x(in, in_dtype, r * ldi + c), v1 = load_x(in, in_dtype, r * ldi + c + 64);
  // fp32 input split over planes (a split-K product): summed in plane order
  for (int p = 1; p < planes; ++p) {
    v0 += load_x(in, in_dtype, p * plane + r * ldi + c);
    v1 += load_x(in, in_dtype, p * plane + r * ldi + c + 64);
  }
  if (PRE && scale) {
    v0 *= scale[c];
    v1 *= scale[c + 64];
  }
  if (ROT) {
    fwht128(v0, v1, lane);
    v0 *= post;
    v1 *= post;
  }
  if (!PRE && scale) {
    v0 *= scale[c];
    v1 *= scale[c + 64];
  }
  store_out(out, out_dtype, r * ldo + c, v0);
  store_out(out, out_dtype, r * ldo + c + 64, v1);
}

// ------------------------------------------------------ routed experts --
// The routed expert forward of a decode batch with QSRT-coded experts, as
// two launches of the fused linear's workgroup (M = 1 row per job):
//   gate/up  job (pair p, matrix j in {w1, w3}, n block, K chunk):
//            h[p, j I + n] = x[t] . W_j(e)[:, n]          (fp32)
//   down     job (pair p, n block of the hidden, K chunk):
//            out[t, n] += sum_p w_p act(h_gate, h_up)[p] . W2(e)[:, n]
// with t = p / topk, e = route_ids[p] (ids outside [0, experts) contribute
// nothing) and act = SiTU / SwiGLU in fp32.  This is the expert MLP of
// scripts/closure_exl3_layer.py:557-598 on weights that
// scripts/stream_k3_pytorch.py:771-775 would decode to dense bf16 first;
// here nothing is decoded to memory and the intermediate stays fp32.  The
// route weight scales the down projection's activation row (linear), and
// the last workgroup of a (token, hidden block) sums every pair's and
// chunk's partial in a fixed order, so the result is deterministic.
struct MoeArgs {
  const void* x;
  int64_t ldx;
  const int* route_ids;
  const float* route_w;
  const kq_qsrt_matrix* mats;  // [experts][3]: w1, w3, w2
  const uint8_t* labels;
  float* h;         // [pairs][2 I]
  float* partial;   // gate/up: [pairs][2][chunks][I]; down: [pairs][chunks][H]
  int* counters;    // gate/up: [pairs][2][I / 128]; down: [tokens][H / 128]
  void* out;
  int64_t ldo, pairs;
  int topk, experts, hidden_tiles, inter_tiles, rate13_n, rate2_n, kbw, chunks, nbw, x_dtype, out_dtype;
  ActParams act;
};

// Stage this wave's tiles of k block kb of a matrix whose record prefix
// sums sit in device memory (prefix[r] = sum of the rates of records
// before r).
__device__ __forceinline__ void prefix_stage(const kq_qsrt_matrix& mt, int k_tiles, int n_tiles, int rate_n, int nb,
                                             int kb, uint32_t* stage, int wave, int lane) {
  const int record = __builtin_amdgcn_readfirstlane(rate_n ? nb : kb);
  const uint32_t p0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)mt.record_prefix[record]);
  const int bits = __builtin_amdgcn_readfirstlane((int)(mt.record_prefix[record + 1] - p0));
  const int64_t record_dw = (int64_t)RECORD_TILES * (rate_n ? k_tiles : n_tiles) * 8;
  stage_wave(reinterpret_cast<const uint32_t*>(mt.payload), (int64_t)p0 * record_dw, bits, rate_n, n_tiles, nb, kb,
             stage, wave, lane);
}

__device__ __forceinline__ int prefix_rate(const kq_qsrt_matrix& mt, int record) {
  record = __builtin_amdgcn_readfirstlane(record);
  return __builtin_amdgcn_readfirstlane((int)(mt.record_prefix[record + 1] - mt.record_prefix[record]));
}

// Sum the partial rows [first, first + count) of a 128-column block into
// dst (fp32 h row or the output in its dtype): 8 threads per column, thread
// r taking rows r, r + 8, ... (loads issued together), then a fixed tree.
__device__ __forceinline__ float sum_partials(const float* q, int64_t stride, int count, int tid) {
  const int r = tid & 7;
  float sum = 0.f;
  for (int i = r; i < count; i += 8)
    sum += __hip_atomic_load(q + (int64_t)i * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 4);
  return sum;
}

template <bool DOWN>
__global__ __launch_bounds__(LIN_THREADS) void moe_kernel(MoeArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lut[65536];
  __shared__ __attribute__((aligned(16))) uint32_t ring[LIN_STAGES][2048];  // 16 waves x 512 bytes
  __shared__ __attribute__((aligned(16))) float xs[lin_max_kb(1) * 128];
  __shared__ float yb[2][128];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = wave >> 3, ntl = wave & 7;
  const int I = a.inter_tiles * TILE;
  const int k_tiles = DOWN ? a.inter_tiles : a.hidden_tiles, n_tiles = DOWN ? a.hidden_tiles : a.inter_tiles;
  const int rate_n = DOWN ? a.rate2_n : a.rate13_n;
  const int n_blocks = n_tiles >> 3, k_blocks = k_tiles >> 3, N = n_tiles * TILE;
  const int n_groups = (n_blocks + a.nbw - 1) / a.nbw;
  int job = (int)blockIdx.x;
  const int chunk = job % a.chunks;
  job /= a.chunks;
  const int nb0 = (job % n_groups) * a.nbw;
  job /= n_groups;
  const int nbc = min(a.nbw, n_blocks - nb0);  // n blocks of this workgroup, one after the other
  const int j = DOWN ? 2 : job % 2;
  const int64_t p = DOWN ? job : job / 2;
  const int64_t t = p / a.topk;
  const int kb0 = chunk * a.kbw;
  const int kbn = min(a.kbw, k_blocks - kb0);
  const int total = nbc * kbn;  // (n block, k block) steps through the ring
  const int e = __builtin_amdgcn_readfirstlane(a.route_ids[p]);
  const bool valid = e >= 0 && e < a.experts;
  kq_qsrt_matrix mt{};
  if (valid) mt = a.mats[(int64_t)e * 3 + j];
  const uint8_t* labels = a.labels + (DOWN ? 3 * 65536 : 0);  // the down projection's rate axis has its own

  int lut_bits = 0;
  if (valid) {
    lut_bits = prefix_rate(mt, rate_n ? nb0 : kb0);
    stage_labels(labels, lut_bits, lut, wave, lane);
#pragma unroll
    for (int s = 0; s < LIN_STAGES; ++s)
      if (s < total) prefix_stage(mt, k_tiles, n_tiles, rate_n, nb0 + s / kbn, kb0 + s % kbn, ring[s], wave, lane);
    // the activation row of this chunk, rotated: one wave per k block
    for (int kbi = wave; kbi < kbn; kbi += 16) {
      const int64_t k = (int64_t)(kb0 + kbi) * 128 + lane;
      float v0, v1;
      if constexpr (DOWN) {
        const float* hp = a.h + p * 2 * I;
        const float wgt = a.route_w[p];
        v0 = activate(a.act, hp[k], hp[I + k]) * wgt;
        v1 = activate(a.act, hp[k + 64], hp[I + k + 64]) * wgt;
      } else {
        v0 = load_x(a.x, a.x_dtype, t * a.ldx + k);
        v1 = load_x(a.x, a.x_dtype, t * a.ldx + k + 64);
      }
      v0 *= mt.suh[k];
      v1 *= mt.suh[k + 64];
      fwht128(v0, v1, lane);
      xs[kbi * 128 + lane] = v0;
      xs[kbi * 128 + lane + 64] = v1;
    }
    wait_own_stage(min(LIN_STAGES, total));  // every wave's labels, then the activation row
    __syncthreads();
  }

  // output scales of the current n block, loaded a block ahead of use
  float sv0 = 0.f, sv1 = 0.f;
  if (valid) {
    sv0 = mt.svh[(int64_t)nb0 * 128 + lane] * (1.f / 128.f);
    sv1 = mt.svh[(int64_t)nb0 * 128 + lane + 64] * (1.f / 128.f);
  }
  float acc[1] = {0.f};
  int nbi = 0, kbi = 0;
  for (int u = 0; u < (valid ? total : nbc); ++u) {
    const int nb = nb0 + nbi;
    if (valid) {
      const int bits = prefix_rate(mt, rate_n ? nb : kb0 + kbi);
      if (bits != lut_bits) {  // the rate changed (uniform): restage the labels
        __syncthreads();
        stage_labels(labels, bits, lut, wave, lane);
        __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
        __syncthreads();
        lut_bits = bits;
      }
      wait_own_stage(min(LIN_STAGES - 1, total - 1 - u));
      accumulate_block<1>(ring[u % LIN_STAGES] + wave * 128, bits, lut, &xs[kbi * 128], 0, half, lane, acc);
      if (u + LIN_STAGES < total) {
        const int un = u + LIN_STAGES;
        prefix_stage(mt, k_tiles, n_tiles, rate_n, nb0 + un / kbn, kb0 + un % kbn, ring[u % LIN_STAGES], wave, lane);
      }
    }
    if (++kbi < kbn && valid) continue;
    // -------- n block nb done: rotate, scale, and hand over its partial --
    kbi = 0;
    ++nbi;
    column_sums<1>(acc);
    if ((lane & 6) == 0) yb[half][ntl * 16 + (lane >> 3) + 8 * (lane & 1)] = acc[0];
    acc[0] = 0.f;
    __syncthreads();
    const int64_t col0 = (int64_t)nb * 128;
    float v0 = 0.f, v1 = 0.f;
    if (wave == 0 && valid) {
      v0 = yb[0][lane] + yb[1][lane];
      v1 = yb[0][lane + 64] + yb[1][lane + 64];
      fwht128(v0, v1, lane);
      v0 *= sv0;
      v1 *= sv1;
    }
    if (valid && nbi < nbc) {  // the next n block's scales
      sv0 = mt.svh[col0 + 128 + lane] * (1.f / 128.f);
      sv1 = mt.svh[col0 + 128 + lane + 64] * (1.f / 128.f);
    }
    if (!DOWN && a.chunks == 1) {
      if (wave == 0) {
        float* hp = a.h + p * 2 * I + j * I + col0;
        hp[lane] = v0;
        hp[lane + 64] = v1;
      }
      __syncthreads();  // yb is rewritten by the next n block
      continue;
    }
    // partials through agent-scope atomics (written through / read past the
    // per-XCD L2s); the last workgroup of the output block sums them in order
    int64_t slot, first;
    int count;
    int* counter;
    if constexpr (DOWN) {
      slot = p * a.chunks + chunk;
      first = t * a.topk * a.chunks;
      count = a.topk * a.chunks;
      counter = a.counters + t * n_blocks + nb;
    } else {
      slot = (p * 2 + j) * a.chunks + chunk;
      first = (p * 2 + j) * a.chunks;
      count = a.chunks;
      counter = a.counters + (p * 2 + j) * n_blocks + nb;
    }
    if (wave == 0) {
      float* q = a.partial + slot * N + col0;
      __hip_atomic_store(q + lane, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(q + lane + 64, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // wave 0's partial stores have completed before the barrier that
    // precedes the count
    if (wave == 0) __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));
    __syncthreads();
    if (tid == 0) s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == count - 1;
    __syncthreads();
    if (s_last) {
      const float sum = sum_partials(a.partial + first * N + col0 + (tid >> 3), N, count, tid);
      if ((tid & 7) == 0) {
        const int c = tid >> 3;
        if constexpr (DOWN) store_out(a.out, a.out_dtype, t * a.ldo + col0 + c, sum);
        else a.h[p * 2 * I + j * I + col0 + c] = sum;
      }
      if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();  // s_last and yb are rewritten by the next n block
  }
}

}  // namespace qsrt
}  // namespace kq

using namespace kq::qsrt;

template <bool FROM_STATES>
static int launch_decode(const int16_t* src, int64_t k_tiles, int64_t n_tiles, int rate_axis, const RecordRates& rates,
                         const uint8_t* tile_bits, const uint8_t* labels, const float* suh, const float* svh,
                         int out_dtype, void* out, int64_t ldo, bool tr, hipStream_t st, const char* fn) {
  const dim3 grid((unsigned)(n_tiles / RECORD_TILES), (unsigned)(k_tiles / RECORD_TILES));
  const int t = tr ? 1 : 0;
  if (out_dtype == KQ_DT_F32)
    decode_kernel<2, FROM_STATES><<<grid, 256, 0, st>>>(src, k_tiles, n_tiles, rate_axis, rates, tile_bits, labels,
                                                        suh, svh, out, ldo, t);
  else if (out_dtype == KQ_DT_BF16)
    decode_kernel<0, FROM_STATES><<<grid, 256, 0, st>>>(src, k_tiles, n_tiles, rate_axis, rates, tile_bits, labels,
                                                        suh, svh, out, ldo, t);
  else
    decode_kernel<1, FROM_STATES><<<grid, 256, 0, st>>>(src, k_tiles, n_tiles, rate_axis, rates, tile_bits, labels,
                                                        suh, svh, out, ldo, t);
  return kq_check_launch(hipGetLastError(), fn);
}

extern "C" int kq_trellis_pack(const int16_t* symbols, int64_t tiles, int bits, int16_t* packed, void* stream) {
  if (bits < 2 || bits > 4) return kq_fail(KQ_ERR_INVALID, "kq_trellis_pack: QSRT supports K=2, K=3, or K=4");
  if (tiles < 0) return kq_fail(KQ_ERR_INVALID, "kq_trellis_pack: negative tile count");
  if (tiles == 0) return KQ_OK;
  if (!symbols || !packed) return kq_fail(KQ_ERR_INVALID, "kq_trellis_pack: null buffer");
  const int64_t n = tiles * TILE * bits;
  pack_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(symbols, tiles, bits, packed);
  return kq_check_launch(hipGetLastError(), "kq_trellis_pack");
}

extern "C" int kq_trellis_unpack(const int16_t* packed, int64_t tiles, int bits, int states, int16_t* out,
                                 void* stream) {
  if (bits < 2 || bits > 4) return kq_fail(KQ_ERR_INVALID, "kq_trellis_unpack: QSRT supports K=2, K=3, or K=4");
  if (tiles < 0) return kq_fail(KQ_ERR_INVALID, "kq_trellis_unpack: negative tile count");
  if (tiles == 0) return KQ_OK;
  if (!packed || !out || kq_misaligned(packed, 2))
    return kq_fail(KQ_ERR_INVALID, "kq_trellis_unpack: null or misaligned buffer");
  const int64_t n = tiles * 256;
  unpack_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(packed, tiles, bits, states ? 1 : 0,
                                                                             out);
  return kq_check_launch(hipGetLastError(), "kq_trellis_unpack");
}

extern "C" int kq_qsrt_decode_weight(const int16_t* payload, int64_t payload_words, int64_t k_tiles,
                                     int64_t n_tiles, int rate_axis, const uint8_t* record_bits,
                                     const uint8_t* labels, const float* suh,
                                     const float* svh, int out_dtype, void* out, int64_t ldo, uint32_t flags,
                                     void* stream) {
  const char* fn = "kq_qsrt_decode_weight";
  if (rate_axis != 0 && rate_axis != 1) return kq_fail(KQ_ERR_INVALID, "%s: rate_axis must be 0 (k) or 1 (n)", fn);
  if (flags & ~(uint32_t)KQ_QSRT_TRANSPOSED) return kq_fail(KQ_ERR_INVALID, "%s: unknown flags", fn);
  if (k_tiles <= 0 || n_tiles <= 0 || k_tiles % RECORD_TILES || n_tiles % RECORD_TILES)
    return kq_fail(KQ_ERR_INVALID, "%s: both dimensions must be positive multiples of 128 (%lld x %lld tiles)", fn,
                   (long long)k_tiles, (long long)n_tiles);
  if (k_tiles / RECORD_TILES > 65535 || n_tiles / RECORD_TILES > 65535)
    return kq_fail(KQ_ERR_LIMIT, "%s: too many blocks", fn);
  if (!payload || !record_bits || !labels || !out)
    return kq_fail(KQ_ERR_INVALID, "%s: null buffer", fn);
  if ((suh == nullptr) != (svh == nullptr)) return kq_fail(KQ_ERR_INVALID, "%s: give both suh and svh or neither", fn);
  if ((out_dtype < KQ_DT_BF16 || out_dtype > KQ_DT_F32) && out_dtype != OUT_E4M3)
    return kq_fail(KQ_ERR_INVALID, "%s: bad output dtype", fn);
  if (out_dtype == OUT_E4M3 && (suh || kq_misaligned(payload, 16) || kq_misaligned(labels, 16)))
    return kq_fail(KQ_ERR_INVALID, "%s: E4M3 bytes need the regularized weight and 16-byte aligned buffers", fn);
  const bool tr = flags & KQ_QSRT_TRANSPOSED;
  const int64_t rows = k_tiles * TILE, cols = n_tiles * TILE;
  if (ldo < (tr ? rows : cols)) return kq_fail(KQ_ERR_INVALID, "%s: ldo too small", fn);
  const int64_t records = (rate_axis ? n_tiles : k_tiles) / RECORD_TILES;
  if (records > MAX_RECORDS)
    return kq_fail(KQ_ERR_LIMIT, "%s: %lld records (at most %d)", fn, (long long)records, MAX_RECORDS);
  const int64_t per_record = (int64_t)RECORD_TILES * (rate_axis ? k_tiles : n_tiles);
  RecordRates rates{};
  int64_t words = 0;
  for (int64_t r = 0; r < records; ++r) {
    const int b = record_bits[r];
    rates.bits[r] = (uint8_t)b;
    if (b < 2 || b > 4) return kq_fail(KQ_ERR_INVALID, "%s: record %lld has rate %d (K2..K4 only)", fn, (long long)r, b);
    words += per_record * TILE * b;
  }
  if (words != payload_words)
    return kq_fail(KQ_ERR_INVALID, "%s: payload has %lld words, the records need %lld", fn,
                   (long long)payload_words, (long long)words);
  if (!kq_misaligned(payload, 16) && !kq_misaligned(labels, 16)) {
    // fast path: LDS labels and rotation; its 16-byte direct loads need a
    // 16-byte aligned payload and label table (record and tile offsets are
    // multiples of 16 bytes)
    LinRecords lr{};
    uint32_t sum = 0;
    for (int64_t r = 0; r < records; ++r) {
      if (r % 8 == 0) lr.prefix8[r / 8] = sum;
      lr.bits[r] = rates.bits[r];
      sum += rates.bits[r];
    }
    int dev = 0, cus = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return kq_check_launch(err, fn);
    // k blocks per workgroup: enough workgroups to fill the device once
    const int64_t n_blocks = n_tiles / RECORD_TILES, k_blocks = k_tiles / RECORD_TILES;
    int64_t kbw = (n_blocks * k_blocks + (cus > 0 ? cus : 1) - 1) / (cus > 0 ? cus : 1);
    kbw = kbw < 1 ? 1 : kbw > k_blocks ? k_blocks : kbw;
    const int64_t chunks = (k_blocks + kbw - 1) / kbw;
    DecArgs da{reinterpret_cast<const uint32_t*>(payload), labels, suh, svh, out, ldo, (int)k_tiles, (int)n_tiles,
               rate_axis, (int)kbw, tr ? 1 : 0, out_dtype,
               out_dtype == OUT_E4M3 && ldo % 4 == 0 && !kq_misaligned(out, 4) ? 1 : 0};
    const dim3 grid((unsigned)(n_blocks * chunks));
    if (suh) decode_fast_kernel<true><<<grid, LIN_THREADS, 0, (hipStream_t)stream>>>(da, lr);
    else decode_fast_kernel<false><<<grid, LIN_THREADS, 0, (hipStream_t)stream>>>(da, lr);
    return kq_check_launch(hipGetLastError(), fn);
  }
  return launch_decode<false>(payload, k_tiles, n_tiles, rate_axis, rates, nullptr, labels, suh, svh, out_dtype,
                              out, ldo, tr, (hipStream_t)stream, fn);
}

extern "C" int kq_qsrt_decode_states(const int16_t* states, int64_t k_tiles, int64_t n_tiles, int rate_axis,
                                     const uint8_t* tile_bits, const uint8_t* labels, const float* suh,
                                     const float* svh, int out_dtype, void* out, int64_t ldo, uint32_t flags,
                                     void* stream) {
  const char* fn = "kq_qsrt_decode_states";
  if (rate_axis != 0 && rate_axis != 1) return kq_fail(KQ_ERR_INVALID, "%s: rate_axis must be 0 (k) or 1 (n)", fn);
  if (flags & ~(uint32_t)KQ_QSRT_TRANSPOSED) return kq_fail(KQ_ERR_INVALID, "%s: unknown flags", fn);
  if (k_tiles <= 0 || n_tiles <= 0 || k_tiles % RECORD_TILES || n_tiles % RECORD_TILES)
    return kq_fail(KQ_ERR_INVALID, "%s: both dimensions must be positive multiples of 128 (%lld x %lld tiles)", fn,
                   (long long)k_tiles, (long long)n_tiles);
  if (k_tiles / RECORD_TILES > 65535 || n_tiles / RECORD_TILES > 65535)
    return kq_fail(KQ_ERR_LIMIT, "%s: too many blocks", fn);
  if (!states || !tile_bits || !labels || !out) return kq_fail(KQ_ERR_INVALID, "%s: null buffer", fn);
  if ((suh == nullptr) != (svh == nullptr)) return kq_fail(KQ_ERR_INVALID, "%s: give both suh and svh or neither", fn);
  if (out_dtype < KQ_DT_BF16 || out_dtype > KQ_DT_F32) return kq_fail(KQ_ERR_INVALID, "%s: bad output dtype", fn);
  const bool tr = flags & KQ_QSRT_TRANSPOSED;
  if (ldo < (tr ? k_tiles * TILE : n_tiles * TILE)) return kq_fail(KQ_ERR_INVALID, "%s: ldo too small", fn);
  return launch_decode<true>(states, k_tiles, n_tiles, rate_axis, RecordRates{}, tile_bits, labels, suh, svh,
                             out_dtype, out, ldo, tr, (hipStream_t)stream, fn);
}

// ---------------------------------------------------------- fused linear --
namespace {

struct LinPlan {
  int mt;      // rows per workgroup (1, 2, 4, 8 or 16)
  int groups;  // row groups
  int kbw;     // k blocks per workgroup
  int chunks;  // workgroups along K
  int64_t counters_bytes, partial_bytes;
};

// K chunk per workgroup: the least (rounds of workgroups) x (fixed cost of a
// workgroup + its k blocks), plus the cost of a cross-workgroup reduction
// when K is split (ties to the larger chunk: fewer partials to sum).  Costs
// in units of one k block of one workgroup (measured: about 1.3 us; a
// workgroup's fixed part, launch to last store, about 4 us; a
// cross-workgroup sum about 2.7 us through the completion counter, about
// 1.8 us polled).
constexpr int LIN_FIXED_KB = 3;
constexpr int LIN_REDUCE_KB = 2;
hipError_t lin_plan(int64_t m, int64_t k_tiles, int64_t n_tiles, LinPlan* p) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  p->mt = m >= 16 ? 16 : m >= 8 ? 8 : m >= 4 ? 4 : m >= 2 ? 2 : 1;
  if (p->mt < m && m < 16) p->mt *= 2;
  p->groups = (int)((m + p->mt - 1) / p->mt);
  const int64_t n_blocks = n_tiles / RECORD_TILES, k_blocks = k_tiles / RECORD_TILES;
  const int64_t slots = cus > 0 ? cus : 1;  // one 16-wave workgroup per CU
  int64_t best = -1;
  const int max_kb = lin_max_kb(p->mt);
  for (int kbw = 1; kbw <= max_kb; ++kbw) {
    const int64_t chunks = (k_blocks + kbw - 1) / kbw;
    const int64_t rounds = (n_blocks * chunks * p->groups + slots - 1) / slots;
    // time in units of one k block per workgroup; summing partials across
    // workgroups costs about LIN_REDUCE_KB more (store, count, reload)
    const int64_t cost = rounds * (LIN_FIXED_KB + kbw) + (chunks > 1 ? LIN_REDUCE_KB : 0);
    if (best < 0 || cost <= best) {
      best = cost;
      p->kbw = kbw;
      p->chunks = (int)chunks;
    }
  }
  // one or two rows per workgroup: partials of every chunk but the last,
  // polled by the last chunk's workgroup; more: every chunk's, and counters
  const bool polled = p->mt <= 2;
  p->counters_bytes = p->chunks > 1 && !polled ? ((int64_t)p->groups * n_blocks * 4 + 255) / 256 * 256 : 0;
  p->partial_bytes = p->chunks > 1 ? (int64_t)(p->chunks - (polled ? 1 : 0)) * m * n_tiles * TILE * 4 : 0;
  return hipSuccess;
}

template <int M>
void launch_linear_m(const LinArgs& a, const LinRecords& rec, bool rot, dim3 grid, hipStream_t st) {
  if (rot) linear_kernel<M, true><<<grid, LIN_THREADS, 0, st>>>(a, rec);
  else linear_kernel<M, false><<<grid, LIN_THREADS, 0, st>>>(a, rec);
}

}  // namespace

// Rows from which kq_qsrt_linear takes the prefill form: the fused kernel
// decodes the weight once per 16 rows, so past two row groups one decode to
// E4M3 label bytes plus the MXFP8 MFMA linear is faster.
static constexpr int64_t PREFILL_ROWS = 33;

// Prefill workspace: rotated activations xr [m, K] (fp32, or bf16 for bf16
// x), the regularized weight's E4M3 bytes [N, K] (an MXFP8 matrix whose
// block scales are all 1, which the linear takes without a scale array),
// the product y fp32 as `slices` K-slice planes [m, N] (split K when the
// output tiles alone would leave CUs idle), and the three-term bf16 split of
// fp32 rows [m, 3K].
struct PrefillLayout {
  int64_t xr, w, y, split, total, split_bytes;
  int slices;
};

static PrefillLayout prefill_layout(int64_t m, int64_t k, int64_t n, bool f32) {
  auto al = [](int64_t v) { return (v + 255) / 256 * 256; };
  PrefillLayout L{};
  L.split_bytes = f32 ? m * 3 * k * 2 : 0;
  L.slices = kq::mx_linear_slices(m, n, (f32 ? 3 * k : k) / 64);
  int64_t o = 0;
  L.xr = o;    o = al(o + m * k * (f32 ? 4 : 2));
  L.w = o;     o = al(o + n * k);
  L.y = o;     o = al(o + m * n * 4 * L.slices);
  L.split = o; o = al(o + L.split_bytes);
  L.total = o;
  return L;
}

extern "C" int64_t kq_qsrt_linear_workspace_size(int64_t m, int64_t k_tiles, int64_t n_tiles) {
  if (m <= 0 || k_tiles <= 0 || n_tiles <= 0 || k_tiles % RECORD_TILES || n_tiles % RECORD_TILES) return 0;
  if (m >= PREFILL_ROWS) return prefill_layout(m, k_tiles * TILE, n_tiles * TILE, true).total;
  LinPlan p;
  if (lin_plan(m, k_tiles, n_tiles, &p) != hipSuccess) return -1;
  return p.counters_bytes + p.partial_bytes;
}

// x @ W for prefill-sized row counts: xr = (x o suh) B_K (unscaled
// transform; bf16 x gives bf16 xr, f16 / fp32 x fp32 xr), W_reg decoded once
// to its E4M3 label bytes [N, K] (exact: W_reg is an MXFP8 matrix with unit
// scales), y = xr W_reg^T on the MXFP8 MFMA linear (fp32 accumulation; fp32
// xr through the exact three-term bf16 split; split over K into planes when
// the output tiles are too few for the CUs), out = (sum of the planes B_N) /
// 128 o svh.
// Without suh / svh the matrix is W_reg itself and both rotations are plain
// conversions.  Argument checks are the caller's.
static int qsrt_prefill(const void* x, int x_dtype, int64_t m, int64_t ldx, const int16_t* payload,
                        int64_t payload_words, int64_t k_tiles, int64_t n_tiles, int rate_axis,
                        const uint8_t* record_bits, const uint8_t* labels, const float* suh, const float* svh,
                        int out_dtype, void* out, int64_t ldo, void* workspace, int64_t ws_bytes, hipStream_t st,
                        const char* fn) {
  const int64_t K = k_tiles * TILE, N = n_tiles * TILE;
  const bool f32 = x_dtype != KQ_DT_BF16;
  const PrefillLayout L = prefill_layout(m, K, N, f32);
  if (L.split_bytes < 0) return kq_fail(KQ_ERR_INVALID, "%s: bad sizes for the prefill product", fn);
  if (!workspace || ws_bytes < L.total || kq_misaligned(workspace, 256))
    return kq_fail(KQ_ERR_INVALID, "%s: workspace needs %lld bytes (256-byte aligned) for %lld rows", fn,
                   (long long)L.total, (long long)m);
  if ((m + 3) / 4 > 65535) return kq_fail(KQ_ERR_LIMIT, "%s: too many rows (%lld)", fn, (long long)m);
  unsigned char* w = static_cast<unsigned char*>(workspace);
  void* xr = w + L.xr;
  uint8_t* wq = w + L.w;
  float* y = reinterpret_cast<float*>(w + L.y);
  const bool rot = suh != nullptr;
  const int xr_dtype = f32 ? KQ_DT_F32 : KQ_DT_BF16;
  const dim3 gin((unsigned)(K / 128), (unsigned)((m + 3) / 4));
  if (rot) rot_rows_kernel<true, true><<<gin, 256, 0, st>>>(x, x_dtype, ldx, m, suh, 1.f, xr, xr_dtype, K);
  else rot_rows_kernel<true, false><<<gin, 256, 0, st>>>(x, x_dtype, ldx, m, nullptr, 1.f, xr, xr_dtype, K);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return kq_check_launch(e, fn);
  int rc = kq_qsrt_decode_weight(payload, payload_words, k_tiles, n_tiles, rate_axis, record_bits, labels, nullptr,
                                 nullptr, OUT_E4M3, wq, K, KQ_QSRT_TRANSPOSED, st);
  if (rc != KQ_OK) return rc;
  if (!kq::mx_linear_planes_ok(f32 ? 3 * K : K, K))
    return kq_fail(KQ_ERR_LIMIT, "%s: %lld rows exceed the prefill product's operand range", fn, (long long)m);
  const uint16_t* a_rows = static_cast<const uint16_t*>(xr);
  if (f32) {
    uint16_t* a3 = reinterpret_cast<uint16_t*>(w + L.split);
    if ((e = kq::split3_rows(static_cast<const float*>(xr), K, m, K, a3, st)) != hipSuccess)
      return kq_check_launch(e, fn);
    a_rows = a3;
  }
  e = kq::mx_linear_planes_unit(a_rows, f32 ? 3 * K : K, wq, y, N, m * N, (int)m, (int)N, (int)(f32 ? 3 * K : K),
                                (int)K, L.slices, st);
  if (e != hipSuccess) return kq_check_launch(e, fn);
  const dim3 gout((unsigned)(N / 128), (unsigned)((m + 3) / 4));
  if (rot)
    rot_rows_kernel<false, true><<<gout, 256, 0, st>>>(y, KQ_DT_F32, N, m, svh, 1.f / 128.f, out, out_dtype, ldo,
                                                       L.slices, m * N);
  else
    rot_rows_kernel<false, false><<<gout, 256, 0, st>>>(y, KQ_DT_F32, N, m, nullptr, 1.f, out, out_dtype, ldo,
                                                        L.slices, m * N);
  return kq_check_launch(hipGetLastError(), fn);
}

extern "C" int kq_qsrt_linear(const void* x, int x_dtype, int64_t m, int64_t ldx, const int16_t* payload,
                              int64_t payload_words, int64_t k_tiles, int64_t n_tiles, int rate_axis,
                              const uint8_t* record_bits, const uint8_t* labels, const float* suh, const float* svh,
                              int out_dtype, void* out, int64_t ldo, void* workspace, int64_t ws_bytes,
                              void* stream) {
  const char* fn = "kq_qsrt_linear";
  if (rate_axis != 0 && rate_axis != 1) return kq_fail(KQ_ERR_INVALID, "%s: rate_axis must be 0 (k) or 1 (n)", fn);
  if (m < 0) return kq_fail(KQ_ERR_INVALID, "%s: negative row count", fn);
  if (k_tiles <= 0 || n_tiles <= 0 || k_tiles % RECORD_TILES || n_tiles % RECORD_TILES)
    return kq_fail(KQ_ERR_INVALID, "%s: both dimensions must be positive multiples of 128 (%lld x %lld tiles)", fn,
                   (long long)k_tiles, (long long)n_tiles);
  if (x_dtype < KQ_DT_BF16 || x_dtype > KQ_DT_F32 || out_dtype < KQ_DT_BF16 || out_dtype > KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "%s: bad activation or output dtype", fn);
  if ((suh == nullptr) != (svh == nullptr)) return kq_fail(KQ_ERR_INVALID, "%s: give both suh and svh or neither", fn);
  const int64_t rows = k_tiles * TILE, cols = n_tiles * TILE;
  if (m == 0) return KQ_OK;
  if (!x || !payload || !record_bits || !labels || !out) return kq_fail(KQ_ERR_INVALID, "%s: null buffer", fn);
  if (kq_misaligned(payload, 16) || kq_misaligned(labels, 16))
    return kq_fail(KQ_ERR_INVALID, "%s: payload and labels must be 16-byte aligned", fn);
  if (ldx < rows || ldo < cols) return kq_fail(KQ_ERR_INVALID, "%s: ldx or ldo too small", fn);
  const int64_t records = (rate_axis ? n_tiles : k_tiles) / RECORD_TILES;
  if (records > MAX_RECORDS)
    return kq_fail(KQ_ERR_LIMIT, "%s: %lld records (at most %d)", fn, (long long)records, MAX_RECORDS);
  const int64_t per_record = (int64_t)RECORD_TILES * (rate_axis ? k_tiles : n_tiles);
  LinRecords rec{};
  int64_t words = 0;
  uint32_t sum = 0;
  for (int64_t r = 0; r < records; ++r) {
    const int b = record_bits[r];
    if (b < 2 || b > 4) return kq_fail(KQ_ERR_INVALID, "%s: record %lld has rate %d (K2..K4 only)", fn, (long long)r, b);
    if (r % 8 == 0) rec.prefix8[r / 8] = sum;
    rec.bits[r] = (uint8_t)b;
    sum += (uint32_t)b;
    words += per_record * TILE * b;
  }
  if (words != payload_words)
    return kq_fail(KQ_ERR_INVALID, "%s: payload has %lld words, the records need %lld", fn,
                   (long long)payload_words, (long long)words);
  if (m >= PREFILL_ROWS)
    return qsrt_prefill(x, x_dtype, m, ldx, payload, payload_words, k_tiles, n_tiles, rate_axis, record_bits,
                        labels, suh, svh, out_dtype, out, ldo, workspace, ws_bytes, (hipStream_t)stream, fn);
  LinPlan p;
  hipError_t e = lin_plan(m, k_tiles, n_tiles, &p);
  if (e != hipSuccess) return kq_check_launch(e, fn);
  const int64_t need = p.counters_bytes + p.partial_bytes;
  if (need > 0 && (!workspace || ws_bytes < need || kq_misaligned(workspace, 256)))
    return kq_fail(KQ_ERR_INVALID, "%s: workspace needs %lld bytes (256-byte aligned, zeroed before first use)", fn,
                   (long long)need);
  const int64_t n_blocks = n_tiles / RECORD_TILES;
  if (n_blocks * p.chunks > 0x7fffffff || p.groups > 65535)
    return kq_fail(KQ_ERR_LIMIT, "%s: too many workgroups", fn);
  LinArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.m = m;
  a.payload = reinterpret_cast<const uint32_t*>(payload);
  a.labels = labels;
  a.suh = suh;
  a.svh = svh;
  a.out = out;
  a.ldo = ldo;
  a.counters = p.counters_bytes > 0 ? static_cast<int*>(workspace) : nullptr;
  a.partial = need > 0 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.counters_bytes) : nullptr;
  a.k_tiles = (int)k_tiles;
  a.n_tiles = (int)n_tiles;
  a.rate_n = rate_axis;
  a.kbw = p.kbw;
  a.chunks = p.chunks;
  a.x_dtype = x_dtype;
  a.out_dtype = out_dtype;
  const dim3 grid((unsigned)(n_blocks * p.chunks), (unsigned)p.groups);
  const bool rot = suh != nullptr;
  const hipStream_t st = (hipStream_t)stream;
  switch (p.mt) {
    case 1: launch_linear_m<1>(a, rec, rot, grid, st); break;
    case 2: launch_linear_m<2>(a, rec, rot, grid, st); break;
    case 4: launch_linear_m<4>(a, rec, rot, grid, st); break;
    case 8: launch_linear_m<8>(a, rec, rot, grid, st); break;
    default: launch_linear_m<16>(a, rec, rot, grid, st); break;
  }
  return kq_check_launch(hipGetLastError(), fn);
}

// --------------------------------------------------------- routed experts --
namespace {

struct MoePlan {
  int kbw13, chunks13, nbw13, kbw2, chunks2, nbw2;
  int64_t h_bytes, part13_bytes, part2_bytes, cnt13_bytes, cnt2_bytes;
};

int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

// Same cost model as the single linear, with nbw n blocks walked one after
// the other by a workgroup (sharing its activation row and labels).
void moe_chunking(int64_t jobs, int64_t n_blocks, int64_t k_blocks, int64_t slots, bool sum_anyway, int* kbw_out,
                  int* chunks_out, int* nbw_out) {
  int64_t best = -1;
  const int64_t max_kb = k_blocks < lin_max_kb(1) ? k_blocks : lin_max_kb(1);
  for (int nbw = 1; nbw <= n_blocks && nbw <= 32; ++nbw) {
    const int64_t groups = (n_blocks + nbw - 1) / nbw;
    for (int kbw = 1; kbw <= max_kb; ++kbw) {
      const int64_t chunks = (k_blocks + kbw - 1) / kbw;
      const int64_t rounds = (jobs * groups * chunks + slots - 1) / slots;
      const int64_t cost = rounds * (LIN_FIXED_KB + (int64_t)nbw * kbw) +
                           (!sum_anyway && chunks > 1 ? LIN_REDUCE_KB : 0);
      if (best < 0 || cost < best || (cost == best && kbw * nbw > *kbw_out * *nbw_out)) {
        best = cost;
        *kbw_out = kbw;
        *chunks_out = (int)chunks;
        *nbw_out = nbw;
      }
    }
  }
}

hipError_t moe_plan(int64_t tokens, int topk, int64_t hidden_tiles, int64_t inter_tiles, MoePlan* p) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int64_t slots = cus > 0 ? cus : 1;
  const int64_t pairs = tokens * topk, H = hidden_tiles * TILE, I = inter_tiles * TILE;
  moe_chunking(pairs * 2, inter_tiles / RECORD_TILES, hidden_tiles / RECORD_TILES, slots, false, &p->kbw13,
               &p->chunks13, &p->nbw13);
  moe_chunking(pairs, hidden_tiles / RECORD_TILES, inter_tiles / RECORD_TILES, slots, true, &p->kbw2, &p->chunks2,
               &p->nbw2);
  p->h_bytes = align256(pairs * 2 * I * 4);
  p->part13_bytes = p->chunks13 > 1 ? align256(pairs * 2 * p->chunks13 * I * 4) : 0;
  p->part2_bytes = align256(pairs * p->chunks2 * H * 4);
  p->cnt13_bytes = p->chunks13 > 1 ? align256(pairs * 2 * (inter_tiles / RECORD_TILES) * 4) : 0;
  p->cnt2_bytes = align256(tokens * (hidden_tiles / RECORD_TILES) * 4);
  return hipSuccess;
}

}  // namespace

extern "C" int64_t kq_qsrt_moe_workspace_size(int64_t tokens, int topk, int64_t hidden_tiles, int64_t inter_tiles) {
  if (tokens <= 0 || topk <= 0 || hidden_tiles <= 0 || inter_tiles <= 0 || hidden_tiles % RECORD_TILES ||
      inter_tiles % RECORD_TILES)
    return 0;
  MoePlan p;
  if (moe_plan(tokens, topk, hidden_tiles, inter_tiles, &p) != hipSuccess) return -1;
  return p.h_bytes + p.part13_bytes + p.part2_bytes + p.cnt13_bytes + p.cnt2_bytes;
}

extern "C" int kq_qsrt_moe_decode(int act, float beta, float linear_beta, const void* x, int x_dtype, int64_t tokens,
                                  int64_t ldx, const int32_t* route_ids, const float* route_weights, int topk,
                                  const kq_qsrt_matrix* mats, int experts, int64_t hidden_tiles, int64_t inter_tiles,
                                  int rate13_axis, int rate2_axis, const uint8_t* labels, int out_dtype, void* out,
                                  int64_t ldo, void* workspace, int64_t ws_bytes, void* stream) {
  const char* fn = "kq_qsrt_moe_decode";
  if (act != KQ_ACT_SITU && act != KQ_ACT_SWIGLU) return kq_fail(KQ_ERR_INVALID, "%s: unknown activation", fn);
  if (tokens < 0 || topk <= 0 || experts <= 0) return kq_fail(KQ_ERR_INVALID, "%s: bad tokens, topk or experts", fn);
  if (hidden_tiles <= 0 || inter_tiles <= 0 || hidden_tiles % RECORD_TILES || inter_tiles % RECORD_TILES)
    return kq_fail(KQ_ERR_INVALID, "%s: hidden and intermediate sizes must be positive multiples of 128", fn);
  if ((rate13_axis != 0 && rate13_axis != 1) || (rate2_axis != 0 && rate2_axis != 1))
    return kq_fail(KQ_ERR_INVALID, "%s: rate axes must be 0 (k) or 1 (n)", fn);
  if (x_dtype < KQ_DT_BF16 || x_dtype > KQ_DT_F32 || out_dtype < KQ_DT_BF16 || out_dtype > KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "%s: bad activation or output dtype", fn);
  if (act == KQ_ACT_SITU && !(beta > 0.f && linear_beta > 0.f))
    return kq_fail(KQ_ERR_INVALID, "%s: SiTU betas must be positive", fn);
  const int64_t H = hidden_tiles * TILE;
  if (ldx < H || ldo < H) return kq_fail(KQ_ERR_INVALID, "%s: ldx or ldo too small", fn);
  if (tokens == 0) return KQ_OK;
  if (!x || !route_ids || !route_weights || !mats || !labels || !out)
    return kq_fail(KQ_ERR_INVALID, "%s: null buffer", fn);
  if (kq_misaligned(labels, 16))  // staged into LDS by 16-byte direct loads
    return kq_fail(KQ_ERR_INVALID, "%s: labels must be 16-byte aligned", fn);
  MoePlan p;
  hipError_t err = moe_plan(tokens, topk, hidden_tiles, inter_tiles, &p);
  if (err != hipSuccess) return kq_check_launch(err, fn);
  const int64_t need = p.h_bytes + p.part13_bytes + p.part2_bytes + p.cnt13_bytes + p.cnt2_bytes;
  if (!workspace || ws_bytes < need || kq_misaligned(workspace, 256))
    return kq_fail(KQ_ERR_INVALID, "%s: workspace needs %lld bytes (256-byte aligned, zeroed before first use)", fn,
                   (long long)need);
  const int64_t pairs = tokens * topk;
  const int64_t groups13 = (inter_tiles / RECORD_TILES + p.nbw13 - 1) / p.nbw13;
  const int64_t groups2 = (hidden_tiles / RECORD_TILES + p.nbw2 - 1) / p.nbw2;
  const int64_t jobs13 = pairs * 2 * groups13 * p.chunks13;
  const int64_t jobs2 = pairs * groups2 * p.chunks2;
  if (jobs13 > 0x7fffffff || jobs2 > 0x7fffffff) return kq_fail(KQ_ERR_LIMIT, "%s: too many workgroups", fn);
  char* ws = static_cast<char*>(workspace);
  MoeArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.route_ids = route_ids;
  a.route_w = route_weights;
  a.mats = mats;
  a.labels = labels;
  a.h = reinterpret_cast<float*>(ws);
  a.out = out;
  a.ldo = ldo;
  a.pairs = pairs;
  a.topk = topk;
  a.experts = experts;
  a.hidden_tiles = (int)hidden_tiles;
  a.inter_tiles = (int)inter_tiles;
  a.rate13_n = rate13_axis;
  a.rate2_n = rate2_axis;
  a.x_dtype = x_dtype;
  a.out_dtype = out_dtype;
  a.act = kq::ActParams{act, beta, linear_beta};
  const hipStream_t st = (hipStream_t)stream;
  MoeArgs g = a;
  g.kbw = p.kbw13;
  g.chunks = p.chunks13;
  g.nbw = p.nbw13;
  g.partial = reinterpret_cast<float*>(ws + p.h_bytes);
  g.counters = reinterpret_cast<int*>(ws + p.h_bytes + p.part13_bytes + p.part2_bytes);
  moe_kernel<false><<<(unsigned)jobs13, LIN_THREADS, 0, st>>>(g);
  if ((err = hipGetLastError()) != hipSuccess) return kq_check_launch(err, fn);
  MoeArgs d = a;
  d.kbw = p.kbw2;
  d.chunks = p.chunks2;
  d.nbw = p.nbw2;
  d.partial = reinterpret_cast<float*>(ws + p.h_bytes + p.part13_bytes);
  d.counters = reinterpret_cast<int*>(ws + p.h_bytes + p.part13_bytes + p.part2_bytes + p.cnt13_bytes);
  moe_kernel<true><<<(unsigned)jobs2, LIN_THREADS, 0, st>>>(d);
  return kq_check_launch(hipGetLastError(), fn);
}
