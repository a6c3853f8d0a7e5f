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
#include "kq_hadamard.h"
#include "kq_internal.h"

namespace kq {
namespace qsrt {

using had::fwht_lines;
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
  if (out_dtype < KQ_DT_BF16 || out_dtype > KQ_DT_F32) return kq_fail(KQ_ERR_INVALID, "%s: bad output dtype", fn);
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
