// MX codec kernels: quantize (dense -> E4M3/E2M1 codes + E8M0 scales),
// dequantize, and nibble pack/unpack.  All are HBM-bound streaming kernels:
// each lane moves one 16-byte vector of the dense side per step and the four
// lanes of a quad own one 32-element block, so the block max is two DPP
// quad permutes and the stores of a wave cover one contiguous range.
#include "kq_common.h"
#include "kq_internal.h"

namespace kq {

// -------------------------------------------------------------- quantize --
// IN: 0 bf16, 1 f16, 2 f32.  FMT: 0 MXFP8-E4M3, 1 MXFP4-E2M1.
// HW: use the gfx950 scaled convert instructions (round to nearest even,
// saturating), otherwise the bit-level software rounding.
typedef uint32_t u32x4_q __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_q __attribute__((ext_vector_type(2)));

// One lane's 16-byte (16-bit inputs) or 32-byte (fp32) share of a block.
template <int IN>
struct QChunk {
  u32x4_q d[IN == 2 ? 2 : 1];
};

template <int IN>
__device__ __forceinline__ QChunk<IN> load_qchunk(const void* __restrict__ in, int64_t elem) {
  QChunk<IN> c;
  if (IN == 2) {
    const u32x4_q* p = reinterpret_cast<const u32x4_q*>(static_cast<const float*>(in) + elem);
    c.d[0] = __builtin_nontemporal_load(p);
    c.d[1] = __builtin_nontemporal_load(p + 1);
  } else {
    c.d[0] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_q*>(static_cast<const uint16_t*>(in) + elem));
  }
  return c;
}

// Quantize one lane's 8 elements of block `blk` (part = lane within the quad
// that owns the block) and store its codes, and the block's scale from part 0.
template <int IN, int FMT, bool HW>
__device__ __forceinline__ void quantize_qchunk(const QChunk<IN>& ch, int64_t blk, int part,
                                                uint8_t* __restrict__ out_q,
                                                uint8_t* __restrict__ out_scale) {
  // 8 elements of this lane as fp32 and, for 16-bit inputs, their raw pairs.
  float x[8];
  uint32_t raw[4];
  if (IN == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = __uint_as_float(ch.d[0][i]);
      x[4 + i] = __uint_as_float(ch.d[1][i]);
    }
  } else {
    raw[0] = ch.d[0][0]; raw[1] = ch.d[0][1]; raw[2] = ch.d[0][2]; raw[3] = ch.d[0][3];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (IN == 0) {
        x[2 * i] = bf16_bits_to_f32(raw[i] & 0xffffu);
        x[2 * i + 1] = bf16_bits_to_f32(raw[i] >> 16);
      } else {
        x[2 * i] = f16_bits_to_f32(raw[i] & 0xffffu);
        x[2 * i + 1] = f16_bits_to_f32(raw[i] >> 16);
      }
    }
  }

  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = quad_max(amax);

  const float qmax = FMT == 0 ? 448.0f : 6.0f;
  const int e = IN == 2 ? mx_block_exponent_f32_log2(amax, qmax) : mx_block_exponent<FMT>(amax);
  const uint32_t sbyte = (uint32_t)(e + 127);
  if (part == 0) out_scale[blk] = (uint8_t)sbyte;

  // The convert instructions read the E8M0 byte from the exponent field of
  // their fp32 scale operand and divide by 2^(byte-127).  Byte 255 (only for
  // an infinite amax) is the E8M0 NaN there, so that block takes the
  // software path.
  const bool hw = HW && sbyte != 255u;
  if (FMT == 0) {
    uint32_t w0 = 0, w1 = 0;
    if (hw) {
      const float sc = __uint_as_float(sbyte << 23);
      short2_t r0 = {0, 0}, r1 = {0, 0};
      if (IN == 0) {
        r0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r0, __builtin_bit_cast(bf16x2_t, raw[0]), sc, false);
        r0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r0, __builtin_bit_cast(bf16x2_t, raw[1]), sc, true);
        r1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r1, __builtin_bit_cast(bf16x2_t, raw[2]), sc, false);
        r1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r1, __builtin_bit_cast(bf16x2_t, raw[3]), sc, true);
      } else if (IN == 1) {
        r0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r0, __builtin_bit_cast(f16x2_t, raw[0]), sc, false);
        r0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r0, __builtin_bit_cast(f16x2_t, raw[1]), sc, true);
        r1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r1, __builtin_bit_cast(f16x2_t, raw[2]), sc, false);
        r1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r1, __builtin_bit_cast(f16x2_t, raw[3]), sc, true);
      } else {
        r0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r0, x[0], x[1], sc, false);
        r0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r0, x[2], x[3], sc, true);
        r1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r1, x[4], x[5], sc, false);
        r1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r1, x[6], x[7], sc, true);
      }
      w0 = __builtin_bit_cast(uint32_t, r0);
      w1 = __builtin_bit_cast(uint32_t, r1);
    } else {
      const float inv = mx_inv_scale(e);
      uint32_t c[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float y = x[i] * inv;
        y = __builtin_amdgcn_fmed3f(y, -448.0f, 448.0f);
        c[i] = f32_to_e4m3_rne(y);
      }
      w0 = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
      w1 = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
    }
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 o = {w0, w1};
    __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(out_q + blk * 32 + part * 8));
  } else {
    uint32_t w = 0;
    if (hw) {
      const float sc = __uint_as_float(sbyte << 23);
      if (IN == 0) {
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(w, __builtin_bit_cast(bf16x2_t, raw[0]), sc, 0);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(w, __builtin_bit_cast(bf16x2_t, raw[1]), sc, 1);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(w, __builtin_bit_cast(bf16x2_t, raw[2]), sc, 2);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(w, __builtin_bit_cast(bf16x2_t, raw[3]), sc, 3);
      } else if (IN == 1) {
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f16(w, __builtin_bit_cast(f16x2_t, raw[0]), sc, 0);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f16(w, __builtin_bit_cast(f16x2_t, raw[1]), sc, 1);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f16(w, __builtin_bit_cast(f16x2_t, raw[2]), sc, 2);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f16(w, __builtin_bit_cast(f16x2_t, raw[3]), sc, 3);
      } else {
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, x[0], x[1], sc, 0);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, x[2], x[3], sc, 1);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, x[4], x[5], sc, 2);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, x[6], x[7], sc, 3);
      }
    } else {
      const float inv = mx_inv_scale(e);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float y = x[i] * inv;
        y = __builtin_amdgcn_fmed3f(y, -6.0f, 6.0f);
        w |= f32_to_e2m1_rne(y) << (4 * i);
      }
    }
    __builtin_nontemporal_store(w, reinterpret_cast<uint32_t*>(out_q + blk * 16 + part * 4));
  }
}

// Each thread handles ITERS chunks 256 apart (a wave covers 16 consecutive
// blocks per step, so every load and store of a wave is one contiguous
// range); all loads are issued before the first block is converted.  With
// contiguous rows the input offset is the chunk index times 8 elements, so
// no division by the row length is needed.  Measured on MI355X (cold):
// MXFP8 at cfg2 is fastest with 2 (6.32 TB/s; 1: 5.78, 4: 6.01), MXFP4 at
// cfg1 with 4 (8.44 us; 2: 8.75, 8: 9.65).
template <int FMT> constexpr int quant_iters() { return FMT == 1 ? 4 : 2; }

template <int IN, int FMT, bool HW, bool CONTIG>
__global__ __launch_bounds__(256) void mx_quantize_kernel(
    const void* __restrict__ in, int64_t ld_in, int64_t nblk, int64_t total_blocks,
    uint8_t* __restrict__ out_q, uint8_t* __restrict__ out_scale) {
  constexpr int QUANT_ITERS = quant_iters<FMT>();
  const int64_t c0 = (int64_t)blockIdx.x * (256 * QUANT_ITERS) + threadIdx.x;
  QChunk<IN> v[QUANT_ITERS];
#pragma unroll
  for (int it = 0; it < QUANT_ITERS; ++it) {
    const int64_t c = c0 + it * 256;
    const int64_t blk = c >> 2;
    if (blk < total_blocks) {  // whole quads are in or out together
      int64_t elem;
      if (CONTIG) {
        elem = c * 8;
      } else {
        const int64_t row = blk / nblk;
        elem = row * ld_in + (blk - row * nblk) * 32 + (c & 3) * 8;
      }
      v[it] = load_qchunk<IN>(in, elem);
    }
  }
#pragma unroll
  for (int it = 0; it < QUANT_ITERS; ++it) {
    const int64_t c = c0 + it * 256;
    const int64_t blk = c >> 2;
    if (blk < total_blocks) quantize_qchunk<IN, FMT, HW>(v[it], blk, (int)(c & 3), out_q, out_scale);
  }
}

// ------------------------------------------------------------ dequantize --
// OUT: 0 bf16, 1 f16, 2 f32.  Each lane expands 8 codes of one block.
template <int FMT, int OUT, bool HW>
__global__ __launch_bounds__(256) void mx_dequant_kernel(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ scale,
    int64_t total_blocks, void* __restrict__ out) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t blk = g >> 2;
  const int part = (int)(g & 3);
  if (blk >= total_blocks) return;
  const uint32_t sb = scale[blk];
  const int64_t e0 = blk * 32 + part * 8;  // first element of this lane

  float v[8];
  if (FMT == 1) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(q + (e0 >> 1));
    if (HW && sb != 255u) {
      const float sc = __uint_as_float(sb << 23);
      float2_t r0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 0);
      float2_t r1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 1);
      float2_t r2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 2);
      float2_t r3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 3);
      v[0] = r0[0]; v[1] = r0[1]; v[2] = r1[0]; v[3] = r1[1];
      v[4] = r2[0]; v[5] = r2[1]; v[6] = r3[0]; v[7] = r3[1];
    } else {
      const float s = e8m0_to_f32(sb);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = e2m1_to_f32((w >> (4 * i)) & 0xfu) * s;
    }
  } else {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 w = *reinterpret_cast<const u32x2*>(q + e0);
    if (HW && sb != 255u) {
      const float sc = __uint_as_float(sb << 23);
      float2_t r0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[0], sc, false);
      float2_t r1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[0], sc, true);
      float2_t r2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[1], sc, false);
      float2_t r3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[1], sc, true);
      v[0] = r0[0]; v[1] = r0[1]; v[2] = r1[0]; v[3] = r1[1];
      v[4] = r2[0]; v[5] = r2[1]; v[6] = r3[0]; v[7] = r3[1];
    } else {
      const float s = e8m0_to_f32(sb);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = e4m3_to_f32((w[i >> 2] >> (8 * (i & 3))) & 0xffu) * s;
    }
  }

  if (OUT == 2) {
    float4_t* p = reinterpret_cast<float4_t*>(static_cast<float*>(out) + e0);
    float4_t a = {v[0], v[1], v[2], v[3]};
    float4_t b = {v[4], v[5], v[6], v[7]};
    __builtin_nontemporal_store(a, p);
    __builtin_nontemporal_store(b, p + 1);
  } else {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = OUT == 0 ? f32x2_to_bf16x2_bits(v[2 * i], v[2 * i + 1])
                      : f32x2_to_f16x2_bits(v[2 * i], v[2 * i + 1]);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + e0));
  }
}

// ------------------------------------------------------ nibble (un)pack --
__global__ __launch_bounds__(256) void unpack_codes_kernel(
    const uint8_t* __restrict__ packed, int64_t n_packed, uint8_t* __restrict__ codes) {
  const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;  // 4 packed bytes
  if (i4 >= n_packed) return;
  if (i4 + 4 <= n_packed) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(packed + i4);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 o;
    // byte j of w -> codes 2j (low nibble), 2j+1 (high nibble)
    const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    o[0] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    o[1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    *reinterpret_cast<u32x2*>(codes + 2 * i4) = o;
  } else {
    for (int64_t j = i4; j < n_packed; ++j) {
      const uint32_t b = packed[j];
      codes[2 * j] = (uint8_t)(b & 0xfu);
      codes[2 * j + 1] = (uint8_t)(b >> 4);
    }
  }
}

__global__ __launch_bounds__(256) void pack_codes_kernel(
    const uint8_t* __restrict__ codes, int64_t n_packed, uint8_t* __restrict__ packed) {
  const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i4 >= n_packed) return;
  if (i4 + 4 <= n_packed) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 c = *reinterpret_cast<const u32x2*>(codes + 2 * i4);
    // even bytes are the low nibbles, odd bytes are shifted up by 4 (mod 256)
    const uint32_t ev = __builtin_amdgcn_perm(c[1], c[0], 0x06040200u);
    const uint32_t od = __builtin_amdgcn_perm(c[1], c[0], 0x07050301u);
    const uint32_t w = ev | ((od << 4) & 0xf0f0f0f0u);
    *reinterpret_cast<uint32_t*>(packed + i4) = w;
  } else {
    for (int64_t j = i4; j < n_packed; ++j)
      packed[j] = (uint8_t)(codes[2 * j] | (uint8_t)(codes[2 * j + 1] << 4));
  }
}

// ------------------------------------------------------ byte decoding --
// table 0: E8M0 scale 2^(b-127); 1: E2M1 code value (codes >= 16 -> NaN);
// 2: float8_e4m3fn value.  OUT: 0 bf16, 1 f16, 2 f32 (exact for every table
// value that the output type can hold).
template <int TABLE, int OUT>
__global__ __launch_bounds__(256) void decode_bytes_kernel(
    const uint8_t* __restrict__ in, int64_t n, void* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint32_t b = in[i];
  float v;
  if (TABLE == 0) v = e8m0_to_f32(b);
  else if (TABLE == 1) v = b < 16u ? e2m1_to_f32(b) : __uint_as_float(0x7fc00000u);
  else v = e4m3_to_f32(b);
  if (OUT == 2) static_cast<float*>(out)[i] = v;
  else if (OUT == 0) static_cast<__bf16*>(out)[i] = (__bf16)v;
  else static_cast<_Float16*>(out)[i] = (_Float16)v;
}

// ------------------------------------------------- MFMA-tiled weight layout --
// One 1 KiB tile per (16-row group rg, 128-column chunk c) of an MXFP4 matrix:
// byte 16*l + j of the tile is packed[16 rg + l % 16][64 c + 16 (l / 16) + j],
// i.e. exactly the B fragment lane l of v_mfma_scale_f32_16x16x128_f8f6f4
// reads (16 rows x 4 E8M0 blocks), and scale tile byte l is
// scale[16 rg + l % 16][4 c + l / 16].  Tiles are stored [rg][c], so a wave
// streaming one row group reads contiguous 1 KiB pieces.
__global__ __launch_bounds__(256) void mx_tile_kernel(const uint8_t* __restrict__ q,
                                                      const uint8_t* __restrict__ s, int64_t rows,
                                                      int64_t k, uint8_t* __restrict__ qt,
                                                      uint8_t* __restrict__ st) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (rg, c, l)
  const int64_t nc = k / 128;
  const int64_t total = rows / 16 * nc * 64;
  if (t >= total) return;
  const int l = (int)(t & 63);
  const int64_t tile = t >> 6;
  const int64_t rg = tile / nc, c = tile - rg * nc;
  const int64_t row = 16 * rg + (l & 15);
  const int g = l >> 4;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  *reinterpret_cast<u32x4*>(qt + 16 * t) =
      *reinterpret_cast<const u32x4*>(q + row * (k / 2) + 64 * c + 16 * g);
  if (st) st[t] = s[row * (k / 32) + 4 * c + g];
}

}  // namespace kq

using namespace kq;

template <int TABLE>
static hipError_t launch_decode(int out_dtype, const uint8_t* in, int64_t n, void* out,
                                hipStream_t st) {
  const dim3 grid((unsigned)((n + 255) / 256));
  if (out_dtype == KQ_DT_F32) decode_bytes_kernel<TABLE, 2><<<grid, 256, 0, st>>>(in, n, out);
  else if (out_dtype == KQ_DT_BF16) decode_bytes_kernel<TABLE, 0><<<grid, 256, 0, st>>>(in, n, out);
  else decode_bytes_kernel<TABLE, 1><<<grid, 256, 0, st>>>(in, n, out);
  return hipGetLastError();
}

extern "C" int kq_decode_bytes(int table, const uint8_t* in, int64_t n, int out_dtype, void* out,
                               void* stream) {
  if (table < KQ_TABLE_E8M0 || table > KQ_TABLE_E4M3)
    return kq_fail(KQ_ERR_INVALID, "kq_decode_bytes: unknown table %d", table);
  if (out_dtype < KQ_DT_BF16 || out_dtype > KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "kq_decode_bytes: unknown output dtype %d", out_dtype);
  if (n < 0) return kq_fail(KQ_ERR_INVALID, "kq_decode_bytes: negative size");
  if (n == 0) return KQ_OK;
  if ((n + 255) / 256 > (int64_t)0x7fffffff)
    return kq_fail(KQ_ERR_LIMIT, "kq_decode_bytes: %lld bytes is too many", (long long)n);
  hipStream_t st = (hipStream_t)stream;
  hipError_t err = table == KQ_TABLE_E8M0 ? launch_decode<0>(out_dtype, in, n, out, st)
                 : table == KQ_TABLE_E2M1 ? launch_decode<1>(out_dtype, in, n, out, st)
                                          : launch_decode<2>(out_dtype, in, n, out, st);
  return kq_check_launch(err, "kq_decode_bytes");
}

template <int IN, int FMT>
static hipError_t launch_quantize(bool hw, const void* in, int64_t ld, int64_t nblk,
                                  int64_t total, void* oq, uint8_t* os, hipStream_t st) {
  const int64_t chunks = total * 4;
  constexpr int QUANT_ITERS = quant_iters<FMT>();
  const dim3 grid((unsigned)((chunks + 256 * QUANT_ITERS - 1) / (256 * QUANT_ITERS)));
  const bool contig = ld == nblk * 32;
  uint8_t* q = (uint8_t*)oq;
  if (hw && contig)
    mx_quantize_kernel<IN, FMT, true, true><<<grid, 256, 0, st>>>(in, ld, nblk, total, q, os);
  else if (hw)
    mx_quantize_kernel<IN, FMT, true, false><<<grid, 256, 0, st>>>(in, ld, nblk, total, q, os);
  else if (contig)
    mx_quantize_kernel<IN, FMT, false, true><<<grid, 256, 0, st>>>(in, ld, nblk, total, q, os);
  else
    mx_quantize_kernel<IN, FMT, false, false><<<grid, 256, 0, st>>>(in, ld, nblk, total, q, os);
  return hipGetLastError();
}

extern "C" int kq_mx_quantize(int fmt, int in_dtype, const void* in, int64_t ld_in,
                              int64_t rows, int64_t k, void* out_q, uint8_t* out_scale,
                              uint32_t flags, void* stream) {
  if (fmt != KQ_FMT_MXFP8_E4M3 && fmt != KQ_FMT_MXFP4_E2M1)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_quantize: unknown format %d", fmt);
  if (in_dtype < KQ_DT_BF16 || in_dtype > KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_quantize: unknown input dtype %d", in_dtype);
  if (rows < 0 || k < 0 || k % 32 != 0)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_quantize: need rows >= 0 and k %% 32 == 0 (k=%lld)",
                   (long long)k);
  if (ld_in < k)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_quantize: ld_in %lld < k %lld", (long long)ld_in,
                   (long long)k);
  const int esz = in_dtype == KQ_DT_F32 ? 4 : 2;
  if ((ld_in * esz) % 16 != 0 || kq_misaligned(in, 16) || kq_misaligned(out_q, 8))
    return kq_fail(KQ_ERR_INVALID,
                   "kq_mx_quantize: input rows must be 16-byte aligned and out_q 8-byte aligned");
  if (rows == 0 || k == 0) return KQ_OK;
  const int64_t nblk = k / 32, total = rows * nblk;
  if (total * 4 / 256 + 1 > (int64_t)0x7fffffff)
    return kq_fail(KQ_ERR_LIMIT, "kq_mx_quantize: %lld blocks is too many", (long long)total);
  const bool hw = (flags & KQ_FLAG_SOFTWARE_CVT) == 0;
  hipStream_t st = (hipStream_t)stream;
  hipError_t err;
  if (fmt == KQ_FMT_MXFP8_E4M3) {
    err = in_dtype == KQ_DT_BF16 ? launch_quantize<0, 0>(hw, in, ld_in, nblk, total, out_q, out_scale, st)
        : in_dtype == KQ_DT_F16  ? launch_quantize<1, 0>(hw, in, ld_in, nblk, total, out_q, out_scale, st)
                                 : launch_quantize<2, 0>(hw, in, ld_in, nblk, total, out_q, out_scale, st);
  } else {
    err = in_dtype == KQ_DT_BF16 ? launch_quantize<0, 1>(hw, in, ld_in, nblk, total, out_q, out_scale, st)
        : in_dtype == KQ_DT_F16  ? launch_quantize<1, 1>(hw, in, ld_in, nblk, total, out_q, out_scale, st)
                                 : launch_quantize<2, 1>(hw, in, ld_in, nblk, total, out_q, out_scale, st);
  }
  return kq_check_launch(err, "kq_mx_quantize");
}

template <int FMT, int OUT>
static hipError_t launch_dequant(bool hw, const uint8_t* q, const uint8_t* s, int64_t total,
                                 void* out, hipStream_t st) {
  const dim3 grid((unsigned)((total * 4 + 255) / 256));
  if (hw)
    mx_dequant_kernel<FMT, OUT, true><<<grid, 256, 0, st>>>(q, s, total, out);
  else
    mx_dequant_kernel<FMT, OUT, false><<<grid, 256, 0, st>>>(q, s, total, out);
  return hipGetLastError();
}

extern "C" int kq_mx_dequant(int fmt, const void* q, const uint8_t* scale, int64_t rows,
                             int64_t k, int out_dtype, void* out, uint32_t flags,
                             void* stream) {
  if (fmt != KQ_FMT_MXFP8_E4M3 && fmt != KQ_FMT_MXFP4_E2M1)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_dequant: unknown format %d", fmt);
  if (out_dtype < KQ_DT_BF16 || out_dtype > KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_dequant: unknown output dtype %d", out_dtype);
  if (rows < 0 || k < 0 || k % 32 != 0)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_dequant: need rows >= 0 and k %% 32 == 0 (k=%lld)",
                   (long long)k);
  if (kq_misaligned(q, fmt == KQ_FMT_MXFP8_E4M3 ? 8 : 4) || kq_misaligned(out, 16))
    return kq_fail(KQ_ERR_INVALID, "kq_mx_dequant: misaligned codes or output");
  if (rows == 0 || k == 0) return KQ_OK;
  const int64_t total = rows * (k / 32);
  if (total * 4 / 256 + 1 > (int64_t)0x7fffffff)
    return kq_fail(KQ_ERR_LIMIT, "kq_mx_dequant: %lld blocks is too many", (long long)total);
  const bool hw = (flags & KQ_FLAG_SOFTWARE_CVT) == 0;
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* qb = (const uint8_t*)q;
  hipError_t err;
  if (fmt == KQ_FMT_MXFP8_E4M3) {
    err = out_dtype == KQ_DT_BF16 ? launch_dequant<0, 0>(hw, qb, scale, total, out, st)
        : out_dtype == KQ_DT_F16  ? launch_dequant<0, 1>(hw, qb, scale, total, out, st)
                                  : launch_dequant<0, 2>(hw, qb, scale, total, out, st);
  } else {
    err = out_dtype == KQ_DT_BF16 ? launch_dequant<1, 0>(hw, qb, scale, total, out, st)
        : out_dtype == KQ_DT_F16  ? launch_dequant<1, 1>(hw, qb, scale, total, out, st)
                                  : launch_dequant<1, 2>(hw, qb, scale, total, out, st);
  }
  return kq_check_launch(err, "kq_mx_dequant");
}

extern "C" int kq_mx_tile_weights(const uint8_t* q, const uint8_t* scale, int64_t mats,
                                  int64_t rows, int64_t k, uint8_t* q_tiled, uint8_t* scale_tiled,
                                  void* stream) {
  if (mats < 0 || rows < 0 || k < 0 || rows % 16 != 0 || k % 128 != 0)
    return kq_fail(KQ_ERR_INVALID,
                   "kq_mx_tile_weights: rows must be a multiple of 16 and k of 128 (rows=%lld k=%lld)",
                   (long long)rows, (long long)k);
  if (kq_misaligned(q, 16) || kq_misaligned(q_tiled, 16))
    return kq_fail(KQ_ERR_INVALID, "kq_mx_tile_weights: packed buffers must be 16-byte aligned");
  if (!scale != !scale_tiled)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_tile_weights: scale and scale_tiled must both be given or both NULL");
  const int64_t per = rows / 16 * (k / 128) * 64;  // lane slots per matrix
  if (per == 0 || mats == 0) return KQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const unsigned grid = (unsigned)((per + 255) / 256);
  for (int64_t m = 0; m < mats; ++m) {
    mx_tile_kernel<<<grid, 256, 0, st>>>(q + m * rows * (k / 2), scale ? scale + m * rows * (k / 32) : nullptr,
                                         rows, k, q_tiled + m * per * 16,
                                         scale_tiled ? scale_tiled + m * per : nullptr);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kq_check_launch(e, "kq_mx_tile_weights");
  }
  return KQ_OK;
}

extern "C" int kq_unpack_codes(const uint8_t* packed, int64_t n_packed, uint8_t* codes,
                               void* stream) {
  if (n_packed < 0) return kq_fail(KQ_ERR_INVALID, "kq_unpack_codes: negative size");
  if (kq_misaligned(packed, 4) || kq_misaligned(codes, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_unpack_codes: misaligned buffers");
  if (n_packed == 0) return KQ_OK;
  const dim3 grid((unsigned)(((n_packed + 3) / 4 + 255) / 256));
  unpack_codes_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(packed, n_packed, codes);
  return kq_check_launch(hipGetLastError(), "kq_unpack_codes");
}

extern "C" int kq_pack_codes(const uint8_t* codes, int64_t n_codes, uint8_t* packed,
                             void* stream) {
  if (n_codes < 0 || n_codes % 2 != 0)
    return kq_fail(KQ_ERR_INVALID, "kq_pack_codes: K must be even (got %lld codes)",
                   (long long)n_codes);
  if (kq_misaligned(packed, 4) || kq_misaligned(codes, 8))
    return kq_fail(KQ_ERR_INVALID, "kq_pack_codes: misaligned buffers");
  const int64_t n_packed = n_codes / 2;
  if (n_packed == 0) return KQ_OK;
  const dim3 grid((unsigned)(((n_packed + 3) / 4 + 255) / 256));
  pack_codes_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(codes, n_packed, packed);
  return kq_check_launch(hipGetLastError(), "kq_pack_codes");
}
