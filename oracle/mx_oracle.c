/*
 * TEST INFRASTRUCTURE ONLY.  CPU restatement of kquant's MX codec, used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker.  Nothing in the kquant_amd product path links or calls it.
 *
 * Each function follows the reference formula step by step, in fp32 as torch
 * does, and rounds to E4M3 / E2M1 by searching the table of representable
 * values (nearest value, ties to the even code), which is a different method
 * from the bit arithmetic of the HIP kernels.
 *
 *   mxo_quantize      kquant/mxfp8.py:34-50  (MXFP8 rule; MXFP4 = same rule
 *                     with E2M1 and 6.0, kquant has no MXFP4 quantizer)
 *   mxo_dequant       kquant/io/mxfp4.py:41-64 and kquant/mxfp8.py:79-84
 *   mxo_pack/unpack   kquant/io/mxfp4.py:19-38
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float f32_from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* value of a float8_e4m3fn byte (0x7f/0xff: NaN) */
float mxo_e4m3_value(uint32_t byte) {
  uint32_t e = (byte >> 3) & 15u, m = byte & 7u;
  float v;
  if ((byte & 0x7fu) == 0x7fu) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
  return (byte & 0x80u) ? -v : v;
}

static const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

float mxo_e2m1_value(uint32_t code) {
  float v = kE2M1[code & 7u];
  return (code & 8u) ? -v : v;
}

/* nearest entry of an ascending table of n magnitudes, ties to even index */
static uint32_t nearest_even(const float* tab, int n, float a) {
  int lo = 0, hi = n - 1;
  if (a >= tab[hi]) return (uint32_t)hi;
  while (hi - lo > 1) {  /* tab[lo] <= a < tab[hi] */
    int mid = (lo + hi) / 2;
    if (tab[mid] <= a) lo = mid; else hi = mid;
  }
  double dl = (double)a - tab[lo], dh = (double)tab[hi] - a;
  if (dl < dh) return (uint32_t)lo;
  if (dh < dl) return (uint32_t)hi;
  return (lo % 2 == 0) ? (uint32_t)lo : (uint32_t)hi;
}

static float g_e4m3_mag[127];
static int g_tables_ready = 0;
static void init_tables(void) {
  if (g_tables_ready) return;
  for (int c = 0; c < 127; ++c) g_e4m3_mag[c] = mxo_e4m3_value((uint32_t)c);
  g_tables_ready = 1;
}

/* torch's fp32 -> float8_e4m3fn cast: nearest, ties to even.  The code after
 * 448 (0x7e) is NaN, so magnitudes past the 448/480 midpoint 464 are NaN and
 * 464 itself ties to the even code 0x7e. */
uint32_t mxo_f32_to_e4m3(float y) {
  init_tables();
  uint32_t sign = (bits_from_f32(y) >> 24) & 0x80u;
  float a = fabsf(y);
  if (isnan(y) || a > 464.0f) return sign | 0x7fu;
  return sign | nearest_even(g_e4m3_mag, 127, a);
}

uint32_t mxo_f32_to_e2m1(float y) {
  uint32_t sign = (bits_from_f32(y) >> 28) & 0x8u;
  return sign | nearest_even(kE2M1, 8, fabsf(y));
}

static float load_elem(const void* in, int dtype, int64_t i) {
  if (dtype == 2) return ((const float*)in)[i];
  uint16_t h = ((const uint16_t*)in)[i];
  if (dtype == 0) return f32_from_bits((uint32_t)h << 16);
  /* fp16 -> fp32 (exact) */
  uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf(1.0f + (float)m / 1024.0f, (int)e - 15);
  return s ? -v : v;
}

/* fmt 0: MXFP8 (E4M3, 448); fmt 1: MXFP4 (E2M1, 6).  dtype 0 bf16, 1 f16,
 * 2 f32.  Input [rows, k] with row stride ld; outputs contiguous. */
void mxo_quantize(int fmt, int dtype, const void* in, int64_t ld, int64_t rows, int64_t k,
                  uint8_t* out_q, uint8_t* out_scale) {
  const float qmax = fmt == 0 ? 448.0f : 6.0f;
  const int64_t nblk = k / 32;
  init_tables();
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < nblk; ++b) {
      float x[32];
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) {
        x[i] = load_elem(in, dtype, r * ld + b * 32 + i);
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
      }
      /* exponent = ceil(log2(amax.clamp(min=1e-30) / E4M3_MAX)).clamp(-127, 128) */
      float clamped = amax < 1e-30f ? 1e-30f : amax;
      float e = ceilf(log2f(clamped / qmax));
      if (e < -127.0f) e = -127.0f;
      if (e > 128.0f) e = 128.0f;
      out_scale[r * nblk + b] = (uint8_t)(int)(e + 127.0f);
      float div = ldexpf(1.0f, (int)e);  /* exp2(exponent); 2^128 -> inf */
      for (int i = 0; i < 32; ++i) {
        float y = x[i] / div;
        if (y < -qmax) y = -qmax;
        if (y > qmax) y = qmax;
        if (fmt == 0) {
          out_q[r * k + b * 32 + i] = (uint8_t)mxo_f32_to_e4m3(y);
        } else {
          uint32_t c = mxo_f32_to_e2m1(y);
          int64_t j = r * (k / 2) + b * 16 + i / 2;
          if (i % 2 == 0) out_q[j] = (uint8_t)c;
          else out_q[j] = (uint8_t)(out_q[j] | (c << 4));
        }
      }
    }
  }
}

/* element-wise torch fp32 -> float8_e4m3fn cast over an array */
void mxo_cast_e4m3(const float* in, int64_t n, uint8_t* out) {
  init_tables();
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)mxo_f32_to_e4m3(in[i]);
}

void mxo_cast_e2m1(const float* in, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)mxo_f32_to_e2m1(in[i]);
}

/* scale_factors: exp2(float(s) - 127) in fp32 */
float mxo_scale_value(uint32_t s) {
  if (s == 255u) return INFINITY;
  return ldexpf(1.0f, (int)s - 127);
}

/* fp32 output [rows, k] */
void mxo_dequant(int fmt, const uint8_t* q, const uint8_t* scale, int64_t rows, int64_t k,
                 float* out) {
  const int64_t nblk = k / 32;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < nblk; ++b) {
      const float s = mxo_scale_value(scale[r * nblk + b]);
      for (int64_t i = b * 32; i < b * 32 + 32; ++i) {
        float v;
        if (fmt == 0) v = mxo_e4m3_value(q[r * k + i]);
        else {
          uint8_t byte = q[r * (k / 2) + i / 2];
          v = mxo_e2m1_value(i % 2 == 0 ? (byte & 15u) : (byte >> 4));
        }
        out[r * k + i] = v * s;
      }
    }
}

void mxo_unpack_codes(const uint8_t* packed, int64_t n, uint8_t* codes) {
  for (int64_t i = 0; i < n; ++i) {
    codes[2 * i] = packed[i] & 0x0f;
    codes[2 * i + 1] = packed[i] >> 4;
  }
}

void mxo_pack_codes(const uint8_t* codes, int64_t n_codes, uint8_t* packed) {
  for (int64_t i = 0; i < n_codes / 2; ++i)
    packed[i] = (uint8_t)(codes[2 * i] | (uint8_t)(codes[2 * i + 1] << 4));
}
