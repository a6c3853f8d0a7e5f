/* TEST INFRASTRUCTURE ONLY - CPU oracle of the SQG trellis quantizer.
 *
 * A restatement of the tail-biting Viterbi search of
 * kquant/csrc/qsrt_quantize_tiles_kernel.cuh:21-471 with the SQG E4M3 labels
 * of kquant/csrc/sqg_quantize.cu:15-125 (the "sqg" path of
 * kquant/sqg_quantizer.py:64-164), in exact fp16 arithmetic:
 *
 *   states are 16-bit windows of the K-bit edge stream; node = the low
 *   16 - K bits; node o at a step is reached from the 2^K nodes
 *   (o >> K) + k 2^(16-2K) with state (k << (16-K)) | o;
 *   w = fp16(x_i); d = fp16(label(state) - w);
 *   cost = fp16(d * d) on a pass's first step (every predecessor but the
 *   forced one at +inf on the closing pass), else fp16(fma(d, d, prev));
 *   each node keeps the first predecessor k with the strictly smallest cost;
 *   argmin over the costs of the primer's second-to-last step (the buffer
 *   the reference reads): smallest cost, ties to the smallest key
 *   (bitrev5(e % 1024 / 32), bitrev5(e % 32), e / 1024) - the order the
 *   kernel's shuffle-down reductions produce;
 *   primer over positions -ctx .. ctx-1 recording decisions of 0 .. ctx-1,
 *   traceback to the node before position 0; closing pass over 0 .. 255
 *   from that node; traceback writes every position's state and label.
 *
 * The procedural control codebooks (quantize_tiles_procedural_cuda,
 * kquant/csrc/sqg_quantize.cu:261-330) run the same search on labels
 * computed per state by the EXL3 decoders of
 * kquant/csrc/exl3_compat/quant/codebook.cuh:
 *   MCG (1, :50-59 and :64-79): x = state * 0xCBAC1FED mod 2^32, then
 *     x = (x & 0x8fff8fff) ^ 0x3b603b60 (lop3 with truth table 0x6a =
 *     (a & b) ^ c), label = fp16(lo + hi) of x's two halves read as fp16;
 *   MUL1 (2, :27-47 and :80-92): x = state * 0x83DCD12D mod 2^32, h = the
 *     fp16 with bits 0x6400 + (sum of x's four bytes) = 1024 + that sum,
 *     label = fp16(h * fp16(0x1eee) + fp16(0xc931)) rounded once (hfma).
 *
 * fp16 values are kept as their bit patterns; every operation is computed
 * exactly in double and rounded once to fp16 (nearest, ties to even,
 * subnormals kept, overflow to +inf), which is the IEEE result. */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static double f16_to_f64(uint16_t h) {
  const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  double v;
  if (e == 0) v = ldexp((double)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexp((double)(1024 + m), e - 25);
  return s ? -v : v;
}

/* Round a double to the nearest fp16 (ties to even). */
static uint16_t f64_to_f16(double x) {
  uint16_t sign = 0;
  if (x < 0 || (x == 0 && signbit(x))) { sign = 0x8000; x = -x; }
  if (isnan(x)) return 0x7e00;
  if (x >= 65520.0) return sign | 0x7c00;  /* 65504 + half ulp rounds to inf */
  if (x < ldexp(1.0, -14)) {               /* subnormal range: units of 2^-24 */
    const double q = x * 16777216.0;
    double r = floor(q);
    const double frac = q - r;
    if (frac > 0.5 || (frac == 0.5 && fmod(r, 2.0) == 1.0)) r += 1.0;
    return sign | (uint16_t)r;             /* r == 1024 is the smallest normal */
  }
  int e;
  const double f = frexp(x, &e);           /* x = f 2^e, f in [0.5, 1) */
  const double q = ldexp(f, 11);           /* 11 significant bits */
  double r = floor(q);
  const double frac = q - r;
  if (frac > 0.5 || (frac == 0.5 && fmod(r, 2.0) == 1.0)) r += 1.0;
  if (r == 2048.0) { r = 1024.0; e += 1; }
  const int be = e - 1 + 15;
  if (be >= 31) return sign | 0x7c00;
  return sign | (uint16_t)(be << 10) | (uint16_t)((int)r - 1024);
}

static uint16_t f32_to_f16(float x) { return f64_to_f16((double)x); }

static uint16_t e4m3_to_f16(uint8_t b) {
  const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  double v = e == 0 ? ldexp((double)m, -9) : ldexp((double)(8 + m), e - 10);
  return f64_to_f16(s ? -v : v);
}

static int less16(uint16_t a, uint16_t b) { return f16_to_f64(a) < f16_to_f64(b); }

static int bitrev5(int v) {
  int r = 0;
  for (int i = 0; i < 5; ++i) r |= ((v >> i) & 1) << (4 - i);
  return r;
}

/* tie order of the argmin: smaller key wins among equal costs */
static int64_t argmin_key(int e) {
  return ((int64_t)bitrev5((e & 1023) >> 5) << 40) | ((int64_t)bitrev5(e & 31) << 32) | (int64_t)(e >> 10);
}

typedef struct {
  int K, edges;
  const uint16_t* lab;  /* fp16 label of every state */
  const uint16_t* w;    /* the tile, fp16 */
  uint16_t* prev;
  uint16_t* cur;
  uint8_t* dec;         /* [256][edges] */
} Trellis;

static void forward(Trellis* t, int roll, int steps, int pre_state, int trace_start) {
  const int K = t->K, edges = t->edges, kr = 16 - K, pstep = 1 << (16 - 2 * K);
  for (int i = 0; i < steps; ++i) {
    const int ri = (i + roll) & 255;
    const double w = f16_to_f64(t->w[ri]);
    uint16_t* tmp = t->prev; t->prev = t->cur; t->cur = tmp;  /* prev now holds the last costs */
    for (int o = 0; o < edges; ++o) {
      int in = o >> K;
      uint16_t best = 0;
      int best_k = 0;
      for (int k = 0; k < (1 << K); ++k, in += pstep) {
        const uint16_t d = f64_to_f16(f16_to_f64(t->lab[(k << kr) | o]) - w);
        const double dd = f16_to_f64(d);
        uint16_t err;
        if (i == 0) {
          err = f64_to_f16(dd * dd);
          if (pre_state >= 0 && in != pre_state) err = 0x7c00;
        } else {
          err = f64_to_f16(dd * dd + f16_to_f64(t->prev[in]));
        }
        if (k == 0) { best = err; best_k = 0; }
        else if (less16(err, best)) { best = err; best_k = k; }
      }
      t->cur[o] = best;
      if (i >= trace_start) t->dec[(size_t)ri * edges + o] = (uint8_t)best_k;
    }
  }
}

/* The reference's argmin reads its "incoming" cost buffer, which after a
 * pass holds the costs of the pass's second-to-last step
 * (qsrt_quantize_tiles_kernel.cuh:343-352 read temp_costs_inc after the
 * swaps of :75-79 and :202-204); entries at +inf are never selected. */
static int argmin_edges(const uint16_t* c, int edges) {
  int best = -1;
  for (int e = 0; e < edges; ++e) {
    if (c[e] == 0x7c00) continue;
    if (best < 0 || less16(c[e], c[best]) || (c[e] == c[best] && argmin_key(e) < argmin_key(best)))
      best = e;
  }
  return best < 0 ? 0 : best;
}

static int argmin_cost(const Trellis* t) { return argmin_edges(t->prev, t->edges); }

/* The argmin alone, for its tests: index of the smallest of `edges` fp16
 * costs (non-negative or +inf) under the tie order above. */
int sqgo_argmin_edges(const uint16_t* costs, int edges) { return argmin_edges(costs, edges); }

static uint16_t procedural_label(int codebook, uint32_t state) {
  if (codebook == 1) {
    const uint32_t x = ((state * 0xCBAC1FEDu) & 0x8fff8fffu) ^ 0x3b603b60u;
    return f64_to_f16(f16_to_f64((uint16_t)(x & 0xffffu)) + f16_to_f64((uint16_t)(x >> 16)));
  }
  const uint32_t x = state * 0x83DCD12Du;
  const uint32_t sum = (x & 0xffu) + ((x >> 8) & 0xffu) + ((x >> 16) & 0xffu) + (x >> 24);
  const double h = f16_to_f64((uint16_t)(0x6400u + sum));
  return f64_to_f16(h * f16_to_f64(0x1eee) + f16_to_f64(0xc931));
}

/* fp16 labels of all 65536 states of procedural codebook 1 (MCG) or 2 (MUL1) */
void sqgo_procedural_labels(int codebook, uint16_t* out) {
  for (uint32_t s = 0; s < 65536; ++s) out[s] = procedural_label(codebook, s);
}

/* The search against fp16 labels in state order. */
void sqgo_quantize_tiles_f16(const float* tiles, int64_t n, const uint16_t* lab, int K, int ctx, float* out_tiles,
                             int16_t* out_states) {
  const int edges = 65536 >> K;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t tile = 0; tile < n; ++tile) {
    uint16_t w[256];
    Trellis t;
    t.K = K;
    t.edges = edges;
    t.lab = lab;
    t.w = w;
    t.prev = (uint16_t*)calloc(edges, sizeof(uint16_t));
    t.cur = (uint16_t*)calloc(edges, sizeof(uint16_t));
    t.dec = (uint8_t*)calloc((size_t)256 * edges, 1);
    for (int i = 0; i < 256; ++i) w[i] = f32_to_f16(tiles[tile * 256 + i]);
    /* primer */
    forward(&t, 256 - ctx, 2 * ctx, -1, ctx);
    int edge = argmin_cost(&t);
    for (int i = 2 * ctx - 1; i >= 0; --i) {
      const int ri = (i + 256 - ctx) & 255;
      const int decision = t.dec[(size_t)ri * edges + edge];
      edge = (decision << (16 - 2 * K)) | (edge >> K);
      if (ri == 0) break;
    }
    const int end_state = edge;
    forward(&t, 0, 256, end_state, 0);
    edge = end_state;
    for (int i = 255; i >= 0; --i) {
      const int decision = t.dec[(size_t)i * edges + edge];
      const int prev = (decision << (16 - 2 * K)) | (edge >> K);
      const int state = ((prev << K) | edge) & 0xffff;
      out_states[tile * 256 + i] = (int16_t)(uint16_t)state;
      out_tiles[tile * 256 + i] = (float)f16_to_f64(lab[state]);
      edge = prev;
    }
    free(t.prev);
    free(t.cur);
    free(t.dec);
  }
}

void sqgo_quantize_tiles(const float* tiles, int64_t n, const uint8_t* lut, int K, int ctx, float* out_tiles,
                         int16_t* out_states) {
  uint16_t* lab = (uint16_t*)malloc(65536 * sizeof(uint16_t));
  for (int s = 0; s < 65536; ++s) lab[s] = e4m3_to_f16(lut[s]);
  sqgo_quantize_tiles_f16(tiles, n, lab, K, ctx, out_tiles, out_states);
  free(lab);
}

/* The fp16 rounding the restatement uses, for its own tests. */
void sqgo_f64_to_f16(const double* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = f64_to_f16(x[i]);
}
