/*
 * kquant_amd — C ABI of the MI355X (gfx950) block-scaled quantization hot path.
 *
 * Every entry point takes raw device pointers, int64 sizes and a HIP stream
 * (passed as void*, a hipStream_t; NULL = the legacy default stream), launches
 * asynchronously on that stream, allocates nothing, and returns KQ_OK (0) or a
 * negative status.  kq_last_error() returns the calling thread's last message.
 * Callers own every buffer (inputs, outputs and workspaces).
 *
 * Formats (the compressed-tensors "mxfp4-pack-quantized" and vLLM MXFP8
 * layouts that kquant uses):
 *   - blocks are 32 consecutive elements along K (the last, contiguous axis);
 *   - E8M0 scale: uint8 [rows, K/32], value 2^(byte-127);
 *   - MXFP4: uint8 [rows, K/2], two E2M1 codes per byte, low nibble = even K;
 *   - MXFP8: uint8 (float8_e4m3fn bits) [rows, K].
 */
#ifndef KQUANT_AMD_H
#define KQUANT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  KQ_OK = 0,
  KQ_ERR_INVALID = -1,  /* bad argument: shape, alignment, enum value   */
  KQ_ERR_HIP = -2,      /* a HIP runtime call failed (launch, query)    */
  KQ_ERR_LIMIT = -3     /* a size exceeds what the kernel supports       */
};

/* element formats */
enum { KQ_FMT_MXFP8_E4M3 = 0, KQ_FMT_MXFP4_E2M1 = 1 };
/* dense element types */
enum { KQ_DT_BF16 = 0, KQ_DT_F16 = 1, KQ_DT_F32 = 2 };
/* flags */
enum {
  /* use the bit-level software rounding instead of the gfx950 convert
     instructions (both are tested to agree byte for byte) */
  KQ_FLAG_SOFTWARE_CVT = 1u
};
/* kq_moe_forward flags: run the grouped GEMMs on the register-staged kernel
   (the path taken when x or the intermediate exceed a 4 GiB buffer range)
   instead of the direct-to-LDS one; both meet the same error bound, and
   differ only by fp32 rounding (they sum each MFMA's k in another order) */
enum { KQ_MOE_REGISTER_STAGED = 1u };
/* kq_moe_forward flags: activation-quantized modes (no kquant counterpart).
   The tokens and the bf16 intermediates are MX-quantized per row with the
   kq_mx_quantize rule (E4M3 for W4A8, E2M1 for W4A4) and every GEMM runs
   on the block-scaled fp8/fp4 MFMA; the result equals an fp32 GEMM over the
   dequantized operands up to summation order */
enum { KQ_MOE_ACT_MXFP8 = 2u, KQ_MOE_ACT_MXFP4 = 4u };
/* kq_syrk_accumulate flags */
enum { KQ_SYRK_OVERWRITE = 1u, KQ_SYRK_SQUARE_WEIGHTS = 2u, KQ_SUM_SQUARE_F64 = 4u };
/* kq_block_ldl flags: also zero the diagonal (finalize_capture_H's
   L[dr, dr] = 0, kquant/exl3_encoder_backend.py:1649-1651) */
enum { KQ_LDL_ZERO_DIAGONAL = 1u };
/* byte tables of kq_decode_bytes */
enum { KQ_TABLE_E8M0 = 0, KQ_TABLE_E2M1 = 1, KQ_TABLE_E4M3 = 2 };
/* expert activations */
enum { KQ_ACT_SITU = 0, KQ_ACT_SWIGLU = 1 };

/* ABI version (major << 16 | minor) and the last error of this thread. */
int kq_version(void);
const char* kq_last_error(void);

/* ---------------------------------------------------------------- codec -- */

/* Quantize a dense [rows, k] matrix (row stride ld_in elements) to MX.
 *
 * MXFP8 replaces kquant/mxfp8.py:11-51 (mxfp8_quantize_cpu):
 *   e = clamp(ceil(log2(max(amax,1e-30)/448)), -127, 128), byte = e + 127,
 *   q = float8_e4m3fn(clamp(x / 2^e, +-448))   (round to nearest even),
 * with the quotient and its log2 each rounded to fp32 as the reference's
 * float32 torch ops do (this decides e only for fp32 inputs whose amax lies a
 * few ulps above 448 * 2^k).
 * MXFP4 is the same rule with (E2M1, 6.0); kquant has no MXFP4 quantizer,
 * its output layout is kquant/io/mxfp4.py:1-8 / pack_codes (:32-38).
 * out_q: uint8 [rows, k] (MXFP8) or [rows, k/2] (MXFP4), contiguous.
 * out_scale: uint8 [rows, k/32], contiguous.  k % 32 == 0.           */
int kq_mx_quantize(int fmt, int in_dtype, const void* in, int64_t ld_in,
                   int64_t rows, int64_t k, void* out_q, uint8_t* out_scale,
                   uint32_t flags, void* stream);

/* Dequantize MX codes + E8M0 scales to a dense [rows, k] matrix.
 * MXFP4 replaces kquant/io/mxfp4.py:52-64 (dequant: E2M1[code]*2^(s-127),
 * fp32), MXFP8 replaces kquant/mxfp8.py:54-84 (mxfp8_dequantize_cpu).
 * out_dtype KQ_DT_F32 is the reference's result; KQ_DT_BF16 / KQ_DT_F16 are
 * that fp32 value rounded to nearest even (scripts/closure_exl3_layer.py:157).
 * Scale byte 255 gives +inf scale (0 * inf = NaN) as exp2(128) does.   */
int kq_mx_dequant(int fmt, const void* q, const uint8_t* scale, int64_t rows,
                  int64_t k, int out_dtype, void* out, uint32_t flags,
                  void* stream);

/* Repack `mats` MXFP4 matrices (packed [rows, k/2] + E8M0 [rows, k/32] each,
 * stacked) into the MFMA-tiled layout kq_moe_forward reads: per matrix,
 * 1 KiB tiles [rows/16][k/128] with tile byte 16*l + j = packed[16 rg + l%16]
 * [64 c + 16 (l/16) + j], and 64-byte scale tiles with byte l =
 * scale[16 rg + l%16][4 c + l/16].  A one-time weight preparation (the role
 * of the external kernel's prepare_weights in scripts/closure_exl3_layer.py:
 * 412-443); same bytes, permuted.  rows % 16 == 0, k % 128 == 0.  scale and
 * scale_tiled may both be NULL (packed bytes only, for X4T-coded scales). */
int kq_mx_tile_weights(const uint8_t* q, const uint8_t* scale, int64_t mats, int64_t rows,
                       int64_t k, uint8_t* q_tiled, uint8_t* scale_tiled, void* stream);

/* Nibble codes <-> packed bytes, kquant/io/mxfp4.py:19-38 (unpack_codes,
 * pack_codes): byte = lo | hi << 4 (mod 256), lo = the even index; codes are
 * OR-ed as whole bytes exactly as the reference does.  n_codes is even. */
int kq_unpack_codes(const uint8_t* packed, int64_t n_packed, uint8_t* codes,
                    void* stream);
int kq_pack_codes(const uint8_t* codes, int64_t n_codes, uint8_t* packed,
                  void* stream);

/* Decode bytes through a format table into a dense array:
 *   KQ_TABLE_E8M0  2^(b-127)        kquant/io/mxfp4.py:41-43 (scale_factors)
 *   KQ_TABLE_E2M1  E2M1_LUT[c]      kquant/io/mxfp4.py:46-49 (code_values);
 *                                   codes >= 16 give NaN (the reference's
 *                                   gather raises IndexError instead)
 *   KQ_TABLE_E4M3  float8_e4m3fn    kquant/sqg_e4m3.py:150-151, 336-353
 *                                   (codebook widening, .view(e4m3).to(dtype)) */
int kq_decode_bytes(int table, const uint8_t* in, int64_t n, int out_dtype, void* out,
                    void* stream);

/* ----------------------------------------------------------- MoE experts -- */

/* Workspace bytes kq_moe_forward needs for these sizes (-1 on bad sizes). */
int64_t kq_moe_workspace_size(int64_t tokens, int topk, int experts, int64_t hidden,
                              int64_t inter);

/* Routed MoE expert forward with MXFP4 expert weights (W4A16):
 *   for every pair (t, s) with e = route_ids[t, s] in [0, experts):
 *     g = x_t W13_e[0:I]^T, u = x_t W13_e[I:2I]^T        (fp32 accumulate)
 *     a = bf16(act(g, u))          SiTU(beta, linear_beta) or SwiGLU
 *     out_t += route_weights[t, s] * (a W2_e^T)          (fp32)
 * which is scripts/closure_exl3_layer.py:557-598 (_reference_rank, tp = 1)
 * with kquant/tp_simulator.py:83-94 (situ) and gate-first w13
 * (closure_exl3_layer.py:420-423); ids outside [0, experts) contribute 0.
 * x bf16 [tokens, hidden] (row stride ldx); route_ids int32 and
 * route_weights fp32 [tokens, topk]; the weights in the kq_mx_tile_weights
 * layout: w13_t / w13_st = tiles of the [experts, 2I, hidden] MXFP4 w13
 * (gate rows first), w2_t / w2_st = tiles of [experts, hidden, I];
 * out [tokens, hidden] bf16 or fp32.
 * hidden % 512 == 0, I % 512 == 0, topk <= 64, experts <= 4096.
 * workspace: >= kq_moe_workspace_size bytes, 256-byte aligned, caller owned;
 * flags: 0, KQ_MOE_REGISTER_STAGED, KQ_MOE_ACT_MXFP8 or KQ_MOE_ACT_MXFP4.
 * results are bitwise reproducible (no floating-point atomics). */
int kq_moe_forward(int activation, float act_beta, float act_linear_beta,
                   const void* x, int64_t ldx, int64_t tokens, int64_t hidden,
                   const int32_t* route_ids, const float* route_weights, int topk,
                   int experts, int64_t inter, const uint8_t* w13_t,
                   const uint8_t* w13_st, const uint8_t* w2_t, const uint8_t* w2_st,
                   int out_dtype, void* out, void* workspace, int64_t workspace_bytes,
                   uint32_t flags, void* stream);

/* Workspace bytes kq_moe_forward_x4t needs (-1 on bad sizes): the
 * kq_moe_forward workspace plus, above 256 routed pairs, one w13 and one w2
 * scale slot per possible grouped-GEMM expert, min(pairs / 17, experts). */
int64_t kq_moe_x4t_workspace_size(int64_t tokens, int topk, int experts, int64_t hidden,
                                  int64_t inter);

/* kq_moe_forward with the expert scales kept X4T-compressed in device memory
 * (kquant/x4t.py's per-expert w1 / w3 / w2 scale planes: fixed streams of
 * `experts` stacked matrices, their exception streams, and per-16-row-tile
 * exception indexes from kq_x4t_tile_index).  The X4T runtime refinement of
 * docs/qsrt-technical-brief.md:446-474, with no allocation, host work or
 * exception search per call: each GEMV workgroup (experts with <= 16 pairs,
 * every expert when decoding) decodes the scales of its own rows - w1 and w3
 * into the gate and up rows of the gate-first w13 - into LDS before its K
 * loop; for the experts on the grouped GEMM one launch after routing expands
 * their scales into workspace slots in the kq_mx_tile_weights scale layout.
 * w13_t / w2_t as for kq_moe_forward.  w1 / w3
 * planes are [inter, hidden / 32], w2 planes [hidden, inter / 32]; hidden
 * and inter at most 8160.  The components must be a valid X4T encoding (as
 * kq_x4t_decode accepts): the expansion does not validate them; with tile
 * indexes that kq_x4t_tile_index made from the same exception streams it
 * accesses no memory outside the buffers described here, whatever they hold.  Same
 * flags and same results, bit for bit, as kq_moe_forward over the decoded
 * scales.  workspace: >= kq_moe_x4t_workspace_size bytes. */
int kq_moe_forward_x4t(int activation, float act_beta, float act_linear_beta,
                       const void* x, int64_t ldx, int64_t tokens, int64_t hidden,
                       const int32_t* route_ids, const float* route_weights, int topk,
                       int experts, int64_t inter, const uint8_t* w13_t, const uint8_t* w2_t,
                       const uint8_t* w1_fixed, const uint32_t* w1_exceptions,
                       const uint32_t* w1_tile_index, const uint8_t* w3_fixed,
                       const uint32_t* w3_exceptions, const uint32_t* w3_tile_index,
                       const uint8_t* w2_fixed, const uint32_t* w2_exceptions,
                       const uint32_t* w2_tile_index, int out_dtype, void* out,
                       void* workspace, int64_t workspace_bytes, uint32_t flags, void* stream);

/* Size of the device array kq_moe_forward_noalloc uses as its workspace. */
#define KQ_MOE_NOALLOC_SCRATCH_BYTES (16ll << 20)

/* kq_moe_forward without a workspace argument: the forward runs in a
 * 16 MiB device array of this library (one per GPU, held until the process
 * ends), so the call allocates nothing.  No counterpart in kquant: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc).  Same arguments (minus the workspace),
 * flags and results, bit for bit, as kq_moe_forward.  Sizes whose
 * kq_moe_workspace_size exceeds KQ_MOE_NOALLOC_SCRATCH_BYTES fail with
 * KQ_ERR_LIMIT (at hidden 7168, intermediate 2048: up to 256 routed pairs,
 * e.g. 32 decode tokens at top-8).  The array keeps the last call's contents;
 * calls that overlap on one GPU (concurrent streams or threads) share it and
 * race, so the caller serializes them. */
int kq_moe_forward_noalloc(int activation, float act_beta, float act_linear_beta,
                           const void* x, int64_t ldx, int64_t tokens, int64_t hidden,
                           const int32_t* route_ids, const float* route_weights, int topk,
                           int experts, int64_t inter, const uint8_t* w13_t,
                           const uint8_t* w13_st, const uint8_t* w2_t, const uint8_t* w2_st,
                           int out_dtype, void* out, uint32_t flags, void* stream);

/* --------------------------------------------------------- dense linear -- */

/* C [m, n] = A [m, k] (bf16, row stride lda) x dequant(W)^T, W [n, k] in
 * w_fmt (MXFP8: E4M3 bytes [n, k]; MXFP4: packed [n, k/2]) with E8M0 scales
 * [n, k/32]; fp32 accumulation, C in bf16 or fp32 (row stride ldc).
 * Replaces the dequantize-then-matmul of kquant's expert/linear oracles
 * (kquant/pack/qsrt_validation.py:249-258, scripts/closure_mxfp8_mlp.py:
 * 146-160: fp32 matmul over dequantized weights) and the external
 * mxfp8_linear.mm call site (scripts/closure_mxfp8_mlp.py:172-177).
 * k % 64 == 0; a, w_q 16-byte aligned. */
int kq_mx_linear(int w_fmt, const void* a, int64_t lda, const void* w_q,
                 const uint8_t* w_scale, int64_t m, int64_t n, int64_t k,
                 int out_dtype, void* c, int64_t ldc, void* stream);

/* C [m, n] = dequant(A) [m, k] x dequant(W) [n, k]^T with both operands
 * MXFP8: A E4M3 bytes [m, k] (row stride lda bytes, lda % 16 == 0) with E8M0
 * scales [m, k/32], W E4M3 bytes [n, k] with E8M0 scales [n, k/32]; the
 * block-scaled fp8 MFMA multiplies the bytes and scales as they are, fp32
 * accumulation, C in bf16 or fp32 (row stride ldc).  This is the operand
 * contract of kquant's production MXFP8 linear (scripts/closure_mxfp8_mlp.py:
 * 146-160 _reference_from_packed: quantize the input, dequantize both
 * operands, fp32 product; :163-187 _production_linear).  a_fmt and w_fmt
 * must be KQ_FMT_MXFP8_E4M3; k % 128 == 0; a_q, w_q 16-byte aligned,
 * scales 4-byte aligned.  workspace (kq_mx_linear_mx_workspace_size bytes,
 * 256-byte aligned, uninitialised) takes both scale planes transposed to
 * [k/128][rows] dwords, the layout the kernel loads a 128-k stage's scales
 * from.  The matrix cores sum the 64 products of a step with a few fp32 ulps
 * of error (measured ~1e-5 relative). */
int64_t kq_mx_linear_mx_workspace_size(int64_t m, int64_t n, int64_t k);
int kq_mx_linear_mx(int a_fmt, const void* a_q, const uint8_t* a_scale, int64_t lda, int w_fmt,
                    const void* w_q, const uint8_t* w_scale, int64_t m, int64_t n, int64_t k,
                    int out_dtype, void* c, int64_t ldc, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* Workspace bytes of kq_mx_linear_mm (the quantized input rows and
 * kq_mx_linear_mx's workspace), -1 on bad sizes. */
int64_t kq_mx_linear_mm_workspace_size(int64_t m, int64_t n, int64_t k);

/* mxfp8_linear.mm of kquant's production MXFP8 linear
 * (scripts/closure_mxfp8_mlp.py:172-177): the input rows A [m, k] (bf16, f16
 * or f32, row stride lda elements) are quantized to MXFP8 with the
 * kq_mx_quantize rule into the workspace (block_fp8_linear.quantize_input,
 * :155), then kq_mx_linear_mx.  w_fmt: KQ_FMT_MXFP8_E4M3; k % 128 == 0;
 * workspace 256-byte aligned, uninitialised. */
int kq_mx_linear_mm(int w_fmt, const void* a, int a_dtype, int64_t lda, const void* w_q,
                    const uint8_t* w_scale, int64_t m, int64_t n, int64_t k, int out_dtype, void* c,
                    int64_t ldc, void* workspace, int64_t workspace_bytes, void* stream);

/* -------------------------------------------------------------- Hessian -- */

/* acc += X^T diag(w) X for X [n, k] (row stride ld elements, k % 8 == 0,
 * 16-byte aligned rows), w fp32 [n] or NULL (all ones).  Replaces the chunked
 * fp32 addmm_ of kquant/candidate_hessian.py:98-105 and
 * kquant/capture.py:713-730 (accumulator.addmm_(x.T, x * w[:, None])).
 * Only upper tiles (tile_row <= tile_col) of acc [k, k] (row stride ld_acc)
 * are written: 256x256 tiles for bf16 rows, 128x128 otherwise; both cover
 * the 128x128 upper tiles, which is what kq_syrk_finalize reads.  With
 * KQ_SYRK_OVERWRITE the tiles are written instead of accumulated (acc need
 * not be initialised).  bf16 rows use bf16 MFMA with exact products; fp16 /
 * fp32 rows and weights use a two-term bf16 split (16 significant bits). */
int kq_syrk_accumulate(int in_dtype, const void* x, int64_t ld, int64_t n, int64_t k,
                       const float* weights, float* acc, int64_t ld_acc, uint32_t flags,
                       void* stream);

/* kq_syrk_accumulate with a workspace for partial tiles.  When the upper
 * 256 x 256 tiles leave the last round of workgroups partly filled (406
 * tiles of k = 7168 on 256 CUs: one full round, then 150 tiles), the tiles
 * of that last round are cut by 64-row steps into 2..16 equal chunks: chunk
 * 0 writes the tile, the others write partial slots, and a second launch
 * adds each tile's slots, in chunk order, to it.  Results are deterministic
 * for a given CU count and agree with kq_syrk_accumulate to fp32 summation
 * order.  Only unweighted bf16 rows take the split; other calls, or a
 * workspace smaller than kq_syrk_accumulate_workspace_size (0 when the
 * split does not pay), run as kq_syrk_accumulate.  workspace: 256-byte
 * aligned, uninitialised, used by one call at a time.  The size function
 * assumes dense rows (ld == k) and the CU count of the current device; the
 * call plans with the CU count of its stream's device, so make that device
 * current when sizing. */
int64_t kq_syrk_accumulate_workspace_size(int in_dtype, int64_t n, int64_t k, int weighted);
int kq_syrk_accumulate_ws(int in_dtype, const void* x, int64_t ld, int64_t n, int64_t k,
                          const float* weights, float* acc, int64_t ld_acc, uint32_t flags,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* out [k, k] = symmetric(acc) / denominator, then
 * diag(out) += damp * mean(diag(out)).  Mirrors the upper tiles written by
 * kq_syrk_accumulate and averages (H + H^T)/2 inside diagonal tiles
 * (kquant/candidate_hessian.py:106-107, kquant/capture.py:861-862); damping
 * is kquant/exl3_encoder_backend.py:1613-1625 (sigma_reg * mean(diag)).
 * acc and out must not alias; k <= 2^20.  Each upper tile of acc is read
 * once (one workgroup per 64 x 64 block and its mirror). */
int kq_syrk_finalize(const float* acc, int64_t ld_acc, int64_t k, double denominator,
                     float damp, float* out, int64_t ld_out, void* stream);

/* Routing sort on its own: the pairs p = t * topk + s of route_ids
 * [tokens, topk] grouped by expert, stable in pair order (ids outside
 * [0, experts) dropped), as the per-expert row selection of
 * kquant/qsrt_candidates.py:264-289 orders them.  Outputs: offsets int64
 * [experts + 1]; rows int32 [pairs] (token t of each sorted pair);
 * optional sorted_pairs int32 [pairs]; optional sorted_weights fp32 [pairs] =
 * pair_weights[pair].  Entries past offsets[experts] are unspecified.
 * workspace: kq_route_sort_workspace_size bytes, 256-byte aligned. */
int64_t kq_route_sort_workspace_size(int64_t tokens, int topk, int experts);
int kq_route_sort(const int32_t* route_ids, int64_t tokens, int topk, int experts,
                  const float* pair_weights, int64_t* offsets, int32_t* rows, int32_t* sorted_pairs,
                  float* sorted_weights, void* workspace, int64_t workspace_bytes, void* stream);

/* Per-group (per-expert) weighted X^T X in one launch: group g owns row-list
 * positions [offsets[g], offsets[g+1]) (offsets: device int64 [groups + 1]);
 * position p is row row_index[p] of x (row p itself when row_index is NULL)
 * with weight weights[p] (squared in fp32 with KQ_SYRK_SQUARE_WEIGHTS, the
 * gate^2 weighting of kquant/qsrt_candidates.py:562; 1 when weights is
 * NULL).  acc: [groups, k, k] fp32, upper tiles overwritten (finish with
 * kq_syrk_finalize_grouped).  The batched form of the per-expert
 * weighted_covariance calls of build_expert_hessians
 * (kquant/qsrt_candidates.py:534-618). */
int kq_syrk_grouped(int in_dtype, const void* x, int64_t ld, const int64_t* offsets, int groups,
                    const int32_t* row_index, const float* weights, int64_t k, float* acc,
                    uint32_t flags, void* stream);

/* out[g] = f64 sum of the group's weights (fp32 squares with
 * KQ_SYRK_SQUARE_WEIGHTS, f64 squares with KQ_SUM_SQUARE_F64; the row count
 * when weights is NULL): the denominators float(w.double().sum()) of
 * kquant/candidate_hessian.py:95 and the Kish sums of :141-153. */
int kq_segment_weight_sums(const float* weights, const int64_t* offsets, int groups, uint32_t flags,
                           double* out, void* stream);

/* out[g] = sym(acc[g]) / denominators[g] (device f64 [groups]); a group with
 * denominator <= 0 gives zeros.  acc, out: [groups, k, k]; no aliasing. */
int kq_syrk_finalize_grouped(const float* acc, int64_t k, int groups, const double* denominators,
                             float* out, void* stream);

/* Sums of covariance_comparison (kquant/candidate_hessian.py:219-258) for
 * fp32 [k, k] reference R and candidate C, in f64: out[8] = {sum (C-R)^2,
 * sum R^2, trace R, trace C, sum diag(R)^2, sum diag(C)^2, diag(R).diag(C),
 * max |C - C^T|}.  workspace: 256 * 8 doubles.  Deterministic. */
int kq_covariance_comparison_sums(const float* reference, const float* candidate, int64_t k,
                                  double* workspace, double* out, void* stream);

/* out [k,k] = ((X + X^T) / 2) with X = torch.lerp(A, B, alpha); A = a, or
 * a_scale * I when a is NULL.  kquant/candidate_hessian.py:115-138
 * (shrink_covariance) and :204-209 (identity target of
 * adaptive_identity_shrinkage).  Contiguous fp32 inputs; out aliases none. */
int kq_sym_lerp(const float* a, float a_scale, const float* b, int64_t k, float alpha,
                float* out, void* stream);

/* Deterministic f64 trace and sum of squares of a contiguous fp32 [k,k]
 * matrix (kquant/candidate_hessian.py:185-191: trace(local64),
 * local64.square()).  workspace: 2 * KQ_COV_STATS_PARTS doubles; out: 2
 * doubles {trace, sum of squares}, both device memory. */
#define KQ_COV_STATS_PARTS 256
int kq_cov_stats(const float* h, int64_t k, double* workspace, double* out, void* stream);

/* ------------------------------------------------ H finalize / block LDL --
 * The Hessian finalize of the trellis encoder
 * (kquant/exl3_encoder_backend.py:1588-1663, finalize_capture_H, and
 * :316-386, block_ldl), fp32 device matrices, row-major. */

/* H *= 1 / count (skipped when count == 0), then
 * diag(H) += sigma_reg * mean(diag(H)) (exl3_encoder_backend.py:1611-1628;
 * the mean is summed in f64 and rounded to fp32).  diag_mean: one float
 * (device) receiving the mean before damping; diag: k floats receiving the
 * damped diagonal, or NULL.  k <= 65535. */
int kq_h_regularize(float* h, int64_t k, int64_t ld, double count, float sigma_reg, float* diag,
                    float* diag_mean, void* stream);

/* In place X <- B S_r X S_c B over `batch` matrices [rows, cols] (row stride
 * ld, matrix stride `stride`), B = blockdiag of the 128 x 128 Sylvester
 * Hadamard / sqrt(128) (kquant/exl3_reference.py:195-212).  sides: 1 = left
 * only (blockwise_preapply_had_l_, exl3_encoder_backend.py:288-299), 2 =
 * right only (blockwise_preapply_had_r_, :302-313), 3 = both (the rotation
 * of finalize_capture_H, :1640-1644, with H *= su^T before the right side
 * and H *= su before the left: row_scale = col_scale = su).  row_scale /
 * col_scale: fp32 vectors or NULL.  The transformed dimensions must be
 * multiples of 128.  Results equal the reference's fp32 matmuls up to fp32
 * rounding (the transform here is a fast Walsh-Hadamard, adds only). */
int kq_blockwise_hadamard(float* x, int64_t rows, int64_t cols, int64_t ld, int64_t batch,
                          int64_t stride, int sides, const float* row_scale, const float* col_scale,
                          void* stream);

/* Lower Cholesky factors L (A = L L^T, zeros above the diagonal) of `batch`
 * symmetric fp32 matrices [n, n]: torch.linalg.cholesky's output
 * (exl3_encoder_backend.py:325-330).  Only the lower triangle of A is read;
 * a == l (same ld and stride) factors in place.  info: batch int32 (device),
 * 0 on success, else the order of the first leading minor that is not
 * positive definite (LAPACK's convention; the factor is then meaningless);
 * -1 if a bounded wait between workgroups of one launch ran out (an internal
 * error; the factor is then meaningless).  workspace:
 * kq_cholesky_workspace_size bytes, not shared by concurrent calls.
 * n, batch <= 65535. */
int64_t kq_cholesky_workspace_size(int64_t n, int64_t batch);
int kq_cholesky(const float* a, int64_t lda, int64_t stride_a, float* l, int64_t ldl,
                int64_t stride_l, int64_t n, int64_t batch, int32_t* info, void* workspace,
                int64_t workspace_bytes, void* stream);

/* The block LDL step of exl3_encoder_backend.py:356-384 in place on lower
 * Cholesky factors: every b x b diagonal block DL_i is inverted, each block
 * column multiplied by its block's inverse (L[:, i] = L[:, i] inv(DL_i)) and
 * the diagonal blocks set to the identity; with KQ_LDL_ZERO_DIAGONAL the
 * diagonal is then zeroed.  b a power of two <= 64, n % b == 0.  workspace:
 * kq_block_ldl_workspace_size bytes. */
int64_t kq_block_ldl_workspace_size(int64_t n, int b, int64_t batch);
int kq_block_ldl(float* l, int64_t ld, int64_t stride, int64_t n, int b, int64_t batch,
                 uint32_t flags, void* workspace, int64_t workspace_bytes, void* stream);

/* --------------------------------------------------------- QSRT trellis --
 * The QSRT-E4M3 trellis bitstream and its weight decode.  A 16 x 16 tile
 * stores 256 K-bit edges (K = 2, 3, 4): 16 spans of 16 symbols, each span K
 * uint16 words MSB first, adjacent words exchanged (kquant/qsrt.py:811-857,
 * pack_trellis_edges / unpack_trellis_edges).  Tiles are [tiles][256] int16
 * symbols and [tiles][16 K] int16 words. */
enum { KQ_QSRT_TRANSPOSED = 1u };

/* Pack the low K bits of every symbol (pack_trellis_edges). */
int kq_trellis_pack(const int16_t* symbols, int64_t tiles, int bits, int16_t* packed, void* stream);

/* Unpack to the K-bit edges (states == 0, unpack_trellis_edges) or to the
 * cyclic 16-bit states (states != 0: unpack_trellis_states,
 * kquant/qsrt.py:860-863 with kquant/exl3_reference.py:37-61). */
int kq_trellis_unpack(const int16_t* packed, int64_t tiles, int bits, int states, int16_t* out,
                      void* stream);

/* Decode a complete packed matrix (the payload of pack_qsrt_trellis,
 * kquant/qsrt.py:983-1013: 128-channel records along the rate axis, record r
 * at rate record_bits[r] (host array), tiles of a record in row-major
 * (k_tile, n_tile) order) to its EXL-oriented weight [K, N] =
 * [16 k_tiles, 16 n_tiles]: decode_qsrt_weight (kquant/exl3_reference.py:
 * 149-192, 270-295) with suh [K] and svh [N] fp32 (device), or the
 * regularized weight (decode_qsrt_regularized_weight) when both are NULL.
 * rate_axis 0 = k, 1 = n.  labels: 3 x 65536 E4M3 bytes (device), the
 * state labels of K2, K3 and K4 (kq_sqg_* / sqg_codebook_bytes).  out:
 * out_dtype values with row stride ldo, [K, N] or, with KQ_QSRT_TRANSPOSED,
 * [N, K] (the loader's dense orientation).  Both dimensions are multiples of
 * 128, at most 1024 records.  The regularized weight is exact; the rotated
 * one equals the reference's fp32 matmuls up to fp32 rounding.  A payload
 * and label table both 16-byte aligned take the direct-load kernel, others
 * a generic one with the same result.  out_dtype KQ_QSRT_OUT_E4M3 writes the
 * regularized weight's E4M3 label bytes themselves (suh = svh = NULL,
 * aligned buffers): the weight operand of an MXFP8 product with unit scales. */
#define KQ_QSRT_OUT_E4M3 3
int kq_qsrt_decode_weight(const int16_t* payload, int64_t payload_words, int64_t k_tiles,
                          int64_t n_tiles, int rate_axis, const uint8_t* record_bits,
                          const uint8_t* labels, const float* suh, const float* svh, int out_dtype,
                          void* out, int64_t ldo, uint32_t flags, void* stream);

/* The same decode from given 16-bit states [k_tiles][n_tiles][256]
 * (decode_qsrt_regularized_weight / decode_qsrt_weight,
 * kquant/exl3_reference.py:149-192, 270-295, which accept any states): tile
 * rates per tile along the rate axis, tile_bits [k_tiles or n_tiles] uint8
 * (device). */
int kq_qsrt_decode_states(const int16_t* states, int64_t k_tiles, int64_t n_tiles, int rate_axis,
                          const uint8_t* tile_bits, const uint8_t* labels, const float* suh,
                          const float* svh, int out_dtype, void* out, int64_t ldo, uint32_t flags,
                          void* stream);

/* A linear layer on a packed QSRT matrix without materializing the weight:
 * out[m, n] = sum_k x[m, k] W[k, n] for m < rows, W the matrix that
 * kq_qsrt_decode_weight would produce from the same arguments (rotated with
 * suh / svh, or regularized when both are NULL).  It replaces the serving
 * use of the decode, which builds the dense weight and then applies it
 * (scripts/stream_k3_pytorch.py:771-775 with decode_qsrt_exl3_weight,
 * kquant/qsrt.py:1107-1141).  x: x_dtype values [rows, ldx >= K]; out:
 * out_dtype values [rows, ldo >= N]; fp32 arithmetic throughout (the
 * activation rows are rotated in fp32, the weight is never rounded to
 * bf16), so the result is the exact product up to fp32 summation order.
 * Up to 32 rows (decode batches) the weight is decoded inside the product,
 * once per 16 rows.  From 33 rows on (prefill) the call runs in four
 * launches: the activation rows rotated by suh and the 128-point blockwise
 * Hadamard, the regularized weight decoded once to its E4M3 labels, the
 * MXFP8 MFMA linear (kq_mx_linear_f32 for fp32 / fp16 x, exact to fp32
 * summation order; kq_mx_linear for bf16 x, whose rotated rows are rounded
 * to bf16 first), and the output rotated by 1/128, the Hadamard and svh.
 * payload and labels must be 16-byte aligned (KQ_ERR_INVALID otherwise).
 * workspace: kq_qsrt_linear_workspace_size(rows, k_tiles, n_tiles) bytes
 * (may be 0), 256-byte aligned and zeroed before its first use with these
 * sizes; each call up to 32 rows leaves it zero again (its completion
 * counters, and for one or two rows the K chunks' partial sums, which the
 * last chunk's workgroup polls), so it serves repeated calls of the same
 * sizes (zero it again before other sizes, and after a prefill-sized call,
 * which uses it as scratch).  Calls sharing a workspace must not overlap.
 * With one or two rows the workgroup of the last K chunk waits for the
 * other chunks' partials (workgroups that precede it in dispatch order and
 * wait on nothing); the wait is bounded, and a partial still missing after
 * it reads as NaN in the output. */
int64_t kq_qsrt_linear_workspace_size(int64_t rows, int64_t k_tiles, int64_t n_tiles);
int kq_qsrt_linear(const void* x, int x_dtype, int64_t rows, int64_t ldx, const int16_t* payload,
                   int64_t payload_words, int64_t k_tiles, int64_t n_tiles, int rate_axis,
                   const uint8_t* record_bits, const uint8_t* labels, const float* suh, const float* svh,
                   int out_dtype, void* out, int64_t ldo, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* One QSRT-coded matrix as kq_qsrt_moe_decode reads it (device pointers):
 * its packed payload (16-byte aligned), record_prefix [records + 1] uint32
 * with record_prefix[r] = the sum of the rates of the records before r (so
 * record r has rate record_prefix[r + 1] - record_prefix[r], 2..4), and its
 * suh [K] / svh [N] fp32 scales. */
typedef struct {
  const int16_t* payload;
  const uint32_t* record_prefix;
  const float* suh;
  const float* svh;
} kq_qsrt_matrix;

/* Routed expert forward of a decode batch with QSRT-coded experts (no
 * kquant counterpart as a kernel: the reference decodes each routed
 * expert's w1 / w3 / w2 to dense bf16, scripts/stream_k3_pytorch.py:771-775,
 * and runs the expert MLP of scripts/closure_exl3_layer.py:557-598):
 *   for every pair (t, s) with e = route_ids[t, s] in [0, experts):
 *     g = x_t W1_e, u = x_t W3_e        (EXL orientation: W1, W3 [H, I])
 *     out_t += route_weights[t, s] * act(g, u) W2_e     (W2 [I, H])
 * in fp32 (the intermediate is not rounded), out = 0 for tokens with no
 * valid expert.  mats: device array [experts][3] (w1, w3, w2) of
 * kq_qsrt_matrix, all experts of one geometry: hidden H = 16 hidden_tiles,
 * intermediate I = 16 inter_tiles (multiples of 128), w1 / w3 records
 * along rate13_axis, w2 along rate2_axis (0 = k, 1 = n), payload sizes as
 * their records require (not checked here: the descriptors live on the
 * device).  x [tokens, ldx >= H] x_dtype, route_ids int32 / route_weights
 * fp32 [tokens, topk], labels (16-byte aligned) 2 x 3 x 65536 E4M3 bytes: the K2..K4 state
 * labels (as kq_qsrt_decode_weight) for w1 / w3, then for w2 (a codebook
 * may depend on the rate axis, kquant/sqg_e4m3.py:305-340), out [tokens,
 * ldo >= H] out_dtype.  Two launches; deterministic.  workspace:
 * kq_qsrt_moe_workspace_size bytes, 256-byte aligned, zeroed before its
 * first use with these sizes (calls leave its counters at zero; zero it
 * again before other sizes); calls sharing it must not overlap. */
int64_t kq_qsrt_moe_workspace_size(int64_t tokens, int topk, int64_t hidden_tiles, int64_t inter_tiles);
int kq_qsrt_moe_decode(int act, float beta, float linear_beta, const void* x, int x_dtype, int64_t tokens,
                       int64_t ldx, const int32_t* route_ids, const float* route_weights, int topk,
                       const kq_qsrt_matrix* mats, int experts, int64_t hidden_tiles, int64_t inter_tiles,
                       int rate13_axis, int rate2_axis, const uint8_t* labels, int out_dtype, void* out,
                       int64_t ldo, void* workspace, int64_t workspace_bytes, void* stream);

/* SQG trellis quantizer: the tail-biting Viterbi search of
 * kquant/csrc/qsrt_quantize_tiles_kernel.cuh with the SQG E4M3 labels of
 * kquant/csrc/sqg_quantize.cu (quantize_tiles_sqg_cuda, :165-342), in the
 * same fp16 arithmetic, decision packing and tie order, so the states and
 * values are those of the reference kernel bit for bit.  tiles / out_tiles
 * fp32 [n_tiles, 256]; out_states int16 [n_tiles, 256] (the cyclic 16-bit
 * states of the path); lut: 65536 E4M3 labels in state order (device);
 * tailbite_context 1..128.  One workgroup per tile, `workgroups` of them
 * over the tiles; workspace: kq_sqg_quantize_workspace_size(bits,
 * workgroups) bytes for the decisions.  Tiles whose every path cost
 * overflows fp16 (|x| in the hundreds) are outside the reference's domain. */
int64_t kq_sqg_quantize_workspace_size(int bits, int workgroups);
int kq_sqg_quantize_tiles(const float* tiles, int64_t n_tiles, const uint8_t* lut, int bits,
                          int tailbite_context, float* out_tiles, int16_t* out_states, void* workspace,
                          int64_t workspace_bytes, int workgroups, void* stream);

/* The same search against a procedural EXL3 control codebook
 * (quantize_tiles_procedural_cuda, kquant/csrc/sqg_quantize.cu:261-330, with
 * the decoders of kquant/csrc/exl3_compat/quant/codebook.cuh):
 *   codebook 1, MCG:  x = state * 0xCBAC1FED mod 2^32,
 *                     x = (x & 0x8fff8fff) ^ 0x3b603b60, label = fp16(lo + hi)
 *                     of the two fp16 halves of x;
 *   codebook 2, MUL1: x = state * 0x83DCD12D mod 2^32, h = fp16(1024 + the
 *                     sum of x's bytes), label = fp16(h * 0x1eee + 0xc931)
 *                     (fp16 bit patterns, one rounding).
 * Arguments and workspace as kq_sqg_quantize_tiles, without the table. */
int kq_sqg_quantize_tiles_procedural(const float* tiles, int64_t n_tiles, int bits, int codebook,
                                     int tailbite_context, float* out_tiles, int16_t* out_states,
                                     void* workspace, int64_t workspace_bytes, int workgroups, void* stream);

/* ---------------------------------------------------- scale-plane codecs --
 * Lossless codings of a uint8 E8M0 scale plane [rows, cols], cols <= 255,
 * rows contiguous.  Variable-length outputs are produced in two calls: a
 * measuring call whose int64 offsets array ends in the total (read it after
 * the stream synchronises, size the output), then an emitting call. */

/* X4T fixed stream and per-tile exception offsets of `mats` stacked planes
 * [mats * rows, cols], rows % 16 == 0, rows * cols < 2^24.
 * kquant/x4t.py:90-130 (pack_x4t_scale_components: per-row adjacent base,
 * lowest base on ties, selector bit = value is base + 1) and :201-234
 * (x4t_scale_storage_bytes / x4t_scale_exception_count).
 * fixed: mats * rows/16 tiles of 16 * (1 + ceil(cols/8)) bytes.
 * tile_offsets: tiles + 1 int64; on completion entry t is the first
 * exception of tile t and entry `tiles` the total.  Matrix m's exceptions
 * are entries [tile_offsets[m * rows/16], tile_offsets[(m+1) * rows/16]). */
int kq_x4t_analyze(const uint8_t* scale, int64_t mats, int64_t rows, int64_t cols,
                   uint8_t* fixed, int64_t* tile_offsets, void* stream);

/* X4T exception words (matrix-local position | value << 24, row-major) at
 * the offsets kq_x4t_analyze produced.  kquant/x4t.py:117-126. */
int kq_x4t_emit_exceptions(const uint8_t* scale, int64_t mats, int64_t rows, int64_t cols,
                           const uint8_t* fixed, const int64_t* tile_offsets,
                           uint32_t* exceptions, void* stream);

/* X4T decode (kquant/x4t.py:477-524, _decode_scale_components) into
 * out [mats * rows, cols].  exception_offsets: mats + 1 int64 giving each
 * matrix's exception range (NULL when mats == 1: all n_exceptions).  With
 * status non-NULL (mats == 1 only) the plane is also validated into
 * status[4] uint32: {selector padding bits set, index of the first exception
 * with a bad or non-increasing position (0xffffffff if none), index of the
 * first exception naming its row's pair (0xffffffff if none), stream not
 * canonical}.  The first failure in that order is the reference's error. */
int kq_x4t_decode(const uint8_t* fixed, const uint32_t* exceptions, int64_t n_exceptions,
                  const int64_t* exception_offsets, int64_t mats, int64_t rows, int64_t cols,
                  uint8_t* out, uint32_t* status, void* stream);

/* Per-tile exception index of `mats` stacked X4T matrices [rows, cols]:
 * index[m * rows/16 + t] = the first entry of matrix m's exception range
 * (exception_offsets[m] .. exception_offsets[m + 1], or all n_exceptions when
 * exception_offsets is NULL and mats == 1) whose position lies at or past
 * tile t's first position; index[mats * rows/16] = n_exceptions.  The same
 * numbers kq_x4t_analyze's tile_offsets hold, recovered from the streams
 * alone (kquant/x4t.py's container keeps only per-matrix offsets,
 * x4t.py:594-602).  One-time preparation for kq_moe_forward_x4t. */
int kq_x4t_tile_index(const uint32_t* exceptions, int64_t n_exceptions,
                      const int64_t* exception_offsets, int64_t mats, int64_t rows, int64_t cols,
                      uint32_t* index, void* stream);

/* KQSC row-palette payload, version 1 (kquant/mxfp4_scale_codec.py:27-85,
 * pack_scale_plane) or 2 (:205-292, pack_scale_plane_compact), tile_rows in
 * 1..255.  row_meta: rows uint32 scratch; tile_offsets: tiles + 1 int64 with
 * tiles = ceil(rows / tile_rows), entry `tiles` = total body bytes.  The
 * payload is 16 + 4 * (tiles + 1) + total bytes; the total must be < 2^32. */
int kq_kqsc_measure(int version, const uint8_t* scale, int64_t rows, int64_t cols, int tile_rows,
                    uint32_t* row_meta, int64_t* tile_offsets, void* stream);
int kq_kqsc_emit(int version, const uint8_t* scale, int64_t rows, int64_t cols, int tile_rows,
                 const uint32_t* row_meta, const int64_t* tile_offsets, uint8_t* payload,
                 void* stream);

/* KQSC tile decode and validation (kquant/mxfp4_scale_codec.py:88-161,
 * unpack_scale_plane; :295-424, unpack_scale_plane_compact) of a device
 * payload whose header and offset table the caller has parsed and checked.
 * status: one uint64, ~0 when valid, else (tile << 20) | key of the first
 * failure in the reference's order (key < 8: tile-level check; key >= 8:
 * 8 + row * 1024 + sub, sub 0 palette escape, 1 adjacent range, 2 selector
 * padding, 3 + 2e bad position / 4 + 2e redundant value of exception e). */
int kq_kqsc_decode(int version, const uint8_t* payload, int64_t payload_bytes, int64_t rows,
                   int64_t cols, int tile_rows, uint8_t* out, uint64_t* status, void* stream);

/* Structural counts of a version-2 payload (kquant/mxfp4_scale_codec.py:427-499,
 * compact_scale_plane_stats): tile_stats [tiles, 3] uint32 {palette escapes,
 * count escapes, exceptions}; status as for kq_kqsc_decode with key 0..4 =
 * explicit bits short / padded, count codes short / padded, accounting. */
int kq_kqsc_stats(const uint8_t* payload, int64_t payload_bytes, int64_t rows, int64_t cols,
                  int tile_rows, uint32_t* tile_stats, uint64_t* status, void* stream);

/* Workspace bytes of kq_mx_linear_f32 (m * 3k bf16), -1 on bad sizes. */
int64_t kq_mx_linear_f32_workspace_size(int64_t m, int64_t k);

/* C [m, n] fp32 = A [m, k] fp32 x dequant(W [n, k])^T at fp32-GEMM accuracy:
 * A is split exactly into three bf16 terms (a = a0 + a1 + a2) written to the
 * workspace as [m, 3k], and one launch of the kq_mx_linear kernel accumulates
 * all three products in fp32 (weight column k' % k for A column k').
 * Replaces the fp32 F.linear over dequantized official weights of
 * kquant/pack/qsrt_validation.py:240-258 (official_expert_output) and the
 * fp32 closure oracles.  k % 64 == 0, lda % 4 == 0; a, w_q, workspace
 * 16-byte aligned. */
int kq_mx_linear_f32(int w_fmt, const float* a, int64_t lda, const void* w_q,
                     const uint8_t* w_scale, int64_t m, int64_t n, int64_t k, float* c,
                     int64_t ldc, void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------- expert MLP helpers --
 * out[r, c] = act(gate[r, c], up[r, c]) computed in fp32 (SiTU with beta /
 * linear_beta, kquant/tp_simulator.py:83-94, or SwiGLU), rounded to
 * out_dtype.  gate and up share the row stride ld_in. */
int kq_expert_activation(int activation, float beta, float linear_beta, int in_dtype,
                         const void* gate, const void* up, int64_t ld_in, int64_t rows,
                         int64_t cols, int out_dtype, void* out, int64_t ld_out, void* stream);

/* out[i] = (sum over p of partials[p * stride + i]) in fp32, summed in order
 * p = 0..parts-1, rounded to out_dtype (kquant/tp_simulator.py:72-80,
 * reduce_partials). */
int kq_reduce_partials(const float* partials, int64_t parts, int64_t stride, int64_t n,
                       int out_dtype, void* out, void* stream);

/* Deterministic f64 sums behind comparison_metrics
 * (kquant/tp_simulator.py:137-160): out[5] = {sum (a - r)^2, max |a - r|,
 * sum r^2, sum a^2, sum r*a} with a - r formed in fp32.  workspace: 256 * 5
 * doubles.  relative_l2 = sqrt(out[0]) / max(sqrt(out[2]), FLT_MIN),
 * cosine = out[4] / (max(sqrt(out[2]), eps) * max(sqrt(out[3]), eps)). */
int kq_comparison_sums(int ref_dtype, const void* reference, int act_dtype, const void* actual,
                       int64_t n, double* workspace, double* out, void* stream);

/* K3 router (kquant/tp_simulator.py:114-134, kimi_topk): scores =
 * sigmoid(logits) in fp32, top-k of scores + bias[e] in descending order
 * (ties to the lower expert id), weights = chosen scores / their sum *
 * routed_scaling_factor.  logits [tokens, experts] (row stride ld),
 * weights fp32 / ids int32 [tokens, topk].  experts <= 1024, topk <= 64. */
int kq_kimi_topk(int logit_dtype, const void* logits, int64_t ld, const float* bias,
                 int64_t tokens, int experts, int topk, float routed_scaling_factor,
                 float* weights, int32_t* ids, void* stream);

/* ------------------------------------------------------------ SQG tables --
 * Tables of kquant/sqg_e4m3.py, 65,536 entries (T12: 4,096), device memory. */
enum { KQ_SQG_RANK_XOR = 0, KQ_SQG_RANK_MIX = 1, KQ_SQG_RANK_K2_OCTILE = 2 };

/* int64 ranks [65536] of every L16 codeword.  KQ_SQG_RANK_XOR:
 * sqg_xor_rank_permutation(bits) (kquant/sqg_e4m3.py:261-285);
 * KQ_SQG_RANK_MIX: sqg_rank_permutation(bits) (:408-438);
 * KQ_SQG_RANK_K2_OCTILE: sqg_k2_eight_stratum_rank_permutation(history_bit)
 * (:356-389, bits ignored). */
int kq_sqg_rank_permutation(int kind, int bits, int history_bit, int64_t* ranks, void* stream);

/* u8 [65536] canonical E4M3 of 1.5 * ndtri((rank + 0.5) / 65536)
 * (sqg_cheb_normal_rank_e4m3_bytes, kquant/sqg_e4m3.py:218-230). */
int kq_sqg_normal_rank_law(uint8_t* law, void* stream);

/* u8 [65536] canonical E4M3 (single zero byte) of fp32 values [65536]
 * (_finite_e4m3_rank_lut, kquant/sqg_e4m3.py:197-208). */
int kq_sqg_finite_rank_lut(const float* values, uint8_t* law, void* stream);

/* status (one uint32, device): bit 0 a NaN byte, bit 1 a decrease between
 * neighbouring entries (kquant/sqg_e4m3.py:209-213). */
int kq_sqg_check_rank_law(const uint8_t* law, uint32_t* status, void* stream);

/* u8 [4096] modal byte of each 16 consecutive ranks, ties to the lower byte
 * (sqg_xor_cheb_t12_rank_lut_bytes, kquant/sqg_e4m3.py:233-257). */
int kq_sqg_modal_compress(const uint8_t* law, uint8_t* t12, void* stream);

/* out[i] = lut[ranks[i] >> shift] for i < n (the label maps of
 * kquant/sqg_e4m3.py:176-179, :289-291, :392-405).  status bit 0: a NaN label
 * was read; bit 1: a rank outside the table (its output byte is 0). */
int kq_sqg_gather(const uint8_t* lut, int64_t lut_len, int shift, const int64_t* ranks, int64_t n,
                  uint8_t* out, uint32_t* status, void* stream);

/* u8 [65536] R44 research labels sqg_e4m3_bytes(bits, "normal")
 * (kquant/sqg_e4m3.py:75-127); status bit 0: a non-finite value. */
int kq_sqg_r44_bytes(int bits, uint8_t* out, uint32_t* status, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KQUANT_AMD_H */
