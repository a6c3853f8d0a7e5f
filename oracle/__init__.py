"""TEST INFRASTRUCTURE ONLY — the CPU oracle of the kquant hot path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or as the timed CPU baseline).
The kquant_amd product path never imports, links or calls anything here.

Contents, each following the cited reference code:
  mx_quantize / mx_dequant / pack_codes / unpack_codes
      C restatement in mx_oracle.c (kquant/mxfp8.py:34-50, 79-84;
      kquant/io/mxfp4.py:19-64), loaded through ctypes.
  weighted_covariance / accumulate_hessian / finalize_damping / covariance_comparison
      numpy restatements of kquant/candidate_hessian.py:70-112, 219-258,
      kquant/capture.py:713-730, kquant/exl3_encoder_backend.py:1613-1625.
  situ / swiglu / reference_rank
      numpy restatements of kquant/tp_simulator.py:83-94 and
      scripts/closure_exl3_layer.py:557-598.
  reduce_partials / kimi_topk / comparison_metrics / expert_output
      kquant/tp_simulator.py:72-80, 114-160; kquant/pack/qsrt_validation.py:240-258.
  sqg_* tables
      kquant/sqg_e4m3.py:38-60, 84-127, 197-302, 356-438.
  sqg_quantize_tiles / procedural_labels / sqg_quantize_tiles_procedural
      C restatement in sqg_viterbi.c of the SQG trellis (Viterbi) quantizer,
      kquant/csrc/qsrt_quantize_tiles_kernel.cuh, kquant/csrc/sqg_quantize.cu,
      and of the MCG / MUL1 procedural codebooks,
      kquant/csrc/exl3_compat/quant/codebook.cuh:27-92.
  scale_plane (submodule): X4T and KQSC scale-plane codecs
      kquant/x4t.py, kquant/mxfp4_scale_codec.py.
  ldl (submodule): the encoder's Hessian finalize — Hadamard rotation,
      regularization, block LDL — kquant/exl3_encoder_backend.py:288-386,
      1588-1663, kquant/exl3_reference.py:195-212.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "libmx_oracle.so"
_lib = None

E2M1_LUT = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run __graft_entry__.build())")
        lib = ctypes.CDLL(str(_LIB_PATH))
        vp, i64, i32, u32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32
        lib.mxo_quantize.argtypes = [i32, i32, vp, i64, i64, i64, vp, vp]
        lib.mxo_quantize.restype = None
        lib.mxo_dequant.argtypes = [i32, vp, vp, i64, i64, vp]
        lib.mxo_dequant.restype = None
        lib.mxo_unpack_codes.argtypes = [vp, i64, vp]
        lib.mxo_unpack_codes.restype = None
        lib.mxo_pack_codes.argtypes = [vp, i64, vp]
        lib.mxo_pack_codes.restype = None
        lib.sqgo_quantize_tiles.argtypes = [vp, ctypes.c_int64, vp, i32, i32, vp, vp]
        lib.sqgo_quantize_tiles.restype = None
        lib.sqgo_quantize_tiles_f16.argtypes = [vp, ctypes.c_int64, vp, i32, i32, vp, vp]
        lib.sqgo_quantize_tiles_f16.restype = None
        lib.sqgo_procedural_labels.argtypes = [i32, vp]
        lib.sqgo_procedural_labels.restype = None
        lib.sqgo_f64_to_f16.argtypes = [vp, ctypes.c_int64, vp]
        lib.sqgo_f64_to_f16.restype = None
        lib.sqgo_argmin_edges.argtypes = [vp, i32]
        lib.sqgo_argmin_edges.restype = i32
        lib.mxo_f32_to_e4m3.argtypes = [ctypes.c_float]
        lib.mxo_f32_to_e4m3.restype = u32
        lib.mxo_f32_to_e2m1.argtypes = [ctypes.c_float]
        lib.mxo_f32_to_e2m1.restype = u32
        lib.mxo_cast_e4m3.argtypes = [vp, i64, vp]
        lib.mxo_cast_e4m3.restype = None
        lib.mxo_cast_e2m1.argtypes = [vp, i64, vp]
        lib.mxo_cast_e2m1.restype = None
        lib.mxo_e4m3_value.argtypes = [u32]
        lib.mxo_e4m3_value.restype = ctypes.c_float
        _lib = lib
    return _lib


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


_DT = {"bf16": 0, "f16": 1, "f32": 2}


def mx_quantize(fmt: str, x: np.ndarray, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """MX quantize of a [rows, k] array.

    fmt: "mxfp8" or "mxfp4".  dtype: "bf16" (x holds uint16 bf16 bit patterns),
    "f16" (float16) or "f32" (float32).  Returns (codes, scales) as uint8:
    codes [rows, k] for MXFP8, [rows, k/2] packed for MXFP4.
    """
    lib = _load()
    if dtype == "bf16":
        x = np.ascontiguousarray(x, dtype=np.uint16)
    elif dtype == "f16":
        x = np.ascontiguousarray(x, dtype=np.float16)
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    f = 0 if fmt == "mxfp8" else 1
    q = np.zeros((rows, k if f == 0 else k // 2), dtype=np.uint8)
    s = np.zeros((rows, k // 32), dtype=np.uint8)
    lib.mxo_quantize(f, _DT[dtype], _ptr(x), k, rows, k, _ptr(q), _ptr(s))
    return q, s


def mx_dequant(fmt: str, q: np.ndarray, s: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
    """fp32 [rows, k] = value(code) * 2^(s-127) (scale byte 255 -> inf).

    ``out`` (optional): a C-contiguous float32 [rows, k] array to write into,
    so that callers dequantizing many matrices reuse one buffer."""
    lib = _load()
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    rows = q.shape[0]
    k = s.shape[1] * 32
    if out is None:
        out = np.empty((rows, k), dtype=np.float32)
    elif out.shape != (rows, k) or out.dtype != np.float32 or not out.flags.c_contiguous:
        raise ValueError("out must be a C-contiguous float32 [rows, k] array")
    lib.mxo_dequant(0 if fmt == "mxfp8" else 1, _ptr(q), _ptr(s), rows, k, _ptr(out))
    return out


def unpack_codes(packed: np.ndarray) -> np.ndarray:
    lib = _load()
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    codes = np.zeros(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    lib.mxo_unpack_codes(_ptr(packed), packed.size, _ptr(codes))
    return codes


def pack_codes(codes: np.ndarray) -> np.ndarray:
    lib = _load()
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    packed = np.zeros(codes.shape[:-1] + (codes.shape[-1] // 2,), dtype=np.uint8)
    lib.mxo_pack_codes(_ptr(codes), codes.size, _ptr(packed))
    return packed


def sqg_quantize_tiles(tiles: np.ndarray, lut: np.ndarray, bits: int, tailbite_context: int = 128):
    """The SQG trellis quantizer (sqg_viterbi.c; kquant/csrc/qsrt_quantize_tiles_kernel.cuh
    with the SQG labels of kquant/csrc/sqg_quantize.cu): tiles float32 [n, 256],
    lut uint8 [65536] E4M3 labels in state order -> (reconstructed float32
    [n, 256], states int16 [n, 256])."""
    lib = _load()
    x = np.ascontiguousarray(tiles, dtype=np.float32).reshape(-1, 256)
    lab = np.ascontiguousarray(lut, dtype=np.uint8)
    out = np.empty_like(x)
    states = np.empty(x.shape, dtype=np.int16)
    lib.sqgo_quantize_tiles(_ptr(x), x.shape[0], _ptr(lab), bits, tailbite_context, _ptr(out), _ptr(states))
    return out, states


def procedural_labels(codebook: int) -> np.ndarray:
    """fp16 labels (as float16) of all 65536 states of the procedural EXL3
    codebook 1 (MCG) or 2 (MUL1), sqg_viterbi.c / codebook.cuh:27-92."""
    if codebook not in (1, 2):
        raise ValueError("procedural codebook must be 1 (MCG) or 2 (MUL1)")
    out = np.empty(65536, dtype=np.uint16)
    _load().sqgo_procedural_labels(codebook, _ptr(out))
    return out.view(np.float16)


def sqg_quantize_tiles_procedural(tiles: np.ndarray, bits: int, codebook: int, tailbite_context: int = 128):
    """The trellis quantizer against a procedural codebook
    (quantize_tiles_procedural_cuda, kquant/csrc/sqg_quantize.cu:261-330)."""
    lib = _load()
    lab = procedural_labels(codebook).view(np.uint16)
    x = np.ascontiguousarray(tiles, dtype=np.float32).reshape(-1, 256)
    out = np.empty_like(x)
    states = np.empty(x.shape, dtype=np.int16)
    lib.sqgo_quantize_tiles_f16(_ptr(x), x.shape[0], _ptr(lab), bits, tailbite_context, _ptr(out), _ptr(states))
    return out, states


def f64_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """sqg_viterbi.c's fp16 rounding (nearest, ties to even), as uint16 bits."""
    lib = _load()
    v = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty(v.shape, dtype=np.uint16)
    lib.sqgo_f64_to_f16(_ptr(v), v.size, _ptr(out))
    return out


def sqg_argmin_edges(costs_f16_bits: np.ndarray) -> int:
    """sqg_viterbi.c's argmin over one cost buffer (uint16 fp16 bits): the
    smallest cost, ties by the key order the reference's reductions give."""
    lib = _load()
    c = np.ascontiguousarray(costs_f16_bits, dtype=np.uint16)
    return int(lib.sqgo_argmin_edges(_ptr(c), c.size))


def f32_to_e4m3(values: np.ndarray) -> np.ndarray:
    """torch's float32 -> float8_e4m3fn cast (ties to even, >464 -> NaN)."""
    lib = _load()
    flat = np.ascontiguousarray(values, dtype=np.float32).ravel()
    out = np.zeros(flat.size, dtype=np.uint8)
    lib.mxo_cast_e4m3(_ptr(flat), flat.size, _ptr(out))
    return out.reshape(np.shape(values))


def f32_to_e2m1(values: np.ndarray) -> np.ndarray:
    """Nearest E2M1 code, ties to the even code, sign kept (no clamping)."""
    lib = _load()
    flat = np.ascontiguousarray(values, dtype=np.float32).ravel()
    out = np.zeros(flat.size, dtype=np.uint8)
    lib.mxo_cast_e2m1(_ptr(flat), flat.size, _ptr(out))
    return out.reshape(np.shape(values))


def e4m3_values(codes: np.ndarray) -> np.ndarray:
    lib = _load()
    table = np.array([lib.mxo_e4m3_value(c) for c in range(256)], dtype=np.float32)
    return table[np.asarray(codes, dtype=np.uint8)]


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest even), returned as uint16 bit patterns."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


# --------------------------------------------------------------- SQG-E4M3 --
# kquant/sqg_e4m3.py:197-302.  Integer/E4M3 table constructions used by the
# QSRT trellis labels; pinned by the SHA-256 known answers of
# tests/test_sqg_e4m3.py:32-69.

TRANSITIONS = 1 << 16


def finite_e4m3_rank_lut(values: np.ndarray) -> np.ndarray:
    """kquant/sqg_e4m3.py:197-214: RNE to E4M3, canonical zero, monotone."""
    if values.ndim != 1 or values.size != TRANSITIONS:
        raise ValueError("SQG rank-law values must contain exactly 65,536 entries")
    raw = f32_to_e4m3(values.astype(np.float32))
    raw[(raw & 0x7F) == 0] = 0
    decoded = e4m3_values(raw)
    if not np.all(np.isfinite(decoded)):
        raise RuntimeError("SQG rank law rounded to a non-finite E4M3 value")
    if not np.all(decoded[1:] >= decoded[:-1]):
        raise RuntimeError("SQG rank law is not monotone after E4M3 rounding")
    return raw


def sqg_cheb_normal_rank_e4m3_bytes() -> np.ndarray:
    """kquant/sqg_e4m3.py:218-230: 1.5 * ndtri((rank + 0.5) / 65536) in f64."""
    from scipy.special import ndtri

    probability = (np.arange(TRANSITIONS, dtype=np.float64) + 0.5) / TRANSITIONS
    return finite_e4m3_rank_lut(1.5 * ndtri(probability))


def sqg_xor_cheb_t12_rank_lut_bytes() -> np.ndarray:
    """kquant/sqg_e4m3.py:233-257: modal byte per 16 ranks, ties -> lower byte."""
    exact = sqg_cheb_normal_rank_e4m3_bytes().reshape(1 << 12, 16)
    out = np.empty(1 << 12, dtype=np.uint8)
    for i, block in enumerate(exact):
        labels, counts = np.unique(block, return_counts=True)
        out[i] = labels[counts == counts.max()].min()
    return out


def _reverse_low_bits(values: np.ndarray, bits: int) -> np.ndarray:
    result = np.zeros_like(values)
    for index in range(bits):
        result |= ((values >> index) & 1) << (bits - 1 - index)
    return result


def sqg_xor_rank_permutation(bits: int) -> np.ndarray:
    """kquant/sqg_e4m3.py:261-285 (carry-mixed SQG rank of every codeword)."""
    if bits not in (2, 3, 4):
        raise ValueError("SQG supports integer K2, K3, or K4")
    width = 16 - bits
    history_mask = (1 << width) - 1
    codeword = np.arange(TRANSITIONS, dtype=np.int64)
    history = codeword >> bits
    branch = codeword & ((1 << bits) - 1)
    mixed = history ^ (history >> 11)
    mixed ^= (mixed << 11) & history_mask
    product = (0x3FA7D929 * mixed + 0xC928FD8E) & 0xFFFFFFFF
    phase = product & history_mask
    syndrome = product >> (32 - bits)
    stratum = _reverse_low_bits(branch, bits) ^ syndrome
    return (stratum << width) | phase


def sqg_xor_cheb_t12_bytes(bits: int) -> np.ndarray:
    """kquant/sqg_e4m3.py:288-302: labels = T12[rank >> 4]."""
    return sqg_xor_cheb_t12_rank_lut_bytes()[sqg_xor_rank_permutation(bits) >> 4]


def _mix_width(values, width, ma, mb, sa, sb, sc):
    """kquant/sqg_e4m3.py:38-60: xorshift / odd multiply mixer modulo 2^width."""
    mask = (1 << width) - 1
    r = values & mask
    for m, s in ((ma | 1, sa), (mb | 1, sb)):
        r ^= r >> min(max(s, 1), width - 1)
        r = (r * m) & mask
    r ^= r >> min(max(sc, 1), width - 1)
    return r & mask


def sqg_rank_permutation(bits: int) -> np.ndarray:
    """kquant/sqg_e4m3.py:408-438 (and :96-115): mix-width SQG rank."""
    width = 16 - bits
    t = np.arange(TRANSITIONS, dtype=np.int64)
    history, branch = t >> bits, t & ((1 << bits) - 1)
    phase = _mix_width(history, width, 0x65AF, 0x16BF, 6, 4, 5)
    syndrome = _mix_width(history ^ 0x5105, width, 0x8693, 0x2A21, 2, 4, 4) & ((1 << bits) - 1)
    stratum = (7 * (_reverse_low_bits(branch, bits) ^ syndrome)) & ((1 << bits) - 1)
    return (stratum << width) | phase


def sqg_k2_eight_stratum_rank_permutation(history_bit: int = 2) -> np.ndarray:
    """kquant/sqg_e4m3.py:356-389: K3 ranks of the codeword with bits 2, h swapped."""
    t = np.arange(TRANSITIONS, dtype=np.int64)
    swap = ((t >> 2) ^ (t >> history_bit)) & 1
    return sqg_rank_permutation(3)[t ^ (swap << 2) ^ (swap << history_bit)]


def sqg_r44_bytes(bits: int) -> np.ndarray:
    """kquant/sqg_e4m3.py:84-127: R44 compander of the clipped mix-rank probability.

    numpy float64 element-wise arithmetic rounds each product and sum
    separately, as the reference's tensor operations do.
    """
    p_coef = (1.25667142, 2.87422731, -9.02398882, 5.36810336, -0.46703015)
    q_coef = (1.0, 2.07630930, -8.08332684, 6.32135736, -1.31208298)
    rank = sqg_rank_permutation(bits)
    prob = np.clip((rank.astype(np.float64) + 0.5) / TRANSITIONS, 1 / 2048, 1 - 1 / 2048)
    a = 2.0 * prob - 1.0
    x = a * a
    num = np.full_like(x, p_coef[-1])
    den = np.full_like(x, q_coef[-1])
    for c in reversed(p_coef[:-1]):
        num = num * x + c
    for c in reversed(q_coef[:-1]):
        den = den * x + c
    values = (1.5 * (a * num / den)).astype(np.float32)
    return f32_to_e4m3(values)


# ---------------------------------------------------------------- Hessian --

def weighted_covariance(rows: np.ndarray, weights: np.ndarray, chunk_rows: int = 256):
    """kquant/candidate_hessian.py:70-112 in numpy float32.

    accumulator.addmm_(values.T, values * w[:, None]) per chunk of rows, then
    / float(sum(w) in f64), then (H + H^T) * 0.5.  Returns (H f32, denom).
    """
    rows = np.asarray(rows)
    weights = np.asarray(weights, dtype=np.float32)
    if rows.ndim != 2 or weights.ndim != 1 or rows.shape[0] != weights.shape[0]:
        raise ValueError("invalid covariance sample shapes")
    if not rows.shape[0] or not rows.shape[1]:
        raise ValueError("covariance samples must be nonempty")
    k = rows.shape[1]
    acc = np.zeros((k, k), dtype=np.float32)
    denom = float(weights.astype(np.float64).sum())
    if not np.isfinite(denom) or denom <= 0:
        raise ValueError("covariance weights must have a positive finite sum")
    for b in range(0, rows.shape[0], chunk_rows):
        v = rows[b : b + chunk_rows].astype(np.float32)
        w = weights[b : b + chunk_rows]
        acc += v.T @ (v * w[:, None])
    cov = acc / np.float32(denom)
    return ((cov + cov.T) * np.float32(0.5)).astype(np.float32), denom


def accumulate_hessian(rows: np.ndarray, weights: np.ndarray, chunk_rows: int = 1024):
    """kquant/capture.py:713-730: unnormalized fp32 accumulator and the f64
    sum of the weights, chunked addmm_."""
    rows = np.asarray(rows)
    weights = np.asarray(weights, dtype=np.float32)
    k = rows.shape[1]
    acc = np.zeros((k, k), dtype=np.float32)
    denom = 0.0
    for b in range(0, rows.shape[0], max(chunk_rows, 1)):
        v = rows[b : b + chunk_rows].astype(np.float32)
        w = weights[b : b + chunk_rows]
        acc += v.T @ (v * w[:, None])
        denom += float(w.astype(np.float64).sum())
    return acc, denom


def damp_diagonal(h: np.ndarray, sigma_reg: float) -> np.ndarray:
    """kquant/exl3_encoder_backend.py:1620-1625: H.diag += sigma * mean(diag)."""
    h = np.array(h, dtype=np.float32, copy=True)
    diag_mean = np.float32(np.diag(h).astype(np.float32).mean(dtype=np.float32))
    idx = np.arange(h.shape[0])
    h[idx, idx] += np.float32(sigma_reg) * diag_mean
    return h


def covariance_comparison(reference: np.ndarray, candidate: np.ndarray) -> dict:
    """kquant/candidate_hessian.py:219-258 (relative Frobenius in f64 etc.)."""
    ref32 = np.asarray(reference, dtype=np.float32)
    cand32 = np.asarray(candidate, dtype=np.float32)
    ref, cand = ref32.astype(np.float64), cand32.astype(np.float64)
    ref_norm = np.linalg.norm(ref)
    rd, cd = np.diag(ref), np.diag(cand)
    dd = np.linalg.norm(rd) * np.linalg.norm(cd)
    tr = np.trace(ref)
    diff = (cand32 - ref32).astype(np.float64)  # (candidate - reference).double(): fp32 difference
    return {
        "relative_frobenius_difference": float(np.linalg.norm(diff) / ref_norm) if ref_norm > 0 else float("inf"),
        "trace_ratio": float(np.trace(cand) / tr) if tr != 0 else float("inf"),
        "diagonal_cosine_similarity": float(rd @ cd / dd) if dd > 0 else 0.0,
        "candidate_symmetry_max_abs": float(np.abs(cand32 - cand32.T).max()),
    }


# -------------------------------------------------------------- MoE expert --

def _sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


def situ(gate: np.ndarray, up: np.ndarray, beta: float = 4.0, linear_beta: float = 25.0) -> np.ndarray:
    """kquant/tp_simulator.py:83-94 in float32 (before the output cast)."""
    g = gate.astype(np.float32)
    u = up.astype(np.float32)
    gate_value = np.float32(beta) * np.tanh(g / np.float32(beta)) * _sigmoid(g)
    up_value = np.float32(linear_beta) * np.tanh(u / np.float32(linear_beta))
    return (gate_value * up_value).astype(np.float32)


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """silu(gate) * up in float32."""
    g = gate.astype(np.float32)
    return (g * _sigmoid(g) * up.astype(np.float32)).astype(np.float32)


def reduce_partials(partials: list[np.ndarray]) -> np.ndarray:
    """kquant/tp_simulator.py:72-80: fp32 sum of rank partials in rank order."""
    acc = np.zeros_like(np.asarray(partials[0], dtype=np.float32))
    for p in partials:
        acc = (acc + np.asarray(p, dtype=np.float32)).astype(np.float32)
    return acc


def kimi_topk(logits: np.ndarray, bias: np.ndarray, topk: int, scale: float = 1.0):
    """kquant/tp_simulator.py:114-134 in float64 arithmetic on fp32 inputs:
    sigmoid scores, top-k of score + bias (descending, lower id on ties),
    weights = chosen scores / their sum * scale.  Returns (weights, ids, keys)."""
    scores = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    keys = scores + bias.astype(np.float64)[None, :]
    order = np.lexsort((np.broadcast_to(np.arange(keys.shape[1]), keys.shape), -keys), axis=1)
    ids = order[:, :topk]
    chosen = np.take_along_axis(scores, ids, axis=1)
    weights = chosen / chosen.sum(axis=1, keepdims=True) * scale
    return weights, ids.astype(np.int32), np.take_along_axis(keys, order, axis=1)


def comparison_metrics(reference: np.ndarray, actual: np.ndarray) -> dict[str, float]:
    """kquant/tp_simulator.py:137-160 in float64 (diff formed in float32)."""
    r = reference.astype(np.float32).ravel()
    a = actual.astype(np.float32).ravel()
    d = (a - r).astype(np.float64)
    r64, a64 = r.astype(np.float64), a.astype(np.float64)
    rn = np.sqrt(np.sum(r64 * r64))
    cos = np.sum(r64 * a64) / np.sqrt(max(np.sum(r64 * r64) * np.sum(a64 * a64), 1e-16))
    return {
        "relative_l2": float(np.sqrt(np.sum(d * d)) / max(rn, np.finfo(np.float32).tiny)),
        "max_abs": float(np.max(np.abs(d))) if d.size else 0.0,
        "cosine": float(cos),
    }


def expert_output(x: np.ndarray, w1: np.ndarray, w3: np.ndarray, w2: np.ndarray,
                  activation: str = "situ") -> np.ndarray:
    """kquant/pack/qsrt_validation.py:240-258 (official_expert_output) with
    dense dequantized matrices [out, in]: float64 products, fp32 activation."""
    x64 = x.astype(np.float64)
    gate = (x64 @ w1.astype(np.float64).T).astype(np.float32)
    up = (x64 @ w3.astype(np.float64).T).astype(np.float32)
    mid = situ(gate, up) if activation == "situ" else swiglu(gate, up)
    return mid.astype(np.float64) @ w2.astype(np.float64).T


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def mx_roundtrip_rows(fmt: str, x: np.ndarray) -> np.ndarray:
    """dequant(quant(x)) row by row for a float32 array holding bf16 values
    (the operand an activation-quantized GEMM multiplies)."""
    q, sc = mx_quantize(fmt, f32_to_bf16_bits(np.asarray(x, np.float32)), "bf16")
    return mx_dequant(fmt, q, sc)


def moe_forward(
    x: np.ndarray,
    route_ids: np.ndarray,
    route_weights: np.ndarray,
    w13: callable,
    w2: callable,
    activation: str = "situ",
    tokens: np.ndarray | None = None,
    intermediate_bf16: bool = True,
    act_format: str | None = None,
) -> np.ndarray:
    """Routed MoE forward of scripts/closure_exl3_layer.py:557-598 (tp=1).

    x: float32 [T, H] (bf16 values); route_ids int [T, k]; route_weights f32
    [T, k]; w13(e) -> float32 [2I, H] (gate rows first), w2(e) -> float32
    [H, I], both dequantized weights.  For every expert: gate/up fp32 GEMMs,
    activation in fp32, the activated intermediate rounded to bf16 (the
    down-projection operand, as F.linear in bf16 makes it), down GEMM in
    fp32, contribution = route_weight * partial, summed per token in fp32.
    ``tokens`` restricts the output to a subset of token rows (the result
    has one row per listed token).

    ``act_format`` "mxfp8" / "mxfp4" restates the activation-quantized mode
    (no kquant counterpart): every token row and every bf16 intermediate row
    is MX-quantized along its length with the rule of ``mx_quantize`` and
    dequantized before its GEMM, so the GEMMs see exactly the operands the
    block-scaled MFMA multiplies.
    """
    act = situ if activation == "situ" else swiglu
    T = x.shape[0]
    if act_format is not None:
        x = mx_roundtrip_rows(act_format, x)
    rows = np.arange(T) if tokens is None else np.asarray(tokens)
    pos = {int(t): i for i, t in enumerate(rows)}
    sub_ids = route_ids[rows]
    out = None
    for e in np.unique(sub_ids):
        sel_t, sel_s = np.nonzero(sub_ids == e)
        tok = rows[sel_t]
        w13e = w13(int(e))
        w2e = w2(int(e))
        inter = w13e.shape[0] // 2
        xe = x[tok].astype(np.float32)
        gate = xe @ w13e[:inter].T
        up = xe @ w13e[inter:].T
        a = act(gate, up)
        if intermediate_bf16:
            a = round_bf16(a)
        if act_format is not None:
            a = mx_roundtrip_rows(act_format, a)
        partial = a @ w2e.T
        if out is None:
            out = np.zeros((rows.size, w2e.shape[0]), dtype=np.float32)
        contrib = route_weights[tok, sel_s][:, None].astype(np.float32) * partial
        np.add.at(out, np.array([pos[int(t)] for t in tok]), contrib)
    return out


def mx_tile(packed: np.ndarray, scale: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """MFMA-tiled MXFP4 layout of one matrix (see kq_mx_tile_weights):
    tiles [rows/16, k/128, 64 lanes, 16 B] and scales [rows/16, k/128, 64]."""
    rows, kh = packed.shape
    k = kh * 2
    p = packed.reshape(rows // 16, 16, k // 128, 4, 16)        # rg, m, c, g, j
    q_t = p.transpose(0, 2, 3, 1, 4).reshape(rows // 16, k // 128, 64, 16)  # lane = g*16 + m
    s = scale.reshape(rows // 16, 16, k // 128, 4)               # rg, m, c, g
    s_t = s.transpose(0, 2, 3, 1).reshape(rows // 16, k // 128, 64)
    return np.ascontiguousarray(q_t), np.ascontiguousarray(s_t)
