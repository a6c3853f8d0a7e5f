"""SQG E4M3 reconstruction tables, built on the GPU.

Drop-in for ``kquant/sqg_e4m3.py``: same names, arguments, byte-exact tables
and errors.  Every table is built by a kernel of ``libkquant_amd.so``
(rank permutations, the finite normal staircase, its modal T12 compression,
the label gathers, the R44 research table) and widened to floating point
with the E4M3 decode kernel.  Tables are cached per device, like the
reference's ``lru_cache``; the default ``device="cpu"`` returns CPU tensors
as the reference does.
"""

from __future__ import annotations

from functools import lru_cache

import torch

from . import _native as N

SQG_NORMAL_E4M3 = "sqg-normal-e4m3"
SQG_CHEB_NORMAL_E4M3 = "sqg-cheb-normal-e4m3"
SQG_CHEB = "sqg_cheb"
SQG_XOR_CHEB_T12 = "sqg_xor_cheb_t12"

_TRANSITIONS = 1 << 16


def _validate(bits: int, mode: str) -> None:
    if isinstance(bits, bool) or not isinstance(bits, int) or bits not in (2, 3, 4):
        raise ValueError("SQG supports integer K2, K3, or K4")
    if mode != "normal":
        raise ValueError("the supported R44 mode is 'normal'")


def _gpu() -> torch.device:
    return N.require_gpu()


def _out(t: torch.Tensor, device) -> torch.Tensor:
    return t.to(device=device).contiguous()


def _status(status: torch.Tensor) -> int:
    return int(status.item()) & 0xFFFFFFFF


# ----------------------------------------------------------- permutations --

@lru_cache(maxsize=None)
def _rank(kind: int, bits: int, history_bit: int, index: int) -> torch.Tensor:
    gpu = torch.device("cuda", index)
    ranks = torch.empty(_TRANSITIONS, dtype=torch.int64, device=gpu)
    N.call("kq_sqg_rank_permutation", kind, bits, history_bit, N.ptr(ranks), N.stream(gpu))
    return ranks


def _rank_on(kind: int, bits: int, history_bit: int = 0) -> torch.Tensor:
    return _rank(kind, bits, history_bit, _gpu().index)


def sqg_rank_permutation(bits: int) -> torch.Tensor:
    """Pre-projection quantile rank of every codeword (kquant/sqg_e4m3.py:408-438)."""

    _validate(bits, "normal")
    return _rank_on(N.SQG_RANK_MIX, bits).cpu()


def sqg_xor_rank_permutation(bits: int) -> torch.Tensor:
    """Primary carry-mixed SQG rank of every codeword (kquant/sqg_e4m3.py:260-285)."""

    _validate(bits, "normal")
    return _rank_on(N.SQG_RANK_XOR, bits).cpu()


def sqg_k2_eight_stratum_rank_permutation(history_bit: int = 2) -> torch.Tensor:
    """State-conditioned eight-stratum K2 labelling (kquant/sqg_e4m3.py:356-389)."""

    if isinstance(history_bit, bool) or not isinstance(history_bit, int):
        raise TypeError("K2 eight-stratum history bit must be an integer")
    if not 2 <= history_bit < 16:
        raise ValueError("K2 eight-stratum history bit must be in [2, 15]")
    return _rank_on(N.SQG_RANK_K2_OCTILE, 2, history_bit).cpu()


# ------------------------------------------------------------- rank laws --

def _check_law(law: torch.Tensor) -> torch.Tensor:
    status = torch.empty(1, dtype=torch.int32, device=law.device)
    N.call("kq_sqg_check_rank_law", N.ptr(law), N.ptr(status), N.stream(law.device))
    s = _status(status)
    if s & 1:
        raise RuntimeError("SQG rank law rounded to a non-finite E4M3 value")
    if s & 2:
        raise RuntimeError("SQG rank law is not monotone after E4M3 rounding")
    return law


def _finite_e4m3_rank_lut(values: torch.Tensor) -> torch.Tensor:
    """Round a monotone real rank law to canonical finite E4M3 bytes."""

    if values.ndim != 1 or values.numel() != _TRANSITIONS:
        raise ValueError("SQG rank-law values must contain exactly 65,536 entries")
    (v,), gpu, host = N.to_gpu([values])
    if not v.is_floating_point() or not bool(torch.isfinite(v).all()):
        raise ValueError("SQG rank-law values must be finite floating point")
    v = N.aligned(v.float(), 4)
    law = torch.empty(_TRANSITIONS, dtype=torch.uint8, device=gpu)
    N.call("kq_sqg_finite_rank_lut", N.ptr(v), N.ptr(law), N.stream(gpu))
    _check_law(law)
    return law if host is None else law.to(host)


@lru_cache(maxsize=None)
def _normal_law(index: int) -> torch.Tensor:
    gpu = torch.device("cuda", index)
    law = torch.empty(_TRANSITIONS, dtype=torch.uint8, device=gpu)
    N.call("kq_sqg_normal_rank_law", N.ptr(law), N.stream(gpu))
    return _check_law(law)


@lru_cache(maxsize=None)
def _t12(index: int) -> torch.Tensor:
    gpu = torch.device("cuda", index)
    t12 = torch.empty(_TRANSITIONS // 16, dtype=torch.uint8, device=gpu)
    N.call("kq_sqg_modal_compress", N.ptr(_normal_law(index)), N.ptr(t12), N.stream(gpu))
    return t12


def sqg_cheb_normal_rank_e4m3_bytes() -> torch.Tensor:
    """Exact full-tail normal staircase: E4M3(1.5 ndtri((rank + 0.5) / 2^16))."""

    return _normal_law(_gpu().index).cpu()


def sqg_xor_cheb_t12_rank_lut_bytes() -> torch.Tensor:
    """The 4 KiB modal T12 staircase (one byte per 16 ranks, ties to the lower byte)."""

    return _t12(_gpu().index).cpu()


# ---------------------------------------------------------------- labels --

def _gather(lut: torch.Tensor, shift: int, ranks: torch.Tensor) -> tuple[torch.Tensor, int]:
    out = torch.empty(ranks.numel(), dtype=torch.uint8, device=ranks.device)
    status = torch.empty(1, dtype=torch.int32, device=ranks.device)
    N.call("kq_sqg_gather", N.ptr(lut), lut.numel(), shift, N.ptr(ranks), ranks.numel(), N.ptr(out),
           N.ptr(status), N.stream(ranks.device))
    return out, _status(status)


def _check_rank_lut(rank_lut: torch.Tensor) -> torch.Tensor:
    if rank_lut.dtype != torch.uint8:
        raise TypeError("SQG rank LUT must contain raw uint8 E4M3 labels")
    if rank_lut.ndim != 1 or rank_lut.numel() != _TRANSITIONS:
        raise ValueError("SQG rank LUT must contain exactly 65,536 labels")
    return rank_lut.detach().to(_gpu()).contiguous()


def _labels_from_rank_lut(rank_lut: torch.Tensor, ranks: torch.Tensor, device) -> torch.Tensor:
    out, status = _gather(rank_lut, 0, ranks)
    if status & 1:
        raise ValueError("SQG rank LUT must contain only finite E4M3 labels")
    return _out(out, device)


def sqg_e4m3_bytes_from_rank_lut(bits: int, rank_lut: torch.Tensor, *, device="cpu") -> torch.Tensor:
    """Map a shared rank-indexed E4M3 law onto the SQG graph (kquant/sqg_e4m3.py:159-187)."""

    _validate(bits, "normal")
    lut = _check_rank_lut(rank_lut)
    return _labels_from_rank_lut(lut, _rank_on(N.SQG_RANK_MIX, bits), device)


def sqg_k2_eight_stratum_e4m3_bytes_from_rank_lut(
    rank_lut: torch.Tensor, *, history_bit: int = 2, device="cpu"
) -> torch.Tensor:
    """Map one shared rank staircase onto state-conditioned K2 octiles."""

    lut = _check_rank_lut(rank_lut)
    sqg_k2_eight_stratum_rank_permutation(history_bit)  # argument checks
    return _labels_from_rank_lut(lut, _rank_on(N.SQG_RANK_K2_OCTILE, 2, history_bit), device)


@lru_cache(maxsize=None)
def _xor_t12_labels(bits: int, index: int) -> torch.Tensor:
    out, status = _gather(_t12(index), 4, _rank(N.SQG_RANK_XOR, bits, 0, index))
    if status:
        raise RuntimeError("SQG T12 label gather failed")
    return out


@lru_cache(maxsize=None)
def _cheb_normal_labels(bits: int, index: int) -> torch.Tensor:
    out, status = _gather(_normal_law(index), 0, _rank(N.SQG_RANK_MIX, bits, 0, index))
    if status:
        raise RuntimeError("SQG rank-law label gather failed")
    return out


@lru_cache(maxsize=None)
def _r44(bits: int, index: int) -> torch.Tensor:
    gpu = torch.device("cuda", index)
    out = torch.empty(_TRANSITIONS, dtype=torch.uint8, device=gpu)
    status = torch.empty(1, dtype=torch.int32, device=gpu)
    N.call("kq_sqg_r44_bytes", bits, N.ptr(out), N.ptr(status), N.stream(gpu))
    if _status(status):
        raise RuntimeError("SQG compander produced a non-finite value")
    return out


def sqg_xor_cheb_t12_bytes(bits: int, *, device="cpu") -> torch.Tensor:
    """Primary QSRT-E4M3 labels: T12[xor_rank >> 4] (kquant/sqg_e4m3.py:288-302)."""

    _validate(bits, "normal")
    return _out(_xor_t12_labels(bits, _gpu().index), device)


def sqg_cheb_normal_e4m3_bytes(bits: int) -> torch.Tensor:
    """The exact normal staircase on the mix-rank graph (kquant/sqg_e4m3.py:233-239)."""

    _validate(bits, "normal")
    return _cheb_normal_labels(bits, _gpu().index).cpu()


def sqg_e4m3_bytes(bits: int, mode: str, *, device="cpu") -> torch.Tensor:
    """The 65,536 R44 research labels (kquant/sqg_e4m3.py:75-137)."""

    _validate(bits, mode)
    return _out(_r44(bits, _gpu().index), device)


def sqg_codebook_bytes(bits: int, codebook: str, *, rate_axis: str | None = None,
                       device="cpu") -> torch.Tensor:
    """State-indexed E4M3 labels of a named SQG codebook (kquant/sqg_e4m3.py:305-340)."""

    if codebook == SQG_XOR_CHEB_T12:
        return sqg_xor_cheb_t12_bytes(bits, device=device)
    if codebook == SQG_NORMAL_E4M3:
        return sqg_e4m3_bytes(bits, "normal", device=device)
    if codebook == SQG_CHEB_NORMAL_E4M3:
        return _out(sqg_cheb_normal_e4m3_bytes(bits), device)
    if codebook == SQG_CHEB:
        if rate_axis not in ("k", "n"):
            raise ValueError("the w2-only K2-Q8H4 profile requires rate_axis 'k' or 'n'")
        law = _normal_law(_gpu().index)
        if bits == 2 and rate_axis == "k":
            return sqg_k2_eight_stratum_e4m3_bytes_from_rank_lut(law, history_bit=4, device=device)
        return sqg_e4m3_bytes_from_rank_lut(bits, law, device=device)
    raise ValueError(f"unsupported SQG codebook: {codebook!r}")


# ---------------------------------------------------------------- widening --

def _widen(raw: torch.Tensor, dtype: torch.dtype, device) -> torch.Tensor:
    if not dtype.is_floating_point:
        raise TypeError("SQG codebook dtype must be floating point")
    gpu = _gpu()
    r = raw.to(gpu).contiguous()
    kernel_dtype = dtype if dtype in N.DTYPE_CODES else torch.float32
    out = torch.empty(r.shape, dtype=kernel_dtype, device=gpu)
    N.call("kq_decode_bytes", N.TABLE_E4M3, N.ptr(r), r.numel(), N.DTYPE_CODES[kernel_dtype],
           N.ptr(out), N.stream(gpu))
    # float32 holds every E4M3 value exactly, so wider types are an exact cast
    return out.to(device=device, dtype=dtype).contiguous()


def sqg_e4m3_codebook(bits: int, mode: str, *, device="cpu", dtype=torch.float16) -> torch.Tensor:
    """The R44 table widened from its exact E4M3 wire values."""

    if not dtype.is_floating_point:
        raise TypeError("SQG codebook dtype must be floating point")
    _validate(bits, mode)
    return _widen(_r44(bits, _gpu().index), dtype, device)


def sqg_e4m3_codebook_from_rank_lut(bits: int, rank_lut: torch.Tensor, *, device="cpu",
                                    dtype=torch.float16) -> torch.Tensor:
    """A shared rank-indexed E4M3 law, labelled and widened."""

    if not dtype.is_floating_point:
        raise TypeError("SQG codebook dtype must be floating point")
    raw = sqg_e4m3_bytes_from_rank_lut(bits, rank_lut, device=_gpu())
    return _widen(raw, dtype, device)


def sqg_codebook(bits: int, codebook: str, *, rate_axis: str | None = None, device="cpu",
                 dtype=torch.float16) -> torch.Tensor:
    """A named SQG codebook widened from its exact E4M3 labels."""

    if not dtype.is_floating_point:
        raise TypeError("SQG codebook dtype must be floating point")
    raw = sqg_codebook_bytes(bits, codebook, rate_axis=rate_axis, device=_gpu())
    return _widen(raw, dtype, device)
