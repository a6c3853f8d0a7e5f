"""X4T exact coding of MXFP4 E8M0 scale planes, on the GPU.

Drop-in for the scale-component surface of ``kquant/x4t.py``:
``pack_x4t_scale_components`` (:90-130), ``x4t_scale_storage_bytes``
(:201-222), ``x4t_scale_exception_count`` (:225-234), ``effective_x4t_bpw``
(:133-139) and the validating decode ``_decode_scale_components``
(:477-524).  Same layouts, canonical choices and error messages:

  fixed stream  per 16-row tile: 16 base bytes, then 16 rows of
                ceil(cols/8) selector bytes (bit c%8 of byte c/8 set when the
                value is base + 1; base = the adjacent pair covering most of
                the row, lowest base on ties);
  exceptions    uint32 ``position | value << 24`` for every value outside its
                row's pair, in row-major position order.

All work runs in ``libkquant_amd.so``; CPU inputs are processed on the
current GPU and results come back on the input's device.  The batched forms
(``pack_x4t_scale_components_batched`` / ``decode_x4t_scale_components_batched``)
code many experts' planes in one launch each, for the all-expert cost pass
and for predecoding the experts a layer is about to use.
"""

from __future__ import annotations

import math

import torch

from . import _native as N

X4T_VERSION = 2
X4T_TILE_ROWS = 16
X4T_POSITION_BITS = 24
X4T_POSITION_MASK = (1 << X4T_POSITION_BITS) - 1

_NONE = 0xFFFFFFFF


def _validate_scale(scale: torch.Tensor) -> tuple[int, int]:
    """kquant/x4t.py:51-68, accepting GPU tensors as well."""

    if (
        scale.dtype != torch.uint8
        or scale.ndim != 2
        or scale.device.type not in ("cpu", "cuda")
        or not scale.is_contiguous()
    ):
        raise ValueError("X4T scale must be a contiguous two-dimensional CPU uint8 tensor")
    rows, columns = map(int, scale.shape)
    if not rows or rows % X4T_TILE_ROWS:
        raise ValueError("X4T scale rows must be a nonzero multiple of 16")
    if not 1 <= columns <= 255:
        raise ValueError("X4T scale columns must lie in 1..255")
    if rows * columns > X4T_POSITION_MASK:
        raise ValueError("X4T logical scale plane exceeds its 24-bit position field")
    return rows, columns


def x4t_fixed_bytes(rows: int, columns: int) -> int:
    """Length of the fixed stream of a [rows, columns] plane."""

    return (rows // X4T_TILE_ROWS) * X4T_TILE_ROWS * (1 + math.ceil(columns / 8))


def _analyze(s: torch.Tensor, mats: int, rows: int, columns: int, gpu: torch.device):
    fixed = torch.empty(mats * x4t_fixed_bytes(rows, columns), dtype=torch.uint8, device=gpu)
    tiles = mats * rows // X4T_TILE_ROWS
    offsets = torch.empty(tiles + 1, dtype=torch.int64, device=gpu)
    N.call("kq_x4t_analyze", N.ptr(s), mats, rows, columns, N.ptr(fixed), N.ptr(offsets),
           N.stream(gpu))
    return fixed, offsets


def _emit(s, mats, rows, columns, fixed, offsets, gpu) -> torch.Tensor:
    total = int(offsets[-1].item())
    exceptions = torch.empty(max(total, 1), dtype=torch.uint32, device=gpu)
    if total:
        N.call("kq_x4t_emit_exceptions", N.ptr(s), mats, rows, columns, N.ptr(fixed),
               N.ptr(offsets), N.ptr(exceptions), N.stream(gpu))
    return exceptions[:total]


def pack_x4t_scale_components(scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Return X4T's fixed stream (uint8) and exception words (uint32)."""

    rows, columns = _validate_scale(scale)
    (s,), gpu, host = N.to_gpu([scale])
    fixed, offsets = _analyze(s, 1, rows, columns, gpu)
    exceptions = _emit(s, 1, rows, columns, fixed, offsets, gpu)
    if host is not None:
        return fixed.to(host), exceptions.to(host)
    return fixed, exceptions


def _exception_total(scale: torch.Tensor) -> int:
    rows, columns = _validate_scale(scale)
    (s,), gpu, _ = N.to_gpu([scale])
    _, offsets = _analyze(s, 1, rows, columns, gpu)
    return int(offsets[-1].item())


def x4t_scale_exception_count(scale: torch.Tensor) -> int:
    """Exact number of uint32 exceptions in a scale plane."""

    return _exception_total(scale)


def x4t_scale_storage_bytes(scale: torch.Tensor) -> int:
    """Fixed-stream plus exception bytes, without materialising them."""

    rows, columns = _validate_scale(scale)
    return x4t_fixed_bytes(rows, columns) + 4 * _exception_total(scale)


def effective_x4t_bpw(scale: torch.Tensor) -> float:
    """Nibble plane plus X4T scale-tensor bytes in bits per weight."""

    rows, columns = _validate_scale(scale)
    return 4.0 + x4t_scale_storage_bytes(scale) * 8 / (rows * columns * 32)


def pack_x4t_scale_components_batched(
    scales: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Code ``mats`` planes [mats, rows, columns] in one pass.

    Returns (fixed uint8 [mats, fixed_bytes], exceptions uint32 [total],
    offsets int64 [mats + 1]); matrix m's exceptions are
    ``exceptions[offsets[m]:offsets[m+1]]`` with matrix-local positions, the
    same words ``pack_x4t_scale_components(scales[m])`` returns.
    """

    if (
        scales.dtype != torch.uint8
        or scales.ndim != 3
        or not scales.is_contiguous()
        or scales.shape[0] < 1
    ):
        raise ValueError("X4T scales must be a contiguous nonempty three-dimensional uint8 tensor")
    mats = int(scales.shape[0])
    rows, columns = _validate_scale(scales[0])
    (s,), gpu, host = N.to_gpu([scales])
    fixed, offsets = _analyze(s, mats, rows, columns, gpu)
    exceptions = _emit(s, mats, rows, columns, fixed, offsets, gpu)
    per_mat = offsets[:: rows // X4T_TILE_ROWS].contiguous()
    out = (fixed.view(mats, -1), exceptions, per_mat)
    if host is not None:
        out = tuple(t.to(host) for t in out)
    return out


def decode_scale_components(
    fixed: torch.Tensor,
    exceptions: torch.Tensor,
    *,
    rows: int,
    columns: int,
) -> torch.Tensor:
    """Validating decode (kquant/x4t.py:477-524), same errors in the same order."""

    selector_bytes = math.ceil(columns / 8)
    tile_bytes = X4T_TILE_ROWS * (1 + selector_bytes)
    if (
        fixed.dtype != torch.uint8
        or fixed.numel() != (rows // X4T_TILE_ROWS) * tile_bytes
        or rows <= 0
        or rows % X4T_TILE_ROWS
        or not 1 <= columns <= 255
        or rows * columns > X4T_POSITION_MASK
    ):
        raise ValueError("X4T fixed scale tensor has invalid geometry")
    if exceptions.dtype != torch.uint32 or exceptions.ndim != 1:
        raise ValueError("X4T exception tensor must be one-dimensional uint32")
    (f, e), gpu, host = N.to_gpu([fixed.reshape(-1), exceptions])
    f = f.contiguous()
    e = N.aligned(e, 4) if e.numel() else torch.empty(1, dtype=torch.uint32, device=gpu)
    out = torch.empty((rows, columns), dtype=torch.uint8, device=gpu)
    status = torch.empty(4, dtype=torch.uint32, device=gpu)
    N.call("kq_x4t_decode", N.ptr(f), N.ptr(e), int(exceptions.numel()), None, 1, rows, columns,
           N.ptr(out), N.ptr(status), N.stream(gpu))
    padding, bad_pos, bad_val, noncanonical = (int(v) for v in status.view(torch.int32).cpu().tolist())
    bad_pos &= _NONE
    bad_val &= _NONE
    if padding:
        raise ValueError("X4T selector has nonzero padding bits")
    if bad_pos != _NONE or bad_val != _NONE:
        if bad_pos <= bad_val:
            raise ValueError("X4T exception positions must be valid and strictly increasing")
        raise ValueError("X4T exception redundantly names an adjacent-palette value")
    if noncanonical:
        raise ValueError("X4T safetensors scale stream is not canonical")
    return out if host is None else out.to(host)


_decode_scale_components = decode_scale_components


def decode_x4t_scale_components_batched(
    fixed: torch.Tensor,
    exceptions: torch.Tensor,
    offsets: torch.Tensor,
    *,
    rows: int,
    columns: int,
) -> torch.Tensor:
    """Trusted predecode of ``mats`` planes into uint8 [mats, rows, columns].

    ``fixed`` [mats, fixed_bytes], ``exceptions`` uint32, ``offsets`` int64
    [mats + 1] as produced by ``pack_x4t_scale_components_batched``.  One
    launch; no validation (use ``decode_scale_components`` on untrusted data).
    """

    mats = int(offsets.numel()) - 1
    if mats < 1 or fixed.dtype != torch.uint8 or fixed.numel() != mats * x4t_fixed_bytes(rows, columns):
        raise ValueError("X4T fixed scale tensor has invalid geometry")
    if exceptions.dtype != torch.uint32 or exceptions.ndim != 1:
        raise ValueError("X4T exception tensor must be one-dimensional uint32")
    if offsets.dtype != torch.int64:
        raise ValueError("X4T exception offsets must be int64")
    (f, e, o), gpu, host = N.to_gpu([fixed.reshape(-1), exceptions, offsets])
    f = f.contiguous()
    o = N.aligned(o, 8)
    e = N.aligned(e, 4) if e.numel() else torch.empty(1, dtype=torch.uint32, device=gpu)
    out = torch.empty((mats, rows, columns), dtype=torch.uint8, device=gpu)
    N.call("kq_x4t_decode", N.ptr(f), N.ptr(e), int(exceptions.numel()), N.ptr(o), mats, rows,
           columns, N.ptr(out), None, N.stream(gpu))
    return out if host is None else out.to(host)


def x4t_tile_index(
    exceptions: torch.Tensor,
    offsets: torch.Tensor,
    *,
    rows: int,
    columns: int,
) -> torch.Tensor:
    """Per-16-row-tile exception index of ``mats`` stacked planes, on the GPU.

    ``exceptions`` uint32 and ``offsets`` int64 [mats + 1] as
    ``pack_x4t_scale_components_batched`` returns them (or as kquant's X4T
    container stores a matrix kind: one exception stream and per-expert
    offsets).  Returns uint32 [mats * rows / 16 + 1]: entry m * rows/16 + t
    is the first exception of matrix m at or past tile t, the last entry the
    total.  The one-time index ``grouped_expert_forward`` needs to expand
    routed experts' scales without searching.
    """

    if exceptions.dtype != torch.uint32 or exceptions.ndim != 1:
        raise ValueError("X4T exception tensor must be one-dimensional uint32")
    if offsets.dtype != torch.int64 or offsets.ndim != 1 or offsets.numel() < 2:
        raise ValueError("X4T exception offsets must be int64 [mats + 1]")
    if rows <= 0 or rows % X4T_TILE_ROWS or not 1 <= columns <= 255 or rows * columns > X4T_POSITION_MASK:
        raise ValueError("X4T plane geometry is invalid")
    mats = int(offsets.numel()) - 1
    (e, o), gpu, _ = N.to_gpu([exceptions, offsets])
    o = N.aligned(o.contiguous(), 8)
    e = N.aligned(e.contiguous(), 4) if e.numel() else torch.zeros(1, dtype=torch.uint32, device=gpu)
    index = torch.empty(mats * (rows // X4T_TILE_ROWS) + 1, dtype=torch.uint32, device=gpu)
    N.call("kq_x4t_tile_index", N.ptr(e), int(exceptions.numel()), N.ptr(o), mats, rows, columns,
           N.ptr(index), N.stream(gpu))
    return index
