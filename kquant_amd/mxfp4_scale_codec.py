"""KQSC exact row-palette coding of the E8M0 scale plane, on the GPU.

Drop-in for ``kquant/mxfp4_scale_codec.py``: ``pack_scale_plane`` (:27-85),
``unpack_scale_plane`` (:88-161), ``effective_mxfp4_bpw`` (:164-172),
``pack_scale_plane_compact`` (:205-292), ``unpack_scale_plane_compact``
(:295-424) and ``compact_scale_plane_stats`` (:427-499), byte-identical
payloads and the same ``ValueError`` messages.

Payload: header ``<4sBBH I H H>`` (magic ``KQSC``, version, tile_rows, 0,
rows, columns, 0), ``tiles + 1`` uint32 body offsets, then per tile of
``tile_rows`` rows:

  version 1  palette0[r] palette1[r] count[r] selectors[r][ceil(cols/8)]
             (position, value) exception pairs
  version 2  palette0[r], 1-bit direction (palette1 = palette0 +/- 1),
             1-bit explicit-palette flag, 2-bit count code (3 = escape),
             explicit palette1 bytes, escaped counts, selectors, exceptions

palette0/palette1 are the row's most and second most frequent values (ties
to the lower value).  Encoding and tile decoding run in
``libkquant_amd.so``; the header and offset table are parsed on the host
because the payload is a host ``bytes`` object in this API.
"""

from __future__ import annotations

import math
import struct

import torch

from . import _native as N

MAGIC = b"KQSC"
VERSION = 1
COMPACT_VERSION = 2
DEFAULT_TILE_ROWS = 16
_HEADER = struct.Struct("<4sBBH I H H")

_ROW_KEY = 8


def _check_scale(scale: torch.Tensor, tile_rows: int) -> tuple[int, int]:
    if (
        scale.dtype != torch.uint8
        or scale.ndim != 2
        or scale.device.type not in ("cpu", "cuda")
    ):
        raise ValueError("scale must be a two-dimensional CPU uint8 tensor")
    rows, columns = map(int, scale.shape)
    if not rows or not columns or columns > 255:
        raise ValueError("scale dimensions must be nonzero and columns must fit uint8")
    if not 1 <= tile_rows <= 255:
        raise ValueError("tile_rows must fit uint8")
    return rows, columns


def _pack(scale: torch.Tensor, tile_rows: int, version: int) -> bytes:
    rows, columns = _check_scale(scale, tile_rows)
    (s,), gpu, _ = N.to_gpu([scale])
    s = s.contiguous()
    tiles = math.ceil(rows / tile_rows)
    meta = torch.empty(rows, dtype=torch.int32, device=gpu)
    offsets = torch.empty(tiles + 1, dtype=torch.int64, device=gpu)
    st = N.stream(gpu)
    N.call("kq_kqsc_measure", version, N.ptr(s), rows, columns, tile_rows, N.ptr(meta),
           N.ptr(offsets), st)
    total = int(offsets[-1].item())
    if total >= 2**32:
        raise ValueError("scale payload exceeds uint32 offset range")
    start = _HEADER.size + 4 * (tiles + 1)
    payload = torch.empty(start + total, dtype=torch.uint8, device=gpu)
    N.call("kq_kqsc_emit", version, N.ptr(s), rows, columns, tile_rows, N.ptr(meta),
           N.ptr(offsets), N.ptr(payload), st)
    return payload.cpu().numpy().tobytes()


def pack_scale_plane(scale: torch.Tensor, *, tile_rows: int = DEFAULT_TILE_ROWS) -> bytes:
    """Pack a two-dimensional uint8 scale plane without numerical loss (version 1)."""

    return _pack(scale, tile_rows, VERSION)


def pack_scale_plane_compact(scale: torch.Tensor, *, tile_rows: int = DEFAULT_TILE_ROWS) -> bytes:
    """Pack with adjacent-palette and sparse-count coding (version 2)."""

    return _pack(scale, tile_rows, COMPACT_VERSION)


def _parse(payload: bytes, version: int, prefix: str):
    """Header and offset table checks of kquant/mxfp4_scale_codec.py:91-111 / :298-318."""

    if len(payload) < _HEADER.size:
        raise ValueError(f"{prefix} payload is truncated before its header")
    magic, ver, tile_rows, reserved0, rows, columns, reserved1 = _HEADER.unpack_from(payload)
    if magic != MAGIC or ver != version:
        raise ValueError(f"{prefix} payload has an unsupported magic or version")
    if reserved0 or reserved1:
        raise ValueError(f"{prefix} payload reserved fields must be zero")
    if not rows or not columns or columns > 255 or not tile_rows:
        raise ValueError(f"{prefix} payload dimensions are invalid")
    tiles = math.ceil(rows / tile_rows)
    start = _HEADER.size + 4 * (tiles + 1)
    if len(payload) < start:
        raise ValueError(f"{prefix} payload is truncated in its offset table")
    offsets = torch.frombuffer(bytearray(payload[_HEADER.size:start]), dtype=torch.int32)
    offsets = offsets.to(torch.int64) & 0xFFFFFFFF
    if int(offsets[0]) != 0 or bool((offsets[1:] < offsets[:-1]).any()):
        raise ValueError(f"{prefix} payload offsets are not monotone from zero")
    if int(offsets[-1]) != len(payload) - start:
        raise ValueError(f"{prefix} payload terminal offset disagrees with its length")
    return tile_rows, rows, columns


_V1_TILE = {
    0: "scale tile is truncated before its fixed fields",
    6: "scale tile exception counts disagree with its length",
    7: "scale payload offsets are not monotone from zero",
}
_V2_TILE = {
    0: "compact scale tile is truncated before its row fields",
    1: "compact scale direction bits has nonzero padding bits",
    2: "compact scale explicit-palette bits has nonzero padding bits",
    3: "compact scale count codes has nonzero padding bits",
    4: "compact scale tile is truncated in its row escapes",
    5: "compact scale count escape is noncanonical",
    6: "compact scale exception counts disagree with its length",
    7: "compact scale payload offsets are not monotone from zero",
}


def _decode_error(key: int, version: int) -> str:
    prefix = "scale" if version == VERSION else "compact scale"
    if key < _ROW_KEY:
        return (_V1_TILE if version == VERSION else _V2_TILE)[key]
    sub = (key - _ROW_KEY) % 1024
    if sub == 0:
        return "compact scale palette escape is noncanonical"
    if sub == 1:
        return "compact scale adjacent palette is out of range"
    if sub == 2:
        return f"{prefix} selector has nonzero padding bits"
    if (sub - 3) % 2 == 0:
        return f"{prefix} exception position is invalid or duplicated"
    return f"{prefix} exception redundantly names a palette value"


def _unpack(payload: bytes, version: int, device) -> torch.Tensor:
    prefix = "scale" if version == VERSION else "compact scale"
    tile_rows, rows, columns = _parse(payload, version, prefix)
    gpu = N.require_gpu()
    data = torch.frombuffer(bytearray(payload), dtype=torch.uint8).to(gpu)
    out = torch.empty((rows, columns), dtype=torch.uint8, device=gpu)
    status = torch.empty(1, dtype=torch.int64, device=gpu)
    N.call("kq_kqsc_decode", version, N.ptr(data), len(payload), rows, columns, tile_rows,
           N.ptr(out), N.ptr(status), N.stream(gpu))
    word = int(status.item()) & 0xFFFFFFFFFFFFFFFF
    if word != 0xFFFFFFFFFFFFFFFF:
        raise ValueError(_decode_error(word & 0xFFFFF, version))
    return out.to(device) if device is not None else out.cpu()


def unpack_scale_plane(payload: bytes, *, device=None) -> torch.Tensor:
    """Decode and validate a row-palette (version 1) scale plane.

    Returns a CPU tensor, as the reference does, unless ``device`` is given.
    """

    return _unpack(payload, VERSION, device)


def unpack_scale_plane_compact(payload: bytes, *, device=None) -> torch.Tensor:
    """Decode and validate a version-2 compact scale plane."""

    return _unpack(payload, COMPACT_VERSION, device)


def effective_mxfp4_bpw(scale: torch.Tensor, payload: bytes) -> float:
    """Exact nibble-plus-compressed-scale storage in bits per weight."""

    if scale.ndim != 2:
        raise ValueError("scale must be two-dimensional")
    weights = int(scale.numel()) * 32
    return (weights // 2 + len(payload)) * 8 / weights


_STATS_ERRORS = {
    0: "compact scale explicit-palette bits has the wrong length",
    1: "compact scale explicit-palette bits has nonzero padding bits",
    2: "compact scale count codes has the wrong length",
    3: "compact scale count codes has nonzero padding bits",
    4: "compact scale payload byte accounting did not close",
}


def compact_scale_plane_stats(payload: bytes) -> dict[str, int]:
    """Structural counts of a version-2 payload (rows, tiles, escapes, exceptions)."""

    if len(payload) < _HEADER.size:
        raise ValueError("compact scale payload is truncated before its header")
    magic, version, tile_rows, reserved0, rows, columns, reserved1 = _HEADER.unpack_from(payload)
    if magic != MAGIC or version != COMPACT_VERSION or reserved0 or reserved1:
        raise ValueError("payload is not a canonical compact scale plane")
    if not rows or not columns or columns > 255 or not tile_rows:
        raise ValueError("compact scale payload dimensions are invalid")
    tiles = math.ceil(rows / tile_rows)
    start = _HEADER.size + 4 * (tiles + 1)
    if len(payload) < start:
        raise ValueError("compact scale payload is truncated in its offset table")
    first, = struct.unpack_from("<I", payload, _HEADER.size)
    last, = struct.unpack_from("<I", payload, _HEADER.size + 4 * tiles)
    if first != 0 or last != len(payload) - start:
        raise ValueError("compact scale payload offsets disagree with its length")
    gpu = N.require_gpu()
    data = torch.frombuffer(bytearray(payload), dtype=torch.uint8).to(gpu)
    per_tile = torch.zeros((tiles, 3), dtype=torch.int32, device=gpu)
    status = torch.empty(1, dtype=torch.int64, device=gpu)
    N.call("kq_kqsc_stats", N.ptr(data), len(payload), rows, columns, tile_rows, N.ptr(per_tile),
           N.ptr(status), N.stream(gpu))
    word = int(status.item()) & 0xFFFFFFFFFFFFFFFF
    if word != 0xFFFFFFFFFFFFFFFF:
        raise ValueError(_STATS_ERRORS[word & 0xFFFFF])
    palette_escapes, count_escapes, exceptions = (
        int(v) for v in per_tile.to(torch.int64).sum(dim=0).cpu().tolist()
    )
    return {
        "rows": rows,
        "tiles": tiles,
        "palette_escapes": palette_escapes,
        "count_escapes": count_escapes,
        "exceptions": exceptions,
    }
