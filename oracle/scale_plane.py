"""TEST INFRASTRUCTURE ONLY — CPU restatements of kquant's lossless E8M0
scale-plane codecs, the checkers of kquant_amd's HIP scale-plane kernels.

  x4t_pack / x4t_decode / x4t_exception_count
      kquant/x4t.py:51-130 (adjacent-pair fixed stream + uint32 exceptions),
      :201-234 (storage accounting), :477-524 (validating decode)
  kqsc_pack_v1 / kqsc_unpack_v1
      kquant/mxfp4_scale_codec.py:27-161 (row-palette tiles, version 1)
  kqsc_pack_v2 / kqsc_unpack_v2 / kqsc_compact_stats
      kquant/mxfp4_scale_codec.py:205-499 (compact version 2)

Each follows the reference step by step (numpy / Python loops; the inputs in
the tests are small).
"""

from __future__ import annotations

import math
import struct
from collections import Counter

import numpy as np

X4T_TILE_ROWS = 16
X4T_POSITION_BITS = 24
X4T_POSITION_MASK = (1 << X4T_POSITION_BITS) - 1
MAGIC = b"KQSC"
HEADER = struct.Struct("<4sBBH I H H")


# ------------------------------------------------------------------- X4T --

def _x4t_validate(scale: np.ndarray) -> tuple[int, int]:
    if scale.dtype != np.uint8 or scale.ndim != 2:
        raise ValueError("X4T scale must be a contiguous two-dimensional CPU uint8 tensor")
    rows, columns = scale.shape
    if not rows or rows % X4T_TILE_ROWS:
        raise ValueError("X4T scale rows must be a nonzero multiple of 16")
    if not 1 <= columns <= 255:
        raise ValueError("X4T scale columns must lie in 1..255")
    if rows * columns > X4T_POSITION_MASK:
        raise ValueError("X4T logical scale plane exceeds its 24-bit position field")
    return rows, columns


def x4t_bases(scale: np.ndarray) -> np.ndarray:
    """Per row, argmax over b in [0, 254] of hist[b] + hist[b+1], lowest b on ties."""
    rows = scale.shape[0]
    indexed = (np.arange(rows, dtype=np.int64)[:, None] << 8) + scale
    histogram = np.bincount(indexed.ravel(), minlength=rows * 256).reshape(rows, 256)
    return np.argmax(histogram[:, :-1] + histogram[:, 1:], axis=1).astype(np.uint8)


def x4t_pack(scale: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    rows, columns = _x4t_validate(scale)
    sb = math.ceil(columns / 8)
    tiles = rows // X4T_TILE_ROWS
    bases = x4t_bases(scale)
    s16 = scale.astype(np.int16)
    b16 = bases.astype(np.int16)
    low = s16 == b16[:, None]
    high = s16 == b16[:, None] + 1
    selectors = np.packbits(high, axis=1, bitorder="little")
    fixed = np.empty((tiles, X4T_TILE_ROWS * (1 + sb)), dtype=np.uint8)
    fixed[:, :X4T_TILE_ROWS] = bases.reshape(tiles, X4T_TILE_ROWS)
    fixed[:, X4T_TILE_ROWS:] = selectors.reshape(tiles, -1)
    coords = np.argwhere(~(low | high))
    if coords.size:
        pos = coords[:, 0].astype(np.uint32) * np.uint32(columns) + coords[:, 1].astype(np.uint32)
        vals = scale[coords[:, 0], coords[:, 1]].astype(np.uint32)
        exc = pos | (vals << np.uint32(X4T_POSITION_BITS))
    else:
        exc = np.empty(0, dtype=np.uint32)
    return fixed.reshape(-1), exc.astype(np.uint32)


def x4t_exception_count(scale: np.ndarray) -> int:
    return int(x4t_pack(scale)[1].size)


def x4t_storage_bytes(scale: np.ndarray) -> int:
    fixed, exc = x4t_pack(scale)
    return int(fixed.size + 4 * exc.size)


def x4t_decode(fixed: np.ndarray, exceptions: np.ndarray, rows: int, columns: int) -> np.ndarray:
    sb = math.ceil(columns / 8)
    tile_bytes = X4T_TILE_ROWS * (1 + sb)
    if fixed.dtype != np.uint8 or fixed.size != (rows // X4T_TILE_ROWS) * tile_bytes:
        raise ValueError("X4T fixed scale tensor has invalid geometry")
    if exceptions.dtype != np.uint32 or exceptions.ndim != 1:
        raise ValueError("X4T exception tensor must be one-dimensional uint32")
    f = fixed.reshape(rows // X4T_TILE_ROWS, tile_bytes)
    bases = f[:, :X4T_TILE_ROWS].reshape(rows)
    selectors = f[:, X4T_TILE_ROWS:].reshape(rows, sb)
    col = np.arange(columns)
    selected = (selectors[:, col // 8].astype(np.int16) >> (col % 8).astype(np.int16)) & 1
    result = np.ascontiguousarray((bases.astype(np.int16)[:, None] + selected).astype(np.uint8))
    if columns % 8 and bool((selectors[:, -1] >> (columns % 8)).any()):
        raise ValueError("X4T selector has nonzero padding bits")
    flat = result.reshape(-1)
    previous = -1
    for entry in exceptions.tolist():
        position = entry & X4T_POSITION_MASK
        value = entry >> X4T_POSITION_BITS
        if position >= flat.size or position <= previous:
            raise ValueError("X4T exception positions must be valid and strictly increasing")
        previous = position
        base = int(bases[position // columns])
        if value in (base, base + 1):
            raise ValueError("X4T exception redundantly names an adjacent-palette value")
        flat[position] = value
    ef, ee = x4t_pack(result)
    if not np.array_equal(ef, fixed.reshape(-1)) or not np.array_equal(ee, exceptions):
        raise ValueError("X4T safetensors scale stream is not canonical")
    return result


# ------------------------------------------------------------------ KQSC --

def _row_palette(row: list[int]) -> tuple[int, int]:
    counts = Counter(row)
    ordered = sorted(counts, key=lambda v: (-counts[v], v))
    first = ordered[0]
    second = first if len(ordered) == 1 else ordered[1]
    return first, second


def _row_fields(row: list[int], sb: int):
    first, second = _row_palette(row)
    selector = bytearray(sb)
    exc: list[tuple[int, int]] = []
    for position, value in enumerate(row):
        if value == second and second != first:
            selector[position // 8] |= 1 << (position % 8)
        elif value != first:
            exc.append((position, value))
    if len(exc) > 255:
        raise ValueError("row exception count does not fit uint8")
    return first, second, bytes(selector), exc


def _check_pack_args(scale: np.ndarray, tile_rows: int) -> tuple[int, int]:
    if scale.dtype != np.uint8 or scale.ndim != 2:
        raise ValueError("scale must be a two-dimensional CPU uint8 tensor")
    rows, columns = scale.shape
    if not rows or not columns or columns > 255:
        raise ValueError("scale dimensions must be nonzero and columns must fit uint8")
    if not 1 <= tile_rows <= 255:
        raise ValueError("tile_rows must fit uint8")
    return rows, columns


def _assemble(version: int, tile_rows: int, rows: int, columns: int, tiles: list[bytes]) -> bytes:
    offsets = [0]
    for t in tiles:
        offsets.append(offsets[-1] + len(t))
    header = HEADER.pack(MAGIC, version, tile_rows, 0, rows, columns, 0)
    return header + struct.pack(f"<{len(offsets)}I", *offsets) + b"".join(tiles)


def kqsc_pack_v1(scale: np.ndarray, tile_rows: int = 16) -> bytes:
    rows, columns = _check_pack_args(scale, tile_rows)
    sb = math.ceil(columns / 8)
    tiles = []
    for start in range(0, rows, tile_rows):
        p0 = bytearray(); p1 = bytearray(); counts = bytearray(); sels = bytearray(); exs = bytearray()
        for r in range(start, min(start + tile_rows, rows)):
            first, second, sel, exc = _row_fields(list(map(int, scale[r])), sb)
            p0.append(first); p1.append(second); counts.append(len(exc)); sels.extend(sel)
            for position, value in exc:
                exs.extend((position, value))
        tiles.append(bytes(p0 + p1 + counts + sels + exs))
    return _assemble(1, tile_rows, rows, columns, tiles)


def _low_bits(values: list[int], bits: int) -> bytes:
    out = bytearray(math.ceil(len(values) * bits / 8))
    for i, v in enumerate(values):
        b = i * bits
        out[b // 8] |= v << (b % 8)
    return bytes(out)


def kqsc_pack_v2(scale: np.ndarray, tile_rows: int = 16) -> bytes:
    rows, columns = _check_pack_args(scale, tile_rows)
    sb = math.ceil(columns / 8)
    tiles = []
    for start in range(0, rows, tile_rows):
        p0 = bytearray(); dirs = []; flags = []; expl = bytearray(); codes = []; ext = bytearray()
        sels = bytearray(); exs = bytearray()
        for r in range(start, min(start + tile_rows, rows)):
            first, second, sel, exc = _row_fields(list(map(int, scale[r])), sb)
            p0.append(first)
            delta = second - first
            if delta in (-1, 1):
                dirs.append(int(delta > 0)); flags.append(0)
            else:
                dirs.append(0); flags.append(1); expl.append(second)
            n = len(exc)
            if n < 3:
                codes.append(n)
            else:
                codes.append(3); ext.append(n)
            sels.extend(sel)
            for position, value in exc:
                exs.extend((position, value))
        tiles.append(bytes(p0) + _low_bits(dirs, 1) + _low_bits(flags, 1) + _low_bits(codes, 2)
                     + bytes(expl) + bytes(ext) + bytes(sels) + bytes(exs))
    return _assemble(2, tile_rows, rows, columns, tiles)


def _parse_header(payload: bytes, version: int, prefix: str):
    if len(payload) < HEADER.size:
        raise ValueError(f"{prefix} payload is truncated before its header")
    magic, ver, tile_rows, r0, rows, columns, r1 = HEADER.unpack_from(payload)
    if magic != MAGIC or ver != version:
        raise ValueError(f"{prefix} payload has an unsupported magic or version")
    if r0 or r1:
        raise ValueError(f"{prefix} payload reserved fields must be zero")
    if not rows or not columns or columns > 255 or not tile_rows:
        raise ValueError(f"{prefix} payload dimensions are invalid")
    tiles = math.ceil(rows / tile_rows)
    start = HEADER.size + 4 * (tiles + 1)
    if len(payload) < start:
        raise ValueError(f"{prefix} payload is truncated in its offset table")
    offsets = struct.unpack_from(f"<{tiles + 1}I", payload, HEADER.size)
    if offsets[0] != 0 or any(a > b for a, b in zip(offsets, offsets[1:])):
        raise ValueError(f"{prefix} payload offsets are not monotone from zero")
    if offsets[-1] != len(payload) - start:
        raise ValueError(f"{prefix} payload terminal offset disagrees with its length")
    return tile_rows, rows, columns, tiles, start, offsets


def kqsc_unpack_v1(payload: bytes) -> np.ndarray:
    tile_rows, rows, columns, tiles, start, offsets = _parse_header(payload, 1, "scale")
    sb = math.ceil(columns / 8)
    result = np.empty((rows, columns), dtype=np.uint8)
    for t in range(tiles):
        r0 = t * tile_rows
        rc = min(tile_rows, rows - r0)
        body = payload[start + offsets[t]: start + offsets[t + 1]]
        if len(body) < rc * (3 + sb):
            raise ValueError("scale tile is truncated before its fixed fields")
        p0, p1, counts = body[:rc], body[rc:2 * rc], body[2 * rc:3 * rc]
        sel0 = 3 * rc
        exc0 = sel0 + rc * sb
        if len(body) != exc0 + 2 * sum(counts):
            raise ValueError("scale tile exception counts disagree with its length")
        cur = exc0
        for lr in range(rc):
            first, second = p0[lr], p1[lr]
            sel = body[sel0 + lr * sb: sel0 + (lr + 1) * sb]
            row = np.full(columns, first, dtype=np.uint8)
            for pos in range(columns):
                if sel[pos // 8] & (1 << (pos % 8)):
                    row[pos] = second
            if columns % 8 and sel[-1] >> (columns % 8):
                raise ValueError("scale selector has nonzero padding bits")
            seen = set()
            for _ in range(counts[lr]):
                pos, val = body[cur], body[cur + 1]
                cur += 2
                if pos >= columns or pos in seen:
                    raise ValueError("scale exception position is invalid or duplicated")
                if val in (first, second):
                    raise ValueError("scale exception redundantly names a palette value")
                seen.add(pos)
                row[pos] = val
            result[r0 + lr] = row
        if cur != len(body):
            raise ValueError("scale tile decoder did not consume its complete body")
    return result


def _unpack_bits(data: bytes, count: int, bits: int, field: str) -> list[int]:
    if len(data) != math.ceil(count * bits / 8):
        raise ValueError(f"compact scale {field} has the wrong length")
    mask = (1 << bits) - 1
    vals = [(data[(i * bits) // 8] >> ((i * bits) % 8)) & mask for i in range(count)]
    used = count * bits
    if used % 8 and data[-1] >> (used % 8):
        raise ValueError(f"compact scale {field} has nonzero padding bits")
    return vals


def kqsc_unpack_v2(payload: bytes) -> np.ndarray:
    tile_rows, rows, columns, tiles, start, offsets = _parse_header(payload, 2, "compact scale")
    sb = math.ceil(columns / 8)
    result = np.empty((rows, columns), dtype=np.uint8)
    for t in range(tiles):
        r0 = t * tile_rows
        rc = min(tile_rows, rows - r0)
        body = payload[start + offsets[t]: start + offsets[t + 1]]
        fb = math.ceil(rc / 8)
        cb = math.ceil(rc * 2 / 8)
        if len(body) < rc + 2 * fb + cb:
            raise ValueError("compact scale tile is truncated before its row fields")
        cur = 0
        p0 = body[cur:cur + rc]; cur += rc
        dirs = _unpack_bits(body[cur:cur + fb], rc, 1, "direction bits"); cur += fb
        flags = _unpack_bits(body[cur:cur + fb], rc, 1, "explicit-palette bits"); cur += fb
        codes = _unpack_bits(body[cur:cur + cb], rc, 2, "count codes"); cur += cb
        n_expl = sum(flags)
        n_ext = sum(c == 3 for c in codes)
        meta_end = cur + n_expl + n_ext
        if len(body) < meta_end + rc * sb:
            raise ValueError("compact scale tile is truncated in its row escapes")
        expl = body[cur:cur + n_expl]; cur += n_expl
        ext = body[cur:cur + n_ext]; cur += n_ext
        counts = []
        ei = 0
        for c in codes:
            if c < 3:
                counts.append(c)
            else:
                n = ext[ei]; ei += 1
                if n < 3:
                    raise ValueError("compact scale count escape is noncanonical")
                counts.append(n)
        sel0 = cur
        exc0 = sel0 + rc * sb
        if len(body) != exc0 + 2 * sum(counts):
            raise ValueError("compact scale exception counts disagree with its length")
        xi = 0
        ecur = exc0
        for lr in range(rc):
            first = p0[lr]
            if flags[lr]:
                second = expl[xi]; xi += 1
                if second - first in (-1, 1):
                    raise ValueError("compact scale palette escape is noncanonical")
            else:
                second = first + (1 if dirs[lr] else -1)
                if not 0 <= second <= 255:
                    raise ValueError("compact scale adjacent palette is out of range")
            sel = body[sel0 + lr * sb: sel0 + (lr + 1) * sb]
            if columns % 8 and sel[-1] >> (columns % 8):
                raise ValueError("compact scale selector has nonzero padding bits")
            row = np.full(columns, first, dtype=np.uint8)
            for pos in range(columns):
                if sel[pos // 8] & (1 << (pos % 8)):
                    row[pos] = second
            seen = set()
            for _ in range(counts[lr]):
                pos, val = body[ecur], body[ecur + 1]
                ecur += 2
                if pos >= columns or pos in seen:
                    raise ValueError("compact scale exception position is invalid or duplicated")
                if val in (first, second):
                    raise ValueError("compact scale exception redundantly names a palette value")
                seen.add(pos)
                row[pos] = val
            result[r0 + lr] = row
        if xi != n_expl or ecur != len(body):
            raise ValueError("compact scale decoder did not consume its complete tile")
    return result


def kqsc_compact_stats(payload: bytes) -> dict:
    if len(payload) < HEADER.size:
        raise ValueError("compact scale payload is truncated before its header")
    magic, ver, tile_rows, r0, rows, columns, r1 = HEADER.unpack_from(payload)
    if magic != MAGIC or ver != 2 or r0 or r1:
        raise ValueError("payload is not a canonical compact scale plane")
    if not rows or not columns or columns > 255 or not tile_rows:
        raise ValueError("compact scale payload dimensions are invalid")
    tiles = math.ceil(rows / tile_rows)
    start = HEADER.size + 4 * (tiles + 1)
    if len(payload) < start:
        raise ValueError("compact scale payload is truncated in its offset table")
    offsets = struct.unpack_from(f"<{tiles + 1}I", payload, HEADER.size)
    if offsets[0] != 0 or offsets[-1] != len(payload) - start:
        raise ValueError("compact scale payload offsets disagree with its length")
    sb = math.ceil(columns / 8)
    pe = ce = ex = 0
    for t in range(tiles):
        rc = min(tile_rows, rows - t * tile_rows)
        body = payload[start + offsets[t]: start + offsets[t + 1]]
        fb = math.ceil(rc / 8)
        cb = math.ceil(rc * 2 / 8)
        flags = _unpack_bits(body[rc + fb: rc + 2 * fb], rc, 1, "explicit-palette bits")
        codes = _unpack_bits(body[rc + 2 * fb: rc + 2 * fb + cb], rc, 2, "count codes")
        tpe, tce = sum(flags), sum(c == 3 for c in codes)
        fixed = rc + 2 * fb + cb + tpe + tce + rc * sb
        eb = len(body) - fixed
        if eb < 0 or eb % 2:
            raise ValueError("compact scale payload byte accounting did not close")
        pe += tpe; ce += tce; ex += eb // 2
    return {"rows": rows, "tiles": tiles, "palette_escapes": pe, "count_escapes": ce, "exceptions": ex}
