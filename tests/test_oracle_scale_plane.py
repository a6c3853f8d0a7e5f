"""Pins of the scale-plane codec oracle (no GPU).

Known answers come from the reference's tests
(tests/test_mxfp4_scale_codec.py, tests/test_x4t.py); hand-assembled byte
strings fix the layouts; brute force fixes the palette and base choices; and
decode(encode(x)) == x over many planes fixes the inverse relation.
"""

from __future__ import annotations

import struct
from collections import Counter

import numpy as np
import pytest

from oracle import scale_plane as sp


def _example_scale() -> np.ndarray:
    # tests/test_mxfp4_scale_codec.py:18-27
    return np.array(
        [
            [120, 121, 120, 121, 122, 120, 121, 120, 119, 121],
            [117] * 10,
            [3, 9, 3, 9, 42, 3, 9, 3, 9, 3],
        ],
        dtype=np.uint8,
    )


def _x4t_scale(rows: int = 32, columns: int = 17) -> np.ndarray:
    # tests/test_x4t.py:14-23
    out = np.empty((rows, columns), dtype=np.uint8)
    for row in range(rows):
        base = 110 + row % 7
        out[row] = [base + (c & 1) for c in range(columns)]
    out[0, 0] = 140
    out[17, columns - 1] = 3
    return out


def planes(seed: int = 0):
    """Planes of the shapes and value mixes the codecs meet."""
    g = np.random.default_rng(seed)
    out = []
    for rows, cols in [(16, 1), (16, 8), (32, 17), (48, 64), (16, 255), (64, 224), (33, 10)]:
        base = g.integers(100, 130, size=(rows, 1))
        plane = base + g.integers(0, 2, size=(rows, cols))
        mask = g.random((rows, cols)) < 0.05
        plane = np.where(mask, g.integers(0, 256, size=(rows, cols)), plane)
        out.append(plane.astype(np.uint8))
    out.append(g.integers(0, 256, size=(32, 40)).astype(np.uint8))       # no structure
    out.append(np.full((16, 9), 255, np.uint8))                           # top boundary
    out.append(np.zeros((16, 9), np.uint8))                               # bottom boundary
    out.append(np.tile(np.array([0, 255], np.uint8), (16, 6)))            # far palette
    return out


# ----------------------------------------------------------------- KQSC --

def test_kqsc_reference_round_trip_and_determinism():
    # tests/test_mxfp4_scale_codec.py:30-47
    scale = _example_scale()
    payload = sp.kqsc_pack_v1(scale, tile_rows=2)
    assert np.array_equal(sp.kqsc_unpack_v1(payload), scale)
    assert payload == sp.kqsc_pack_v1(scale.copy(), tile_rows=2)
    assert (scale.size * 16 + len(payload)) * 8 / (scale.size * 32) > 4.0


def test_kqsc_reference_terminal_offset():
    # tests/test_mxfp4_scale_codec.py:50-58
    payload = bytearray(sp.kqsc_pack_v1(_example_scale(), tile_rows=2))
    prior = struct.unpack_from("<I", payload, 16 + 4)[0]
    struct.pack_into("<I", payload, 16 + 2 * 4, prior)
    with pytest.raises(ValueError, match="terminal offset"):
        sp.kqsc_unpack_v1(bytes(payload))


def test_kqsc_reference_rejects_non_uint8():
    # tests/test_mxfp4_scale_codec.py:61-63
    with pytest.raises(ValueError, match="CPU uint8"):
        sp.kqsc_pack_v1(np.ones((2, 8), dtype=np.int16))


def test_kqsc_reference_compact_stats():
    # tests/test_mxfp4_scale_codec.py:66-83
    scale = np.array([[120 + (c & 1) for c in range(112)] for _ in range(16)], dtype=np.uint8)
    scale[0, 0] = 122
    payload = sp.kqsc_pack_v2(scale, tile_rows=16)
    assert np.array_equal(sp.kqsc_unpack_v2(payload), scale)
    assert len(payload) < len(sp.kqsc_pack_v1(scale, tile_rows=16))
    assert sp.kqsc_compact_stats(payload) == {
        "rows": 16, "tiles": 1, "palette_escapes": 0, "count_escapes": 0, "exceptions": 1,
    }


def test_kqsc_reference_adjacent_boundary_escape():
    # tests/test_mxfp4_scale_codec.py:86-91
    scale = np.array([[0, 0, 0, 0], [255, 255, 255, 255]], dtype=np.uint8)
    assert np.array_equal(sp.kqsc_unpack_v2(sp.kqsc_pack_v2(scale)), scale)


def test_kqsc_hand_assembled_bytes():
    # one row [5, 6, 5, 9]: palette (5, 6), selector bit 1, exception (3, 9)
    scale = np.array([[5, 6, 5, 9]], dtype=np.uint8)
    header1 = b"KQSC" + bytes([1, 16, 0, 0]) + (1).to_bytes(4, "little") + bytes([4, 0, 0, 0])
    body1 = bytes([5, 6, 1, 0b0010, 3, 9])
    assert sp.kqsc_pack_v1(scale) == header1 + struct.pack("<2I", 0, 6) + body1
    # v2: palette0 5, direction +1, no explicit palette, count code 1
    header2 = header1[:4] + bytes([2]) + header1[5:]
    body2 = bytes([5, 0b1, 0b0, 0b01, 0b0010, 3, 9])
    assert sp.kqsc_pack_v2(scale) == header2 + struct.pack("<2I", 0, 7) + body2
    # a constant row: explicit palette1 equal to palette0, no selectors set
    flat = np.array([[7, 7, 7]], dtype=np.uint8)
    body = sp.kqsc_pack_v2(flat)[16 + 8:]
    assert body == bytes([7, 0, 0b1, 0, 7, 0])


def test_kqsc_palette_brute_force():
    for plane in planes(1):
        for row in plane:
            vals, counts = np.unique(row, return_counts=True)
            order = np.lexsort((vals, -counts))
            first = int(vals[order[0]])
            second = int(vals[order[1]]) if len(vals) > 1 else first
            assert sp._row_palette(list(map(int, row))) == (first, second)


@pytest.mark.parametrize("tile_rows", [1, 2, 5, 16, 255])
def test_kqsc_round_trips(tile_rows):
    for plane in planes(2):
        p1 = sp.kqsc_pack_v1(plane, tile_rows=tile_rows)
        p2 = sp.kqsc_pack_v2(plane, tile_rows=tile_rows)
        assert np.array_equal(sp.kqsc_unpack_v1(p1), plane)
        assert np.array_equal(sp.kqsc_unpack_v2(p2), plane)
        stats = sp.kqsc_compact_stats(p2)
        expected_exc = 0
        pal = cnt = 0
        for row in plane:
            first, second = sp._row_palette(list(map(int, row)))
            n = int(np.sum((row != first) & (row != second)))
            expected_exc += n
            pal += abs(second - first) != 1
            cnt += n >= 3
        assert stats["exceptions"] == expected_exc
        assert stats["palette_escapes"] == pal and stats["count_escapes"] == cnt


def test_kqsc_decode_errors():
    plane = planes(3)[2]
    payload = bytearray(sp.kqsc_pack_v1(plane, tile_rows=16))
    start = 16 + 4 * 3
    bad = bytearray(payload)
    bad[start + 2 * 16] += 1          # row 0 count off by one
    with pytest.raises(ValueError, match="counts disagree"):
        sp.kqsc_unpack_v1(bytes(bad))
    bad = bytearray(payload)
    bad[start + 3 * 16 + 2] |= 0x80   # row 0 selector padding (17 columns)
    with pytest.raises(ValueError, match="padding"):
        sp.kqsc_unpack_v1(bytes(bad))
    bad = bytearray(payload)
    bad[4] = 3
    with pytest.raises(ValueError, match="magic or version"):
        sp.kqsc_unpack_v1(bytes(bad))


# ------------------------------------------------------------------- X4T --

def test_x4t_reference_known_answers():
    # tests/test_x4t.py:26-49
    scale = _x4t_scale()
    fixed, exc = sp.x4t_pack(scale)
    again = sp.x4t_pack(scale.copy())
    assert np.array_equal(fixed, again[0]) and np.array_equal(exc, again[1])
    assert sp.x4t_storage_bytes(scale) == fixed.size + 4 * exc.size
    assert 4.0 + sp.x4t_storage_bytes(scale) * 8 / (scale.size * 32) < 4.25
    fixed, exc = sp.x4t_pack(_x4t_scale(columns=8))
    assert fixed.dtype == np.uint8 and exc.dtype == np.uint32
    assert exc.size == 2 and int(exc[0]) & sp.X4T_POSITION_MASK == 0
    with pytest.raises(ValueError, match="multiple of 16"):
        sp.x4t_pack(np.zeros((15, 8), dtype=np.uint8))


def test_x4t_hand_assembled():
    # row 0 [7, 8, 20]: pair (7, 8) covers two values -> base 7, bit 1, one exception
    # rows 1..15 [1, 1, 1]: pairs (0, 1) and (1, 2) tie -> lowest base 0, all bits set
    scale = np.ones((16, 3), dtype=np.uint8)
    scale[0] = [7, 8, 20]
    fixed, exc = sp.x4t_pack(scale)
    assert fixed.tolist() == [7] + [0] * 15 + [0b010] + [0b111] * 15
    assert exc.tolist() == [2 | (20 << 24)]


def _brute_base(row: np.ndarray) -> int:
    best, best_b = -1, 0
    for b in range(255):
        covered = sum(1 for v in row.tolist() if v == b or v == b + 1)
        if covered > best:
            best, best_b = covered, b
    return best_b


def test_x4t_base_brute_force_and_round_trip():
    for plane in planes(4):
        if plane.shape[0] % 16:
            continue
        bases = sp.x4t_bases(plane)
        assert [_brute_base(r) for r in plane] == bases.tolist()
        fixed, exc = sp.x4t_pack(plane)
        assert np.array_equal(sp.x4t_decode(fixed, exc, *plane.shape), plane)
        covered = (plane == bases[:, None]) | (plane.astype(np.int16) == bases[:, None] + 1)
        assert exc.size == int((~covered).sum())
        assert np.all(np.diff((exc & sp.X4T_POSITION_MASK).astype(np.int64)) > 0)


def test_x4t_decode_errors():
    plane = planes(5)[2]  # 32 x 17
    fixed, exc = sp.x4t_pack(plane)
    assert exc.size >= 2
    f = fixed.copy()
    f[16 + 2] |= 0x80  # row 0 selector padding
    with pytest.raises(ValueError, match="padding"):
        sp.x4t_decode(f, exc, 32, 17)
    e = exc[::-1].copy()
    with pytest.raises(ValueError, match="strictly increasing"):
        sp.x4t_decode(fixed, e, 32, 17)
    e = exc.copy()
    row = int(e[0] & sp.X4T_POSITION_MASK) // 17
    base = int(fixed[(row // 16) * 16 * 4 + row % 16])
    e[0] = (e[0] & sp.X4T_POSITION_MASK) | (base << 24)
    with pytest.raises(ValueError, match="adjacent-palette"):
        sp.x4t_decode(fixed, e, 32, 17)
    # a constant row of 100 codes canonically as base 99 with every bit set;
    # base 100 with no bits decodes to the same row but is not canonical
    flat = plane.copy()
    flat[1] = 100
    fixed, exc = sp.x4t_pack(flat)
    assert fixed[1] == 99 and fixed[16 + 3 * 1: 16 + 3 * 1 + 3].tolist() == [0xFF, 0xFF, 0x01]
    f = fixed.copy()
    f[1] = 100
    f[16 + 3: 16 + 6] = 0
    with pytest.raises(ValueError, match="not canonical"):
        sp.x4t_decode(f, exc, 32, 17)
