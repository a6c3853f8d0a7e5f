"""X4T and KQSC scale-plane codecs on the GPU against the CPU oracle.

Byte-exact encodings, exact decodes, the reference's known answers
(tests/test_x4t.py, tests/test_mxfp4_scale_codec.py), the production scale
planes of a routed expert (w2 [7168, 64], w1/w3 [2048, 224]) at full size,
and corrupted streams: every corruption must give the same outcome (the same
error message, or the same decoded plane) as the oracle's validating decode.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from kquant_amd import mxfp4_scale_codec as kqsc
from kquant_amd import x4t
from oracle import scale_plane as sp
from tests.test_oracle_scale_plane import _example_scale, _x4t_scale, planes

pytestmark = pytest.mark.gpu


def _outcome(fn, *args, **kw):
    try:
        out = fn(*args, **kw)
    except ValueError as exc:
        return ("error", str(exc))
    if isinstance(out, torch.Tensor):
        out = out.cpu().numpy()
    return ("ok", out)


def _same(a, b) -> bool:
    if a[0] != b[0]:
        return False
    if a[0] == "error":
        return a[1] == b[1]
    if isinstance(a[1], dict):
        return a[1] == b[1]
    return np.array_equal(np.asarray(a[1]), np.asarray(b[1]))


def _production_planes():
    g = np.random.default_rng(11)
    out = []
    for rows, cols in [(7168, 64), (2048, 224)]:
        # E8M0 scales of a trained layer: rows sit on one or two adjacent
        # exponents with a thin tail
        base = g.integers(112, 122, size=(rows, 1))
        plane = base + (g.random((rows, cols)) < 0.4)
        tail = g.random((rows, cols)) < 0.01
        plane = np.where(tail, base + g.integers(-6, 4, size=(rows, cols)), plane)
        out.append(np.clip(plane, 0, 255).astype(np.uint8))
    return out


# ------------------------------------------------------------------- X4T --

def test_x4t_pack_matches_oracle(gpu):
    for plane in planes(0) + planes(7) + _production_planes():
        if plane.shape[0] % 16:
            continue
        want_f, want_e = sp.x4t_pack(plane)
        for src in (torch.from_numpy(plane), torch.from_numpy(plane).to(gpu)):
            fixed, exc = x4t.pack_x4t_scale_components(src)
            assert fixed.device == src.device and exc.dtype == torch.uint32
            assert np.array_equal(fixed.cpu().numpy(), want_f)
            assert np.array_equal(exc.cpu().numpy(), want_e)
        t = torch.from_numpy(plane)
        assert x4t.x4t_scale_exception_count(t) == want_e.size
        assert x4t.x4t_scale_storage_bytes(t) == want_f.size + 4 * want_e.size


def test_x4t_reference_known_answers_on_gpu(gpu):
    # tests/test_x4t.py:26-49
    scale = torch.from_numpy(_x4t_scale())
    fixed, exc = x4t.pack_x4t_scale_components(scale)
    again = x4t.pack_x4t_scale_components(scale.clone())
    assert torch.equal(fixed, again[0])
    assert torch.equal(exc.view(torch.int32), again[1].view(torch.int32))
    assert x4t.x4t_scale_storage_bytes(scale) == fixed.numel() + 4 * exc.numel()
    assert x4t.effective_x4t_bpw(scale) < 4.25
    fixed, exc = x4t.pack_x4t_scale_components(torch.from_numpy(_x4t_scale(columns=8)))
    assert fixed.dtype == torch.uint8 and exc.dtype == torch.uint32
    assert int(exc.numel()) == 2
    assert int(exc.view(torch.int32)[0]) & x4t.X4T_POSITION_MASK == 0
    with pytest.raises(ValueError, match="multiple of 16"):
        x4t.pack_x4t_scale_components(torch.zeros((15, 8), dtype=torch.uint8))


def test_x4t_decode_round_trip(gpu):
    for plane in planes(1) + _production_planes():
        if plane.shape[0] % 16:
            continue
        fixed, exc = sp.x4t_pack(plane)
        out = x4t.decode_scale_components(
            torch.from_numpy(fixed), torch.from_numpy(exc), rows=plane.shape[0], columns=plane.shape[1]
        )
        assert out.device.type == "cpu"
        assert np.array_equal(out.numpy(), plane)


def test_x4t_batched_pack_and_predecode(gpu):
    g = np.random.default_rng(3)
    mats = np.stack([planes(int(s))[2] for s in g.integers(0, 1000, size=6)])  # 6 x 32 x 17
    fixed, exc, offsets = x4t.pack_x4t_scale_components_batched(torch.from_numpy(mats).to(gpu))
    assert offsets.tolist()[0] == 0 and offsets.tolist()[-1] == exc.numel()
    for m in range(mats.shape[0]):
        want_f, want_e = sp.x4t_pack(mats[m])
        assert np.array_equal(fixed[m].cpu().numpy(), want_f)
        a, b = offsets[m].item(), offsets[m + 1].item()
        assert np.array_equal(exc[a:b].cpu().numpy(), want_e)
    out = x4t.decode_x4t_scale_components_batched(fixed, exc, offsets, rows=32, columns=17)
    assert np.array_equal(out.cpu().numpy(), mats)


def test_x4t_corrupted_streams_match_oracle(gpu):
    g = np.random.default_rng(5)
    plane = planes(6)[2]  # 32 x 17, with exceptions
    rows, cols = plane.shape
    fixed, exc = sp.x4t_pack(plane)
    assert exc.size >= 3
    cases = []
    for _ in range(150):
        f, e = fixed.copy(), exc.copy()
        kind = g.integers(0, 4)
        if kind == 0:
            f[g.integers(0, f.size)] = g.integers(0, 256)
        elif kind == 1:
            i = g.integers(0, e.size)
            e[i] = (e[i] & sp.X4T_POSITION_MASK) | (np.uint32(g.integers(0, 256)) << np.uint32(24))
        elif kind == 2:
            i = g.integers(0, e.size)
            e[i] = (e[i] & ~np.uint32(sp.X4T_POSITION_MASK)) | np.uint32(g.integers(0, rows * cols + 4))
        else:
            e = e[g.permutation(e.size)]
        cases.append((f, e))
    cases.append((fixed, exc[:-1]))  # a dropped exception leaves a non-canonical plane
    for f, e in cases:
        want = _outcome(sp.x4t_decode, f, e, rows, cols)
        got = _outcome(x4t.decode_scale_components, torch.from_numpy(f), torch.from_numpy(e),
                       rows=rows, columns=cols)
        assert _same(got, want), (got[1] if got[0] == "error" else "ok", want[1] if want[0] == "error" else "ok")


# ------------------------------------------------------------------ KQSC --

@pytest.mark.parametrize("tile_rows", [1, 2, 7, 16, 255])
def test_kqsc_pack_matches_oracle(gpu, tile_rows):
    for plane in planes(8):
        t = torch.from_numpy(plane)
        p1 = kqsc.pack_scale_plane(t, tile_rows=tile_rows)
        p2 = kqsc.pack_scale_plane_compact(t, tile_rows=tile_rows)
        assert p1 == sp.kqsc_pack_v1(plane, tile_rows=tile_rows)
        assert p2 == sp.kqsc_pack_v2(plane, tile_rows=tile_rows)
        assert np.array_equal(kqsc.unpack_scale_plane(p1).numpy(), plane)
        assert np.array_equal(kqsc.unpack_scale_plane_compact(p2).numpy(), plane)
        assert kqsc.compact_scale_plane_stats(p2) == sp.kqsc_compact_stats(p2)


def test_kqsc_production_planes(gpu):
    for plane in _production_planes():
        t = torch.from_numpy(plane).to(gpu)
        p1 = kqsc.pack_scale_plane(t)
        p2 = kqsc.pack_scale_plane_compact(t)
        assert p1 == sp.kqsc_pack_v1(plane)
        assert p2 == sp.kqsc_pack_v2(plane)
        assert torch.equal(kqsc.unpack_scale_plane(p1, device=gpu), t)
        assert torch.equal(kqsc.unpack_scale_plane_compact(p2, device=gpu), t)
        assert kqsc.compact_scale_plane_stats(p2) == sp.kqsc_compact_stats(p2)


def test_kqsc_reference_known_answers_on_gpu(gpu):
    # tests/test_mxfp4_scale_codec.py:30-91
    scale = torch.from_numpy(_example_scale())
    payload = kqsc.pack_scale_plane(scale, tile_rows=2)
    assert torch.equal(kqsc.unpack_scale_plane(payload), scale)
    assert kqsc.effective_mxfp4_bpw(scale, payload) > 4.0
    assert payload == kqsc.pack_scale_plane(scale.clone(), tile_rows=2)
    bad = bytearray(payload)
    prior = struct.unpack_from("<I", bad, 16 + 4)[0]
    struct.pack_into("<I", bad, 16 + 2 * 4, prior)
    with pytest.raises(ValueError, match="terminal offset"):
        kqsc.unpack_scale_plane(bytes(bad))
    with pytest.raises(ValueError, match="CPU uint8"):
        kqsc.pack_scale_plane(torch.ones((2, 8), dtype=torch.int16))
    scale = torch.tensor([[120 + (c & 1) for c in range(112)] for _ in range(16)], dtype=torch.uint8)
    scale[0, 0] = 122
    payload = kqsc.pack_scale_plane_compact(scale, tile_rows=16)
    assert torch.equal(kqsc.unpack_scale_plane_compact(payload), scale)
    assert len(payload) < len(kqsc.pack_scale_plane(scale, tile_rows=16))
    assert kqsc.compact_scale_plane_stats(payload) == {
        "rows": 16, "tiles": 1, "palette_escapes": 0, "count_escapes": 0, "exceptions": 1,
    }
    scale = torch.tensor([[0, 0, 0, 0], [255, 255, 255, 255]], dtype=torch.uint8)
    assert torch.equal(kqsc.unpack_scale_plane_compact(kqsc.pack_scale_plane_compact(scale)), scale)


@pytest.mark.parametrize("version", [1, 2])
def test_kqsc_corrupted_payloads_match_oracle(gpu, version):
    g = np.random.default_rng(20 + version)
    pack = sp.kqsc_pack_v1 if version == 1 else sp.kqsc_pack_v2
    ref_unpack = sp.kqsc_unpack_v1 if version == 1 else sp.kqsc_unpack_v2
    unpack = kqsc.unpack_scale_plane if version == 1 else kqsc.unpack_scale_plane_compact
    sources = [planes(9)[3], planes(9)[7], planes(9)[6]]  # 48x64, 32x40 random, 33x10
    n_err = 0
    for plane in sources:
        for tile_rows in (5, 16):
            payload = pack(plane, tile_rows=tile_rows)
            tiles = -(-plane.shape[0] // tile_rows)
            body0 = 16 + 4 * (tiles + 1)
            for trial in range(60):
                bad = bytearray(payload)
                if trial % 10 == 0:
                    at = int(g.integers(0, body0))         # header or offset table
                else:
                    at = int(g.integers(body0, len(bad)))  # a tile body
                bad[at] = int(g.integers(0, 256))
                if trial % 15 == 7:
                    bad = bad[: int(g.integers(body0, len(bad)))]
                want = _outcome(ref_unpack, bytes(bad))
                got = _outcome(unpack, bytes(bad))
                assert _same(got, want), (at, got[1] if got[0] == "error" else "ok",
                                          want[1] if want[0] == "error" else "ok")
                n_err += want[0] == "error"
                if version == 2:
                    assert _same(_outcome(kqsc.compact_scale_plane_stats, bytes(bad)),
                                 _outcome(sp.kqsc_compact_stats, bytes(bad)))
    assert n_err > 50
