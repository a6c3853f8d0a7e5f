"""The oracle against the golden fixtures of tests/golden (no GPU).

The fixtures were written by tests/golden/make_golden.py from the reference
implementation (in the build container) for the functions no reference test
or closed form pins: the SQG tables without a hash in tests/test_sqg_e4m3.py
and mxfp8_quantize_cpu on float32 blocks next to a scale boundary.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict:
    return json.loads((GOLDEN / name).read_text())


def sha(a: np.ndarray, dtype) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=dtype).tobytes()).hexdigest()


def oracle_tables() -> dict:
    law = oracle.sqg_cheb_normal_rank_e4m3_bytes()
    out = {
        "sqg_cheb_normal_rank_e4m3_bytes": (law, np.uint8),
        "sqg_xor_cheb_t12_rank_lut_bytes": (oracle.sqg_xor_cheb_t12_rank_lut_bytes(), np.uint8),
    }
    for bits in (2, 3, 4):
        mix = oracle.sqg_rank_permutation(bits)
        out[f"sqg_rank_permutation_k{bits}"] = (mix, np.int64)
        out[f"sqg_xor_rank_permutation_k{bits}"] = (oracle.sqg_xor_rank_permutation(bits), np.int64)
        out[f"sqg_e4m3_bytes_normal_k{bits}"] = (oracle.sqg_r44_bytes(bits), np.uint8)
        out[f"sqg_cheb_normal_e4m3_bytes_k{bits}"] = (law[mix], np.uint8)
        out[f"sqg_xor_cheb_t12_bytes_k{bits}"] = (oracle.sqg_xor_cheb_t12_bytes(bits), np.uint8)
        out[f"sqg_cheb_k{bits}_n"] = (law[mix], np.uint8)
        k_axis = law[oracle.sqg_k2_eight_stratum_rank_permutation(4)] if bits == 2 else law[mix]
        out[f"sqg_cheb_k{bits}_k"] = (k_axis, np.uint8)
    for h in (2, 4, 9, 15):
        out[f"sqg_k2_eight_stratum_rank_permutation_h{h}"] = (
            oracle.sqg_k2_eight_stratum_rank_permutation(h), np.int64)
    return out


def test_sqg_tables_match_golden():
    golden = load("sqg_tables.json")
    tables = oracle_tables()
    assert set(tables) == set(golden)
    for name, (table, dtype) in tables.items():
        entry = golden[name]
        assert table.size == entry["numel"], name
        for i, v in entry["samples"]:
            assert int(table[i]) == v, (name, i)
        assert sha(table, dtype) == entry["sha256"], name


def test_golden_agrees_with_reference_test_constants():
    # tests/test_sqg_e4m3.py:32-37 (the hashes the reference's own tests hold)
    golden = load("sqg_tables.json")
    assert golden["sqg_xor_cheb_t12_rank_lut_bytes"]["sha256"] == (
        "cca11fe5744c9c93a34f4217f342fbc0f74ecc8a007c076582424a505fc9da5e")
    assert golden["sqg_xor_cheb_t12_bytes_k2"]["sha256"] == (
        "62027916386245a84c86156a0a08b6cf07e41548871af0e56fb40780558f6293")


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_sqg_rank_permutations_are_bijective_and_span_strata(bits):
    # tests/test_sqg_e4m3.py:73-78, 92-98
    width = 16 - bits
    for ranks in (oracle.sqg_rank_permutation(bits), oracle.sqg_xor_rank_permutation(bits)):
        assert np.array_equal(np.sort(ranks), np.arange(1 << 16))
        strata = (ranks >> width).reshape(1 << width, 1 << bits)
        assert np.array_equal(np.sort(strata, axis=1),
                              np.broadcast_to(np.arange(1 << bits), strata.shape))


def test_mxfp8_f32_boundaries_match_golden():
    d = load("mxfp8_f32_boundaries.json")
    x = np.array(d["input_f32_bits"], dtype=np.uint32).view(np.float32).reshape(d["shape"])
    q, s = oracle.mx_quantize("mxfp8", x, "f32")
    assert np.array_equal(q.ravel(), np.array(d["q_bytes"], dtype=np.uint8))
    assert np.array_equal(s.ravel(), np.array(d["scale_bytes"], dtype=np.uint8))
    # the fixture does exercise the f32 log2 rounding: the exact exponent
    # (no rounding of log2) differs from the reference on some blocks
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    quot = (np.maximum(amax, np.float32(1e-30)) / np.float32(448)).astype(np.float32)
    mant, ex = np.frexp(quot.astype(np.float64))
    exact = np.clip(ex - 1 + (mant != 0.5), -127, 128) + 127
    assert np.sum(exact != s.ravel()) >= 10
