"""SQG tables built on the GPU (kquant_amd.sqg_e4m3) against the golden
digests, the reference's own known answers (tests/test_sqg_e4m3.py) and the
oracle; plus the fp32 MXFP8 boundary fixture through the quantize kernel."""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import _native as N
from kquant_amd import mxfp8
from kquant_amd import sqg_e4m3 as S
from tests.test_oracle_golden import load

pytestmark = pytest.mark.gpu

REFERENCE_SHA = {  # tests/test_sqg_e4m3.py:32-37
    "t12": "cca11fe5744c9c93a34f4217f342fbc0f74ecc8a007c076582424a505fc9da5e",
    2: "62027916386245a84c86156a0a08b6cf07e41548871af0e56fb40780558f6293",
    3: "afe7b3633e7d243b00b379b18ec4dca573722b3727cafef47fcb6470d7e7e6c9",
    4: "5a9620f0c4d8f0a60d0b6fbea921dcecbd193e6febf31043aaa6403c20389c2f",
}


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().cpu().numpy().tobytes()).hexdigest()


def test_reference_t12_known_answers(gpu):
    table = S.sqg_xor_cheb_t12_rank_lut_bytes()
    assert table.dtype == torch.uint8 and table.shape == (1 << 12,)
    assert sha(table) == REFERENCE_SHA["t12"]
    for bits in (2, 3, 4):
        ranks = S.sqg_xor_rank_permutation(bits)
        labels = S.sqg_xor_cheb_t12_bytes(bits)
        width = 16 - bits
        strata = (ranks >> width).reshape(1 << width, 1 << bits)
        assert torch.equal(torch.sort(ranks).values, torch.arange(1 << 16))
        assert torch.equal(torch.sort(strata, dim=1).values, torch.arange(1 << bits).expand_as(strata))
        assert torch.equal(labels, table[ranks >> 4])
        assert torch.equal(labels, S.sqg_codebook_bytes(bits, S.SQG_XOR_CHEB_T12))
        assert not bool(((labels & 0x7F) == 0).logical_and(labels != 0).any())
        assert sha(labels) == REFERENCE_SHA[bits]


def test_every_table_matches_golden(gpu):
    golden = load("sqg_tables.json")
    built = {
        "sqg_cheb_normal_rank_e4m3_bytes": S.sqg_cheb_normal_rank_e4m3_bytes(),
        "sqg_xor_cheb_t12_rank_lut_bytes": S.sqg_xor_cheb_t12_rank_lut_bytes(),
    }
    for bits in (2, 3, 4):
        built[f"sqg_rank_permutation_k{bits}"] = S.sqg_rank_permutation(bits)
        built[f"sqg_xor_rank_permutation_k{bits}"] = S.sqg_xor_rank_permutation(bits)
        built[f"sqg_e4m3_bytes_normal_k{bits}"] = S.sqg_e4m3_bytes(bits, "normal")
        built[f"sqg_cheb_normal_e4m3_bytes_k{bits}"] = S.sqg_cheb_normal_e4m3_bytes(bits)
        built[f"sqg_xor_cheb_t12_bytes_k{bits}"] = S.sqg_xor_cheb_t12_bytes(bits)
        for axis in ("k", "n"):
            built[f"sqg_cheb_k{bits}_{axis}"] = S.sqg_codebook_bytes(bits, S.SQG_CHEB, rate_axis=axis)
    for h in (2, 4, 9, 15):
        built[f"sqg_k2_eight_stratum_rank_permutation_h{h}"] = S.sqg_k2_eight_stratum_rank_permutation(h)
    assert set(built) == set(golden)
    for name, table in built.items():
        assert table.device.type == "cpu"
        assert str(table.dtype).replace("torch.", "") == golden[name]["dtype"], name
        assert sha(table) == golden[name]["sha256"], name


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_reference_codebook_properties(gpu, bits):
    # tests/test_sqg_e4m3.py:81-131
    raw = S.sqg_e4m3_bytes(bits, "normal")
    codebook = S.sqg_e4m3_codebook(bits, "normal")
    assert raw.dtype == torch.uint8 and codebook.dtype == torch.float16
    assert torch.equal(codebook.to(torch.float8_e4m3fn).view(torch.uint8), raw)
    assert bool(torch.isfinite(codebook).all())
    ranks = S.sqg_rank_permutation(bits)
    assert ranks.dtype == torch.int64
    rank_lut = torch.arange(1 << 16, dtype=torch.int64).remainder(126).to(torch.uint8)
    expected = rank_lut.index_select(0, ranks)
    assert torch.equal(S.sqg_e4m3_bytes_from_rank_lut(bits, rank_lut), expected)
    widened = S.sqg_e4m3_codebook_from_rank_lut(bits, rank_lut)
    assert torch.equal(widened.to(torch.float8_e4m3fn).view(torch.uint8), expected)
    law = S.sqg_cheb_normal_rank_e4m3_bytes()
    assert torch.equal(S.sqg_cheb_normal_e4m3_bytes(bits), law.index_select(0, ranks))
    assert not torch.equal(S.sqg_cheb_normal_e4m3_bytes(bits), raw)
    for dtype in (torch.float32, torch.bfloat16, torch.float64):
        wide = S.sqg_codebook(bits, S.SQG_XOR_CHEB_T12, dtype=dtype)
        ref = S.sqg_xor_cheb_t12_bytes(bits).view(torch.float8_e4m3fn).to(dtype)
        assert wide.dtype == dtype and torch.equal(wide, ref)


def test_reference_errors(gpu):
    rank_lut = torch.zeros(1 << 16, dtype=torch.uint8)
    rank_lut[0] = 0x7F
    with pytest.raises(ValueError, match="finite E4M3"):
        S.sqg_e4m3_bytes_from_rank_lut(2, rank_lut)
    with pytest.raises(ValueError, match="requires rate_axis"):
        S.sqg_codebook_bytes(2, S.SQG_CHEB)
    with pytest.raises(ValueError, match="K2, K3, or K4"):
        S.sqg_xor_cheb_t12_bytes(5)
    with pytest.raises(TypeError, match="floating point"):
        S.sqg_codebook(2, S.SQG_XOR_CHEB_T12, dtype=torch.int32)
    with pytest.raises(ValueError, match=r"\[2, 15\]"):
        S.sqg_k2_eight_stratum_rank_permutation(16)


def test_finite_rank_lut_on_gpu(gpu):
    p = (torch.arange(1 << 16, dtype=torch.float64) + 0.5) / (1 << 16)
    values = 1.5 * torch.special.ndtri(p)
    law = S._finite_e4m3_rank_lut(values)
    assert torch.equal(law, S.sqg_cheb_normal_rank_e4m3_bytes())
    ref = oracle.finite_e4m3_rank_lut(values.numpy())
    assert np.array_equal(law.numpy(), ref)
    with pytest.raises(RuntimeError, match="not monotone"):
        S._finite_e4m3_rank_lut(values.flip(0))
    with pytest.raises(ValueError, match="finite floating point"):
        bad = values.clone()
        bad[3] = float("nan")
        S._finite_e4m3_rank_lut(bad)
    with pytest.raises(RuntimeError, match="non-finite"):
        S._finite_e4m3_rank_lut(torch.full((1 << 16,), 500.0))


@pytest.mark.parametrize("flags", [0, N.FLAG_SOFTWARE_CVT], ids=["hw", "sw"])
def test_mxfp8_f32_boundary_golden(gpu, flags):
    d = load("mxfp8_f32_boundaries.json")
    bits = np.array(d["input_f32_bits"], dtype=np.uint32)
    x = torch.from_numpy(bits.view(np.float32).reshape(d["shape"]).copy()).to(gpu)
    rows, k = x.shape
    q = torch.empty(rows, k, dtype=torch.uint8, device=gpu)
    s = torch.empty(rows, k // 32, dtype=torch.uint8, device=gpu)
    N.call("kq_mx_quantize", N.FMT_MXFP8_E4M3, N.DT_F32, N.ptr(x), k, rows, k, N.ptr(q), N.ptr(s),
           flags, N.stream(gpu))
    assert np.array_equal(s.cpu().numpy().ravel(), np.array(d["scale_bytes"], dtype=np.uint8))
    assert np.array_equal(q.cpu().numpy().ravel(), np.array(d["q_bytes"], dtype=np.uint8))
    if flags == 0:
        q2, s2 = mxfp8.mxfp8_quantize(x)
        assert np.array_equal(q2.view(torch.uint8).cpu().numpy().ravel(), np.array(d["q_bytes"], np.uint8))
