"""GPU parity of the SQG trellis quantizer (kq_sqg_quantize_tiles) with the
C oracle (oracle/sqg_viterbi.c, the reference kernel's search restated in
exact fp16): states and values bit-exact, for K2/K3/K4, full and short
tail-biting contexts, tie-heavy tiles (zeros, constants, tiles made of label
values) and more tiles than workgroups; and the same search against the MCG
and MUL1 procedural codebooks."""

from __future__ import annotations

import types

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import sqg_quantizer
from kquant_amd.sqg_e4m3 import sqg_xor_cheb_t12_bytes

pytestmark = pytest.mark.gpu


def _tiles(bits: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    lut = oracle.sqg_xor_cheb_t12_bytes(bits)
    labels = oracle.e4m3_values(lut)
    return np.stack([
        rng.standard_normal(256),
        rng.standard_normal(256) * 0.3,
        np.zeros(256),                                 # every path ties
        np.full(256, 0.5),
        labels[rng.integers(0, 65536, 256)],           # exact label values
        rng.standard_normal(256) * 3.0,
    ]).astype(np.float32)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("ctx", [128, 16])
def test_matches_oracle_bit_exact(gpu, bits, ctx):
    x = _tiles(bits, 10 * bits + ctx)
    lut_np = oracle.sqg_xor_cheb_t12_bytes(bits)
    want_vals, want_states = oracle.sqg_quantize_tiles(x, lut_np, bits, ctx)
    lut = sqg_xor_cheb_t12_bytes(bits, device=gpu)
    assert np.array_equal(lut.cpu().numpy(), lut_np)
    vals, states = sqg_quantizer.quantize_tiles_sqg(torch.from_numpy(x).to(gpu), lut, bits, ctx)
    mism = np.flatnonzero((states.cpu().numpy() != want_states).any(axis=1))
    print(f"K{bits} ctx {ctx}: mismatching tiles {mism.tolist()}", flush=True)
    assert mism.size == 0
    assert np.array_equal(vals.cpu().numpy(), want_vals)


def test_more_tiles_than_workgroups_and_install_hook(gpu, monkeypatch):
    bits = 3
    x = np.concatenate([_tiles(bits, s) for s in range(2)])  # 12 tiles
    lut_np = oracle.sqg_xor_cheb_t12_bytes(bits)
    want_vals, want_states = oracle.sqg_quantize_tiles(x, lut_np, bits, 32)
    monkeypatch.setattr(sqg_quantizer, "_workgroups", lambda device: 5)
    module = types.SimpleNamespace(quantize_tiles=lambda tiles, args: ("original", args))
    sqg_quantizer.install_sqg_quantizer(module)
    sqg_quantizer.install_sqg_quantizer(module)  # idempotent
    assert module.quantize_tiles(None, {})[0] == "original"
    args = {"devices": [gpu], "K": bits, "tailbite_context": 32,
            "sqg_e4m3_luts_by_bits": {3: torch.from_numpy(lut_np)}}
    vals, states = module.quantize_tiles(torch.from_numpy(x).to(gpu), args)
    assert np.array_equal(states.cpu().numpy(), want_states)
    assert np.array_equal(vals.cpu().numpy(), want_vals)
    with pytest.raises(ValueError, match="missing rate-specific SQG K3 LUT"):
        module.quantize_tiles(torch.from_numpy(x).to(gpu), {**args, "sqg_e4m3_luts_by_bits": {2: None}})


@pytest.mark.parametrize("codebook", [1, 2])
@pytest.mark.parametrize("bits,ctx", [(2, 128), (3, 16), (4, 128), (4, 16)])
def test_procedural_codebooks_match_oracle_bit_exact(gpu, codebook, bits, ctx):
    """MCG (1) and MUL1 (2) labels computed per state in the kernel against
    the oracle's tables (pinned by their closed forms on the CPU)."""
    rng = np.random.default_rng(100 * codebook + 10 * bits + ctx)
    labels = oracle.procedural_labels(codebook).astype(np.float32)
    x = np.stack([
        rng.standard_normal(256),
        rng.standard_normal(256) * 0.3,
        np.zeros(256),
        labels[rng.integers(0, 65536, 256)],
        rng.standard_normal(256) * 2.0,
    ]).astype(np.float32)
    want_vals, want_states = oracle.sqg_quantize_tiles_procedural(x, bits, codebook, ctx)
    vals, states = sqg_quantizer.quantize_tiles_procedural(torch.from_numpy(x).to(gpu), bits, codebook, ctx)
    mism = np.flatnonzero((states.cpu().numpy() != want_states).any(axis=1))
    print(f"codebook {codebook} K{bits} ctx {ctx}: mismatching tiles {mism.tolist()}", flush=True)
    assert mism.size == 0
    assert np.array_equal(vals.cpu().numpy(), want_vals)


def test_install_hook_routes_none_to_mcg(gpu):
    """A None entry of sqg_e4m3_luts_by_bits selects the MCG control
    (kquant/sqg_quantizer.py:99-119, tests/test_sqg_quantizer.py:11-48)."""
    x = np.random.default_rng(7).standard_normal((3, 256)).astype(np.float32)
    want_vals, want_states = oracle.sqg_quantize_tiles_procedural(x, 2, 1, 128)
    module = types.SimpleNamespace(quantize_tiles=lambda tiles, args: "upstream")
    sqg_quantizer.install_sqg_quantizer(module)
    vals, states = module.quantize_tiles(torch.from_numpy(x).to(gpu), {
        "K": 2, "devices": [gpu], "sqg_e4m3_luts_by_bits": {2: None, 3: None, 4: None}})
    assert np.array_equal(states.cpu().numpy(), want_states)
    assert np.array_equal(vals.cpu().numpy(), want_vals)
    with pytest.raises(ValueError, match="1 \\(MCG\\) or 2 \\(MUL1\\)"):
        sqg_quantizer.quantize_tiles_procedural(torch.from_numpy(x).to(gpu), 2, 3)
