"""Pins of the MoE oracle and host-side validation (no GPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import moe


def test_situ_known_answer():
    # tests/test_tp_simulator.py:66-74
    gate = np.array([[-5.0, 0.0, 5.0]], np.float32)
    up = np.array([[30.0, -2.0, 3.0]], np.float32)
    g64, u64 = gate.astype(np.float64), up.astype(np.float64)
    expected = 4.0 * np.tanh(g64 / 4.0) / (1 + np.exp(-g64)) * (25.0 * np.tanh(u64 / 25.0))
    assert np.allclose(oracle.situ(gate, up), expected, rtol=2e-6, atol=2e-6)


def test_swiglu_closed_form():
    g = np.linspace(-8, 8, 101, dtype=np.float32)
    u = np.linspace(3, -3, 101, dtype=np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(oracle.swiglu(g, u), ref, rtol=1e-6, atol=1e-6)


def _brute_force(x, ids, w, w13, w2, act):
    """Per-pair float64 loop: an independent restatement of the routed sum."""
    T, k = ids.shape
    inter = w13.shape[1] // 2
    out = np.zeros((T, w2.shape[1]), dtype=np.float64)
    f = {"situ": lambda g, u: 4 * np.tanh(g / 4) / (1 + np.exp(-g)) * 25 * np.tanh(u / 25),
         "swiglu": lambda g, u: g / (1 + np.exp(-g)) * u}[act]
    for t in range(T):
        for s in range(k):
            e = ids[t, s]
            g = w13[e, :inter].astype(np.float64) @ x[t].astype(np.float64)
            u = w13[e, inter:].astype(np.float64) @ x[t].astype(np.float64)
            a = oracle.round_bf16(f(g, u).astype(np.float32)).astype(np.float64)
            out[t] += w[t, s] * (w2[e].astype(np.float64) @ a)
    return out


@pytest.mark.parametrize("act", ["situ", "swiglu"])
def test_oracle_moe_matches_per_pair_brute_force(act):
    rng = np.random.default_rng(0)
    T, k, E, H, I = 9, 3, 5, 64, 32
    x = oracle.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    w = rng.uniform(0, 1, (T, k)).astype(np.float32)
    w13 = (rng.standard_normal((E, 2 * I, H)) * 0.1).astype(np.float32)
    w2 = (rng.standard_normal((E, H, I)) * 0.1).astype(np.float32)
    got = oracle.moe_forward(x, ids, w, lambda e: w13[e], lambda e: w2[e], act)
    ref = _brute_force(x, ids, w, w13, w2, act)
    assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    sub = oracle.moe_forward(x, ids, w, lambda e: w13[e], lambda e: w2[e], act, tokens=np.array([7, 2]))
    assert np.allclose(sub, got[[7, 2]], rtol=0, atol=1e-5 * np.abs(ref).max())


def test_grouped_forward_validates_before_gpu():
    x = torch.zeros(4, 512, dtype=torch.bfloat16)
    ids = torch.zeros(4, 2, dtype=torch.int32)
    w = torch.ones(4, 2)
    w13q = torch.zeros(2, 1024, 256, dtype=torch.uint8)
    w13s = torch.zeros(2, 1024, 16, dtype=torch.uint8)
    w2q = torch.zeros(2, 512, 256, dtype=torch.uint8)
    w2s = torch.zeros(2, 512, 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match="activation"):
        moe.grouped_expert_forward(x, ids, w, w13q, w13s, w2q, w2s, activation="gelu")
    with pytest.raises(TypeError):
        moe.grouped_expert_forward(x, ids, w, w13q.float(), w13s, w2q, w2s)
    with pytest.raises(ValueError, match="w2_packed"):
        moe.grouped_expert_forward(x, ids, w, w13q, w13s, w2q[:, :256], w2s, activation="situ")
    with pytest.raises(ValueError, match="topk"):
        moe.grouped_expert_forward(x, ids[:, :1], w, w13q, w13s, w2q, w2s)
