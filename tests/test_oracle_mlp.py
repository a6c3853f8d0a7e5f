"""Pins of the expert-MLP helper oracles (no GPU): the reference's known
answers (tests/test_tp_simulator.py) and closed forms."""

from __future__ import annotations

import numpy as np
import torch

import oracle


def test_kimi_topk_reference_known_answer():
    # tests/test_tp_simulator.py:49-63: the bias selects but does not weight
    logits = np.array([[0.0, 1.0, 2.0, 3.0]], dtype=np.float32)
    weights, ids, _ = oracle.kimi_topk(logits, np.array([10.0, 0, 0, 0]), 2, 2.0)
    assert ids.tolist() == [[0, 3]]
    raw = torch.tensor(logits).sigmoid()[0, [0, 3]].double().numpy()
    assert np.allclose(weights[0], 2.0 * raw / raw.sum(), rtol=1e-12)


def test_kimi_topk_matches_torch_topk():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(64, 384, generator=g)
    bias = torch.randn(384, generator=g) * 0.1
    scores = logits.sigmoid()
    ref_ids = torch.topk(scores + bias, k=8, dim=-1, sorted=True).indices
    _, ids, _ = oracle.kimi_topk(logits.numpy(), bias.numpy(), 8)
    assert np.array_equal(ids, ref_ids.numpy())


def test_situ_reference_known_answer():
    # tests/test_tp_simulator.py:66-74
    gate = torch.tensor([[-5.0, 0.0, 5.0]])
    up = torch.tensor([[30.0, -2.0, 3.0]])
    expected = 4.0 * torch.tanh(gate / 4.0) * torch.sigmoid(gate) * (25.0 * torch.tanh(up / 25.0))
    assert np.allclose(oracle.situ(gate.numpy(), up.numpy()), expected.numpy(), rtol=1e-6, atol=1e-7)


def test_reduce_partials_reassembles_row_parallel_linear():
    # tests/test_tp_simulator.py:35-46: row-parallel partials sum to the linear
    g = np.random.default_rng(8)
    x = g.standard_normal((2, 17)).astype(np.float32)
    w = g.standard_normal((11, 17)).astype(np.float32)
    parts = [x[:, i::3] @ w[:, i::3].T for i in range(3)]
    assert np.allclose(oracle.reduce_partials(parts), x @ w.T, rtol=2e-6, atol=2e-6)


def test_comparison_metrics_closed_forms():
    r = np.random.default_rng(1).standard_normal(1000).astype(np.float32)
    same = oracle.comparison_metrics(r, r)
    assert same["relative_l2"] == 0.0 and same["max_abs"] == 0.0 and abs(same["cosine"] - 1) < 1e-12
    double = oracle.comparison_metrics(r, 2 * r)
    assert abs(double["relative_l2"] - 1.0) < 1e-12 and abs(double["cosine"] - 1.0) < 1e-12
    assert double["max_abs"] == float(np.abs(r).max())
    e = np.zeros(4, np.float32)
    f = np.zeros(4, np.float32)
    e[0], f[1] = 1.0, 3.0
    assert oracle.comparison_metrics(e, f)["cosine"] == 0.0


def test_expert_output_with_identity_weights_is_the_activation():
    x = np.random.default_rng(2).standard_normal((5, 8)).astype(np.float32)
    eye = np.eye(8, dtype=np.float32)
    out = oracle.expert_output(x, eye, 0.5 * eye, eye)
    assert np.allclose(out, oracle.situ(x, 0.5 * x), rtol=1e-7, atol=1e-9)
