"""Pins of the Hessian oracle and of the host-side Hessian API (no GPU).

Known answers come from the reference's tests (tests/test_candidate_hessian.py
and tests/test_capture.py); the chunked fp32 oracle is also checked against an
exact float64 evaluation, which the mathematics fixes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import candidate_hessian as ch
from kquant_amd import workloads

# (rows, weights, expected) known answers transcribed from the reference tests
KATS = [
    # tests/test_candidate_hessian.py:16-25 (denominator 6.0)
    ([[1.0, 2.0], [3.0, 4.0], [-1.0, 2.0]], [1.0, 2.0, 3.0], None),
    # tests/test_capture.py:136-139
    ([[1, 2], [3, 4]], [0.5, 1.25], None),
    # tests/test_capture.py:140-143
    ([[1, 2, 3, 4], [2, 0, 1, 3]], [0.25, 2.0], None),
    # tests/test_capture.py:168-178 (single rows, unit weight)
    ([[3, 4]], [1.0], [[9, 12], [12, 16]]),
    ([[2, 0, 1, 3]], [1.0], [[4, 0, 2, 6], [0, 0, 0, 0], [2, 0, 1, 3], [6, 0, 3, 9]]),
    # tests/test_capture.py:196-207
    ([[1, 2]], [1.0], [[1, 2], [2, 4]]),
    ([[1, 2, 3, 4]], [1.0], [[1, 2, 3, 4], [2, 4, 6, 8], [3, 6, 9, 12], [4, 8, 12, 16]]),
]


def _expected(rows, weights, expected):
    if expected is not None:
        return np.array(expected, dtype=np.float32)
    x = np.array(rows, dtype=np.float32)
    w = np.array(weights, dtype=np.float32)
    return (x.T @ (x * w[:, None])) / w.sum()


@pytest.mark.parametrize("case", range(len(KATS)))
def test_oracle_weighted_covariance_known_answers(case):
    rows, weights, expected = KATS[case]
    h, denom = oracle.weighted_covariance(np.array(rows, np.float32), np.array(weights, np.float32), 2)
    assert np.allclose(h, _expected(rows, weights, expected), rtol=1e-6, atol=1e-6)
    assert denom == pytest.approx(float(np.sum(weights)))
    if case == 0:
        assert denom == 6.0


def test_oracle_accumulate_is_unnormalised():
    x = np.array([[1, 2], [3, 4]], np.float32)
    w = np.array([0.5, 1.25], np.float32)
    acc, denom = oracle.accumulate_hessian(x, w, chunk_rows=1)
    assert np.allclose(acc, x.T @ (x * w[:, None]))
    assert denom == pytest.approx(1.75)


@pytest.mark.parametrize("weighted", [False, True])
def test_oracle_chunked_fp32_close_to_exact_f64(weighted):
    x = workloads.student_t4(2048, 192, seed=3).float().numpy()
    w = np.random.default_rng(0).uniform(0, 2, 2048).astype(np.float32) if weighted else np.ones(2048, np.float32)
    h, denom = oracle.weighted_covariance(x, w, 256)
    x64 = x.astype(np.float64)
    exact = x64.T @ (x64 * w[:, None].astype(np.float64)) / w.astype(np.float64).sum()
    metrics = oracle.covariance_comparison(exact, h)
    assert metrics["relative_frobenius_difference"] < 1e-6
    assert metrics["candidate_symmetry_max_abs"] == 0.0


def test_oracle_damping_adds_mean_diagonal():
    h = np.diag(np.array([1.0, 2.0, 3.0, 6.0], np.float32))
    d = oracle.damp_diagonal(h, 0.01)
    assert np.allclose(np.diag(d), np.diag(h) + 0.01 * 3.0)
    assert np.array_equal(d - np.diag(np.diag(d)), h - np.diag(np.diag(h)))


def test_covariance_comparison_metric_definition():
    # tests/test_candidate_hessian.py:30-43 endpoints, on the oracle metric
    g = np.eye(3, dtype=np.float32)
    l = np.diag(np.array([2.0, 3.0, 4.0], np.float32))
    m = oracle.covariance_comparison(g, l)
    assert m["trace_ratio"] == 3.0
    assert m["relative_frobenius_difference"] == pytest.approx(np.sqrt(1 + 4 + 9) / np.sqrt(3))
    assert m["candidate_symmetry_max_abs"] == 0.0


# ---------------------------------------- host-side validation (no GPU work)

@pytest.mark.parametrize(
    "rows,weights,error",
    [
        (torch.empty(0, 2), torch.empty(0), "nonempty"),
        (torch.ones(2, 2), torch.ones(3), "shapes"),
        (torch.ones(2, 2), torch.tensor([1.0, -1.0]), "nonnegative"),
        (torch.ones(2, 2), torch.zeros(2), "positive"),
    ],
)
def test_weighted_covariance_rejects_bad_samples(rows, weights, error):
    # tests/test_candidate_hessian.py:46-57
    with pytest.raises(ValueError, match=error):
        ch.weighted_covariance(rows, weights, device=torch.device("cpu"))


def test_shrink_covariance_rejects_invalid_alpha():
    with pytest.raises(ValueError, match="alpha"):
        ch.shrink_covariance(torch.eye(2), torch.eye(2), 1.1)


