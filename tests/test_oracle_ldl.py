"""Pins the CPU oracle of the encoder's Hessian finalize (oracle/ldl.py).

Each check is fixed by mathematics or by the reference's own definitions,
not by retyping the oracle: the Hadamard closed form and orthogonality, the
block LDL identity H = L_u D L_u^T, the textbook LDL^T at b = 1, and a planted
mistake in each of the first two caught.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ldl


def _spd(n: int, seed: int, rows: int | None = None) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows or 2 * n, n))
    h = x.T @ x / x.shape[0]
    return h + 0.025 * np.diag(h).mean() * np.eye(n)


@pytest.mark.parametrize("size", [1, 2, 8, 128])
def test_hadamard_closed_form_and_orthogonal(size):
    h = ldl.normalized_hadamard(size)
    i, j = np.meshgrid(np.arange(size), np.arange(size), indexing="ij")
    signs = np.vectorize(lambda a: (-1) ** bin(a).count("1"))(i & j)
    assert np.array_equal(h * np.sqrt(size), signs)  # Sylvester order, exl3_reference.py:195-212
    assert np.allclose(h @ h.T, np.eye(size), atol=1e-12)


def test_hadamard_planted_transpose_is_caught():
    # Sylvester's matrix is symmetric, so a transposed operand would pass;
    # a row-reversed (wrong-order) matrix must not
    h = ldl.normalized_hadamard(8)
    assert np.array_equal(h, h.T)
    assert not np.array_equal(h[::-1], ldl.normalized_hadamard(8))


def test_blockwise_rotation_equals_dense_block_product():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((256, 384))
    rs, cs = rng.choice([-1.0, 1.0], 256), rng.choice([-1.0, 1.0], 384)
    b_rows = np.kron(np.eye(2), ldl.normalized_hadamard(128))
    b_cols = np.kron(np.eye(3), ldl.normalized_hadamard(128))
    want = b_rows @ np.diag(rs) @ x @ np.diag(cs) @ b_cols
    assert np.allclose(ldl.blockwise_hadamard(x, 3, rs, cs), want, atol=1e-12)
    assert np.allclose(ldl.blockwise_hadamard(x, 1), b_rows @ x, atol=1e-12)
    assert np.allclose(ldl.blockwise_hadamard(x, 2), x @ b_cols, atol=1e-12)


@pytest.mark.parametrize("b", [1, 4, 16])
def test_block_ldl_reconstructs_h(b):
    h = _spd(64, b)
    lu = ldl.block_ldl(h, b)
    d = ldl.block_diagonal_d(h, b)
    assert np.allclose(lu @ d @ lu.T, h, rtol=1e-10, atol=1e-12)
    for i in range(64 // b):
        blk = slice(i * b, (i + 1) * b)
        assert np.array_equal(lu[blk, blk], np.eye(b))
    assert np.allclose(np.triu(lu, 1), 0.0)


def test_block_ldl_b1_is_textbook_ldlt():
    h = _spd(32, 7)
    lower = np.linalg.cholesky(h)
    assert np.allclose(ldl.block_ldl(h, 1), lower / np.diag(lower)[None, :], atol=1e-12)


def test_block_ldl_planted_mistake_is_caught():
    h = _spd(48, 9)
    lu = ldl.block_ldl(h, 16)
    d = ldl.block_diagonal_d(h, 16)
    wrong = lu.copy()
    wrong[32:48, 16:32] = wrong[32:48, 16:32].T  # a transposed block
    assert not np.allclose(wrong @ d @ wrong.T, h, rtol=1e-6)


def test_regularize_and_finalize():
    h = _spd(128, 3) * 10.0
    reg, diag, mean = ldl.regularize(h, 10.0, 0.025)
    assert np.isclose(mean, np.diag(h / 10.0).mean())
    assert np.allclose(np.diag(reg), np.diag(h / 10.0) * 1.0 + 0.025 * mean)
    assert np.allclose(diag, np.diag(reg))
    same, _, zero_mean = ldl.regularize(h, 0, 0.025)  # count 0: untouched
    assert zero_mean == 0.0 and np.array_equal(same, h)
    su = np.random.default_rng(4).choice([-1.0, 1.0], 128)
    q_fallback, rot, lower, _ = ldl.finalize(h, 10.0, 0.025, su)
    assert not q_fallback and np.allclose(np.diag(lower), 0.0)
    assert np.allclose(rot, ldl.blockwise_hadamard(reg, 3, su, su))
    assert ldl.finalize(h, 0, 0.025, su)[0] and ldl.finalize(h, 0, 0.025, su)[2] is None
