"""TEST INFRASTRUCTURE ONLY — CPU oracle of the encoder's Hessian finalize.

numpy restatements (f64 unless stated) of:
  normalized_hadamard     kquant/exl3_reference.py:195-212 (Sylvester order,
                          [[M, M], [M, -M]], scaled by 1/sqrt(size))
  blockwise_hadamard      kquant/exl3_encoder_backend.py:288-313
                          (blockwise_preapply_had_l_ / _r_) and the rotation
                          of finalize_capture_H, :1640-1644
  regularize              kquant/exl3_encoder_backend.py:1611-1628
  block_ldl               kquant/exl3_encoder_backend.py:316-386 (Cholesky by
                          numpy.linalg.cholesky, a library routine; the
                          diagonal-block inverses and block-column products)
  finalize                kquant/exl3_encoder_backend.py:1588-1663 with the
                          sign vector su given (the reference draws it from
                          torch.randn)

Pinned by tests/test_oracle_ldl.py: Hadamard orthogonality and the closed form
H[i][j] = (-1)^popcount(i & j) / sqrt(n); the block LDL identity
L_u D L_u^T = H with D_i = DL_i DL_i^T; b = 1 reducing to the textbook LDL^T;
the rotation commuting with the closed-form matrix product.
Only tests/ may import this module.
"""

from __future__ import annotations

import numpy as np


def normalized_hadamard(size: int = 128) -> np.ndarray:
    if size <= 0 or size & (size - 1):
        raise ValueError("Hadamard size must be a positive power of two")
    m = np.ones((1, 1))
    while m.shape[0] < size:
        m = np.block([[m, m], [m, -m]])
    return m / np.sqrt(size)


def blockwise_hadamard(x: np.ndarray, sides: int, row_scale=None, col_scale=None, size: int = 128) -> np.ndarray:
    """B S_r X S_c B restricted to the requested sides (1 left, 2 right, 3 both)."""
    x = np.array(x, dtype=np.float64)
    if row_scale is not None:
        x = x * np.asarray(row_scale, dtype=np.float64)[:, None]
    if col_scale is not None:
        x = x * np.asarray(col_scale, dtype=np.float64)[None, :]
    had = normalized_hadamard(size)
    rows, cols = x.shape
    if sides & 2:
        x = (x.reshape(rows, cols // size, size) @ had).reshape(rows, cols)
    if sides & 1:
        x = (had @ x.reshape(rows // size, size, cols)).reshape(rows, cols)
    return x


def regularize(h: np.ndarray, count: float, sigma_reg: float) -> tuple[np.ndarray, np.ndarray, float]:
    """H /= count; diag += sigma * mean(diag) (count 0: mean 0, H unchanged).
    Returns (H, damped diag, mean)."""
    h = np.array(h, dtype=np.float64)
    mean = 0.0
    if count > 0:
        h = h / count
        mean = float(np.diag(h).mean())
    idx = np.arange(h.shape[0])
    h[idx, idx] += sigma_reg * mean
    return h, h[idx, idx].copy(), mean


def block_ldl(h: np.ndarray, b: int) -> np.ndarray:
    """Unit block-lower L_u with H = L_u D L_u^T (D block diagonal)."""
    h = np.asarray(h, dtype=np.float64)
    n = h.shape[0]
    if n % b:
        raise ValueError("n must be a multiple of b")
    lower = np.linalg.cholesky(h)
    m = n // b
    out = lower.copy()
    for i in range(m):
        blk = slice(i * b, (i + 1) * b)
        inv = np.linalg.inv(lower[blk, blk])
        out[:, blk] = lower[:, blk] @ inv
        out[blk, blk] = np.eye(b)
    return out


def block_diagonal_d(h: np.ndarray, b: int) -> np.ndarray:
    """D of the block LDL: D_i = DL_i DL_i^T from the Cholesky factor."""
    lower = np.linalg.cholesky(np.asarray(h, dtype=np.float64))
    n = h.shape[0]
    d = np.zeros_like(lower)
    for i in range(n // b):
        blk = slice(i * b, (i + 1) * b)
        d[blk, blk] = lower[blk, blk] @ lower[blk, blk].T
    return d


def finalize(h: np.ndarray, count: float, sigma_reg: float, su: np.ndarray, b: int = 16):
    """(q_fallback, rotated H, L with zero diagonal or None, damped diag)."""
    h, diag, mean = regularize(h, count, sigma_reg)
    q_fallback = count == 0 or mean < 1e-20
    su = np.asarray(su, dtype=np.float64).reshape(-1)
    h = blockwise_hadamard(h, 3, su, su)
    lower = None
    if not q_fallback:
        lower = block_ldl(h, b)
        idx = np.arange(h.shape[0])
        lower[idx, idx] = 0.0
    return q_fallback, h, lower, diag
