"""Input builders shared by the codec tests (CPU and GPU)."""

from __future__ import annotations

import numpy as np


def finite_bf16_patterns() -> np.ndarray:
    """All 65,536 bf16 bit patterns except infinities and NaNs."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    exp = (bits >> 7) & 0xFF
    return bits[exp != 0xFF].astype(np.uint16)


def exhaustive_scale_blocks(qmax: float, span_hi: int, span_lo: int) -> np.ndarray:
    """Blocks that put every finite bf16 value under a sweep of block scales.

    Each block holds one setter A = qmax * 2^t (so the block exponent is t)
    and up to 31 bf16 values of one binade E.  For every binade, t runs over
    E - span_hi .. E + span_lo, so v / 2^t sweeps from the top of the target
    format's range down past its smallest subnormal.  Returns uint16 bf16 bit
    patterns of shape [blocks, 32].
    """
    vals = finite_bf16_patterns()
    exps = ((vals.astype(np.uint32) >> 7) & 0xFF).astype(np.int64)
    blocks = []
    for e_biased in range(0, 255):
        group = vals[exps == e_biased]
        e_unb = max(e_biased, 1) - 127
        for t in range(e_unb - span_hi, e_unb + span_lo + 1):
            with np.errstate(over="ignore"):
                setter = np.float32(np.ldexp(np.float64(qmax), t))
            sbits = int(setter.view(np.uint32))
            if not np.isfinite(setter) or setter == 0 or (sbits & 0xFFFF):
                continue  # not an exact, finite, nonzero bf16
            for i in range(0, group.size, 31):
                chunk = group[i : i + 31]
                blk = np.zeros(32, dtype=np.uint16)
                blk[0] = sbits >> 16
                blk[1 : 1 + chunk.size] = chunk
                blocks.append(blk)
    return np.stack(blocks)


def random_blocks_bf16(n_blocks: int, seed: int = 0) -> np.ndarray:
    """Random bf16 blocks whose elements span ~24 binades below the block max,
    with exact E2M1/E4M3 rounding ties planted."""
    rng = np.random.default_rng(seed)
    top = rng.integers(-100, 100, size=(n_blocks, 1))
    expo = top - rng.integers(0, 24, size=(n_blocks, 32))
    mant = rng.integers(0, 128, size=(n_blocks, 32))
    sign = rng.integers(0, 2, size=(n_blocks, 32))
    v = np.ldexp(1.0 + mant / 128.0, expo) * np.where(sign, -1.0, 1.0)
    bits = (v.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    # zero blocks and blocks with zeros / negative zeros
    bits[:: 97] = 0
    bits[1:: 89, ::3] = 0x8000
    return bits
