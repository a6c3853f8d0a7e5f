"""Write the golden fixtures of this directory from the reference implementation.

Run in the build container only (``python tests/golden/make_golden.py``): it
imports kquant from /root/reference to record outputs that no reference test
or closed form pins:

* the SQG tables without a hash in the reference's tests (the mix-width rank
  permutation, the R44 research table, the full 65,536-entry ndtri
  staircase and the codebooks built from it), as SHA-256 digests plus
  evenly spaced samples;
* ``mxfp8_quantize_cpu`` on float32 blocks whose amax sits within a few ulps
  of 448 * 2^k, where the f32 ``log2`` of the reference decides the scale.

The fixtures are data (inputs and expected outputs); nothing here is loaded
at test time except the JSON files.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REFERENCE = Path("/root/reference")


def _table(t) -> dict:
    t = t.contiguous()
    n = int(t.numel())
    idx = sorted(set(list(range(0, n, max(1, n // 64))) + [n - 1]))
    return {
        "dtype": str(t.dtype).replace("torch.", ""),
        "numel": n,
        "sha256": hashlib.sha256(t.numpy().tobytes()).hexdigest(),
        "samples": [[i, int(t[i])] for i in idx],
    }


def sqg_fixture(S) -> dict:
    out = {}
    for bits in (2, 3, 4):
        out[f"sqg_rank_permutation_k{bits}"] = _table(S.sqg_rank_permutation(bits))
        out[f"sqg_xor_rank_permutation_k{bits}"] = _table(S.sqg_xor_rank_permutation(bits))
        out[f"sqg_e4m3_bytes_normal_k{bits}"] = _table(S.sqg_e4m3_bytes(bits, "normal"))
        out[f"sqg_cheb_normal_e4m3_bytes_k{bits}"] = _table(S.sqg_cheb_normal_e4m3_bytes(bits))
        out[f"sqg_xor_cheb_t12_bytes_k{bits}"] = _table(S.sqg_xor_cheb_t12_bytes(bits))
        for axis in ("k", "n"):
            out[f"sqg_cheb_k{bits}_{axis}"] = _table(
                S.sqg_codebook_bytes(bits, "sqg_cheb", rate_axis=axis)
            )
    out["sqg_cheb_normal_rank_e4m3_bytes"] = _table(S.sqg_cheb_normal_rank_e4m3_bytes())
    out["sqg_xor_cheb_t12_rank_lut_bytes"] = _table(S.sqg_xor_cheb_t12_rank_lut_bytes())
    for h in (2, 4, 9, 15):
        out[f"sqg_k2_eight_stratum_rank_permutation_h{h}"] = _table(
            S.sqg_k2_eight_stratum_rank_permutation(h)
        )
    return out


def _boundary_blocks() -> np.ndarray:
    g = np.random.default_rng(2024)
    blocks = []
    for k in (-133, -130, -127, -126, -100, -60, -20, -1, 0, 1, 5, 20, 60, 100, 120, 127):
        base = np.float32(np.ldexp(np.float64(448.0), k))
        cands = [base]
        lo = hi = base
        for _ in range(3):
            lo = np.nextafter(lo, np.float32(0))
            hi = np.nextafter(hi, np.float32(np.inf))
            cands += [lo, hi]
        for amax in cands:
            if not np.isfinite(amax) or amax == 0:
                continue
            blk = (g.uniform(-1, 1, 32) * np.float64(amax)).astype(np.float32)
            blk[g.integers(0, 32)] = amax if g.random() < 0.5 else -amax
            blocks.append(blk)
    for amax in (np.float32(3.4e38), np.float32(1e-40), np.float32(1e-45), np.float32(0.0)):
        blk = (g.uniform(-1, 1, 32) * np.float64(amax)).astype(np.float32)
        blk[0] = amax
        blocks.append(blk)
    if len(blocks) % 2:
        blocks.append(np.zeros(32, np.float32))
    return np.stack(blocks).reshape(-1, 64)


def mxfp8_fixture(M) -> dict:
    import torch

    x = _boundary_blocks()
    q, s = M.mxfp8_quantize_cpu(torch.from_numpy(x))
    return {
        "shape": list(x.shape),
        "input_f32_bits": x.view(np.uint32).ravel().tolist(),
        "q_bytes": q.view(torch.uint8).numpy().ravel().tolist(),
        "scale_bytes": s.numpy().ravel().tolist(),
    }


def main() -> None:
    sys.path.insert(0, str(REFERENCE))
    from kquant import mxfp8 as M
    from kquant import sqg_e4m3 as S

    (HERE / "sqg_tables.json").write_text(json.dumps(sqg_fixture(S), indent=1) + "\n")
    (HERE / "mxfp8_f32_boundaries.json").write_text(json.dumps(mxfp8_fixture(M)) + "\n")


if __name__ == "__main__":
    main()
