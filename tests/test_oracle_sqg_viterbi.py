"""Pins the C oracle of the SQG trellis quantizer (oracle/sqg_viterbi.c):
its fp16 rounding against numpy's float16 conversion, and the search by
properties a wrong index, sign or rounding would break - the result is a
closed cyclic trellis path whose values are its labels, and its fp16 path
cost (the quantity the search minimises, rounded as it rounds) is no larger
than that of any path one edge away with the same boundary state."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import qsrt


def test_fp16_rounding_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000) * np.exp2(rng.integers(-30, 18, 20000)),
        np.array([65504.0, 65519.99, 65520.0, 1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001,
                  3 * 2.0 ** -26, 0.0, -0.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]),
    ])
    got = oracle.f64_to_f16_bits(x)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


def _path_cost(states: np.ndarray, w16: np.ndarray, lab16: np.ndarray) -> np.float16:
    """fp16 cost of a closed path as the closing pass accumulates it."""
    cost = None
    for i in range(256):
        d = np.float16(np.float64(lab16[states[i]]) - np.float64(w16[i]))
        dd = np.float64(d) * np.float64(d)
        cost = np.float16(dd) if cost is None else np.float16(dd + np.float64(cost))
    return cost


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_search_is_optimal_against_one_edge_changes(bits):
    lut = oracle.sqg_xor_cheb_t12_bytes(bits)
    x = np.random.default_rng(bits).standard_normal((2, 256)).astype(np.float32)
    out, states = oracle.sqg_quantize_tiles(x, lut, bits, 16)
    lab16 = oracle.e4m3_values(lut).astype(np.float16)
    span = -(-16 // bits)
    rng = np.random.default_rng(10 + bits)
    for t in range(2):
        st = states[t].view(np.uint16).astype(np.int64)
        edges = st & ((1 << bits) - 1)
        assert np.array_equal(qsrt.reconstruct_trellis_states(edges, bits).view(np.uint16), st)
        assert np.array_equal(out[t], lab16[st].astype(np.float32))
        w16 = x[t].astype(np.float16)
        best = _path_cost(st, w16, lab16)
        # one-edge changes that keep the node before position 0 (the closing
        # pass's fixed boundary): positions whose edge is not in that node
        for p in rng.choice(np.arange(0, 256 - span), 24, replace=False):
            alt = edges.copy()
            alt[p] = (alt[p] + rng.integers(1, 1 << bits)) % (1 << bits)
            alt_states = qsrt.reconstruct_trellis_states(alt, bits).view(np.uint16).astype(np.int64)
            assert _path_cost(alt_states, w16, lab16) >= best
        # rate-distortion sanity: about 6 dB per bit (a wrong search is far worse)
        assert float(((out[t] - x[t]) ** 2).mean()) < 0.15 * (2.0 ** (-2 * (bits - 2)))
