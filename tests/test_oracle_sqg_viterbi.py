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


def _state_products(mult: int) -> np.ndarray:
    """state * mult mod 2^32 for every 16-bit state (numpy's uint32 wraps)."""
    return np.arange(65536, dtype=np.uint32) * np.uint32(mult)


def test_mcg_labels_follow_their_bit_layout():
    """MCG (kquant/csrc/exl3_compat/quant/codebook.cuh:50-59; multiplier of
    kquant/exl3_encoder_backend.py:24).  The mask keeps sign, exponent bits
    0-1 and the mantissa of each half; the xor sets the exponent's top bits
    to 011 and flips bit 1, so each half is a random sign times
    2^(e - 15) (1 + m/1024) with e in 12..15: |label| < 4 and, for
    equidistributed products, E[label^2] = 2 E[h^2] with
    E[h^2] = (1/4)(4^-3 + 4^-2 + 4^-1 + 1)(7/3) = 595/768."""
    lab = oracle.procedural_labels(1).astype(np.float64)
    assert np.all(np.abs(lab) < 4.0)
    assert abs(lab.mean()) < 0.01
    assert abs(lab.std() / np.sqrt(2 * 595 / 768) - 1.0) < 0.002
    # the two halves read as fp16 numbers and added in float32 (exact for
    # these exponents) with one rounding to fp16: numpy's own arithmetic
    x = (_state_products(0xCBAC1FED) & np.uint32(0x8FFF8FFF)) ^ np.uint32(0x3B603B60)
    halves = x.view(np.float16).reshape(-1, 2).astype(np.float32)
    assert np.array_equal(oracle.procedural_labels(1), (halves[:, 0] + halves[:, 1]).astype(np.float16))


def test_mul1_labels_are_scaled_byte_sums():
    """MUL1 (codebook.cuh:27-47, 80-92; multiplier of
    kquant/exl3_encoder_backend.py:25): the byte sum s of the product, mean
    510 and standard deviation sqrt(4 (2^16 - 1) / 12) = 147.8 for uniform
    bytes, standardised as (s - 510) / 147.7, to within the fp16 rounding of
    the constants and the result (<= 0.0045 over the label range)."""
    s = _state_products(0x83DCD12D).view(np.uint8).reshape(-1, 4).astype(np.int64).sum(axis=1)
    lab = oracle.procedural_labels(2).astype(np.float64)
    assert np.abs(lab - (s - 510) / 147.7).max() <= 0.0045
    assert abs(s.mean() - 510) < 1.0 and abs(s.std() - np.sqrt(4 * 65535 / 12)) < 0.5
    assert abs(lab.std() - 1.0) < 0.005
    # one label per byte sum: the map s -> label is monotone
    order = np.argsort(s, kind="stable")
    assert np.all(np.diff(lab[order]) >= 0)


@pytest.mark.parametrize("codebook,bits", [(1, 2), (2, 3), (1, 4), (2, 4)])
def test_procedural_search_is_optimal_against_one_edge_changes(codebook, bits):
    lab16 = oracle.procedural_labels(codebook)
    x = np.random.default_rng(20 + bits).standard_normal((1, 256)).astype(np.float32)
    out, states = oracle.sqg_quantize_tiles_procedural(x, bits, codebook, 16)
    span = -(-16 // bits)
    rng = np.random.default_rng(30 + bits)
    st = states[0].view(np.uint16).astype(np.int64)
    edges = st & ((1 << bits) - 1)
    assert np.array_equal(qsrt.reconstruct_trellis_states(edges, bits).view(np.uint16), st)
    assert np.array_equal(out[0], lab16[st].astype(np.float32))
    w16 = x[0].astype(np.float16)
    best = _path_cost(st, w16, lab16)
    for p in rng.choice(np.arange(0, 256 - span), 24, replace=False):
        alt = edges.copy()
        alt[p] = (alt[p] + rng.integers(1, 1 << bits)) % (1 << bits)
        alt_states = qsrt.reconstruct_trellis_states(alt, bits).view(np.uint16).astype(np.int64)
        assert _path_cost(alt_states, w16, lab16) >= best
    assert float(((out[0] - x[0]) ** 2).mean()) < 0.15 * (2.0 ** (-2 * (bits - 2)))


def _reference_argmin(costs: np.ndarray, bits: int) -> int:
    """The reference kernel's argmin procedure, step by step
    (kquant/csrc/qsrt_quantize_tiles_kernel.cuh:330-412): strided per-thread
    scans keeping the first strictly smaller cost, warp shuffle-down trees
    (a lane past the warp's end reads its own value; strictly smaller
    wins), per-warp results in shared slots, and warp 0's final tree.  K2:
    1024 threads with stride 1024; K3/K4: threads 0..511 each run two
    streams (from t and from t + 512, stride 1024) into slots w and 16 + w."""
    edges = costs.size

    def scan(start, stride, nthreads):
        t = np.arange(nthreads)
        best_v, best_i = np.full(nthreads, np.inf), np.full(nthreads, -1)
        for j in range(-(-(edges - start) // stride)):
            e = start + t + j * stride
            v = np.where(e < edges, costs[np.minimum(e, edges - 1)], np.inf)
            take = v < best_v
            best_v, best_i = np.where(take, v, best_v), np.where(take, e, best_i)
        return best_v, best_i

    def warp_tree(v, i):
        v, i = v.reshape(-1, 32), i.reshape(-1, 32)
        lanes = np.arange(32)
        for off in (16, 8, 4, 2, 1):
            src = np.where(lanes + off < 32, lanes + off, lanes)
            ov, oi = v[:, src], i[:, src]
            take = ov < v
            v, i = np.where(take, ov, v), np.where(take, oi, i)
        return v[:, 0], i[:, 0]

    if bits == 2:
        slot_v, slot_i = warp_tree(*scan(0, 1024, 1024))
    else:
        a_v, a_i = warp_tree(*scan(0, 1024, 512))
        b_v, b_i = warp_tree(*scan(512, 1024, 512))
        slot_v, slot_i = np.concatenate([a_v, b_v]), np.concatenate([a_i, b_i])
    return int(warp_tree(slot_v, slot_i)[1][0])


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_argmin_tie_order_follows_the_reference_reduction(bits):
    """Pins the closed-form tie key of the oracle's argmin against the
    reference's reduction procedure simulated step by step: cost buffers
    whose minimum is shared by 2, 3 or many entries (some +inf entries,
    which are never picked), and buffers of few distinct values."""
    edges = 65536 >> bits
    rng = np.random.default_rng(bits)
    cases = 0
    for trial in range(60):
        c = rng.choice(np.array([0.75, 1.0, 2.0, np.inf]), size=edges, p=[0.0, 0.6, 0.3, 0.1])
        ties = rng.choice(edges, size=[2, 3, 17][trial % 3], replace=False)
        c[ties] = 0.5
        if trial % 5 == 0:                       # few values: the minimum everywhere
            c = rng.choice(np.array([0.5, 1.0]), size=edges)
        bits16 = c.astype(np.float16).view(np.uint16)
        want = _reference_argmin(c, bits)
        assert oracle.sqg_argmin_edges(bits16) == want, (trial, sorted(ties.tolist()))
        cases += 1
    assert cases == 60
