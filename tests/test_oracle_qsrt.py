"""Pins the CPU oracle of the QSRT trellis bitstream and decode
(oracle/qsrt.py) with the reference's own known answers and closed forms."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import qsrt


@pytest.mark.parametrize(
    ("bits", "expected_prefix"),
    [  # kquant tests/test_qsrt.py:215-231 (native pack.cu word order)
        (2, [6939] * 6),
        (3, [30469, 1337, 1337, 14711, 14711, 30469]),
        (4, [17767, 291, -12817, -30293, 17767, 291]),
    ],
)
def test_pack_matches_reference_word_prefixes(bits, expected_prefix):
    indices = (np.arange(256) % (1 << bits)).astype(np.int16)[None]
    packed = qsrt.pack_trellis_edges(indices, bits)
    assert packed.shape == (1, 16 * bits)
    assert packed[0, : len(expected_prefix)].tolist() == expected_prefix
    assert np.array_equal(qsrt.unpack_trellis_edges(packed, bits), indices)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_pack_keeps_only_low_bits(bits):
    rng = np.random.default_rng(100 + bits)
    indices = rng.integers(-32768, 32768, (7, 256))
    got = qsrt.unpack_trellis_edges(qsrt.pack_trellis_edges(indices, bits), bits)
    assert np.array_equal(got.astype(np.int64), indices & ((1 << bits) - 1))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_states_follow_the_scalar_recurrence(bits):
    # kquant tests/test_qsrt.py:254-268: warm up on the tile's last edges, then
    # state = ((state << K) | edge) & 0xFFFF
    rng = np.random.default_rng(175 + bits)
    edges = rng.integers(0, 1 << bits, (3, 5, 256))
    want = np.zeros_like(edges)
    for idx in np.ndindex(3, 5):
        state = 0
        for e in edges[idx][-((16 + bits - 1) // bits):]:
            state = ((state << bits) | int(e)) & 0xFFFF
        for i, e in enumerate(edges[idx]):
            state = ((state << bits) | int(e)) & 0xFFFF
            want[idx][i] = state
    assert np.array_equal(qsrt.reconstruct_trellis_states(edges, bits).view(np.uint16), want)
    # a closed path round-trips through its packed edges
    states = qsrt.reconstruct_trellis_states(edges[0], bits)
    back = qsrt.reconstruct_trellis_states(qsrt.unpack_trellis_edges(qsrt.pack_trellis_edges(states, bits), bits),
                                           bits)
    assert np.array_equal(back, states)


def test_tensor_core_permutation_is_a_bijection_with_known_entries():
    perm = qsrt.tensor_core_permutation()
    assert sorted(perm.tolist()) == list(range(256))
    # thread 0: rows 0, 1, 8, 9 of column 0 then column 8; thread 1 starts at row 2
    assert perm[:9].tolist() == [0, 16, 128, 144, 8, 24, 136, 152, 32]


def test_decode_custom_codebook_places_each_state_once():
    # kquant tests/test_sqg_e4m3.py:163-173: states 0..255 decode to a
    # permutation of the first 256 labels
    labels = oracle.sqg_xor_cheb_t12_bytes(3)
    states = np.arange(256, dtype=np.int16).reshape(1, 1, 256)
    decoded = qsrt.decode_regularized_weight(states, labels)
    assert decoded.shape == (16, 16)
    assert np.array_equal(np.sort(decoded.ravel()), np.sort(oracle.e4m3_values(labels[:256])))
    # and element t sits at row-major position perm[t]
    perm = qsrt.tensor_core_permutation()
    assert np.array_equal(decoded.ravel()[perm], oracle.e4m3_values(labels[:256]))


@pytest.mark.parametrize("rate_axis", ["k", "n"])
def test_payload_round_trip_and_rotation(rate_axis):
    rng = np.random.default_rng(7)
    k_tiles, n_tiles = (16, 8) if rate_axis == "k" else (8, 16)
    record_bits = (2, 4)
    states = np.zeros((k_tiles, n_tiles, 256), dtype=np.int16)
    labels = {b: oracle.sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)}
    for kt in range(k_tiles):
        for nt in range(n_tiles):
            bits = record_bits[(kt if rate_axis == "k" else nt) // 8]
            states[kt, nt] = qsrt.reconstruct_trellis_states(rng.integers(0, 1 << bits, 256), bits)
    payload = qsrt.pack_payload(states, record_bits, rate_axis)
    assert payload.size == k_tiles * n_tiles * 16 * 3  # six bits per coefficient pair on average
    assert np.array_equal(qsrt.unpack_payload_states(payload, k_tiles, n_tiles, record_bits, rate_axis), states)
    reg = qsrt.decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, rate_axis, labels)
    suh = rng.choice([-1.0, 1.0], k_tiles * 16)
    svh = rng.uniform(0.5, 2.0, n_tiles * 16)
    full = qsrt.decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, rate_axis, labels, suh, svh)
    # the rotation is orthogonal up to the scales: undo it in closed form
    h = oracle.ldl.normalized_hadamard(128)
    bk = np.kron(np.eye(k_tiles // 8), h)
    bn = np.kron(np.eye(n_tiles // 8), h)
    undone = bk.T @ (full / suh[:, None] / svh[None, :]) @ bn.T
    assert np.allclose(undone, reg, atol=1e-9)


def test_situ64_is_the_pinned_fp32_situ_in_double():
    """situ64 restates kquant/tp_simulator.py:83-94 in f64; oracle.situ (the
    fp32 restatement, pinned by the reference's known answers in the GPU MLP
    tests) must agree to fp32 rounding, and the closed forms hold: 0 at
    g = 0 or u = 0, odd in u, and -> beta * linear_beta * tanh(u / lb) for
    large g."""
    rng = np.random.default_rng(3)
    g = rng.standard_normal(4096) * 6
    u = rng.standard_normal(4096) * 40
    a64 = qsrt.situ64(g, u)
    a32 = oracle.situ(g.astype(np.float32), u.astype(np.float32)).astype(np.float64)
    assert np.allclose(a64, a32, rtol=2e-6, atol=1e-6)
    assert np.all(qsrt.situ64(np.zeros(8), u[:8]) == 0) and np.all(qsrt.situ64(g[:8], np.zeros(8)) == 0)
    assert np.allclose(qsrt.situ64(g, -u), -a64)
    assert np.allclose(qsrt.situ64(np.full(4, 60.0), u[:4]), 4.0 * 25.0 * np.tanh(u[:4] / 25.0))


def test_linear_and_expert_oracles_reduce_to_the_decoded_weight():
    """qsrt_linear with one-hot rows returns rows of decode_qsrt_weight; the
    expert oracle is linear in the route weights and ignores invalid ids."""
    rng = np.random.default_rng(4)
    labels = {b: oracle.sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)}
    k_tiles, n_tiles, bits = 16, 8, (3, 2)
    states = np.stack([qsrt.reconstruct_trellis_states(rng.integers(0, 8, (n_tiles, 256)), 3)
                       for _ in range(k_tiles)]).astype(np.int16)
    payload = qsrt.pack_payload(states, bits, "k")
    w = qsrt.decode_qsrt_weight(payload, k_tiles, n_tiles, bits, "k", labels)
    rows = np.array([0, 5, 130, 255])
    x = np.zeros((4, k_tiles * 16))
    x[np.arange(4), rows] = 1.0
    assert np.array_equal(qsrt.qsrt_linear(x, payload, k_tiles, n_tiles, bits, "k", labels), w[rows])

    def mat(k, n, axis):
        recs = (k if axis == "k" else n) // 128
        per = 8 * ((n if axis == "k" else k) // 16)
        return (rng.integers(-32768, 32768, per * 16 * 3 * recs).astype(np.int16), (3,) * recs,
                rng.uniform(0.5, 1.5, k), rng.uniform(0.5, 1.5, n))

    experts = [(mat(256, 128, "n"), mat(256, 128, "n"), mat(128, 256, "k")) for _ in range(2)]
    x = rng.standard_normal((1, 256)) * 0.05
    one = qsrt.qsrt_expert_forward(x, [[0, 1]], [[1.0, 0.0]], experts, 256, 128, labels, labels)
    two = qsrt.qsrt_expert_forward(x, [[0, 1]], [[2.0, 0.0]], experts, 256, 128, labels, labels)
    skip = qsrt.qsrt_expert_forward(x, [[0, 7]], [[1.0, 3.0]], experts, 256, 128, labels, labels)
    assert np.allclose(two, 2 * one) and np.array_equal(skip, one) and np.abs(one).max() > 0
