"""TEST INFRASTRUCTURE ONLY — CPU oracle of the QSRT trellis bitstream and
its weight decode.

numpy restatements of:
  pack_trellis_edges / unpack_trellis_edges   kquant/qsrt.py:811-857 (16 spans
      of 16 symbols, K bits each, MSB first; adjacent uint16 words swapped)
  reconstruct_trellis_states                  kquant/exl3_reference.py:37-61
      (state = low 16 bits of (previous << K) | edge, cyclic in the tile)
  tensor_core_permutation                     kquant/exl3_reference.py:88-108
  decode_regularized_weight                   kquant/exl3_reference.py:110-147
      (state -> E4M3 label, tiles to [K, N] in row-major element order)
  decode_qsrt_weight                          kquant/exl3_reference.py:149-192,
      270-295 (per-record rate tables, then B_K W B_N with suh / svh)
  record tile order of a packed payload       kquant/qsrt.py:974-1018
  qsrt_linear                                 x @ decode_qsrt_weight(...), the
      dense serving use (scripts/stream_k3_pytorch.py:771-775)
Pinned in tests/test_oracle_qsrt.py by the reference's own known answers
(tests/test_qsrt.py:215-268: packed word prefixes, low-bit round trips, the
scalar recurrence) and tests/test_sqg_e4m3.py:163-200 (custom-codebook and
rate-table decodes).  Only tests/ may import this module.
"""

from __future__ import annotations

import numpy as np

from . import e4m3_values
from .ldl import blockwise_hadamard

TILE = 16
TILE_VALUES = 256


def pack_trellis_edges(indices: np.ndarray, bits: int) -> np.ndarray:
    values = np.asarray(indices, dtype=np.int64) & ((1 << bits) - 1)
    lead = values.shape[:-1]
    spans = values.reshape(*lead, TILE, TILE)
    shifts = np.arange(bits - 1, -1, -1)
    stream = ((spans[..., None] >> shifts) & 1).reshape(*lead, TILE, bits, 16)
    words = (stream << np.arange(15, -1, -1)).sum(axis=-1).reshape(*lead, TILE * bits)
    swapped = words.reshape(*lead, -1, 2)[..., ::-1].reshape(*lead, TILE * bits)
    return swapped.astype(np.uint16).view(np.int16)


def unpack_trellis_edges(packed: np.ndarray, bits: int) -> np.ndarray:
    words = np.asarray(packed).view(np.uint16).astype(np.int64)
    lead = words.shape[:-1]
    words = words.reshape(*lead, -1, 2)[..., ::-1].reshape(*lead, TILE, bits)
    stream = ((words[..., None] >> np.arange(15, -1, -1)) & 1).reshape(*lead, TILE, TILE, bits)
    values = (stream << np.arange(bits - 1, -1, -1)).sum(axis=-1)
    return values.reshape(*lead, TILE_VALUES).astype(np.int16)


def reconstruct_trellis_states(edges: np.ndarray, bits: int) -> np.ndarray:
    edges = np.asarray(edges, dtype=np.int64) & ((1 << bits) - 1)
    states = np.zeros_like(edges)
    for lag in range(-(-16 // bits)):
        states |= np.roll(edges, lag, axis=-1) << (lag * bits)
    return (states & 0xFFFF).astype(np.uint16).view(np.int16)


def tensor_core_permutation() -> np.ndarray:
    perm = np.zeros(TILE_VALUES, dtype=np.int64)
    for thread in range(32):
        row0 = (thread % 4) * 2
        rows = (row0, row0 + 1, row0 + 8, row0 + 9)
        col0 = thread // 4
        for j in range(8):
            perm[thread * 8 + j] = rows[j % 4] * TILE + col0 + 8 * (j // 4)
    return perm


def decode_regularized_weight(states: np.ndarray, labels: np.ndarray) -> np.ndarray:
    """states [K/16, N/16, 256] -> float32 [K, N] through E4M3 labels [65536]."""
    states = np.asarray(states)
    values = e4m3_values(np.asarray(labels, dtype=np.uint8)[states.view(np.uint16).astype(np.int64)])
    k_tiles, n_tiles, _ = states.shape
    tiles = np.empty_like(values)
    tiles[..., tensor_core_permutation()] = values
    return tiles.reshape(k_tiles, n_tiles, TILE, TILE).transpose(0, 2, 1, 3).reshape(
        k_tiles * TILE, n_tiles * TILE).astype(np.float32)


def record_tiles_order(k_tiles: int, n_tiles: int, rate_axis: str, record_tiles: int = 8):
    """(k_tile, n_tile) of every tile in payload order, record by record."""
    order = []
    records = (k_tiles if rate_axis == "k" else n_tiles) // record_tiles
    for record in range(records):
        base = record * record_tiles
        if rate_axis == "k":
            order += [(kt, nt) for kt in range(base, base + record_tiles) for nt in range(n_tiles)]
        else:
            order += [(kt, nt) for kt in range(k_tiles) for nt in range(base, base + record_tiles)]
    return order


def pack_payload(states: np.ndarray, record_bits, rate_axis: str) -> np.ndarray:
    """Concatenated packed words of every record (pack_qsrt_trellis's payload)."""
    k_tiles, n_tiles, _ = states.shape
    pieces = []
    order = record_tiles_order(k_tiles, n_tiles, rate_axis)
    per = len(order) // len(record_bits)
    for record, bits in enumerate(record_bits):
        tiles = np.stack([states[kt, nt] for kt, nt in order[record * per:(record + 1) * per]])
        pieces.append(pack_trellis_edges(tiles, bits).reshape(-1))
    return np.concatenate(pieces)


def unpack_payload_states(payload: np.ndarray, k_tiles: int, n_tiles: int, record_bits,
                          rate_axis: str) -> np.ndarray:
    order = record_tiles_order(k_tiles, n_tiles, rate_axis)
    per = len(order) // len(record_bits)
    states = np.zeros((k_tiles, n_tiles, TILE_VALUES), dtype=np.int16)
    cursor = 0
    for record, bits in enumerate(record_bits):
        words = payload[cursor:cursor + per * TILE * bits].reshape(per, TILE * bits)
        cursor += per * TILE * bits
        tile_states = reconstruct_trellis_states(unpack_trellis_edges(words, bits), bits)
        for (kt, nt), st in zip(order[record * per:(record + 1) * per], tile_states):
            states[kt, nt] = st
    return states


def decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, rate_axis, labels_by_bits, suh=None, svh=None,
                       record_tiles: int = 8) -> np.ndarray:
    """Full decode: per-record rate tables, then (suh, svh given) the rotation
    diag(suh) B_K W B_N diag(svh) in f64; float32 [K, N] regularized otherwise."""
    states = unpack_payload_states(payload, k_tiles, n_tiles, record_bits, rate_axis)
    weight = np.zeros((k_tiles * TILE, n_tiles * TILE), dtype=np.float32)
    for record, bits in enumerate(record_bits):
        sl = slice(record * record_tiles, (record + 1) * record_tiles)
        if rate_axis == "k":
            weight[sl.start * TILE:sl.stop * TILE] = decode_regularized_weight(states[sl], labels_by_bits[bits])
        else:
            weight[:, sl.start * TILE:sl.stop * TILE] = decode_regularized_weight(states[:, sl],
                                                                                labels_by_bits[bits])
    if suh is None:
        return weight
    w = blockwise_hadamard(weight, 3)
    return w * np.asarray(suh, dtype=np.float64)[:, None] * np.asarray(svh, dtype=np.float64)[None, :]


def qsrt_linear(x, payload, k_tiles, n_tiles, record_bits, rate_axis, labels_by_bits, suh=None, svh=None):
    """x [M, K] @ W in f64, W = decode_qsrt_weight(...) (the dense serving
    path: decode, then the linear; scripts/stream_k3_pytorch.py:771-775)."""
    weight = decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, rate_axis, labels_by_bits, suh, svh)
    return np.asarray(x, dtype=np.float64) @ np.asarray(weight, dtype=np.float64)


def situ64(gate, up, beta: float = 4.0, linear_beta: float = 25.0):
    """kquant/tp_simulator.py:83-94 in f64: beta tanh(g / beta) sigmoid(g) *
    linear_beta tanh(u / linear_beta)."""
    g = np.asarray(gate, dtype=np.float64)
    u = np.asarray(up, dtype=np.float64)
    return beta * np.tanh(g / beta) / (1.0 + np.exp(-g)) * (linear_beta * np.tanh(u / linear_beta))


def qsrt_expert_forward(x, route_ids, route_weights, experts, hidden, inter, labels13, labels2,
                        rate13_axis="n", rate2_axis="k", activation="situ"):
    """The routed expert MLP (scripts/closure_exl3_layer.py:557-598 with
    situ) on QSRT experts decoded in f64: experts[e] = (w1, w3, w2), each
    (payload, record_bits, suh, svh); W1, W3 [H, I], W2 [I, H] in the EXL
    orientation; ids outside [0, E) contribute nothing."""
    x = np.asarray(x, dtype=np.float64)
    out = np.zeros((x.shape[0], hidden))
    ht, it = hidden // TILE, inter // TILE
    cache = {}

    def weight(e, j):
        if (e, j) not in cache:
            payload, bits, suh, svh = experts[e][j]
            kt, nt, axis, labels = (ht, it, rate13_axis, labels13) if j < 2 else (it, ht, rate2_axis, labels2)
            cache[e, j] = decode_qsrt_weight(payload, kt, nt, bits, axis, labels, suh, svh)
        return cache[e, j]

    for t in range(x.shape[0]):
        for e, w in zip(np.asarray(route_ids[t]).tolist(), np.asarray(route_weights[t], dtype=np.float64).tolist()):
            if not 0 <= e < len(experts):
                continue
            g, u = x[t] @ weight(e, 0), x[t] @ weight(e, 1)
            a = situ64(g, u) if activation == "situ" else g / (1.0 + np.exp(-g)) * u
            out[t] += w * (a @ weight(e, 2))
    return out
