"""GPU parity of the QSRT trellis bitstream and weight decode
(kq_trellis_pack / kq_trellis_unpack / kq_qsrt_decode_weight /
kq_qsrt_decode_states) against oracle/qsrt.py: bit-exact for words, edges,
states and the regularized weight (E4M3 labels are exact in fp32); the
rotated weight within 2e-6 of max |ref| (fp32 transform vs the f64 oracle).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import exl3_reference as xr
from kquant_amd import qsrt
from kquant_amd.sqg_e4m3 import sqg_e4m3_codebook
from oracle import qsrt as oq

pytestmark = pytest.mark.gpu

_LABELS = {b: oracle.sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)}


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_pack_unpack_match_oracle(gpu, bits):
    rng = np.random.default_rng(bits)
    indices = rng.integers(-32768, 32768, (33, 256)).astype(np.int16)
    packed = qsrt.pack_trellis_edges(torch.from_numpy(indices).to(gpu), bits)
    want = oq.pack_trellis_edges(indices, bits)
    assert np.array_equal(packed.cpu().numpy(), want)
    edges = qsrt.unpack_trellis_edges(packed, bits)
    assert np.array_equal(edges.cpu().numpy(), oq.unpack_trellis_edges(want, bits))
    states = qsrt.unpack_trellis_states(packed, bits)
    assert np.array_equal(states.cpu().numpy(),
                          oq.reconstruct_trellis_states(oq.unpack_trellis_edges(want, bits), bits))
    # the reference's word-order known answer through the GPU
    ar = torch.arange(256, dtype=torch.int16)[None] % (1 << bits)
    prefix = {2: [6939] * 6, 3: [30469, 1337, 1337, 14711, 14711, 30469],
              4: [17767, 291, -12817, -30293, 17767, 291]}[bits]
    assert qsrt.pack_trellis_edges(ar.to(gpu), bits)[0, :6].tolist() == prefix


def _random_matrix(k_tiles, n_tiles, rate_axis, record_bits, seed):
    rng = np.random.default_rng(seed)
    states = np.zeros((k_tiles, n_tiles, 256), dtype=np.int16)
    for kt in range(k_tiles):
        for nt in range(n_tiles):
            bits = record_bits[(kt if rate_axis == "k" else nt) // 8]
            states[kt, nt] = oq.reconstruct_trellis_states(rng.integers(0, 1 << bits, 256), bits)
    return states, oq.pack_payload(states, record_bits, rate_axis)


@pytest.mark.parametrize("rate_axis", ["k", "n"])
def test_payload_decode_matches_oracle(gpu, rate_axis):
    k_tiles, n_tiles = (24, 16) if rate_axis == "k" else (16, 24)
    record_bits = (2, 4, 3)
    states, payload = _random_matrix(k_tiles, n_tiles, rate_axis, record_bits, 5)
    p = torch.from_numpy(payload).to(gpu)
    reg = qsrt.decode_qsrt_payload(p, k_tiles=k_tiles, n_tiles=n_tiles, rate_axis=rate_axis,
                                   record_bits=record_bits)
    want = oq.decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, rate_axis, _LABELS)
    assert np.array_equal(reg.cpu().numpy(), want)
    rng = np.random.default_rng(6)
    suh = rng.choice([-1.0, 1.0], k_tiles * 16).astype(np.float32)
    svh = rng.uniform(0.5, 2.0, n_tiles * 16).astype(np.float32)
    full = qsrt.decode_qsrt_payload(p, k_tiles=k_tiles, n_tiles=n_tiles, rate_axis=rate_axis,
                                    record_bits=record_bits, suh=torch.from_numpy(suh), svh=torch.from_numpy(svh))
    ref = oq.decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, rate_axis, _LABELS, suh, svh)
    assert np.abs(full.cpu().numpy() - ref).max() <= 2e-6 * np.abs(ref).max()
    tr = qsrt.decode_qsrt_payload(p, k_tiles=k_tiles, n_tiles=n_tiles, rate_axis=rate_axis,
                                  record_bits=record_bits, suh=torch.from_numpy(suh), svh=torch.from_numpy(svh),
                                  out_dtype=torch.bfloat16, transposed=True)
    assert torch.equal(tr.cpu(), full.cpu().T.to(torch.bfloat16))


def test_payload_decode_k3_expert_shape(gpu):
    """w1 of a Kimi-K3 expert: EXL [K=3584, N=3072], rate axis n, 24 records."""
    k_tiles, n_tiles = 224, 192
    record_bits = (2, 4) * 2 + (3,) * 20
    rng = np.random.default_rng(9)
    edges = [rng.integers(0, 1 << record_bits[r], (k_tiles, 8, 256)) for r in range(24)]
    states = np.concatenate([oq.reconstruct_trellis_states(e, record_bits[r]) for r, e in enumerate(edges)], axis=1)
    payload = oq.pack_payload(states, record_bits, "n")
    got = qsrt.decode_qsrt_payload(torch.from_numpy(payload).to(gpu), k_tiles=k_tiles, n_tiles=n_tiles,
                                   rate_axis="n", record_bits=record_bits)
    want = oq.decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, "n", _LABELS)
    assert np.array_equal(got.cpu().numpy(), want)


def test_dropin_reference_decoders(gpu):
    # custom E4M3 codebook (kquant tests/test_sqg_e4m3.py:163-173)
    states = torch.arange(256, dtype=torch.int16).reshape(1, 1, 256)
    codebook = sqg_e4m3_codebook(3, "normal")
    got = xr.decode_regularized_weight(states.to(gpu), codebook_values=codebook)
    want = oq.decode_regularized_weight(states.numpy(), codebook.to(torch.float8_e4m3fn).view(torch.uint8).numpy())
    assert got.shape == (16, 16) and np.array_equal(got.cpu().numpy(), want)
    # per-tile rates (kquant tests/test_sqg_e4m3.py:176-200), arbitrary states
    st = torch.arange(3 * 3 * 256, dtype=torch.int32).to(torch.int16).reshape(3, 3, 256)
    for rate_axis in ("k", "n"):
        got = xr.decode_qsrt_regularized_weight(st.to(gpu), rate_axis=rate_axis, tile_bits=(2, 3, 4),
                                                codebook=xr.CODEBOOK_SQG_XOR_CHEB_T12)
        pieces = []
        for tile, bits in enumerate((2, 3, 4)):
            sel = st.narrow(0 if rate_axis == "k" else 1, tile, 1).numpy()
            pieces.append(oq.decode_regularized_weight(sel, _LABELS[bits]))
        assert np.array_equal(got.cpu().numpy(), np.concatenate(pieces, axis=0 if rate_axis == "k" else 1))
    # edges -> states
    edges = torch.randint(0, 8, (4, 256), generator=torch.Generator().manual_seed(2))
    assert np.array_equal(xr.reconstruct_trellis_states(edges.to(gpu), 3).cpu().numpy(),
                          oq.reconstruct_trellis_states(edges.numpy(), 3))
    assert torch.equal(xr.tensor_core_permutation(), torch.from_numpy(oq.tensor_core_permutation()))


def test_payload_decode_paths_agree(gpu):
    """A 4-byte-aligned payload takes the LDS decode, a 2-byte-aligned one the
    first kernel: the regularized weights agree bit for bit, the rotated ones
    to fp32 rounding."""
    from kquant_amd import _native as N

    k_tiles, n_tiles, record_bits = 16, 24, (2, 4, 3)
    _, payload = _random_matrix(k_tiles, n_tiles, "n", record_bits, 17)
    buf = torch.zeros(payload.size + 2, dtype=torch.int16, device=gpu)
    buf[1:1 + payload.size] = torch.from_numpy(payload).to(gpu)
    odd = buf[1:1 + payload.size]  # 2-byte aligned
    even = torch.from_numpy(payload).to(gpu)
    assert odd.data_ptr() % 4 == 2 and even.data_ptr() % 4 == 0
    labels = qsrt.rate_labels(rate_axis="n", device=gpu)
    rng = np.random.default_rng(18)
    suh = torch.from_numpy(rng.choice([-1.0, 1.0], k_tiles * 16).astype(np.float32)).to(gpu)
    svh = torch.from_numpy(rng.uniform(0.5, 2.0, n_tiles * 16).astype(np.float32)).to(gpu)
    outs = {}
    for name, p in (("odd", odd), ("even", even)):
        for rot in (False, True):
            out = torch.empty(k_tiles * 16, n_tiles * 16, device=gpu)
            N.call("kq_qsrt_decode_weight", N.ptr(p), p.numel(), k_tiles, n_tiles, 1, bytes(record_bits),
                   N.ptr(labels), N.ptr(suh) if rot else None, N.ptr(svh) if rot else None, N.DT_F32, N.ptr(out),
                   n_tiles * 16, 0, N.stream(gpu))
            outs[name, rot] = out.cpu().numpy()
    assert np.array_equal(outs["odd", False], outs["even", False])
    ref = outs["even", True]
    assert np.abs(outs["odd", True] - ref).max() <= 2e-6 * np.abs(ref).max()
