"""GPU parity of the routed expert forward on QSRT-coded experts
(kq_qsrt_moe_decode through kquant_amd.qsrt.qsrt_expert_forward) against
oracle/qsrt.py (each expert's w1 / w3 / w2 decoded in f64, the expert MLP
in f64): fp32 arithmetic throughout, so within 2e-5 of max |ref|.  Covers
mixed record rates, several K chunks of the gate/up projection, invalid
expert ids, SiTU and SwiGLU, bf16 and fp32 activations, and a Kimi-K3
TP12-local geometry (H = 3584, I = 256, top-16) checked against the decoded
weights' dense product."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import qsrt
from oracle import qsrt as oq

pytestmark = pytest.mark.gpu

_LABELS = {b: oracle.sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)}


def _matrix(rng, k, n, axis):
    records = (k if axis == "k" else n) // 128
    bits = tuple(int(b) for b in rng.integers(2, 5, records))
    per_record = 8 * ((n if axis == "k" else k) // 16)
    words = sum(per_record * 16 * b for b in bits)
    payload = rng.integers(-32768, 32768, words).astype(np.int16)
    suh = (rng.choice([-1.0, 1.0], k) * rng.uniform(0.5, 1.5, k)).astype(np.float32)
    svh = rng.uniform(0.5, 2.0, n).astype(np.float32)
    return payload, bits, suh, svh


def _experts(seed, count, hidden, inter):
    rng = np.random.default_rng(seed)
    spec = [(_matrix(rng, hidden, inter, "n"), _matrix(rng, hidden, inter, "n"), _matrix(rng, inter, hidden, "k"))
            for _ in range(count)]

    def as_torch(m):
        return tuple(torch.from_numpy(v) if isinstance(v, np.ndarray) else v for v in m)

    dev = qsrt.QSRTExperts([as_torch(s[0]) for s in spec], [as_torch(s[1]) for s in spec],
                           [as_torch(s[2]) for s in spec], hidden=hidden, inter=inter)
    return spec, dev


@pytest.mark.parametrize("activation,x_dtype", [("situ", torch.float32), ("swiglu", torch.bfloat16)])
def test_routed_forward_matches_oracle(gpu, activation, x_dtype):
    hidden, inter, count, tokens, topk = 640, 256, 5, 3, 4
    spec, experts = _experts(7, count, hidden, inter)
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((tokens, hidden)) * 0.05).astype(np.float32)
    ids = rng.integers(0, count, (tokens, topk)).astype(np.int32)
    ids[0, 1] = -1  # ids outside [0, experts) contribute nothing
    ids[2, 3] = count + 2
    wts = rng.uniform(0.1, 1.0, (tokens, topk)).astype(np.float32)
    xt = torch.from_numpy(x).to(gpu).to(x_dtype)
    got = qsrt.qsrt_expert_forward(xt, torch.from_numpy(ids).to(gpu), torch.from_numpy(wts).to(gpu), experts,
                                   activation=activation, out_dtype=torch.float32)
    ref = oq.qsrt_expert_forward(xt.float().cpu().numpy(), ids, wts, spec, hidden, inter, _LABELS, _LABELS,
                                 activation=activation)
    assert np.abs(got.cpu().numpy() - ref).max() <= 2e-5 * np.abs(ref).max()


def test_tokens_without_valid_experts_give_zero_and_calls_repeat_exactly(gpu):
    hidden, inter = 256, 256
    _, experts = _experts(9, 3, hidden, inter)
    x = torch.randn(2, hidden, device=gpu) * 0.05
    ids = torch.tensor([[-1, 5], [0, 2]], dtype=torch.int32, device=gpu)
    wts = torch.ones(2, 2, device=gpu)
    first = qsrt.qsrt_expert_forward(x, ids, wts, experts, out_dtype=torch.float32)
    assert torch.count_nonzero(first[0]).item() == 0
    for _ in range(3):  # the workspace counters are back at zero after every call
        assert torch.equal(qsrt.qsrt_expert_forward(x, ids, wts, experts, out_dtype=torch.float32), first)


def test_tp12_geometry_matches_dense_product(gpu):
    """Kimi-K3 at TP12: H = 3584, the rank's 256 intermediate channels,
    top-16 routing; reference = the decoded weights (kq_qsrt_decode_weight,
    pinned against the oracle elsewhere) applied in f64."""
    hidden, inter, count, tokens, topk = 3584, 256, 20, 2, 16
    rng = np.random.default_rng(11)
    mats = []
    for e in range(count):
        row = []
        for kind in ("w1", "w3", "w2"):
            k, n, axis = (hidden, inter, "n") if kind != "w2" else (inter, hidden, "k")
            payload, bits, suh, svh = _matrix(rng, k, n, axis)
            row.append((torch.from_numpy(payload).to(gpu), bits, torch.from_numpy(suh).to(gpu),
                        torch.from_numpy(svh).to(gpu)))
        mats.append(row)
    experts = qsrt.QSRTExperts([m[0] for m in mats], [m[1] for m in mats], [m[2] for m in mats], hidden=hidden,
                               inter=inter)
    x = torch.randn(tokens, hidden, device=gpu) * 0.05
    ids = torch.stack([torch.randperm(count, device=gpu)[:topk] for _ in range(tokens)]).to(torch.int32)
    wts = torch.rand(tokens, topk, device=gpu)
    got = qsrt.qsrt_expert_forward(x.to(torch.bfloat16), ids, wts, experts, out_dtype=torch.float32).double()

    def dense(e, j):
        payload, bits, suh, svh = mats[e][j]
        k, n, axis = (hidden, inter, "n") if j < 2 else (inter, hidden, "k")
        return qsrt.decode_qsrt_payload(payload, k_tiles=k // 16, n_tiles=n // 16, rate_axis=axis, record_bits=bits,
                                        suh=suh, svh=svh).double()

    xb = x.to(torch.bfloat16).double()
    ref = torch.zeros(tokens, hidden, dtype=torch.float64, device=gpu)
    for t in range(tokens):
        for s in range(topk):
            e = int(ids[t, s])
            g, u = xb[t] @ dense(e, 0), xb[t] @ dense(e, 1)
            a = 4.0 * torch.tanh(g / 4.0) * torch.sigmoid(g) * 25.0 * torch.tanh(u / 25.0)
            ref[t] += float(wts[t, s]) * (a @ dense(e, 2))
    assert (got - ref).abs().max().item() <= 2e-5 * ref.abs().max().item()


def test_workgroups_walking_several_n_blocks_match_oracle(gpu):
    """16 tokens x top-8: the planner lets a gate/up workgroup walk both n
    blocks of a matrix (records of different rates along n, so the labels
    are restaged between them) and a down workgroup several hidden blocks."""
    hidden, inter, count, tokens, topk = 640, 256, 6, 16, 8
    spec, experts = _experts(13, count, hidden, inter)
    rng = np.random.default_rng(14)
    x = (rng.standard_normal((tokens, hidden)) * 0.05).astype(np.float32)
    ids = np.stack([rng.permutation(count + 2)[:topk] for _ in range(tokens)]).astype(np.int32) - 1
    wts = rng.uniform(0.1, 1.0, (tokens, topk)).astype(np.float32)
    got = qsrt.qsrt_expert_forward(torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
                                   torch.from_numpy(wts).to(gpu), experts, out_dtype=torch.float32)
    ref = oq.qsrt_expert_forward(x, ids, wts, spec, hidden, inter, _LABELS, _LABELS)
    assert np.abs(got.cpu().numpy() - ref).max() <= 2e-5 * np.abs(ref).max()
