"""Expert-MLP helpers on the GPU against the oracle: the activation kernel,
rank-partial reduction, the K3 router, the comparison metrics, the fp32
linear (three-term bf16 split), the fp32 single-expert MLP and the source
reconstruction.  fp32 tolerances are stated per test."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import linear, moe, tp_simulator as tp
from kquant_amd import mxfp4 as kq_mxfp4
from kquant_amd.source_weights import PackedMXFP4Matrix, dequant_packed_matrix

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_situ_and_swiglu(gpu, dtype):
    g = torch.Generator().manual_seed(0)
    gate = (torch.randn(37, 300, generator=g) * 6).to(dtype)
    up = (torch.randn(37, 300, generator=g) * 40).to(dtype)
    for fn, ref_fn in ((tp.situ, oracle.situ), (tp.swiglu, oracle.swiglu)):
        got = fn(gate.to(gpu), up.to(gpu))
        assert got.dtype == dtype and got.device.type == "cuda"
        ref = ref_fn(gate.float().numpy(), up.float().numpy())
        if dtype == torch.float32:
            # fp32 tanh / exp differ from numpy's by a few ulps
            assert np.allclose(got.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
        else:
            r = torch.from_numpy(ref).to(dtype).float().numpy()
            eps = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
            assert np.allclose(got.float().cpu().numpy(), r, rtol=eps, atol=1e-3 * eps)
    # tests/test_tp_simulator.py:66-74 through the CPU entry
    gate = torch.tensor([[-5.0, 0.0, 5.0]])
    up = torch.tensor([[30.0, -2.0, 3.0]])
    expected = 4.0 * torch.tanh(gate / 4.0) * torch.sigmoid(gate) * (25.0 * torch.tanh(up / 25.0))
    got = tp.situ(gate, up)
    assert got.device.type == "cpu"
    torch.testing.assert_close(got, expected)


def test_activation_accuracy_sweep(gpu):
    """The epilogue activations (hardware exp2 / reciprocal, a fitted tanh
    polynomial below |y| = 0.625) against float64 SiTU / SwiGLU over a wide
    fp32 grid: tiny values, both signs, the tanh branch point, saturation and
    exp overflow (|x| up to 200).  Bar: a few ulp relative plus 1e-30
    absolute (denormal-range sigmoid tails)."""
    mags = np.concatenate([np.geomspace(1e-20, 1e-3, 64), np.linspace(1e-3, 3.0, 900),
                           np.array([0.625 * 4, 0.625 * 4 * (1 - 2 ** -23), 0.625 * 25, 0.625 * 25 * (1 + 2 ** -23)]),
                           np.linspace(3.0, 200.0, 400)])
    vals = np.concatenate([mags, -mags, [0.0, -0.0]]).astype(np.float32)
    gate = torch.from_numpy(np.repeat(vals, 16).reshape(-1, 16))
    up = torch.from_numpy(np.tile(vals[:: max(1, len(vals) // 16)][:16], (len(vals), 1)).astype(np.float32))
    g64, u64 = gate.double().numpy(), up.double().numpy()
    sig = 1.0 / (1.0 + np.exp(-g64))
    refs = {"situ": 4.0 * np.tanh(g64 / 4.0) * sig * (25.0 * np.tanh(u64 / 25.0)), "swiglu": g64 * sig * u64}
    for name, fn in (("situ", tp.situ), ("swiglu", tp.swiglu)):
        got = fn(gate.to(gpu), up.to(gpu)).cpu().double().numpy()
        ref = refs[name]
        assert np.isfinite(got).all()
        err = np.abs(got - ref) / (np.abs(ref) * 2.0 ** -23 + 1e-30)
        print(f"{name}: max error {err.max():.2f} ulp (fp32 relative)", flush=True)
        assert err.max() <= 16.0


def test_reduce_partials(gpu):
    g = torch.Generator().manual_seed(1)
    parts = [torch.randn(6, 129, generator=g) for _ in range(5)]
    got = tp.reduce_partials([p.to(gpu) for p in parts], dtype=torch.float32)
    ref = oracle.reduce_partials([p.numpy() for p in parts])
    assert np.array_equal(got.cpu().numpy(), ref)  # same fp32 order: bit-exact
    got16 = tp.reduce_partials(parts, dtype=torch.bfloat16)
    assert got16.dtype == torch.bfloat16
    assert torch.equal(got16, torch.from_numpy(ref).to(torch.bfloat16))
    with pytest.raises(ValueError, match="at least one partial"):
        tp.reduce_partials([], dtype=torch.float32)


def test_kimi_topk(gpu):
    # tests/test_tp_simulator.py:49-63
    logits = torch.tensor([[0.0, 1.0, 2.0, 3.0]])
    weights, ids = tp.kimi_topk(logits, torch.tensor([10.0, 0.0, 0.0, 0.0]), 2, routed_scaling_factor=2.0)
    assert ids.tolist() == [[0, 3]] and ids.dtype == torch.int32 and weights.dtype == torch.float32
    raw = logits.sigmoid()[0, ids[0].long()]
    torch.testing.assert_close(weights[0], 2.0 * raw / raw.sum())
    # K3 shape: 384 experts, top-8; and a 1024-expert, top-64 edge case
    for tokens, experts, k, dt in ((500, 384, 8, torch.float32), (33, 1024, 64, torch.bfloat16)):
        g = torch.Generator().manual_seed(experts)
        lg = torch.randn(tokens, experts, generator=g).to(dt)
        bias = torch.randn(experts, generator=g) * 0.05
        w, i = tp.kimi_topk(lg.to(gpu), bias.to(gpu), k, routed_scaling_factor=2.5)
        rw, ri, keys = oracle.kimi_topk(lg.float().numpy(), bias.numpy(), k, 2.5)
        gaps = np.diff(keys[:, : k + 1], axis=1)
        clear = np.all(np.abs(gaps) > 1e-5, axis=1)  # rows without a near-tie
        assert clear.mean() > 0.5
        gi = i.cpu().numpy()
        assert np.array_equal(gi[clear], ri[clear])
        assert np.allclose(w.cpu().numpy()[clear], rw[clear], rtol=2e-6, atol=1e-7)
        # every row, near-ties included: the chosen keys are a top-k, in order
        all_keys = 1.0 / (1.0 + np.exp(-lg.float().numpy().astype(np.float64))) + bias.numpy()
        chosen = np.take_along_axis(all_keys, gi.astype(np.int64), axis=1)
        assert np.allclose(chosen, keys[:, :k], rtol=0, atol=1e-5)
        assert np.all([len(set(r)) == k for r in gi.tolist()])


def test_comparison_metrics(gpu):
    g = torch.Generator().manual_seed(4)
    ref = torch.randn(1000, 77, generator=g)
    act = ref + 1e-3 * torch.randn(1000, 77, generator=g)
    got = tp.comparison_metrics(ref.to(gpu), act.to(torch.bfloat16).to(gpu))
    want = oracle.comparison_metrics(ref.numpy(), act.to(torch.bfloat16).float().numpy())
    for key in ("relative_l2", "max_abs", "cosine"):
        assert abs(got[key] - want[key]) <= 1e-6 * max(1.0, abs(want[key])), key


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("m,n,k", [(1, 256, 7168), (77, 300, 2048), (256, 512, 1024)])
def test_fp32_source_linear(gpu, fmt, m, n, k):
    """fp32 sources reach fp32-GEMM accuracy: max |C - R| / max |R| <= 1e-5 (bar 2e-3)."""
    print(f"case fp32 linear {fmt} m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    x = torch.randn(m, k, generator=g) * torch.exp(0.5 * torch.randn(k, generator=g))
    if fmt == "mxfp4":
        q, s = kq_mxfp4.mxfp4_quantize(w)
        wd = oracle.mx_dequant("mxfp4", q.cpu().numpy(), s.cpu().numpy())
        c = linear.mxfp4_linear(x.to(gpu), q, s)
    else:
        from kquant_amd import mxfp8
        q, s = mxfp8.mxfp8_quantize(w)
        wd = oracle.mx_dequant("mxfp8", q.view(torch.uint8).cpu().numpy(), s.cpu().numpy())
        c = linear.mxfp8_linear(x.to(gpu), q, s)
    assert c.dtype == torch.float32
    ref = x.double().numpy() @ wd.astype(np.float64).T
    err = np.abs(c.cpu().numpy() - ref).max() / np.abs(ref).max()
    print(f"fp32 linear max-rel {err:.2e}", flush=True)
    assert err <= 1e-5


def _expert(g, rows, cols):
    w = (torch.randn(rows, cols, generator=g) * 0.02).to(torch.bfloat16)
    q, s = kq_mxfp4.mxfp4_quantize(w)
    return q.cpu(), s.cpu()


def test_expert_output_matches_fp32_oracle(gpu):
    """official_expert_output semantics at K3 shapes (H 7168, I 2048), 64 rows."""
    g = torch.Generator().manual_seed(9)
    hidden, inter = 7168, 2048
    w1, w3, w2 = _expert(g, inter, hidden), _expert(g, inter, hidden), _expert(g, hidden, inter)
    x = torch.randn(64, hidden, generator=g)
    got = moe.expert_output(x.to(gpu), w1, w3, PackedMXFP4Matrix(*w2))
    assert got.dtype == torch.float32 and got.shape == (64, hidden)
    dq = [oracle.mx_dequant("mxfp4", q.numpy(), s.numpy()) for q, s in (w1, w3, w2)]
    ref = oracle.expert_output(x.numpy(), *dq)
    err = np.abs(got.cpu().numpy() - ref).max() / np.abs(ref).max()
    print(f"expert_output max-rel {err:.2e}", flush=True)
    assert err <= 2e-3
    assert np.linalg.norm(got.cpu().numpy() - ref) / np.linalg.norm(ref) <= 1e-5


def test_reconstruct_and_packed_matrix(gpu):
    g = torch.Generator().manual_seed(10)
    q, s = _expert(g, 64, 256)
    s = s.clone()
    s[0, 0] = 250
    out = moe.reconstruct_source({"w1": {"packed": q, "scale": s}}, gpu, scale_byte_max=140)
    clamped = np.minimum(s.numpy(), 140)
    ref = oracle.round_bf16(oracle.mx_dequant("mxfp4", q.numpy(), clamped))
    assert out["w1"].dtype == torch.bfloat16 and out["w1"].device.type == "cuda"
    assert np.array_equal(out["w1"].float().cpu().numpy(), ref)
    full = dequant_packed_matrix(PackedMXFP4Matrix(q, s), device=gpu)
    assert full.dtype == torch.float32 and full.is_contiguous()
    assert np.array_equal(full.cpu().numpy(), oracle.mx_dequant("mxfp4", q.numpy(), s.numpy()))
    host = dequant_packed_matrix(PackedMXFP4Matrix(q, s))
    assert host.device.type == "cpu" and torch.equal(host, full.cpu())
