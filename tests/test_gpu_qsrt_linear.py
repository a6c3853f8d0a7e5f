"""GPU parity of the fused QSRT linear (kq_qsrt_linear through
kquant_amd.qsrt.qsrt_linear) against oracle/qsrt.py (x @ the decoded weight,
f64).  One-hot activation rows read the regularized weight back exactly
(each output is one product 1 * label plus exact zeros), which pins the
state windows, label lookup and tensor-core order bit for bit; random rows
through the rotated weight must agree with the f64 product to within 4e-6
of max |ref| for fp32 output (fp32 products and sums over K <= 2048), and
bf16 output must be that result rounded once (within one bf16 ulp of the
f64 value).  Row counts cover every row tile (1, 2, 4, 8), several row
groups, single- and multi-chunk K splits, both rate axes and mixed rates,
and the prefill form past FUSED_MAX_ROWS rows (fp32 rows within 8e-6 of max
|ref|, one-hot rows bit-exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import qsrt
from oracle import qsrt as oq

pytestmark = pytest.mark.gpu

_LABELS = {b: oracle.sqg_xor_cheb_t12_bytes(b) for b in (2, 3, 4)}


def _random_matrix(k_tiles, n_tiles, rate_axis, record_bits, seed):
    rng = np.random.default_rng(seed)
    states = np.zeros((k_tiles, n_tiles, 256), dtype=np.int16)
    for kt in range(k_tiles):
        for nt in range(n_tiles):
            bits = record_bits[(kt if rate_axis == "k" else nt) // 8]
            states[kt, nt] = oq.reconstruct_trellis_states(rng.integers(0, 1 << bits, 256), bits)
    return oq.pack_payload(states, record_bits, rate_axis)


def _scales(k_tiles, n_tiles, seed):
    rng = np.random.default_rng(seed)
    suh = rng.choice([-1.0, 1.0], k_tiles * 16).astype(np.float32) * rng.uniform(0.5, 1.5, k_tiles * 16)
    svh = rng.uniform(0.5, 2.0, n_tiles * 16).astype(np.float32)
    return suh.astype(np.float32), svh


@pytest.mark.parametrize("rate_axis", ["k", "n"])
def test_one_hot_rows_read_the_weight_exactly(gpu, rate_axis):
    k_tiles, n_tiles = (24, 16) if rate_axis == "k" else (16, 24)
    record_bits = (2, 4, 3)
    payload = _random_matrix(k_tiles, n_tiles, rate_axis, record_bits, 11)
    want = oq.decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, rate_axis, _LABELS)
    rows = np.arange(0, k_tiles * 16, 7)  # every residue of the tile rows and both k halves
    x = np.zeros((rows.size, k_tiles * 16), dtype=np.float32)
    x[np.arange(rows.size), rows] = 1.0
    p = torch.from_numpy(payload).to(gpu)
    for r0 in range(0, rows.size, qsrt.FUSED_MAX_ROWS):  # the fused kernel, in batches it takes
        xs = torch.from_numpy(x[r0:r0 + qsrt.FUSED_MAX_ROWS]).to(gpu)
        got = qsrt.qsrt_linear(xs, p, k_tiles=k_tiles, n_tiles=n_tiles, rate_axis=rate_axis,
                               record_bits=record_bits)
        assert got.dtype == torch.float32
        assert np.array_equal(got.cpu().numpy(), want[rows[r0:r0 + qsrt.FUSED_MAX_ROWS]])


@pytest.mark.parametrize("rate_axis,m,shape,record_bits", [
    ("n", 1, (16, 24), (3, 2, 4)),
    ("n", 2, (128, 16), (4, 3)),
    ("k", 3, (24, 16), (2, 4, 3)),
    ("k", 8, (64, 8), (3, 3, 2, 2, 4, 4, 3, 2)),
    ("n", 13, (32, 32), (2, 3, 4, 3)),
    ("k", 29, (16, 40), (4, 2)),
])
def test_rotated_product_matches_oracle(gpu, rate_axis, m, shape, record_bits):
    k_tiles, n_tiles = shape
    payload = _random_matrix(k_tiles, n_tiles, rate_axis, record_bits, m)
    suh, svh = _scales(k_tiles, n_tiles, m + 1)
    x = np.random.default_rng(m + 2).standard_normal((m, k_tiles * 16)).astype(np.float32)
    ref = oq.qsrt_linear(x, payload, k_tiles, n_tiles, record_bits, rate_axis, _LABELS, suh, svh)
    args = dict(k_tiles=k_tiles, n_tiles=n_tiles, rate_axis=rate_axis, record_bits=record_bits,
                suh=torch.from_numpy(suh), svh=torch.from_numpy(svh))
    p = torch.from_numpy(payload).to(gpu)
    xg = torch.from_numpy(x).to(gpu)
    got = qsrt.qsrt_linear(xg, p, **args).cpu().numpy().astype(np.float64)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 4e-6 * scale
    # bf16 output: the fp32 result rounded once
    got16 = qsrt.qsrt_linear(xg, p, out_dtype=torch.bfloat16, **args).cpu().float().numpy()
    assert np.all(np.abs(got16 - ref) <= np.abs(ref) * 2.0 ** -8 + 4e-6 * scale)
    # bf16 activations: the same product of the bf16-rounded rows
    xb = xg.to(torch.bfloat16)
    refb = oq.qsrt_linear(xb.float().cpu().numpy(), payload, k_tiles, n_tiles, record_bits, rate_axis, _LABELS,
                          suh, svh)
    gotb = qsrt.qsrt_linear(xb, p, out_dtype=torch.float32, **args).cpu().numpy()
    assert np.abs(gotb - refb).max() <= 4e-6 * np.abs(refb).max()


def test_matches_decode_then_matmul_and_reuses_workspace(gpu):
    """Kimi-K3 w1 geometry (EXL [K=3584, N=3072], 24 records along n):
    several calls in a row, shrinking and growing, each with the workspace
    that calls of its row count share (left zero by every call)."""
    k_tiles, n_tiles = 224, 192
    record_bits = (2, 4) * 2 + (3,) * 20
    g = torch.Generator(device=gpu).manual_seed(3)
    words = sum(8 * k_tiles * 16 * b for b in record_bits)
    p = torch.randint(-32768, 32768, (words,), dtype=torch.int16, generator=g, device=gpu)
    suh = torch.randn(k_tiles * 16, generator=g, device=gpu).sign()
    svh = torch.rand(n_tiles * 16, generator=g, device=gpu) + 0.5
    args = dict(k_tiles=k_tiles, n_tiles=n_tiles, rate_axis="n", record_bits=record_bits, suh=suh, svh=svh)
    w = qsrt.decode_qsrt_payload(p, **args).double()
    for m in (4, 1, 16, 5):
        x = torch.randn(m, k_tiles * 16, generator=g, device=gpu)
        ref = x.double() @ w
        got = qsrt.qsrt_linear(x, p, **args).double()
        assert (got - ref).abs().max().item() <= 4e-6 * ref.abs().max().item(), m
    assert qsrt.qsrt_linear(torch.empty(0, k_tiles * 16, device=gpu), p, **args).shape == (0, n_tiles * 16)


def test_argument_errors(gpu):
    p = torch.zeros(8 * 8 * 16 * 3 * 2, dtype=torch.int16, device=gpu)
    x = torch.zeros(1, 128, device=gpu)
    with pytest.raises(ValueError, match="features"):
        qsrt.qsrt_linear(torch.zeros(1, 64, device=gpu), p, k_tiles=8, n_tiles=16, rate_axis="n", record_bits=(3, 3))
    with pytest.raises(ValueError, match="K2, K3, or K4"):
        qsrt.qsrt_linear(x, p, k_tiles=8, n_tiles=16, rate_axis="n", record_bits=(3, 5))
    with pytest.raises(RuntimeError, match="payload has"):
        qsrt.qsrt_linear(x, p, k_tiles=8, n_tiles=16, rate_axis="n", record_bits=(3, 2))


def test_launcher_in_a_graph_replays_the_eager_result(gpu):
    """The prepared launcher captured in a HIP graph: every replay (with eager
    work and synchronizations between) equals the eager call bit for bit,
    since the K split and its summation order are fixed."""
    k_tiles, n_tiles = 64, 24
    record_bits = (3, 2, 4)
    payload = torch.from_numpy(_random_matrix(k_tiles, n_tiles, "n", record_bits, 21)).to(gpu)
    suh, svh = (torch.from_numpy(v).to(gpu) for v in _scales(k_tiles, n_tiles, 22))
    x = torch.randn(3, k_tiles * 16, generator=torch.Generator(device=gpu).manual_seed(23), device=gpu)
    args = dict(k_tiles=k_tiles, n_tiles=n_tiles, rate_axis="n", record_bits=record_bits, suh=suh, svh=svh)
    eager = qsrt.qsrt_linear(x, payload, **args)
    out = torch.empty_like(eager)
    run = qsrt.qsrt_linear_launcher(x, payload, out, **args)
    run()
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for i in range(4):
        out.zero_()
        qsrt.qsrt_linear(x[:1], payload, **args)  # eager work sharing nothing with the graph
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i


@pytest.mark.parametrize("m", [1, 2])
def test_polled_partials_start_every_call_from_zero(gpu, m):
    """One or two rows: the K chunks' partials are polled by the last chunk's
    workgroup, in a workspace that each call must leave zero.  28 chunks of
    one k block each; calls with different rows in a row (eager and graph
    replays with new rows copied in) each match their own product, a repeat
    of the first rows matches it bit for bit, and zero rows give +0.0
    everywhere (a partial is stored as -0.0 when it is zero)."""
    k_tiles, n_tiles = 224, 16
    record_bits = (3, 2)
    payload = torch.from_numpy(_random_matrix(k_tiles, n_tiles, "n", record_bits, 61)).to(gpu)
    suh, svh = (torch.from_numpy(v).to(gpu) for v in _scales(k_tiles, n_tiles, 62))
    args = dict(k_tiles=k_tiles, n_tiles=n_tiles, rate_axis="n", record_bits=record_bits, suh=suh, svh=svh)
    w = qsrt.decode_qsrt_payload(payload, **args).double()
    g = torch.Generator(device=gpu).manual_seed(63 + m)
    xs = [torch.randn(m, k_tiles * 16, generator=g, device=gpu) for _ in range(3)]

    def check(got, x):
        ref = x.double() @ w
        assert (got.double() - ref).abs().max().item() <= 4e-6 * ref.abs().max().item()

    first = qsrt.qsrt_linear(xs[0], payload, **args)
    check(first, xs[0])
    check(qsrt.qsrt_linear(xs[1], payload, **args), xs[1])
    assert torch.equal(qsrt.qsrt_linear(xs[0], payload, **args), first)
    zero = qsrt.qsrt_linear(torch.zeros(m, k_tiles * 16, device=gpu), payload, **args)
    assert torch.equal(zero, torch.zeros_like(zero)) and not torch.signbit(zero).any()

    xin = xs[0].clone()
    out = torch.empty_like(first)
    run = qsrt.qsrt_linear_launcher(xin, payload, out, **args)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for i, x in enumerate(xs + xs[:1]):
        xin.copy_(x)
        qsrt.qsrt_linear(xs[2][:1], payload, **args)  # eager work sharing nothing with the graph
        graph.replay()
        torch.cuda.synchronize()
        check(out, x)
        if i == 3:
            assert torch.equal(out, first)


def test_every_finite_e4m3_label_converts_exactly(gpu):
    """Labels equal to the state's low byte (the two NaN codes mapped to
    zero) put every finite E4M3 code into the weight; identity activation
    rows read W back, which must equal the oracle's E4M3 values exactly."""
    from kquant_amd import _native as N

    k_tiles, n_tiles, bits = 8, 16, (3, 2)
    payload = _random_matrix(k_tiles, n_tiles, "n", bits, 31)
    table = (np.arange(65536) & 0xFF).astype(np.uint8)
    table[(table & 0x7F) == 0x7F] = 0
    labels = torch.from_numpy(np.stack([table] * 3)).to(gpu)
    want = oq.decode_qsrt_weight(payload, k_tiles, n_tiles, bits, "n", {2: table, 3: table, 4: table})
    assert len(np.unique(want)) == 253  # every finite code (the two zeros compare equal)
    p = torch.from_numpy(payload).to(gpu)
    x = torch.eye(k_tiles * 16, device=gpu)
    out = torch.empty(k_tiles * 16, n_tiles * 16, device=gpu)
    need = int(N.library().kq_qsrt_linear_workspace_size(x.shape[0], k_tiles, n_tiles))
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=gpu)
    N.call("kq_qsrt_linear", N.ptr(x), N.DT_F32, x.shape[0], x.shape[1], N.ptr(p), p.numel(), k_tiles, n_tiles, 1,
           bytes(bits), N.ptr(labels), None, None, N.DT_F32, N.ptr(out), out.shape[1], N.ptr(ws), need,
           N.stream(gpu))
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("pad", [0, 4, 3])
def test_e4m3_label_bytes_every_code(gpu, transposed, pad):
    """kq_qsrt_decode_weight to KQ_QSRT_OUT_E4M3 (the prefill's weight):
    every finite code's byte, [K, N] and [N, K], with 4-byte aligned output
    rows (the byte tile and 4-byte stores) and with a row stride that is not
    (one byte per store); the bytes past each row stay untouched."""
    from kquant_amd import _native as N

    k_tiles, n_tiles, bits = 16, 24, (3, 2, 4)
    payload = _random_matrix(k_tiles, n_tiles, "n", bits, 41)
    table = (np.arange(65536) & 0xFF).astype(np.uint8)
    table[(table & 0x7F) == 0x7F] = 0
    labels = torch.from_numpy(np.stack([table] * 3)).to(gpu)
    want = oq.decode_qsrt_weight(payload, k_tiles, n_tiles, bits, "n", {2: table, 3: table, 4: table})
    if transposed:
        want = want.T
    want8 = torch.from_numpy(np.ascontiguousarray(want)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    rows, cols = want.shape
    ldo = cols + pad
    out = torch.full((rows, ldo), 0xA5, dtype=torch.uint8, device=gpu)
    p = torch.from_numpy(payload).to(gpu)
    N.call("kq_qsrt_decode_weight", N.ptr(p), p.numel(), k_tiles, n_tiles, 1, bytes(bits), N.ptr(labels), None,
           None, N.QSRT_OUT_E4M3, N.ptr(out), ldo, 1 if transposed else 0, N.stream(gpu))
    got = out.cpu().numpy()
    assert np.array_equal(got[:, :cols], want8)
    assert (got[:, cols:] == 0xA5).all()


@pytest.mark.parametrize("rate_axis,m,shape,record_bits", [
    ("n", qsrt.FUSED_MAX_ROWS + 1, (32, 16), (3, 4)),
    ("k", 100, (24, 40), (2, 4, 3)),
    ("n", 257, (64, 24), (4, 2, 3)),
])
def test_prefill_rows_match_oracle(gpu, rate_axis, m, shape, record_bits):
    """More than FUSED_MAX_ROWS rows take kq_qsrt_linear's prefill form
    (rows rotated, the regularized weight decoded once to E4M3 label bytes,
    the MXFP8 MFMA linear, the output rotated).  fp32 rows keep fp32
    accuracy (exact three-term bf16 split): within 8e-6 of max |ref| of the
    f64 product, rotated or regularized; bf16 rows are rotated to bf16, so
    their bar is bf16 rounding of the rotated rows (4e-3 of max |ref|)."""
    k_tiles, n_tiles = shape
    payload = _random_matrix(k_tiles, n_tiles, rate_axis, record_bits, m + 40)
    suh, svh = _scales(k_tiles, n_tiles, m + 41)
    x = np.random.default_rng(m + 42).standard_normal((m, k_tiles * 16)).astype(np.float32)
    p = torch.from_numpy(payload).to(gpu)
    xg = torch.from_numpy(x).to(gpu)
    base = dict(k_tiles=k_tiles, n_tiles=n_tiles, rate_axis=rate_axis, record_bits=record_bits)
    for rotated in (True, False):
        args = dict(base, suh=torch.from_numpy(suh), svh=torch.from_numpy(svh)) if rotated else base
        ref = oq.qsrt_linear(x, payload, k_tiles, n_tiles, record_bits, rate_axis, _LABELS,
                             suh if rotated else None, svh if rotated else None)
        got = qsrt.qsrt_linear(xg, p, **args).cpu().numpy().astype(np.float64)
        rel = np.abs(got - ref).max() / np.abs(ref).max()
        print(f"prefill m={m} rotated={rotated} fp32 max-rel {rel:.2e}", flush=True)
        assert rel <= 8e-6
        xb = xg.to(torch.bfloat16)
        refb = oq.qsrt_linear(xb.float().cpu().numpy(), payload, k_tiles, n_tiles, record_bits, rate_axis,
                              _LABELS, suh if rotated else None, svh if rotated else None)
        gotb = qsrt.qsrt_linear(xb, p, out_dtype=torch.float32, **args).cpu().numpy().astype(np.float64)
        relb = np.abs(gotb - refb).max() / np.abs(refb).max()
        print(f"prefill m={m} rotated={rotated} bf16 rows max-rel {relb:.2e}", flush=True)
        assert relb <= (4e-3 if rotated else 8e-6)


@pytest.mark.parametrize("k_tiles,n_tiles,record_bits", [(16, 24, (2, 4, 3)), (64, 24, (4, 3, 2))])
def test_prefill_one_hot_rows_read_the_weight_exactly(gpu, k_tiles, n_tiles, record_bits):
    """One-hot fp32 rows through the prefill form of the regularized product
    return the weight bit for bit: the E4M3 label bytes the decode writes,
    their unit block scales and the exact split; at K = 1024 (342 rows, four
    output tiles) the product is also split over K into fp32 planes."""
    payload = _random_matrix(k_tiles, n_tiles, "n", record_bits, 61)
    want = oq.decode_qsrt_weight(payload, k_tiles, n_tiles, record_bits, "n", _LABELS)
    rows = np.arange(0, k_tiles * 16, 3)
    assert rows.size > qsrt.FUSED_MAX_ROWS
    x = np.zeros((rows.size, k_tiles * 16), dtype=np.float32)
    x[np.arange(rows.size), rows] = 1.0
    got = qsrt.qsrt_linear(torch.from_numpy(x).to(gpu), torch.from_numpy(payload).to(gpu), k_tiles=k_tiles,
                           n_tiles=n_tiles, rate_axis="n", record_bits=record_bits)
    assert np.array_equal(got.cpu().numpy(), want[rows])


def test_payload_alignment(gpu):
    """The fast kernels stage 16-byte pieces by direct loads: the decode
    entry point takes its first kernel for a payload 4 bytes past a 16-byte
    boundary (same weight), the linear entry point rejects one, and the
    Python functions copy such a payload to an aligned buffer."""
    from kquant_amd import _native as N

    k_tiles, n_tiles, bits = 16, 16, (3, 2)  # two 128-column records along n
    payload = _random_matrix(k_tiles, n_tiles, "n", bits, 71)
    big = torch.zeros(payload.size + 16, dtype=torch.int16, device=gpu)
    p = big[2:2 + payload.size]
    p.copy_(torch.from_numpy(payload))
    assert p.data_ptr() % 16 == 4
    labels = qsrt.rate_labels(device=gpu)
    want = qsrt.decode_qsrt_payload(p.clone(), k_tiles=k_tiles, n_tiles=n_tiles, rate_axis="n", record_bits=bits)
    out = torch.empty_like(want)
    N.call("kq_qsrt_decode_weight", N.ptr(p), p.numel(), k_tiles, n_tiles, 1, bytes(bits), N.ptr(labels), None,
           None, N.DT_F32, N.ptr(out), out.shape[1], 0, N.stream(gpu))
    assert torch.equal(out, want)
    x = torch.randn(2, k_tiles * 16, device=gpu)
    y = torch.empty(2, n_tiles * 16, device=gpu)
    need = int(N.library().kq_qsrt_linear_workspace_size(2, k_tiles, n_tiles))
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        N.call("kq_qsrt_linear", N.ptr(x), N.DT_F32, 2, x.shape[1], N.ptr(p), p.numel(), k_tiles, n_tiles, 1,
               bytes(bits), N.ptr(labels), None, None, N.DT_F32, N.ptr(y), y.shape[1], N.ptr(ws), need,
               N.stream(gpu))
    args = dict(k_tiles=k_tiles, n_tiles=n_tiles, rate_axis="n", record_bits=bits)
    assert torch.equal(qsrt.qsrt_linear(x, p, **args), qsrt.qsrt_linear(x, p.clone(), **args))
    with pytest.raises(ValueError, match="16-byte aligned"):
        qsrt.qsrt_linear_launcher(x, p, y, **args)
    with pytest.raises(ValueError, match="record rates"):
        qsrt.qsrt_linear(x, p.clone(), k_tiles=k_tiles, n_tiles=n_tiles, rate_axis="n", record_bits=(3,))


def test_chunks_spanning_records_of_different_rates(gpu):
    """K = 5120 along the rate axis k with alternating record rates: the
    planner gives a workgroup two or more k blocks, so it crosses records of
    different rates and restages the label table mid-chunk."""
    k_tiles, n_tiles = 320, 64
    record_bits = (2, 4, 3) * 13 + (4,)
    payload = _random_matrix(k_tiles, n_tiles, "k", record_bits, 51)
    suh, svh = _scales(k_tiles, n_tiles, 52)
    x = np.random.default_rng(53).standard_normal((1, k_tiles * 16)).astype(np.float32)
    ref = oq.qsrt_linear(x, payload, k_tiles, n_tiles, record_bits, "k", _LABELS, suh, svh)
    got = qsrt.qsrt_linear(torch.from_numpy(x).to(gpu), torch.from_numpy(payload).to(gpu), k_tiles=k_tiles,
                           n_tiles=n_tiles, rate_axis="k", record_bits=record_bits, suh=torch.from_numpy(suh),
                           svh=torch.from_numpy(svh)).cpu().numpy()
    assert np.abs(got - ref).max() <= 4e-6 * np.abs(ref).max()
