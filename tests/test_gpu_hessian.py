"""GPU parity of the Hessian (SYRK) kernels.

Bar: covariance_comparison relative Frobenius difference <= 1e-5 against the
chunked fp32 oracle (kquant/candidate_hessian.py:98-107) and against exact
float64 sums.  At the benchmark size (65,536 x 7,168) the full oracle is too
slow on a CPU; there the check uses exact float64 dot products of 4,096
sampled entries, the exact trace and the symmetry of the result.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import _native as N
from kquant_amd import candidate_hessian as ch
from kquant_amd import workloads
from tests.test_oracle_hessian import KATS, _expected

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _rel_fro(ref: np.ndarray, got: np.ndarray) -> float:
    return oracle.covariance_comparison(ref, got)["relative_frobenius_difference"]


@pytest.mark.parametrize("case", range(len(KATS)))
def test_reference_known_answers_on_gpu(gpu, case):
    rows, weights, expected = KATS[case]
    h, denom = ch.weighted_covariance(
        torch.tensor(rows, dtype=torch.float32), torch.tensor(weights), device=torch.device("cpu")
    )
    assert h.device.type == "cpu"
    torch.testing.assert_close(h, torch.from_numpy(_expected(rows, weights, expected)))
    torch.testing.assert_close(h, h.T)
    assert denom == pytest.approx(float(sum(weights)))


@pytest.mark.parametrize("n,k", [(4096, 640), (1000, 256), (63, 128), (4097, 136), (257, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_unweighted_matches_oracle(gpu, n, k, dtype):
    print(f"case syrk n={n} k={k} {dtype}", flush=True)
    x = workloads.student_t4(n, k, seed=n + k, dtype=dtype)
    ones = torch.ones(n)
    h, denom = ch.weighted_covariance(x, ones, device=gpu, return_cpu=True)
    ref, rden = oracle.weighted_covariance(x.float().numpy(), ones.numpy(), 256)
    assert denom == rden
    assert _rel_fro(ref, h.numpy()) <= TOL
    x64 = x.double().numpy()
    assert _rel_fro(x64.T @ x64 / n, h.numpy()) <= TOL
    assert torch.equal(h, h.T)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_weighted_matches_oracle(gpu, dtype):
    n, k = 3000, 384
    x = workloads.student_t4(n, k, seed=11, dtype=dtype)
    w = torch.rand(n, generator=torch.Generator().manual_seed(2)) * 2.0
    w[::7] = 0.0
    h, denom = ch.weighted_covariance(x, w, device=gpu)
    ref, _ = oracle.weighted_covariance(x.float().numpy(), w.numpy(), 256)
    assert _rel_fro(ref, h.numpy()) <= TOL
    acc, d2 = ch.accumulate_hessian(x, w, device=gpu)
    racc, rd2 = oracle.accumulate_hessian(x.float().numpy(), w.numpy(), 1024)
    assert _rel_fro(racc, acc.cpu().numpy()) <= TOL
    assert d2 == pytest.approx(rd2)


def test_damped_hessian(gpu):
    n, k = 2048, 512
    x = workloads.student_t4(n, k, seed=5)
    h, denom = ch.damped_hessian(x, damp=0.01)
    ref, _ = oracle.weighted_covariance(x.float().numpy(), np.ones(n, np.float32), 256)
    ref = oracle.damp_diagonal(ref, 0.01)
    assert denom == n
    assert _rel_fro(ref, h.cpu().numpy()) <= TOL
    d = torch.diagonal(h).cpu().double()
    assert torch.allclose(d, torch.from_numpy(np.diag(ref).copy()).double(), rtol=1e-5, atol=0)


def test_cfg4_full_size_sampled_entries(gpu):
    """65,536 Student-t(4) bf16 rows at K = 7,168 with the 0.01 * mean(diag)
    damping of benchmark configuration 4 (i), against exact float64 values:
    sampled entries of X^T X / n plus the damping on the diagonal ones, and
    the trace (1.01 times the exact undamped trace)."""
    n, k = 65536, 7168
    g = torch.Generator(device=gpu).manual_seed(0)
    z0 = torch.randn(n, k, generator=g, device=gpu)
    chi = torch.zeros(n, k, device=gpu)
    for _ in range(4):
        chi += torch.randn(n, k, generator=g, device=gpu).square()
    x = (z0 / torch.sqrt(chi / 4.0)).to(torch.bfloat16)
    del z0, chi
    damp = 0.01
    h, denom = ch.damped_hessian(x, damp=damp)
    torch.cuda.synchronize()
    assert denom == n
    assert torch.equal(h, h.T)
    trace_exact = float(x.float().square().sum(dtype=torch.float64)) / n
    shift = damp * trace_exact / k  # damp * mean(diag) of the exact undamped H
    # checker: exact float64 dot products of sampled entries (torch on the GPU)
    rng = np.random.default_rng(0)
    i = torch.from_numpy(rng.integers(0, k, 4096)).to(gpu)
    j = torch.from_numpy(rng.integers(0, k, 4096)).to(gpu)
    j[:512] = i[:512]  # include diagonal entries
    exact = torch.zeros(4096, dtype=torch.float64, device=gpu)
    for c in range(0, 4096, 512):
        exact[c:c + 512] = (x[:, i[c:c + 512]].double() * x[:, j[c:c + 512]].double()).sum(0) / n
    exact += (i == j).double() * shift
    got = h[i, j].double()
    rel = float(torch.linalg.vector_norm(got - exact) / torch.linalg.vector_norm(exact))
    print(f"cfg4 damped sampled-entry relative error {rel:.3e}", flush=True)
    assert rel <= TOL
    diag = (i == j).nonzero().flatten()
    rel_diag = float(torch.linalg.vector_norm(got[diag] - exact[diag]) / torch.linalg.vector_norm(exact[diag]))
    assert rel_diag <= TOL
    trace_damped = trace_exact * (1.0 + damp)
    assert abs(float(torch.trace(h.double())) - trace_damped) / trace_damped <= 1e-6


def test_cfg4_expert_bench_workload_sampled_entries(gpu):
    """Configuration 4 (ii) exactly as bench.py runs it: 524,288 Zipf-routed
    rows of K = 2,048 over 384 experts (up to ~60k rows each), gate^2
    weights, one grouped launch with in-kernel ranking by row count.  The 10
    largest and 10 smallest non-empty experts are each checked on 4,096
    entries (a 64 x 64 block of random rows and columns, 8 of them on the
    diagonal) against exact float64 weighted dot products, and on their
    trace against its exact float64 value."""
    rows, gates, offsets, counts = workloads.cfg4_expert_rows(gpu)
    k = rows.shape[1]
    h, den = ch.expert_hessians_from_rows(rows, offsets, gates, square_weights=True)
    torch.cuda.synchronize()
    nonempty = torch.nonzero(counts).flatten()
    order = nonempty[torch.argsort(counts[nonempty], descending=True)]
    check = order[:10].tolist() + order[-10:].tolist()
    assert counts[check[0]] > 50000 and counts[check[-1]] <= 3
    rng = np.random.default_rng(3)
    g2 = gates.float().square().double()  # weights = fp32 gate^2, as the reference forms them
    worst = 0.0
    for e in check:
        a, b = int(offsets[e]), int(offsets[e + 1])
        xe = rows[a:b].double()
        we = g2[a:b]
        denom = float(we.sum())
        assert float(den[e]) == pytest.approx(denom, rel=1e-12)
        i = torch.from_numpy(rng.choice(k, 64, replace=False)).to(gpu)
        j = torch.from_numpy(rng.choice(k, 64, replace=False)).to(gpu)
        j[:8] = i[:8]  # a few diagonal entries in the block
        exact = (xe[:, i] * we[:, None]).T @ xe[:, j] / denom
        got = h[e][i][:, j].double()
        rel = float(torch.linalg.matrix_norm(got - exact) / torch.linalg.matrix_norm(exact))
        worst = max(worst, rel)
        assert rel <= TOL, (e, int(counts[e]), rel)
        trace_exact = float((xe.square() * we[:, None]).sum()) / denom
        # the trace sums ~60k positive fp32-accumulated terms per diagonal entry: the 1e-5 bar
        assert abs(float(torch.trace(h[e].double())) - trace_exact) / trace_exact <= TOL, e
        assert torch.equal(h[e], h[e].T)
    print(f"cfg4 (ii) bench workload: worst sampled-entry relative error {worst:.3e}", flush=True)


def test_repeat_runs_are_bitwise_identical(gpu):
    x = workloads.student_t4(4096, 512, seed=9).to(gpu)
    a, _ = ch.damped_hessian(x, damp=0.0)
    b, _ = ch.damped_hessian(x, damp=0.0)
    assert torch.equal(a, b)


def test_shrinkage_matches_reference_formulas(gpu):
    # tests/test_candidate_hessian.py:73-110 on GPU tensors
    rows = torch.tensor([[1.0, 0.0], [0.0, 2.0], [1.0, 2.0], [-1.0, 1.0]])
    weights = torch.ones(4)
    local, _ = ch.weighted_covariance(rows, weights, device=gpu, return_cpu=False)
    actual, evidence = ch.adaptive_identity_shrinkage(local, weights, max_local_alpha=0.6)
    assert evidence["effective_sample_size"] == pytest.approx(4.0)
    assert 0.0 <= evidence["local_alpha"] <= 0.6
    assert evidence["identity_scale"] == pytest.approx(float(torch.trace(local) / 2))
    torch.testing.assert_close(torch.trace(actual), torch.trace(local))
    torch.testing.assert_close(actual, actual.T)

    rows = torch.tensor([[3.0, 0.0], [0.0, 1.0], [2.0, -1.0], [-2.0, 1.0]])
    weights = torch.tensor([1.0, 2.0, 1.0, 0.5])
    local, _ = ch.weighted_covariance(rows, weights, device=gpu, return_cpu=False)
    actual, evidence = ch.adaptive_identity_shrinkage(local, weights)
    identity_scale = float(torch.trace(local) / local.shape[0])
    expected = torch.lerp(torch.eye(2, device=gpu) * identity_scale, local, evidence["local_alpha"])
    torch.testing.assert_close(actual, expected)

    g, l = torch.eye(3), torch.diag(torch.tensor([2.0, 3.0, 4.0]))
    torch.testing.assert_close(ch.shrink_covariance(g, l, 0), g)
    torch.testing.assert_close(ch.shrink_covariance(g, l, 1), l)
    torch.testing.assert_close(ch.shrink_covariance(g, l, 0.25), 0.75 * g + 0.25 * l)
    diagnostics = ch.covariance_comparison(g, l)
    assert diagnostics["trace_ratio"] == 3.0


def test_weighted_effective_sample_size_tracks_weight_concentration(gpu):
    # tests/test_candidate_hessian.py:65-70
    assert ch.weighted_effective_sample_size(torch.ones(8)) == pytest.approx(8.0)
    concentrated = ch.weighted_effective_sample_size(torch.tensor([10.0, 1.0, 1.0, 1.0]))
    assert 1.0 < concentrated < 4.0
    assert concentrated == pytest.approx(13.0 ** 2 / 103.0, rel=1e-12)


def _routing(tokens, topk, experts, seed):
    g = np.random.default_rng(seed)
    p = np.arange(1, experts + 1, dtype=np.float64) ** -1.1
    p /= p.sum()
    ids = np.stack([g.choice(experts, size=topk, replace=False, p=p) for _ in range(tokens)])
    ids = ids.astype(np.int32)
    ids[g.random(ids.shape) < 0.02] = -1          # dropped slots
    ids[ids == experts - 1] = experts + 3         # expert E-1 never receives rows
    gates = g.random(ids.shape).astype(np.float32)
    return ids, gates


@pytest.mark.parametrize("k", [256, 200])
def test_expert_hessians_match_per_expert_oracle(gpu, k):
    """All experts in one routing sort + one grouped SYRK launch vs the oracle's
    weighted_covariance of each expert's rows (token order, weight g^2)."""
    tokens, topk, experts = 1500, 4, 12
    x = workloads.student_t4(tokens, k, seed=5)
    ids, gates = _routing(tokens, topk, experts, 6)
    h, den, counts = ch.expert_hessians(x.to(gpu), torch.from_numpy(ids), torch.from_numpy(gates), experts)
    assert h.shape == (experts, k, k) and den.dtype == torch.float64
    xf = x.float().numpy()
    for e in range(experts):
        mask = ids == e
        rows = np.nonzero(mask.any(axis=1))[0]
        assert int(counts[e]) == len(rows)
        if not len(rows):
            assert float(den[e]) == 0.0 and not torch.any(h[e] != 0)
            continue
        w = (gates * mask).sum(axis=1)[rows]
        w2 = (w * w).astype(np.float32)
        ref, denom = oracle.weighted_covariance(xf[rows], w2)
        assert float(den[e]) == pytest.approx(denom, rel=1e-12)
        got = h[e].cpu().numpy()
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel <= 1e-5, (e, rel)
        assert np.array_equal(got, got.T)


def test_expert_hessians_from_rows_cfg4_expert_shape(gpu):
    """Pre-grouped rows at the expert-down width K = 2048 (config 4 ii), unit
    and fp32-squared weights, group sizes 0 .. 700."""
    k = 2048
    sizes = [0, 1, 7, 64, 700, 130]
    n = sum(sizes)
    x = workloads.student_t4(n, k, seed=8)
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]), dtype=torch.int64)
    w = torch.rand(n, generator=torch.Generator().manual_seed(2))
    for weights, square in ((None, False), (w, True)):
        h, den = ch.expert_hessians_from_rows(x.to(gpu), offsets, weights, square_weights=square)
        for gi, (a, b) in enumerate(zip(offsets[:-1].tolist(), offsets[1:].tolist())):
            if a == b:
                assert float(den[gi]) == 0.0
                continue
            ww = np.ones(b - a, np.float32) if weights is None else (w[a:b].numpy() ** 2).astype(np.float32)
            ref, denom = oracle.weighted_covariance(x[a:b].float().numpy(), ww)
            rel = np.linalg.norm(h[gi].cpu().numpy() - ref) / np.linalg.norm(ref)
            assert float(den[gi]) == pytest.approx(denom, rel=1e-12)
            assert rel <= 1e-5, (gi, rel)


@pytest.mark.parametrize("k", [200, 520])
def test_expert_hessians_from_rows_edge_tiles(gpu, k):
    """Weighted grouped rows at widths that end inside a 256-feature tile
    (the direct-load kernel reads a valid chunk for features past k), plain
    fp32 weights with zeros, an empty group first and last, ragged steps."""
    sizes = [0, 5, 40, 333, 17, 0]
    n = sum(sizes)
    x = workloads.student_t4(n, k, seed=k)
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]), dtype=torch.int64)
    w = torch.rand(n, generator=torch.Generator().manual_seed(k)) * 3.0
    w[::5] = 0.0
    h, den = ch.expert_hessians_from_rows(x.to(gpu), offsets, w)
    for gi, (a, b) in enumerate(zip(offsets[:-1].tolist(), offsets[1:].tolist())):
        if a == b or not float(w[a:b].sum()):
            assert float(den[gi]) == 0.0 and not torch.any(h[gi] != 0)
            continue
        ref, denom = oracle.weighted_covariance(x[a:b].float().numpy(), w[a:b].numpy())
        got = h[gi].cpu().numpy()
        assert float(den[gi]) == pytest.approx(denom, rel=1e-12)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5, gi
        assert np.array_equal(got, got.T)


def test_build_expert_hessians_composes_reference_steps(gpu):
    """kquant/qsrt_candidates.py:534-618 on one expert, both H2 policies and a
    nonzero H13 alpha, against the tested primitives composed as the reference does."""
    g = torch.Generator().manual_seed(12)
    n, hdim, idim = 300, 512, 256
    inputs = torch.randn(n, hdim, generator=g)
    middle = torch.randn(n, idim, generator=g) * 0.3
    gates = torch.rand(n, generator=g)
    global_h13 = torch.eye(hdim) * 0.5
    global_h2 = torch.eye(idim)
    w = gates.float().square()
    for h13_alpha, h2_alpha in ((0.0, None), (0.3, 0.5)):
        h13, h2, ev = ch.build_expert_hessians(inputs.to(gpu), gates.to(gpu), middle.to(gpu),
                                               global_h13=global_h13, global_h2=global_h2, device=gpu,
                                               h13_alpha=h13_alpha, h2_alpha=h2_alpha)
        assert ev["gate_square_sum"] == pytest.approx(float(w.double().sum()), rel=1e-12)
        local_h2, _ = ch.weighted_covariance(middle, w, device=gpu, return_cpu=False)
        if h2_alpha is None:
            want_h2, sh = ch.adaptive_identity_shrinkage(local_h2, w, max_local_alpha=0.75)
            assert ev["h2_local_alpha"] == pytest.approx(sh["local_alpha"], rel=1e-6)
        else:
            scale = float(torch.trace(local_h2) / idim)
            want_h2 = ch.shrink_covariance(torch.eye(idim, device=gpu) * scale, local_h2, h2_alpha)
        assert ch.covariance_comparison(want_h2, h2)["relative_frobenius_difference"] <= 1e-5
        if h13_alpha == 0.0:
            assert torch.equal(h13.cpu(), global_h13)
        else:
            local_h13, _ = ch.weighted_covariance(inputs, w, device=gpu, return_cpu=False)
            want = ch.shrink_covariance(global_h13.to(gpu), local_h13, h13_alpha)
            assert ch.covariance_comparison(want, h13)["relative_frobenius_difference"] <= 1e-5


def test_covariance_comparison_matches_oracle(gpu):
    g = torch.Generator().manual_seed(13)
    a = torch.randn(300, 300, generator=g)
    r = a @ a.T / 300
    c = r + 1e-4 * torch.randn(300, 300, generator=g)
    got = ch.covariance_comparison(r.to(gpu), c.to(gpu))
    want = oracle.covariance_comparison(r.numpy(), c.numpy())
    for key, value in want.items():
        assert got[key] == pytest.approx(value, rel=1e-9, abs=1e-12), key


@pytest.mark.parametrize("n,k", [(4096, 2048), (2048, 6144), (3001, 520)])
def test_split_launch_matches_plain_launch(gpu, n, k):
    """The chunked-tail launch (kq_syrk_accumulate_ws; chunk counts for 256
    CUs): 36 tiles all in the chunked tail (6 chunks), 300 tiles with a full
    round then 5 chunks, and 6 ragged edge tiles (k = 520) over a row count
    that is not a multiple of 32, in 10 chunks.  Written (overwrite) and
    accumulated onto a prefilled accumulator; against exact float64 X^T X
    and the one-tile-per-workgroup launch; repeat calls bitwise identical."""
    print(f"case split syrk n={n} k={k}", flush=True)
    lib = N.library()
    need = int(lib.kq_syrk_accumulate_workspace_size(N.DT_BF16, n, k, 0))
    assert need > 0, "the split launch should pay for this shape"
    assert lib.kq_syrk_accumulate_workspace_size(N.DT_BF16, n, k, 1) == 0  # weighted rows: plain launch
    x = workloads.student_t4(n, k, seed=n + 3 * k, dtype=torch.bfloat16).to(gpu)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu).fill_(0xFF)  # slots need no initialisation
    st = N.stream(gpu)
    acc_plain = torch.zeros(k, k, dtype=torch.float32, device=gpu)
    N.call("kq_syrk_accumulate", N.DT_BF16, N.ptr(x), k, n, k, None, N.ptr(acc_plain), k, N.SYRK_OVERWRITE, st)
    runs = []
    for _ in range(2):
        acc = torch.full((k, k), float("nan"), dtype=torch.float32, device=gpu)
        N.call("kq_syrk_accumulate_ws", N.DT_BF16, N.ptr(x), k, n, k, None, N.ptr(acc), k, N.SYRK_OVERWRITE,
               N.ptr(ws), need, st)
        runs.append(acc)
    upper = torch.ones(k, k, dtype=torch.bool, device=gpu).triu()  # the lower triangle is not written
    assert torch.equal(runs[0][upper], runs[1][upper])
    got = runs[0][upper].double()
    x64 = x.double()
    exact = (x64.T @ x64)[upper]
    rel = float(torch.linalg.vector_norm(got - exact) / torch.linalg.vector_norm(exact))
    plain = acc_plain[upper].double()
    rel_plain = float(torch.linalg.vector_norm(got - plain) / torch.linalg.vector_norm(plain))
    print(f"split vs exact {rel:.2e}, vs plain {rel_plain:.2e}", flush=True)
    assert rel <= TOL and rel_plain <= TOL
    # accumulate mode: acc0 + X^T X
    acc0 = torch.randn(k, k, generator=torch.Generator(device=gpu).manual_seed(1), device=gpu)
    acc = acc0.clone()
    N.call("kq_syrk_accumulate_ws", N.DT_BF16, N.ptr(x), k, n, k, None, N.ptr(acc), k, 0, N.ptr(ws), need, st)
    want = acc0[upper].double() + exact
    rel_acc = float(torch.linalg.vector_norm(acc[upper].double() - want) / torch.linalg.vector_norm(want))
    assert rel_acc <= TOL


def _finalize_expected(acc: np.ndarray, k: int, inv: np.float32, tile: int = 128) -> np.ndarray:
    """sym(acc) * inv from the computed region only: entries with
    tile(i) <= tile(j) (128-wide tiles; a diagonal tile holds both halves),
    the rest mirrored, each product rounded to fp32, and inside diagonal tiles
    (H + H^T) / 2 of the scaled entries (kquant's symmetrisation)."""
    a = acc[:k, :k].astype(np.float32)
    t = np.arange(k) // tile
    full = np.where(t[:, None] <= t[None, :], a, a.T)
    v = (full * inv).astype(np.float32)
    avg = ((v + v.T) * np.float32(0.5)).astype(np.float32)
    return np.where(t[:, None] == t[None, :], avg, v)


@pytest.mark.parametrize("k, ld", [(64, 64), (200, 208), (333, 340), (1000, 1000)])
def test_finalize_is_bitwise_mirror_scale_average(gpu, k, ld):
    """kq_syrk_finalize and kq_syrk_finalize_grouped on an accumulator whose
    never-computed lower tiles hold NaN (they must not be read), widths that
    end inside a 64-block and a 128-tile, a padded row stride, one group
    without weight (zeros)."""
    g = torch.Generator().manual_seed(k)
    acc = torch.randn(ld, ld, generator=g, dtype=torch.float32) * 3.0
    t = torch.arange(ld) // 128
    acc[t[:, None] > t[None, :]] = float("nan")
    denom = 7.25
    out = torch.full((ld, ld), -1.0, device=gpu)
    N.call("kq_syrk_finalize", N.ptr(acc.to(gpu)), ld, k, float(denom), 0.0, N.ptr(out), ld, N.stream(gpu))
    want = _finalize_expected(acc.numpy(), k, np.float32(1.0 / denom))
    got = out.cpu().numpy()
    assert np.array_equal(got[:k, :k], want)
    assert np.all(got[:k, k:] == -1.0) and np.all(got[k:, :] == -1.0)

    accg = torch.stack([acc[:k, :k], acc[:k, :k] * 0.5, acc[:k, :k]]).contiguous().to(gpu)
    dens = torch.tensor([denom, 3.0, 0.0], dtype=torch.float64, device=gpu)
    outg = torch.empty_like(accg)
    N.call("kq_syrk_finalize_grouped", N.ptr(accg), k, 3, N.ptr(dens), N.ptr(outg), N.stream(gpu))
    outg = outg.cpu().numpy()
    assert np.array_equal(outg[0], want)
    assert np.array_equal(outg[1], _finalize_expected(accg[1].cpu().numpy(), k, np.float32(1.0 / 3.0)))
    # no weight: acc * 0, i.e. zeros where acc is finite and NaN where it is not
    assert np.array_equal(outg[2], _finalize_expected(acc.numpy(), k, np.float32(0.0)), equal_nan=True)
