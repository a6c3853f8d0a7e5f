"""GPU parity of the encoder's Hessian finalize: blockwise Hadamard rotation,
batched Cholesky, block LDL and finalize_capture_H
(kquant/exl3_encoder_backend.py:288-386, 1588-1663).

Oracle: oracle/ldl.py in f64 (numpy's Cholesky as the factorization).  The
GPU computes in fp32 as the reference does, so the bars are fp32 ones:
rotation within 2e-6 of max |ref|; Cholesky with backward error
||L L^T - A|| / ||A|| <= 2e-6 and forward error <= 2e-5 (relative Frobenius,
on matrices of condition number ~30-1000); block LDL and finalize within 1e-4.
"""

from __future__ import annotations

import io
import re
from contextlib import redirect_stdout

import numpy as np
import pytest
import torch

from kquant_amd import _native as N
from kquant_amd import exl3_encoder_backend as eb
from oracle import ldl

pytestmark = pytest.mark.gpu


def _spd(n: int, seed: int, rows: int | None = None, damp: float = 0.025) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows or 2 * n, n))
    h = x.T @ x / x.shape[0]
    return (h + damp * np.diag(h).mean() * np.eye(n)).astype(np.float32)


def _rel(ref: np.ndarray, got: np.ndarray) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(np.asarray(got, dtype=np.float64) - ref) / np.linalg.norm(ref))


def _cholesky(a: torch.Tensor, batch: int = 1, in_place: bool = False):
    n = a.shape[-1]
    out = a if in_place else torch.full_like(a, float("nan"))
    ws = torch.empty(int(N.library().kq_cholesky_workspace_size(n, batch)), dtype=torch.uint8, device=a.device)
    info = torch.full((batch,), -7, dtype=torch.int32, device=a.device)
    N.call("kq_cholesky", N.ptr(a), n, n * n, N.ptr(out), n, n * n, n, batch, N.ptr(info), N.ptr(ws),
           ws.numel(), N.stream(a.device))
    return out, info


@pytest.mark.parametrize("sides", [1, 2, 3])
@pytest.mark.parametrize("scaled", [False, True])
def test_hadamard_matches_oracle(gpu, sides, scaled):
    rng = np.random.default_rng(sides)
    x = rng.standard_normal((2, 256, 384)).astype(np.float32)
    rs = rng.choice([-1.0, 1.0], 256).astype(np.float32) if scaled else None
    cs = rng.choice([-1.0, 1.0], 384).astype(np.float32) if scaled else None
    if sides == 1:
        x = x[:, :, :300].copy()  # the untransformed dimension may be ragged
        cs = cs[:300].copy() if scaled else None
    t = torch.from_numpy(x).to(gpu)
    rst = None if rs is None else torch.from_numpy(rs).to(gpu)
    cst = None if cs is None else torch.from_numpy(cs).to(gpu)
    rows, cols = x.shape[1:]
    N.call("kq_blockwise_hadamard", N.ptr(t), rows, cols, cols, 2, rows * cols, sides, N.ptr(rst), N.ptr(cst),
           N.stream(gpu))
    got = t.cpu().numpy()
    for b in range(2):
        ref = ldl.blockwise_hadamard(x[b], sides, rs, cs)
        assert np.abs(got[b] - ref).max() <= 2e-6 * np.abs(ref).max()


def test_dropin_hadamard_in_place(gpu):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((128, 256)).astype(np.float32)
    t = torch.from_numpy(x).to(gpu)
    eb.blockwise_preapply_had_r_(t, 128)
    eb.blockwise_preapply_had_l_(t, 128)
    ref = ldl.blockwise_hadamard(x, 3)
    assert np.abs(t.cpu().numpy() - ref).max() <= 4e-6 * np.abs(ref).max()
    with pytest.raises(AssertionError):
        eb.blockwise_preapply_had_l_(torch.zeros(100, 128, device=gpu), 128)


@pytest.mark.parametrize("n", [1, 64, 100, 200, 1000])
def test_cholesky_matches_numpy(gpu, n):
    a = _spd(n, n)
    got, info = _cholesky(torch.from_numpy(a).to(gpu))
    assert int(info.item()) == 0
    lower = got.cpu().numpy()
    assert np.array_equal(np.triu(lower, 1), np.zeros_like(lower))
    ref = np.linalg.cholesky(a.astype(np.float64))
    back = _rel(a, lower.astype(np.float64) @ lower.T.astype(np.float64))
    fwd = _rel(ref, lower)
    print(f"cholesky n={n}: backward {back:.2e} forward {fwd:.2e}", flush=True)
    assert back <= 2e-6 and fwd <= 2e-5


def test_cholesky_batched_and_in_place(gpu):
    batch, n = 4, 2048
    a = np.stack([_spd(n, 10 + i) for i in range(batch)])
    t = torch.from_numpy(a).to(gpu)
    got, info = _cholesky(t.clone(), batch, in_place=True)
    assert info.cpu().tolist() == [0] * batch
    lower = got.cpu().numpy()
    for i in range(batch):
        assert _rel(np.linalg.cholesky(a[i].astype(np.float64)), lower[i]) <= 2e-5
    # out of place gives the same bits
    again, _ = _cholesky(t, batch)
    assert torch.equal(again, got)


@pytest.mark.parametrize("batch,n", [(8, 300), (12, 777)])
def test_cholesky_super_panels(gpu, batch, n):
    """Batches of 8 and more factor four 64-column panels per trailing
    update (column updates inside the panel launches, diagonal blocks
    factored by the workgroup that completes them): every matrix against
    numpy's f64 factor, ragged last panels included."""
    a = np.stack([_spd(n, 100 + i) for i in range(batch)])
    got, info = _cholesky(torch.from_numpy(a).to(gpu), batch)
    assert info.cpu().tolist() == [0] * batch
    lower = got.cpu().numpy()
    for i in range(batch):
        assert np.array_equal(np.triu(lower[i], 1), np.zeros((n, n), dtype=lower.dtype))
        back = _rel(a[i], lower[i].astype(np.float64) @ lower[i].T.astype(np.float64))
        fwd = _rel(np.linalg.cholesky(a[i].astype(np.float64)), lower[i])
        assert back <= 2e-6 and fwd <= 2e-5, (i, back, fwd)
    bad = a.copy()
    bad[5][200, 200] = -1.0
    _, info = _cholesky(torch.from_numpy(bad).to(gpu), batch)
    assert info.cpu().tolist()[5] == 201 and sum(info.cpu().tolist()) == 201


def test_cholesky_large(gpu):
    """H13-sized (7168): input and residual built with f64 GEMMs on the GPU."""
    n = 7168
    g = torch.Generator(device=gpu).manual_seed(5)
    x = torch.randn(n + n // 2, n, generator=g, device=gpu, dtype=torch.float64)
    a64 = x.T @ x / x.shape[0]
    a64 += 0.025 * torch.diagonal(a64).mean() * torch.eye(n, device=gpu, dtype=torch.float64)
    del x
    a = a64.float()
    got, info = _cholesky(a)
    assert int(info.item()) == 0
    l64 = got.double()
    back = float(torch.linalg.vector_norm(l64 @ l64.T - a.double()) / torch.linalg.vector_norm(a.double()))
    print(f"cholesky n={n}: backward {back:.2e}", flush=True)
    assert back <= 2e-6


def test_cholesky_reports_leading_minor(gpu):
    n = 150
    good = _spd(n, 1)
    bad = np.eye(n, dtype=np.float32)
    bad[70, 70] = -1.0
    worse = _spd(n, 2)
    worse[:, 130] = worse[130, :] = 0.0  # minor of order 131 singular
    t = torch.from_numpy(np.stack([good, bad, worse])).to(gpu)
    _, info = _cholesky(t, 3)
    assert info.cpu().tolist() == [0, 71, 131]


@pytest.mark.parametrize("b", [1, 16, 64])
def test_block_ldl_matches_oracle(gpu, b):
    n = 512
    a = _spd(n, b)
    h = torch.from_numpy(a).to(gpu)
    lower, h_cpu = eb.block_ldl(h, b, {}, False)
    assert lower.data_ptr() == h.data_ptr() and h_cpu.device.type == "cpu"
    assert torch.equal(h_cpu, torch.from_numpy(a))
    assert _rel(ldl.block_ldl(a, b), lower.cpu().numpy()) <= 1e-4


def test_block_ldl_retries_with_damping(gpu):
    n, rows = 256, 64  # rank-deficient covariance pushed below positive definite
    rng = np.random.default_rng(8)
    x = rng.standard_normal((rows, n))
    h64 = x.T @ x / rows
    h64 -= 1e-3 * np.diag(h64).mean() * np.eye(n)
    h = torch.from_numpy(h64.astype(np.float32)).to(gpu)
    buf = io.StringIO()
    with redirect_stdout(buf):
        lower, h_cpu = eb.block_ldl(h, 16, {"sigma_reg": 0.025}, False)
    attempts = re.findall(r"attempt (\d+)/10", buf.getvalue())
    assert attempts and attempts[-1] == str(len(attempts))
    damped = h64.astype(np.float32).astype(np.float64)
    for _ in attempts:
        damped[np.arange(n), np.arange(n)] += 2.0 * 0.025 * np.diag(damped).mean()
    assert np.allclose(h_cpu.numpy(), damped, rtol=1e-6, atol=1e-7)
    assert _rel(ldl.block_ldl(damped, 16), lower.cpu().numpy()) <= 1e-4


def test_block_ldl_gives_up_after_ten_retries(gpu):
    h = torch.eye(128, device=gpu)
    h[3, 3] = -1e6  # no amount of 2 * sigma * mean(diag) damping fixes it
    with redirect_stdout(io.StringIO()), pytest.raises(torch.linalg.LinAlgError):
        eb.block_ldl(h, 16, {}, False)


@pytest.mark.parametrize("k", [256, 1024])
def test_finalize_capture_h_matches_oracle(gpu, k):
    rows = 3 * k
    rng = np.random.default_rng(k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    acc = x.astype(np.float64).T @ x.astype(np.float64)
    h_data = {"H": torch.from_numpy(acc.astype(np.float32)).to(gpu), "count": rows, "finalized": False}
    torch.manual_seed(11)
    q_fallback, h_rot, lower, su, diag = eb.finalize_capture_H(h_data, {"sigma_reg": 0.025}, False)
    torch.manual_seed(11)  # su drawn as the reference draws it
    want_su = (torch.randn(k, device=gpu).sign() + 1e-5).sign().to(torch.float).unsqueeze(1)
    assert torch.equal(su, want_su) and h_data["finalized"] and h_data["su"] is su
    ref_fb, ref_rot, ref_lower, ref_diag = ldl.finalize(acc.astype(np.float32), rows, 0.025, su.cpu().numpy())
    assert q_fallback is False and ref_fb is False
    assert _rel(ref_diag, diag.cpu().numpy()) <= 1e-6
    assert h_rot.device.type == "cpu" and _rel(ref_rot, h_rot.numpy()) <= 1e-5
    assert _rel(ref_lower, lower.cpu().numpy()) <= 1e-4
    assert torch.count_nonzero(torch.diagonal(lower)) == 0
    # finalized entries come back unchanged on a second call
    again = eb.finalize_capture_H(h_data, {"sigma_reg": 0.025}, False)
    assert again[2] is lower


def test_finalize_capture_h_without_samples(gpu):
    h_data = {"H": torch.zeros(128, 128, device=gpu), "count": 0, "finalized": False}
    q_fallback, h_rot, lower, su, diag = eb.finalize_capture_H(h_data, {}, False)
    assert q_fallback is True and lower is None and su.shape == (128, 1)
    assert torch.count_nonzero(h_rot) == 0


def test_block_ldl_batched(gpu):
    experts, n = 5, 256
    a = np.stack([_spd(n, 40 + e) for e in range(experts)])
    a[3, 17, 17] = -5.0
    lower, info = eb.block_ldl_batched(torch.from_numpy(a).to(gpu), 16)
    info = info.cpu().tolist()
    assert info[3] > 0 and [v for i, v in enumerate(info) if i != 3] == [0] * (experts - 1)
    got = lower.cpu().numpy()
    for e in range(experts):
        if e != 3:
            assert _rel(ldl.block_ldl(a[e], 16), got[e]) <= 1e-4


@pytest.mark.parametrize("ld", [260, 257])
def test_hadamard_ragged_rows_and_row_strides(gpu, ld):
    """Right-side rotation of a [200, 256] matrix inside a wider buffer: the
    last row block is ragged (single-element path), ld = 260 keeps 16-byte
    rows (vector path for full blocks), ld = 257 does not (single-element
    path throughout); padding columns stay untouched."""
    rng = np.random.default_rng(ld)
    rows, cols = 200, 256
    buf = rng.standard_normal((rows, ld)).astype(np.float32)
    cs = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    t = torch.from_numpy(buf).to(gpu)
    cst = torch.from_numpy(cs).to(gpu)
    N.call("kq_blockwise_hadamard", N.ptr(t), rows, cols, ld, 1, 0, 2, None, N.ptr(cst), N.stream(gpu))
    got = t.cpu().numpy()
    ref = ldl.blockwise_hadamard(buf[:, :cols], 2, None, cs)
    assert np.abs(got[:, :cols] - ref).max() <= 2e-6 * np.abs(ref).max()
    assert np.array_equal(got[:, cols:], buf[:, cols:])
