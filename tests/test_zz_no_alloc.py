"""kq_moe_forward_noalloc: the routed MoE forward with its workspace in the
library's own device array (no allocation per call).

It runs the kernels of kq_moe_forward on the same arguments, so its output
must equal that entry point's bit for bit.  Every check makes two calls in a
row on the shared array, the second with fewer tokens, so the second runs
over what the first left behind.  Both calls go through the C ABI.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from kquant_amd import _native as N
from kquant_amd import moe, workloads


def _args(prep, x, ids, w, act, out, flags):
    head = (N.ACT_SITU if act == "situ" else N.ACT_SWIGLU, 4.0, 25.0, N.ptr(x), x.shape[1], x.shape[0],
            x.shape[1], N.ptr(ids), N.ptr(w), ids.shape[1], prep.experts, prep.inter,
            N.ptr(prep.w13_tiles), N.ptr(prep.w13_scale_tiles), N.ptr(prep.w2_tiles),
            N.ptr(prep.w2_scale_tiles), N.DTYPE_CODES[out.dtype], N.ptr(out))
    return head, (flags, N.stream(x.device))


def _with_workspace(prep, x, ids, w, act, out_dtype, flags):
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    nbytes = N.library().kq_moe_workspace_size(x.shape[0], ids.shape[1], prep.experts, prep.hidden, prep.inter)
    ws = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device=x.device)  # stale contents
    head, (fl, st) = _args(prep, x, ids, w, act, out, flags)
    N.call("kq_moe_forward", *head, N.ptr(ws), nbytes, fl, st)
    return out


def _noalloc(prep, x, ids, w, act, out_dtype, flags):
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    head, tail = _args(prep, x, ids, w, act, out, flags)
    N.call("kq_moe_forward_noalloc", *head, *tail)
    return out


def _routing(T, k, E, g, hot=None):
    rows = []
    for _ in range(T):
        perm = torch.randperm(E, generator=g)[:k]
        if hot is not None and hot not in perm:
            perm[0] = hot
        rows.append(perm)
    ids = torch.stack(rows).to(torch.int32)
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    return ids, w


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["bf16", "mxfp8", "mxfp4"])
def test_noalloc_matches_workspace_forward(gpu, mode):
    """320 routed pairs (grouped GEMM for the hot expert, GEMV for the
    rest), then 20 pairs (decode routing), in each activation mode."""
    flags = {"bf16": 0, "mxfp8": N.MOE_ACT_MXFP8, "mxfp4": N.MOE_ACT_MXFP4}[mode]
    E, H, I, k = 8, 512, 1024, 4
    prep = moe.prepare_expert_weights(*workloads.quantized_experts(range(E), E, H, I, seed=11, device=gpu))
    g = torch.Generator().manual_seed(5)
    for T, act in ((80, "situ"), (5, "swiglu")):
        print(f"noalloc {mode} T={T} {act}", flush=True)
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(gpu)
        ids, w = _routing(T, k, E, g, hot=0)
        ids[0, 1] = -3  # an invalid id contributes nothing, on both paths
        ids, w = ids.to(gpu), w.to(gpu)
        for out_dtype in (torch.float32, torch.bfloat16):
            ref = _with_workspace(prep, x, ids, w, act, out_dtype, flags)
            got = _noalloc(prep, x, ids, w, act, out_dtype, flags)
            torch.cuda.synchronize()
            assert torch.isfinite(ref.float()).all()
            assert torch.equal(got, ref), f"{mode} T={T} {out_dtype}"


@pytest.mark.gpu
def test_noalloc_decode_at_serving_shape(gpu):
    """Hidden 7168, intermediate 2048, top-8 decode batches of 32 tokens
    (256 pairs, the largest decode routing, near the 16 MiB limit) and then
    1 token."""
    E, H, I, k = 24, 7168, 2048, 8
    prep = moe.prepare_expert_weights(*workloads.quantized_experts(range(E), E, H, I, seed=12, device=gpu))
    g = torch.Generator().manual_seed(6)
    need = N.library().kq_moe_workspace_size(32, k, E, H, I)
    assert need <= N.MOE_NOALLOC_SCRATCH_BYTES
    for T in (32, 1):
        print(f"noalloc serving shape T={T}", flush=True)
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(gpu)
        ids, w = _routing(T, k, E, g)
        ids, w = ids.to(gpu), w.to(gpu)
        ref = _with_workspace(prep, x, ids, w, "situ", torch.float32, 0)
        got = _noalloc(prep, x, ids, w, "situ", torch.float32, 0)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"T={T}"


def test_noalloc_rejects_sizes_beyond_its_scratch():
    """A call needing more than KQ_MOE_NOALLOC_SCRATCH_BYTES fails on the
    host with KQ_ERR_LIMIT before anything is launched (no GPU needed)."""
    lib = N.library()
    T, k, E, H, I = 8192, 8, 384, 7168, 2048
    assert lib.kq_moe_workspace_size(T, k, E, H, I) > N.MOE_NOALLOC_SCRATCH_BYTES
    p = ctypes.c_void_p(4096)  # never dereferenced: the size check comes first
    rc = lib.kq_moe_forward_noalloc(N.ACT_SITU, 4.0, 25.0, p, H, T, H, p, p, k, E, I, p, p, p, p,
                                    N.DT_F32, p, 0, None)
    assert rc == N.KQ_ERR_LIMIT
    msg = lib.kq_last_error().decode()
    assert "kq_moe_forward_noalloc" in msg and "scratch" in msg
    # bad arguments keep kq_moe_forward's own errors
    rc = lib.kq_moe_forward_noalloc(N.ACT_SITU, 4.0, 25.0, p, H, 4, H, p, p, k, E, I, p, None, p, p,
                                    N.DT_F32, p, 0, None)
    assert rc == N.KQ_ERR_INVALID and b"null scale tiles" in lib.kq_last_error()
