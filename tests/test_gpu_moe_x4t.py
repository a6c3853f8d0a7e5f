"""GPU parity of the routed MoE forward over X4T-coded expert scales
(kq_moe_forward_x4t) and of the per-tile exception index (kq_x4t_tile_index).

The forward expands the routed experts' w1 / w3 / w2 X4T planes into
per-call scale slots and runs the same GEMM kernels as kq_moe_forward, so
the bar is bitwise equality with kq_moe_forward over the dense scales: in
each routing regime (decode, one-workgroup prep, multi-block prep), each
mode (bf16 activations on the direct-to-LDS or register-staged GEMMs, W4A8,
W4A4), with stale slots from earlier calls, and under HIP graph replay.
Plain kq_moe_forward is itself pinned to the fp32 oracle in test_gpu_moe.py,
and the X4T forward is also checked against that oracle directly.
The tile index is checked against numpy.searchsorted over each matrix's
exception positions and against the encoder's own per-tile offsets.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kquant_amd import moe, workloads, x4t

pytestmark = pytest.mark.gpu


def _index_expected(exc: np.ndarray, offsets: np.ndarray, rows: int, cols: int) -> np.ndarray:
    tiles = rows // 16
    pos = (exc & 0xFFFFFF).astype(np.int64)
    out = []
    for m in range(len(offsets) - 1):
        lo, hi = int(offsets[m]), int(offsets[m + 1])
        starts = np.arange(tiles, dtype=np.int64) * 16 * cols
        out.append(lo + np.searchsorted(pos[lo:hi], starts, side="left"))
    out.append([int(offsets[-1])])
    return np.concatenate(out)


@pytest.mark.parametrize("cols", [1, 37, 224])
def test_tile_index_matches_searchsorted(gpu, cols):
    mats, rows = 5, 96
    g = torch.Generator().manual_seed(cols)
    planes = torch.randint(118, 122, (mats, rows, cols), generator=g, dtype=torch.uint8)
    planes[1] = 120                                   # a matrix with no exceptions
    planes[3, 40:] = torch.randint(90, 150, (rows - 40, cols), generator=g, dtype=torch.uint8)
    planes[4, :, 0] = 200                             # exceptions in column 0 only
    fixed, exc, offsets = x4t.pack_x4t_scale_components_batched(planes.to(gpu))
    index = x4t.x4t_tile_index(exc, offsets, rows=rows, columns=cols)
    want = _index_expected(exc.cpu().numpy().astype(np.int64), offsets.cpu().numpy(), rows, cols)
    assert np.array_equal(index.cpu().numpy().astype(np.int64), want)
    # the encoder's per-tile offsets (kq_x4t_analyze) are the same numbers
    _, tile_offsets = x4t._analyze(planes.to(gpu).contiguous(), mats, rows, cols, gpu)
    assert np.array_equal(tile_offsets.cpu().numpy(), want)


def test_tile_index_single_matrix_without_offsets(gpu):
    rows, cols = 32, 9
    plane = torch.randint(100, 140, (rows, cols), generator=torch.Generator().manual_seed(2),
                          dtype=torch.uint8)
    fixed, exc = x4t.pack_x4t_scale_components(plane)
    offsets = torch.tensor([0, exc.numel()], dtype=torch.int64)
    index = x4t.x4t_tile_index(exc, offsets, rows=rows, columns=cols)
    want = _index_expected(exc.numpy().astype(np.int64), offsets.numpy(), rows, cols)
    assert np.array_equal(index.cpu().numpy().astype(np.int64), want)


def _weights(E, H, I, seed, gpu, spread=()):
    """Quantizer-made MXFP4 experts; the experts in ``spread`` get scale
    planes with many X4T exceptions (bytes spread over 112..127)."""
    w13q, w13s, w2q, w2s = workloads.quantized_experts(range(E), E, H, I, seed=seed, device=gpu)
    g = torch.Generator(device=gpu).manual_seed(seed)
    for e in spread:
        w13s[e] = torch.randint(112, 128, w13s[e].shape, generator=g, device=gpu, dtype=torch.uint8)
        w2s[e] = torch.randint(112, 128, w2s[e].shape, generator=g, device=gpu, dtype=torch.uint8)
    return w13q, w13s, w2q, w2s


_MODES = {
    "bf16": {},
    "bf16_register_staged": {"register_staged": True},
    "w4a8": {"activation_format": "mxfp8"},
    "w4a4": {"activation_format": "mxfp4"},
}


@pytest.mark.parametrize("mode", list(_MODES))
@pytest.mark.parametrize("T", [1, 4, 100, 600])
def test_x4t_forward_bitwise_equals_dense(gpu, mode, T):
    """T=1: 4 pairs over 8 experts (fewer slots than experts); T=4: decode
    routing; T=100: one-workgroup prep with GEMV and grouped-GEMM experts;
    T=600: multi-block prep.  Expert 7 is never routed."""
    k, E, H, I = 4, 8, 512, 1024
    g = torch.Generator().manual_seed(T)
    p = torch.tensor([0.4, 0.2, 0.15, 0.1, 0.08, 0.05, 0.02, 0.0])
    ids = torch.stack([torch.multinomial(p, k, replacement=False, generator=g) for _ in range(T)])
    ids = ids.to(torch.int32)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    weights = _weights(E, H, I, 21, gpu, spread=(1, 5))
    dense = moe.prepare_expert_weights(*weights)
    coded = moe.prepare_expert_weights(*weights, scale_format="x4t")
    assert coded.scale_format == "x4t" and coded.w13_scale_tiles is None
    assert torch.equal(coded.w13_tiles, dense.w13_tiles) and torch.equal(coded.w2_tiles, dense.w2_tiles)
    args = (x.to(gpu), ids.to(gpu), w.to(gpu))
    want = moe.grouped_expert_forward(*args, dense, **_MODES[mode])
    got = moe.grouped_expert_forward(*args, coded, **_MODES[mode])
    print(f"x4t forward T={T} {mode}: max |diff| {(got - want).abs().max().item():.3e}", flush=True)
    assert torch.equal(got, want)


def test_x4t_stale_slots_and_rerouting(gpu):
    """Slots hold the previous call's experts (or poison): each call's
    expansion rewrites every slot it uses before the GEMMs read it."""
    k, E, H, I = 8, 16, 512, 512
    weights = _weights(E, H, I, 31, gpu, spread=(2, 9))
    dense = moe.prepare_expert_weights(*weights)
    coded = moe.prepare_expert_weights(*weights, scale_format="x4t")
    g = torch.Generator().manual_seed(3)
    for step, T in enumerate([2, 2, 40, 2, 300]):
        ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
        x = torch.randn(T, H, generator=g).to(torch.bfloat16)
        w = torch.rand(T, k, generator=g)
        args = (x.to(gpu), ids.to(gpu), w.to(gpu))
        want = moe.grouped_expert_forward(*args, dense)
        if step % 2:
            for buf in moe._WORKSPACES.values():
                buf.fill_(0xA5)
        got = moe.grouped_expert_forward(*args, coded)
        assert torch.equal(got, want), f"step {step} T={T}"


def test_x4t_components_from_container_layout(gpu):
    """prepare_expert_weights_x4t over host components in kquant's X4T
    container layout (per matrix kind: fixed stream, exception stream,
    per-expert exception offsets)."""
    k, E, H, I, T = 4, 6, 1024, 512, 24
    w13q, w13s, w2q, w2s = _weights(E, H, I, 41, gpu, spread=(0,))
    comps = []
    for plane in (w13s[:, :I], w13s[:, I:], w2s):
        comps.append(tuple(t.cpu() for t in x4t.pack_x4t_scale_components_batched(plane.contiguous())))
    coded = moe.prepare_expert_weights_x4t(w13q.cpu(), w2q.cpu(), *comps)
    dense = moe.prepare_expert_weights(w13q, w13s, w2q, w2s)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.rand(T, k, generator=g)
    args = (x.to(gpu), ids.to(gpu), w.to(gpu))
    assert torch.equal(moe.grouped_expert_forward(*args, coded), moe.grouped_expert_forward(*args, dense))
    with pytest.raises(ValueError, match="invalid geometry"):
        moe.prepare_expert_weights_x4t(w13q, w2q, comps[0], comps[2], comps[2])
    with pytest.raises(ValueError, match="expected"):
        moe.prepare_expert_weights_x4t(w13q, w2q, coded.w1_scale_x4t, coded.w3_scale_x4t, coded.w1_scale_x4t)


def test_x4t_graph_replay(gpu):
    """The X4T forward captured in a HIP graph: replays with new routings
    copied into the captured inputs (eager work and synchronisation between
    replays) each match the eager dense-scale forward bit for bit."""
    k, E, H, I, T = 4, 12, 512, 512, 4
    weights = _weights(E, H, I, 51, gpu, spread=(3,))
    dense = moe.prepare_expert_weights(*weights)
    coded = moe.prepare_expert_weights(*weights, scale_format="x4t")
    g = torch.Generator().manual_seed(5)

    def routing():
        ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
        return ids.to(gpu), torch.rand(T, k, generator=g).to(gpu), torch.randn(T, H, generator=g).to(
            torch.bfloat16).to(gpu)

    s_ids, s_w, s_x = routing()
    moe.grouped_expert_forward(s_x, s_ids, s_w, coded)  # warm the workspace outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        s_out = moe.grouped_expert_forward(s_x, s_ids, s_w, coded)
    for rep in range(4):
        ids, w, x = routing()
        s_ids.copy_(ids)
        s_w.copy_(w)
        s_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        want = moe.grouped_expert_forward(x, ids, w, dense)
        torch.cuda.synchronize()
        assert torch.equal(s_out, want), f"replay {rep}"


@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_x4t_decode_real_shapes(gpu, tokens):
    """Configuration 5 shapes (hidden 7168, intermediate 2048, 384 experts,
    top-8): X4T planes w1 / w3 [2048, 224], w2 [7168, 64].  One token takes
    the fused decode of at most 8 pairs, four tokens (32 pairs) the wide
    decode kernel, 16 tokens the routed-list path."""
    ids, w = workloads.random_routing(tokens, seed=100 + tokens)
    x = torch.randn(tokens, 7168, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    weights = workloads.quantized_experts(ids.flatten().tolist(), device=gpu)
    dense = moe.prepare_expert_weights(*weights)
    coded = moe.prepare_expert_weights(*weights, scale_format="x4t")
    args = (x.to(gpu), ids.to(gpu), w.to(gpu))
    assert torch.equal(moe.grouped_expert_forward(*args, coded), moe.grouped_expert_forward(*args, dense))


@pytest.mark.parametrize("T", [2, 3, 4])
def test_x4t_wide_decode_exception_heavy(gpu, T):
    """9 to 32 pairs at intermediate 2048 (the wide decode kernel decodes
    each unit's half of two scale tiles in the workgroup), three experts
    with exception-heavy planes (more than 64 exceptions per pair of tiles,
    which the kernel loads past its prefetched words): bitwise the
    dense-scale forward, bf16 and fp32 outputs."""
    k, E, H, I = 8, 12, 512, 2048
    g = torch.Generator().manual_seed(70 + T)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    weights = _weights(E, H, I, 71, gpu, spread=(0, 4, 9))
    dense = moe.prepare_expert_weights(*weights)
    coded = moe.prepare_expert_weights(*weights, scale_format="x4t")
    args = (x.to(gpu), ids.to(gpu), w.to(gpu))
    for out_dtype in (torch.bfloat16, torch.float32):
        want = moe.grouped_expert_forward(*args, dense, out_dtype=out_dtype)
        got = moe.grouped_expert_forward(*args, coded, out_dtype=out_dtype)
        assert torch.equal(got, want), out_dtype


@pytest.mark.parametrize("T", [4, 600])
def test_x4t_forward_matches_oracle(gpu, T):
    """The X4T-scale forward against oracle.moe_forward on the dequantized
    weights directly (kquant/x4t.py:477-524 decodes the planes to the dense
    scales the oracle dequantizes with), at a decode routing (T=4: every
    expert on the GEMV kernel, scales decoded in its prologue) and a prefill
    routing (T=600: expanded scale slots for the grouped-GEMM experts, GEMV
    for the rest), W4A16 and W4A4, with exception-heavy planes on two experts."""
    import oracle

    k, E, H, I = 4, 8, 512, 1024
    g = torch.Generator().manual_seed(40 + T)
    p = torch.tensor([0.4, 0.2, 0.15, 0.1, 0.08, 0.05, 0.02, 0.0])
    ids = torch.stack([torch.multinomial(p, k, replacement=False, generator=g) for _ in range(T)])
    ids = ids.to(torch.int32)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    weights = _weights(E, H, I, 23, gpu, spread=(0, 3))
    coded = moe.prepare_expert_weights(*weights, scale_format="x4t")
    w13q, w13s, w2q, w2s = (t.cpu().numpy() for t in weights)

    def w13(e):
        return oracle.mx_dequant("mxfp4", w13q[e], w13s[e])

    def w2(e):
        return oracle.mx_dequant("mxfp4", w2q[e], w2s[e])

    args = (x.to(gpu), ids.to(gpu), w.to(gpu))
    for fmt in ("bf16", "mxfp4"):
        got = moe.grouped_expert_forward(*args, coded, activation_format=fmt).cpu().numpy()
        ref = oracle.moe_forward(x.float().numpy(), ids.numpy(), w.numpy(), w13, w2, "situ",
                                 act_format=None if fmt == "bf16" else fmt)
        err = np.abs(got.astype(np.float64) - ref) / np.abs(ref).max()
        print(f"x4t forward vs oracle T={T} {fmt}: max rel {err.max():.2e}", flush=True)
        if fmt == "bf16":
            assert err.max() <= 2e-3
        else:  # the W4A4 bars of test_gpu_moe.py
            assert np.mean(err <= 1e-5) >= 0.999 and err.max() <= 0.05
