"""GPU parity of the routed MXFP4 MoE expert forward (kq_moe_forward).

Oracle: scripts/closure_exl3_layer.py:557-598 restated in numpy fp32 over the
oracle-dequantized MXFP4 weights, with the activated intermediate rounded to
bf16 (the down-projection operand).  Bar: max |out - ref| / max |ref| <= 2e-3
on fp32 output.  Both kernel shapes are covered: experts with <= 16 routed
pairs (GEMV path) and more (grouped GEMM path).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import moe, workloads

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _deq(q: torch.Tensor, s: torch.Tensor) -> np.ndarray:
    return oracle.mx_dequant("mxfp4", q.cpu().numpy(), s.cpu().numpy())


def _oracle(x, ids, w, weights, act, tokens=None):
    w13q, w13s, w2q, w2s = weights
    cache = {}

    def w13(e):
        if ("a", e) not in cache:
            cache[("a", e)] = _deq(w13q[e], w13s[e])
        return cache[("a", e)]

    def w2(e):
        if ("b", e) not in cache:
            cache[("b", e)] = _deq(w2q[e], w2s[e])
        return cache[("b", e)]

    return oracle.moe_forward(x.float().cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(),
                              w13, w2, act, tokens=tokens)


def _max_rel(ref, got):
    return float(np.abs(got.astype(np.float64) - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("act", ["situ", "swiglu"])
@pytest.mark.parametrize("T", [40, 80])
def test_small_config_both_paths(gpu, act, T):
    """T=40 (160 pairs): decode routing, every expert on the GEMV kernel, the
    experts with more than 16 pairs split into entries of at most 16.  T=80
    (320 pairs): every expert has 29..80 pairs, all on the grouped GEMM."""
    k, E, H, I = 4, 8, 512, 1024
    g = torch.Generator().manual_seed(1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    # expert 0 gets every token, the others <= 16 pairs each
    ids = torch.stack([torch.cat([torch.tensor([0]), 1 + torch.randperm(E - 1, generator=g)[: k - 1]])
                       for _ in range(T)]).to(torch.int32)
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    weights = workloads.quantized_experts(range(E), E, H, I, seed=3, device=gpu)
    out = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), *weights, activation=act)
    ref = _oracle(x, ids, w, weights, act)
    rel = _max_rel(ref, out.cpu().numpy())
    print(f"moe small-config {act} max-rel {rel:.2e}", flush=True)
    assert rel <= TOL
    out16 = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), *weights, activation=act,
                                       out_dtype=torch.bfloat16)
    assert torch.equal(out16.cpu(), out.cpu().to(torch.bfloat16))


def test_invalid_ids_contribute_nothing(gpu):
    T, k, E, H, I = 6, 3, 4, 512, 512
    g = torch.Generator().manual_seed(2)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.tensor([[0, 1, -1], [2, 4, 3], [1, 1, 0], [3, 2, 1], [-5, 0, 2], [1, 3, 0]], dtype=torch.int32)
    w = torch.rand(T, k, generator=g)
    weights = workloads.quantized_experts(range(E), E, H, I, seed=4, device=gpu)
    out = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), *weights)
    valid = (ids >= 0) & (ids < E)
    ref = _oracle(x, torch.where(valid, ids, torch.zeros_like(ids)), w * valid, weights, "situ")
    assert _max_rel(ref, out.cpu().numpy()) <= TOL


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_no_valid_pair_gives_zeros(gpu, out_dtype):
    T, k, E, H, I = 5, 2, 4, 512, 512
    ids = torch.tensor([[-1, 4], [7, -2], [4, 4], [-1, -1], [100, 5]], dtype=torch.int32)
    w = torch.rand(T, k)
    weights = workloads.quantized_experts(range(E), E, H, I, seed=4, device=gpu)
    x = torch.randn(T, H).to(torch.bfloat16)
    out = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), *weights, out_dtype=out_dtype)
    assert out.dtype == out_dtype and torch.count_nonzero(out) == 0


@pytest.mark.parametrize("inter", [512, 1024, 2048, 4096])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_per_pair_decode_matches_listed_path_bitwise(gpu, out_dtype, inter):
    """At most 8 pairs the forward skips the routing launch (one gate/up
    workgroup per pair) and fuses the down projection with the combine, with
    dense or X4T-coded scales.  Its output is bitwise that of the routed-list
    path, which the same 4 tokens take when 5 more tokens (18 pairs) ride
    along (a token's output depends only on its own pairs): here with an
    expert repeated across tokens, invalid ids, a token with no valid expert,
    and each intermediate width that selects its own instantiation of the
    fused down kernel (2 / 4 / 8 / 16 K steps)."""
    T, k, E, H, I = 4, 2, 4, 512, inter
    ids = torch.tensor([[1, 3], [3, -1], [0, 99], [-2, -1]], dtype=torch.int32)
    w = torch.rand(T, k, generator=torch.Generator().manual_seed(8))
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    extra = 5
    ids_l = torch.cat([ids, torch.randint(0, E, (extra, k), generator=torch.Generator().manual_seed(10),
                                          dtype=torch.int32)])
    w_l = torch.cat([w, torch.rand(extra, k, generator=torch.Generator().manual_seed(11))])
    x_l = torch.cat([x, torch.randn(extra, H, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)])
    raw = workloads.quantized_experts(range(E), E, H, I, seed=5, device=gpu)
    dense = moe.prepare_expert_weights(*raw)
    x4t = moe.prepare_expert_weights(*raw, scale_format="x4t")
    outs = {}
    for name, prep in (("dense", dense), ("x4t", x4t)):
        outs[f"fused_{name}"] = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), prep,
                                                           out_dtype=out_dtype)
        outs[f"listed_{name}"] = moe.grouped_expert_forward(x_l.to(gpu), ids_l.to(gpu), w_l.to(gpu), prep,
                                                            out_dtype=out_dtype)[:T]
    fused = outs["fused_dense"]
    for name, got in outs.items():
        assert torch.equal(got, fused), name
    assert torch.count_nonzero(fused[3]) == 0
    valid = (ids >= 0) & (ids < E)
    ref = _oracle(x, torch.where(valid, ids, torch.zeros_like(ids)), w * valid, raw, "situ")
    assert _max_rel(ref, fused.float().cpu().numpy()) <= (TOL if out_dtype == torch.float32 else 2 ** -8)
    again = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), x4t, out_dtype=out_dtype)
    assert torch.equal(again, fused)


@pytest.mark.parametrize("inter", [1024, 2048])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [2, 4])
def test_wide_decode_matches_listed_path_bitwise(gpu, T, out_dtype, inter):
    """9 .. 32 pairs with dense scales also skip the routing launch: the
    per-pair gate/up GEMV groups each expert's pairs into entries of up to 16
    token slots itself, and one kernel runs the down projection of every
    entry and the combine.  Bitwise against the routed-list path (the same
    tokens with 5 more riding along, 72 pairs) and against the X4T-scale
    forward (which keeps the listed path above 8 pairs): with one expert
    taking all 8 slots of a token (and, at 4 tokens, 17 or more pairs in
    all: two entries), experts repeated across tokens, invalid ids and a
    token with no valid expert."""
    k, E, H, I = 8, 8, 512, inter
    g = torch.Generator().manual_seed(20 + T)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    ids[0] = 1                                  # one expert in all 8 slots of token 0
    ids[1, :3] = torch.tensor([1, -1, 99], dtype=torch.int32)
    if T == 4:
        ids[2, :] = 1                           # >= 17 pairs of expert 1: entries of 16 + the rest
        ids[3, :] = torch.tensor([-1, -2, 8, 99, -1, 100, -7, 8], dtype=torch.int32)  # nothing valid
    w = torch.rand(T, k, generator=g)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    extra = 5
    ids_l = torch.cat([ids, torch.randint(0, E, (extra, k), generator=g, dtype=torch.int32)])
    w_l = torch.cat([w, torch.rand(extra, k, generator=g)])
    x_l = torch.cat([x, torch.randn(extra, H, generator=g).to(torch.bfloat16)])
    raw = workloads.quantized_experts(range(E), E, H, I, seed=6, device=gpu)
    dense = moe.prepare_expert_weights(*raw)
    x4t = moe.prepare_expert_weights(*raw, scale_format="x4t")
    print(f"case wide decode T={T} inter={I} {out_dtype}", flush=True)
    wide = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), dense, out_dtype=out_dtype)
    listed = moe.grouped_expert_forward(x_l.to(gpu), ids_l.to(gpu), w_l.to(gpu), dense, out_dtype=out_dtype)[:T]
    listed_x4t = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), x4t, out_dtype=out_dtype)
    assert torch.equal(wide, listed)
    assert torch.equal(wide, listed_x4t)
    if T == 4:
        assert torch.count_nonzero(wide[3]) == 0
    valid = (ids >= 0) & (ids < E)
    ref = _oracle(x, torch.where(valid, ids, torch.zeros_like(ids)), w * valid, raw, "situ")
    assert _max_rel(ref, wide.float().cpu().numpy()) <= (TOL if out_dtype == torch.float32 else 2 ** -8)
    again = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), dense, out_dtype=out_dtype)
    assert torch.equal(again, wide)


@pytest.mark.parametrize("T", [1, 4])
def test_decode_without_routing_launch_graph_replay(gpu, T):
    """The decode paths without a routing launch (8 pairs: per-pair gate/up
    + fused down; 32 pairs: grouped entries + the 9-32 pair down kernel)
    captured in a HIP graph: replays with new routings, tokens and weights
    copied into the captured inputs (eager work and synchronisation between
    replays) each equal the eager forward bit for bit."""
    k, E, H, I = 8, 16, 512, 1024
    raw = workloads.quantized_experts(range(E), E, H, I, seed=9, device=gpu)
    prep = moe.prepare_expert_weights(*raw)
    g = torch.Generator().manual_seed(30 + T)

    def routing():
        ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
        if T > 1:
            ids[1, 0] = ids[0, 0]  # an expert shared by two tokens
        return ids.to(gpu), torch.rand(T, k, generator=g).to(gpu), torch.randn(T, H, generator=g).to(
            torch.bfloat16).to(gpu)

    s_ids, s_w, s_x = routing()
    moe.grouped_expert_forward(s_x, s_ids, s_w, prep)  # warm the workspace outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        s_out = moe.grouped_expert_forward(s_x, s_ids, s_w, prep)
    for rep in range(4):
        ids, w, x = routing()
        s_ids.copy_(ids)
        s_w.copy_(w)
        s_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        want = moe.grouped_expert_forward(x, ids, w, prep)
        torch.cuda.synchronize()
        assert torch.equal(s_out, want), f"replay {rep}"


@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_decode_real_shapes(gpu, tokens):
    """Configuration 5: hidden 7168, intermediate 2048, 384 experts, top-8."""
    ids, w = workloads.random_routing(tokens, seed=tokens)
    x = torch.randn(tokens, 7168, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    check = np.arange(tokens)  # every token: at 16 tokens every routed expert's GEMV entries
    weights = workloads.quantized_experts(ids.flatten().tolist(), device=gpu)
    out = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), *weights)
    ref = _cfg3_oracle(x, ids, w, weights, check, "bf16")
    rel = _max_rel(ref, out.cpu().numpy())
    print(f"moe decode T={tokens} max-rel {rel:.2e}", flush=True)
    assert rel <= TOL


@pytest.mark.parametrize("distinct", [1, 4, 16])
@pytest.mark.parametrize("tokens", [1, 4])
def test_decode_tp12_shard_shape(gpu, tokens, distinct):
    """The reference's published routed-MoE decode shape (Kimi-K3 TP12 shard:
    hidden 3584, 256 intermediate channels per rank, top-16,
    docs/qsrt-technical-brief.md:458-470): an intermediate size that is a
    multiple of 256 only, accepted for bf16-activation decode batches.  Each
    token's 16 slots cycle over ``distinct`` experts (repeated experts in one
    token), dense and X4T-coded scales, against the oracle and bitwise against
    each other."""
    E, H, I, k = 64, 3584, 256, 16
    g = torch.Generator().manual_seed(tokens * 100 + distinct)
    ids = torch.stack([torch.randperm(E, generator=g)[:distinct].repeat(k // distinct) for _ in range(tokens)])
    ids = ids.to(torch.int32)
    w = torch.softmax(torch.randn(tokens, k, generator=g), dim=-1)
    x = torch.randn(tokens, H, generator=g).to(torch.bfloat16)
    raw = workloads.quantized_experts(torch.unique(ids).tolist(), E, H, I, seed=7, device=gpu)
    dense = moe.prepare_expert_weights(*raw)
    x4t = moe.prepare_expert_weights(*raw, scale_format="x4t")
    out = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), dense)
    out_x4t = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), x4t)
    assert torch.equal(out, out_x4t)
    ref = _oracle(x, ids, w, raw, "situ")
    rel = _max_rel(ref, out.cpu().numpy())
    print(f"moe tp12 T={tokens} distinct={distinct} max-rel {rel:.2e}", flush=True)
    assert rel <= TOL


def test_tile_layout_matches_oracle(gpu):
    w13q, w13s, w2q, w2s = workloads.quantized_experts([0, 2], 3, 512, 1024, seed=8, device=gpu)
    prep = moe.prepare_expert_weights(w13q, w13s, w2q, w2s)
    for e in (0, 2):
        qt, st = oracle.mx_tile(w13q[e].cpu().numpy(), w13s[e].cpu().numpy())
        assert np.array_equal(prep.w13_tiles[e].cpu().numpy().reshape(qt.shape), qt)
        assert np.array_equal(prep.w13_scale_tiles[e].cpu().numpy().reshape(st.shape), st)
        qt, st = oracle.mx_tile(w2q[e].cpu().numpy(), w2s[e].cpu().numpy())
        assert np.array_equal(prep.w2_tiles[e].cpu().numpy().reshape(qt.shape), qt)
        assert np.array_equal(prep.w2_scale_tiles[e].cpu().numpy().reshape(st.shape), st)


@pytest.mark.parametrize("register_staged", [False, True])
def test_many_tiles_per_workgroup(gpu, register_staged):
    """More row tiles than one pass of the persistent grid, experts spanning
    several 256-row tiles with ragged last tiles (waves past the expert's rows
    idle), a GEMV-path expert, and one expert with no pairs; both grouped GEMM
    kernels checked against the oracle on every token."""
    T, k, E, H, I = 8192, 4, 10, 512, 512
    g = torch.Generator().manual_seed(11)
    # skewed popularity: expert 9 never routed, expert 8 gets exactly 5 pairs
    p = torch.tensor([0.3, 0.2, 0.15, 0.12, 0.1, 0.07, 0.04, 0.02])
    ids = torch.stack([torch.multinomial(p, k, replacement=False, generator=g) for _ in range(T)])
    ids[:5, 0] = 8
    ids = ids.to(torch.int32)
    counts = torch.bincount(ids.flatten().long(), minlength=E)
    assert counts[9] == 0 and counts[8] == 5 and (counts[:8] % 256 != 0).all()
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    weights = workloads.quantized_experts(range(E), E, H, I, seed=12, device=gpu)
    prep = moe.prepare_expert_weights(*weights)
    out = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), prep,
                                     register_staged=register_staged)
    ref = _oracle(x, ids, w, weights, "situ")
    rel = _max_rel(ref, out.cpu().numpy())
    print(f"moe many-tiles register_staged={register_staged} max-rel {rel:.2e}", flush=True)
    assert rel <= TOL
    out2 = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), prep,
                                      register_staged=register_staged)
    assert torch.equal(out, out2)
    other = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), prep,
                                       register_staged=not register_staged)
    # another fp32 summation order can move a gate/up value across a bf16
    # rounding boundary of the intermediate, which the down GEMM carries on
    assert _max_rel(out.cpu().numpy().astype(np.float64), other.cpu().numpy()) <= 2e-4


# Bars of the activation-quantized modes against the oracle on the same
# quantized operands (element error / max |ref|):
#  * W4A4: the E2M1 x E2M1 MFMA sums exactly in fp32, so the GEMMs differ
#    from the oracle only by summation order; 99.9 % of elements within 1e-5.
#    The rest come from an intermediate moved across a bf16 rounding boundary
#    and so across an MX step (a few per million elements), which changes
#    that pair's row by up to one step: all within 0.05.
#  * W4A8: the E4M3 x E2M1 MFMA does not sum at full fp32 precision (its
#    products span ~2^17 within one instruction): ~1 % of the bf16
#    intermediates differ from an fp32 or fp64 GEMM on the same operands by
#    one ulp, and E4M3's finer steps turn more of those into requantized
#    elements; 99 % within 1e-3 (observed 99.9 %), all within 2e-2
#    (observed max 3e-3).
_MX_BARS = {"mxfp4": (1e-5, 0.999, 0.05), "mxfp8": (1e-3, 0.99, 2e-2)}


def _check_operand_exact(ref: np.ndarray, got: np.ndarray, fmt: str) -> float:
    tight, frac, worst = _MX_BARS[fmt]
    rel = np.abs(got.astype(np.float64) - ref) / np.abs(ref).max()
    assert np.mean(rel <= tight) >= frac, f"only {np.mean(rel <= tight):.5f} of elements within {tight}"
    assert rel.max() <= worst
    return float(np.median(rel))


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
@pytest.mark.parametrize("T", [6, 600])
def test_activation_quantized_matches_operand_oracle(gpu, fmt, T):
    """W4A8 / W4A4 modes.  T=6 (24 pairs): decode routing, every expert on the
    GEMV kernel.  T=600 (2400 pairs): expert 0 with every token on the grouped
    GEMM (3 row tiles, the last ragged), experts with <= 16 pairs on the
    GEMV kernel, the rest on the grouped GEMM."""
    k, E, H, I = 4, 12, 512, 1024
    g = torch.Generator().manual_seed(21 + T)
    x = (torch.randn(T, H, generator=g) * torch.exp(0.5 * torch.randn(H, generator=g))).to(torch.bfloat16)
    p = torch.tensor([0.02] * (E - 1))
    p[-1] = 0.0005
    ids = torch.stack([torch.cat([torch.tensor([0]), 1 + torch.multinomial(p, k - 1, generator=g)]) for _ in range(T)])
    ids = ids.to(torch.int32)
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    weights = workloads.quantized_experts(range(E), E, H, I, seed=22, device=gpu)
    out = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), *weights, activation_format=fmt)
    ref = _oracle_mx(x, ids, w, weights, fmt)
    med = _check_operand_exact(ref, out.cpu().numpy(), fmt)
    print(f"moe {fmt} T={T} median rel {med:.2e}", flush=True)
    again = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), *weights, activation_format=fmt)
    assert torch.equal(out, again)


def _oracle_mx(x, ids, w, weights, fmt, tokens=None):
    w13q, w13s, w2q, w2s = weights
    cache = {}

    def w13(e):
        if ("a", e) not in cache:
            cache[("a", e)] = _deq(w13q[e], w13s[e])
        return cache[("a", e)]

    def w2(e):
        if ("b", e) not in cache:
            cache[("b", e)] = _deq(w2q[e], w2s[e])
        return cache[("b", e)]

    return oracle.moe_forward(x.float().cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), w13, w2,
                              "situ", tokens=tokens, act_format=fmt)


# ------------------------------------------------ configuration 3 at bench size --
def cfg3_check_tokens(ids: torch.Tensor, tile: int = 128) -> np.ndarray:
    """Tokens of the configuration-3 routing that cover the first and the
    last pair of every ``tile``-row tile of every expert on the grouped-GEMM
    path (more than 16 pairs; pairs sit in an expert's rows in token order):
    128-row tiles are the W4A16 grouped GEMM's, and their boundaries include
    those of the 256-row tiles of the activation-quantized kernels.  Plus one
    token of every expert on the GEMV path (1..16 pairs) and every token with
    more than one GEMV-path slot.  (No token of this routing is routed only
    to GEMV-path experts.)"""
    flat = ids.flatten().long()
    counts = torch.bincount(flat, minlength=384)
    sel = set()
    for e in torch.nonzero(counts > 16).flatten().tolist():
        pos = torch.nonzero(flat == e).flatten()
        for first in range(0, pos.numel(), tile):
            last = min(first + tile, pos.numel()) - 1
            sel.add(int(pos[first]) // ids.shape[1])
            sel.add(int(pos[last]) // ids.shape[1])
    gemv = (counts >= 1) & (counts <= 16)
    for e in torch.nonzero(gemv).flatten().tolist():
        sel.add(int(torch.nonzero((ids == e).any(1)).flatten()[0]))
    multi = torch.nonzero(gemv[ids.long()].sum(1) > 1).flatten().tolist()
    sel.update(multi)
    return np.array(sorted(sel))


@pytest.fixture(scope="module")
def cfg3(gpu):
    ids, w = workloads.zipf_routing(8192)
    x = torch.randn(8192, 7168, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    weights = workloads.quantized_experts(torch.unique(ids).tolist(), device=gpu)
    prep = moe.prepare_expert_weights(*weights)
    return ids, w, x, weights, prep


def _cfg3_oracle(x, ids, w, weights, check, fmt):
    """oracle.moe_forward on the checked tokens only, every expert's weights
    dequantized by the C oracle into two reused buffers."""
    w13q, w13s, w2q, w2s = weights
    b13 = np.empty((w13q.shape[1], w13s.shape[2] * 32), np.float32)
    b2 = np.empty((w2q.shape[1], w2s.shape[2] * 32), np.float32)

    def w13(e):
        return oracle.mx_dequant("mxfp4", w13q[e].cpu().numpy(), w13s[e].cpu().numpy(), out=b13)

    def w2(e):
        return oracle.mx_dequant("mxfp4", w2q[e].cpu().numpy(), w2s[e].cpu().numpy(), out=b2)

    sel = torch.from_numpy(check)
    return oracle.moe_forward(x[sel].float().numpy(), ids[sel].numpy(), w[sel].numpy(), w13, w2, "situ",
                              act_format=None if fmt == "bf16" else fmt)


@pytest.mark.parametrize("fmt", ["bf16", "mxfp8", "mxfp4"])
def test_cfg3_bench_size_covers_every_tile_kind(gpu, cfg3, fmt):
    """Configuration 3 at bench size (8192 tokens, Zipf(1.1) top-8 over 384
    experts, 205 active) in the W4A16, W4A8 and W4A4 modes: the output rows
    of cfg3_check_tokens (first and last row of every 128-row tile of every
    grouped-GEMM expert, every GEMV-path expert) against the oracle, and two
    runs bitwise equal."""
    ids, w, x, weights, prep = cfg3
    check = cfg3_check_tokens(ids)
    assert len(check) >= 1000
    counts = torch.bincount(ids.flatten().long(), minlength=384)
    # some expert's last 128-row tile ends inside its second 64-row wave half
    assert bool(((counts > 16) & (counts % 128 > 64)).any())
    out = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), prep, activation_format=fmt)
    again = moe.grouped_expert_forward(x.to(gpu), ids.to(gpu), w.to(gpu), prep, activation_format=fmt)
    assert torch.equal(out, again)
    got = out[torch.from_numpy(check).to(gpu)].cpu().numpy()
    ref = _cfg3_oracle(x, ids, w, weights, check, fmt)
    if fmt == "bf16":
        rel = _max_rel(ref, got)
        print(f"moe cfg3 W4A16 {len(check)} tokens max-rel {rel:.2e}", flush=True)
        assert rel <= TOL
    else:
        med = _check_operand_exact(ref, got, fmt)
        print(f"moe cfg3 {fmt} {len(check)} tokens median rel {med:.2e}", flush=True)
