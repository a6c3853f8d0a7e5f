"""Seeded synthetic inputs of the benchmark configurations.

The reference publishes no dataset for this path; each generator follows the
recipe of one benchmark configuration (BASELINE.json ``configs``) with a
seeded CPU ``torch.Generator`` so every run sees the same bytes.

  cfg1  MXFP4 expert weight [7168, 2048] bf16, N(0, 0.02), 0.1 % outliers x20
  cfg2  MXFP8 linear W [12288, 7168] bf16 N(0, 0.015); X [4096, 7168] bf16
        N(0, 1) times a per-channel lognormal(0, 0.5) factor
  cfg3  MoE prefill: 384 experts, hidden 7168, intermediate 2048, 8192 tokens,
        top-8 routing from softmax(randn + log Zipf(1.1) popularity)
  cfg4  Hessian rows: Student-t(4) activations, bf16
  cfg5  MoE decode: 1 / 4 / 16 tokens, 8 random distinct experts per token
"""

from __future__ import annotations

import hashlib
import math

import torch

HIDDEN = 7168
INTER = 2048
EXPERTS = 384
TOPK = 8


def sha256(t: torch.Tensor) -> str:
    t = t.detach().contiguous().cpu()
    return hashlib.sha256(t.view(torch.uint8).numpy().tobytes()).hexdigest()


def cfg1_weight(rows: int = 7168, cols: int = 2048, seed: int = 0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=g) * 0.02
    mask = torch.rand(rows, cols, generator=g) < 1e-3
    w[mask] *= 20.0
    return w.to(torch.bfloat16)


def cfg2_weight(rows: int = 12288, cols: int = HIDDEN, seed: int = 0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(rows, cols, generator=g) * 0.015).to(torch.bfloat16)


def cfg2_activations(tokens: int = 4096, cols: int = HIDDEN, seed: int = 1) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    channel = torch.exp(0.5 * torch.randn(cols, generator=g))
    return (torch.randn(tokens, cols, generator=g) * channel).to(torch.bfloat16)


def student_t4(rows: int, cols: int, seed: int = 0, dtype=torch.bfloat16) -> torch.Tensor:
    """X = Z0 / sqrt((Z1^2 + ... + Z4^2) / 4): Student-t with 4 d.o.f."""
    g = torch.Generator().manual_seed(seed)
    z0 = torch.randn(rows, cols, generator=g)
    chi = torch.zeros(rows, cols)
    for _ in range(4):
        chi += torch.randn(rows, cols, generator=g).square()
    return (z0 / torch.sqrt(chi / 4.0)).to(dtype)


def zipf_routing(
    tokens: int,
    experts: int = EXPERTS,
    topk: int = TOPK,
    exponent: float = 1.1,
    seed: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k routing with Zipf expert popularity.

    p_k ~ k^-exponent over a seeded permutation of expert ids; logits =
    randn + ln p; top-k of softmax; weights = renormalized top-k probs.
    Returns (ids int32 [tokens, topk], weights float32 [tokens, topk]).
    """
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(experts, generator=g)
    rank = torch.empty(experts, dtype=torch.float64)
    rank[perm] = torch.arange(1, experts + 1, dtype=torch.float64)
    logp = (-exponent * torch.log(rank)).float()
    logits = torch.randn(tokens, experts, generator=g) + logp
    probs = torch.softmax(logits, dim=-1)
    top, ids = torch.topk(probs, topk, dim=-1)
    weights = top / top.sum(dim=-1, keepdim=True)
    return ids.to(torch.int32), weights.float()


def cfg4_expert_rows(device, tokens: int = 65536, k: int = INTER, experts: int = EXPERTS, seed: int = 1):
    """Configuration 4 (ii): every expert's routed rows at K = 2048, grouped.

    The routing is ``zipf_routing(tokens)`` (configuration 3's recipe); expert
    e owns rows [offsets[e], offsets[e + 1]) of ``rows`` (bf16 [pairs, k],
    Student-t(4), generated on ``device`` in slabs by a seeded device
    generator) with one gate per row (``gates`` fp32 [pairs], U(0, 1)).
    Returns (rows, gates, offsets int64 [experts + 1] on the CPU, counts).
    """
    ids, _ = zipf_routing(tokens, experts)
    counts = torch.bincount(ids[ids >= 0].flatten().long(), minlength=experts)
    offsets = torch.zeros(experts + 1, dtype=torch.int64)
    offsets[1:] = torch.cumsum(counts, 0)
    pairs = int(offsets[-1])
    g = torch.Generator(device=device).manual_seed(seed)
    rows = torch.empty(pairs, k, dtype=torch.bfloat16, device=device)
    for c0 in range(0, pairs, 65536):
        n = min(65536, pairs - c0)
        z = torch.randn(n, k, generator=g, device=device)
        chi = sum(torch.randn(n, k, generator=g, device=device).square() for _ in range(4))
        rows[c0:c0 + n] = (z / torch.sqrt(chi / 4)).to(torch.bfloat16)
    gates = torch.rand(pairs, generator=g, device=device)
    return rows, gates, offsets, counts


def random_routing(tokens: int, experts: int = EXPERTS, topk: int = TOPK, seed: int = 0):
    """Decode routing: per token randperm(experts)[:topk], softmax(randn(topk)) weights."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(experts, generator=g)[:topk] for _ in range(tokens)])
    weights = torch.softmax(torch.randn(tokens, topk, generator=g), dim=-1)
    return ids.to(torch.int32), weights.float()


def expert_weights_bf16(
    experts: int, hidden: int = HIDDEN, inter: int = INTER, seed: int = 0, std: float = 0.02
) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense bf16 expert weights: w13 [E, 2*inter, hidden] (gate rows first)
    and w2 [E, hidden, inter]."""
    g = torch.Generator().manual_seed(seed)
    w13 = (torch.randn(experts, 2 * inter, hidden, generator=g) * std).to(torch.bfloat16)
    w2 = (torch.randn(experts, hidden, inter, generator=g) * std).to(torch.bfloat16)
    return w13, w2


def bytes_per_expert(hidden: int = HIDDEN, inter: int = INTER) -> int:
    """MXFP4 bytes (codes + E8M0 scales) of one expert's w13 + w2."""
    w13 = 2 * inter * hidden // 2 + 2 * inter * hidden // 32
    w2 = hidden * inter // 2 + hidden * inter // 32
    return w13 + w2


def moe_flops(pairs: int, hidden: int = HIDDEN, inter: int = INTER) -> float:
    """2 * pairs * (2*inter*hidden + hidden*inter): gate/up and down GEMMs."""
    return 2.0 * pairs * (2 * inter * hidden + hidden * inter)


def syrk_flops(rows: int, k: int) -> float:
    """Useful SYRK flops N*K*(K+1) (upper triangle incl. diagonal, x2 flops/MAC)."""
    return float(rows) * k * (k + 1)


def log2_ceil(x: float) -> int:
    return int(math.ceil(math.log2(x)))


def quantized_experts(
    needed,
    experts: int = EXPERTS,
    hidden: int = HIDDEN,
    inter: int = INTER,
    seed: int = 0,
    std: float = 0.02,
    device: torch.device | str = "cuda",
):
    """MXFP4 expert weights produced by the MXFP4 quantizer from N(0, std).

    Returns (w13_packed [E, 2I, H/2], w13_scale [E, 2I, H/32], w2_packed
    [E, H, I/2], w2_scale [E, H, I/32]) on ``device``.  Only the experts in
    ``needed`` are generated (each from its own seeded generator, so a
    subset reproduces the same bytes); the others are zero.
    """
    from .mxfp4 import mxfp4_quantize

    device = torch.device(device)
    w13q = torch.zeros(experts, 2 * inter, hidden // 2, dtype=torch.uint8, device=device)
    w13s = torch.zeros(experts, 2 * inter, hidden // 32, dtype=torch.uint8, device=device)
    w2q = torch.zeros(experts, hidden, inter // 2, dtype=torch.uint8, device=device)
    w2s = torch.zeros(experts, hidden, inter // 32, dtype=torch.uint8, device=device)
    for e in sorted({int(v) for v in needed}):
        g = torch.Generator(device=device).manual_seed(seed * 100003 + e)
        w13 = (torch.randn(2 * inter, hidden, generator=g, device=device) * std).to(torch.bfloat16)
        w2 = (torch.randn(hidden, inter, generator=g, device=device) * std).to(torch.bfloat16)
        w13q[e], w13s[e] = mxfp4_quantize(w13)
        w2q[e], w2s[e] = mxfp4_quantize(w2)
    return w13q, w13s, w2q, w2s
