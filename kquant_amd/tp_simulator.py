"""Expert-path helpers of ``kquant/tp_simulator.py`` on the GPU.

``situ`` (:83-94), ``reduce_partials`` (:72-80), ``kimi_topk`` (:114-134)
and ``comparison_metrics`` (:137-160), with the reference's signatures and
result types.  Each runs a kernel of ``libkquant_amd.so``; CPU inputs are
processed on the current GPU and results return on the input's device.
"""

from __future__ import annotations

import math

import torch

from . import _native as N

_METRIC_PARTS = 256
_METRIC_FIELDS = 5


def _flat(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in N.DTYPE_CODES:
        t = t.float()
    return t.contiguous().reshape(-1)


def _activation(kind: int, gate: torch.Tensor, up: torch.Tensor, beta: float,
                linear_beta: float, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    if gate.shape != up.shape:
        raise ValueError("gate and up must have the same shape")
    out_dtype = gate.dtype if out_dtype is None else out_dtype
    kernel_out = out_dtype if out_dtype in N.DTYPE_CODES else torch.float32
    (g, u), gpu, host = N.to_gpu([gate, up])
    g, u = _flat(g), _flat(u)
    if u.dtype != g.dtype:
        u = u.to(g.dtype)
    n = g.numel()
    out = torch.empty(n, dtype=kernel_out, device=gpu)
    if n:
        N.call("kq_expert_activation", kind, float(beta), float(linear_beta), N.DTYPE_CODES[g.dtype],
               N.ptr(g), N.ptr(u), n, 1, n, N.DTYPE_CODES[kernel_out], N.ptr(out), n, N.stream(gpu))
    out = out.reshape(gate.shape).to(out_dtype)
    return out if host is None else out.to(host)


def situ(gate: torch.Tensor, up: torch.Tensor, *, beta: float = 4.0,
         linear_beta: float = 25.0) -> torch.Tensor:
    """beta tanh(g/beta) sigmoid(g) * linear_beta tanh(u/linear_beta), in fp32, as gate's dtype."""

    return _activation(N.ACT_SITU, gate, up, beta, linear_beta)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(g) * u in fp32, as gate's dtype (the SwiGLU expert activation)."""

    return _activation(N.ACT_SWIGLU, gate, up, 1.0, 1.0)


def reduce_partials(partials: list[torch.Tensor], *, dtype: torch.dtype) -> torch.Tensor:
    """Sum rank partials in fp32 in rank order, then round to ``dtype``."""

    if not partials:
        raise ValueError("at least one partial is required")
    shape = partials[0].shape
    if any(p.shape != shape for p in partials):
        raise ValueError("partials must share one shape")
    moved, gpu, host = N.to_gpu(partials)
    stacked = torch.stack([p.float() for p in moved]).contiguous()
    n = stacked[0].numel()
    kernel_out = dtype if dtype in N.DTYPE_CODES else torch.float32
    out = torch.empty(n, dtype=kernel_out, device=gpu)
    if n:
        N.call("kq_reduce_partials", N.ptr(stacked), len(partials), n, n, N.DTYPE_CODES[kernel_out],
               N.ptr(out), N.stream(gpu))
    out = out.reshape(shape).to(dtype)
    return out if host is None else out.to(host)


def kimi_topk(router_logits: torch.Tensor, correction_bias: torch.Tensor, topk: int, *,
              routed_scaling_factor: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """K3's one-group sigmoid router with biased selection -> (weights fp32, ids int32)."""

    if router_logits.ndim != 2:
        raise ValueError("router logits must be [tokens, experts]")
    tokens, experts = map(int, router_logits.shape)
    if correction_bias.numel() != experts:
        raise ValueError("correction bias must have one entry per expert")
    (logits, bias), gpu, host = N.to_gpu([router_logits, correction_bias])
    logits = _flat(logits).reshape(tokens, experts)
    bias = bias.float().contiguous()
    weights = torch.empty(tokens, topk, dtype=torch.float32, device=gpu)
    ids = torch.empty(tokens, topk, dtype=torch.int32, device=gpu)
    N.call("kq_kimi_topk", N.DTYPE_CODES[logits.dtype], N.ptr(logits), experts, N.ptr(bias), tokens,
           experts, int(topk), float(routed_scaling_factor), N.ptr(weights), N.ptr(ids),
           N.stream(gpu))
    if host is not None:
        return weights.to(host), ids.to(host)
    return weights, ids


def comparison_sums(reference: torch.Tensor, actual: torch.Tensor) -> tuple[float, ...]:
    """(sum d^2, max |d|, sum r^2, sum a^2, sum r a) in float64, d = a - r in fp32."""

    if reference.shape != actual.shape:
        raise ValueError("reference and actual must have the same shape")
    (r, a), gpu, _ = N.to_gpu([reference, actual])
    r, a = _flat(r), _flat(a)
    ws = torch.empty(_METRIC_PARTS * _METRIC_FIELDS, dtype=torch.float64, device=gpu)
    out = torch.empty(_METRIC_FIELDS, dtype=torch.float64, device=gpu)
    N.call("kq_comparison_sums", N.DTYPE_CODES[r.dtype], N.ptr(r), N.DTYPE_CODES[a.dtype], N.ptr(a),
           r.numel(), N.ptr(ws), N.ptr(out), N.stream(gpu))
    return tuple(float(v) for v in out.cpu().tolist())


def comparison_metrics(reference: torch.Tensor, actual: torch.Tensor) -> dict[str, float]:
    """relative_l2, max_abs and cosine of actual against reference (float32 results)."""

    s_dd, m_d, s_rr, s_aa, s_ra = comparison_sums(reference, actual)
    tiny = float(torch.finfo(torch.float32).tiny)
    eps = 1e-8
    relative = math.sqrt(s_dd) / max(math.sqrt(s_rr), tiny)
    cosine = s_ra / math.sqrt(max(s_rr * s_aa, eps * eps))
    as_f32 = lambda v: float(torch.tensor(v, dtype=torch.float32))  # noqa: E731
    return {"relative_l2": as_f32(relative), "max_abs": as_f32(m_d), "cosine": as_f32(cosine)}
