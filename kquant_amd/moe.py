"""Routed MoE expert forward over MXFP4-packed expert weights (W4A16).

``grouped_expert_forward`` computes, for every (token, slot) routed pair, the
gate/up projections, the activation (SiTU or SwiGLU), the down projection and
the route-weighted sum per token, exactly as kquant's routed reference
(scripts/closure_exl3_layer.py:557-598, ``_reference_rank`` with tp = 1) does
with dequantized weights; all of it runs in ``kq_moe_forward`` (one stream, a
cached device workspace, no host synchronisation).

Layouts (compressed-tensors MXFP4, kquant/io/mxfp4.py:1-8):
  w13_packed uint8 [E, 2I, H/2], w13_scale uint8 [E, 2I, H/32] (gate rows
  first, then up rows: the "w31"/gate-first order of
  scripts/closure_exl3_layer.py:420-423); w2_packed uint8 [E, H, I/2],
  w2_scale uint8 [E, H, I/32].
"""

from __future__ import annotations

import torch

from . import _native as N

_WORKSPACES: dict[torch.device, torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    buf = _WORKSPACES.get(device)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORKSPACES[device] = buf
    return buf


def situ(gate: torch.Tensor, up: torch.Tensor, *, beta: float = 4.0,
         linear_beta: float = 25.0) -> torch.Tensor:
    """kquant/tp_simulator.py:83-94 (host-side helper, computed with torch)."""
    gate_value = beta * torch.tanh(gate.float() / beta) * torch.sigmoid(gate.float())
    up_value = linear_beta * torch.tanh(up.float() / linear_beta)
    return (gate_value * up_value).to(gate.dtype)


def grouped_expert_forward(
    x: torch.Tensor,
    route_ids: torch.Tensor,
    route_weights: torch.Tensor,
    w13_packed: torch.Tensor,
    w13_scale: torch.Tensor,
    w2_packed: torch.Tensor,
    w2_scale: torch.Tensor,
    *,
    activation: str = "situ",
    beta: float = 4.0,
    linear_beta: float = 25.0,
    out_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Route-weighted expert outputs ``[T, H]`` (fp32 by default, as the
    reference's accumulator is)."""

    if activation not in ("situ", "swiglu"):
        raise ValueError(f"unsupported activation {activation!r}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("out_dtype must be float32 or bfloat16")
    if x.ndim != 2:
        raise ValueError("x must be [tokens, hidden]")
    tokens, hidden = x.shape
    if route_ids.shape != route_weights.shape or route_ids.ndim != 2 or route_ids.shape[0] != tokens:
        raise ValueError("route_ids and route_weights must both be [tokens, topk]")
    for t in (w13_packed, w13_scale, w2_packed, w2_scale):
        if t.dtype != torch.uint8:
            raise TypeError(f"expected uint8 packed weights and scales, got {t.dtype}")
    experts = w13_packed.shape[0]
    inter = w13_packed.shape[1] // 2
    if w13_packed.shape != (experts, 2 * inter, hidden // 2):
        raise ValueError(f"w13_packed shape {tuple(w13_packed.shape)} != {(experts, 2 * inter, hidden // 2)}")
    if w13_scale.shape != (experts, 2 * inter, hidden // 32):
        raise ValueError("w13_scale shape does not match w13_packed")
    if w2_packed.shape != (experts, hidden, inter // 2):
        raise ValueError(f"w2_packed shape {tuple(w2_packed.shape)} != {(experts, hidden, inter // 2)}")
    if w2_scale.shape != (experts, hidden, inter // 32):
        raise ValueError("w2_scale shape does not match w2_packed")
    topk = route_ids.shape[1]
    xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
    ids = route_ids.to(torch.int32)
    rw = route_weights.to(torch.float32)
    (xb, ids, rw, w13q, w13s, w2q, w2s), gpu, host = N.to_gpu(
        [xb, ids, rw, w13_packed, w13_scale, w2_packed, w2_scale])
    xb, ids, rw = N.aligned(xb), N.aligned(ids), N.aligned(rw)
    w13q, w13s, w2q, w2s = (N.aligned(t) for t in (w13q, w13s, w2q, w2s))
    out = torch.empty(tokens, hidden, dtype=out_dtype, device=gpu)
    lib = N.library()
    nbytes = int(lib.kq_moe_workspace_size(tokens, topk, experts, hidden, inter))
    if nbytes < 0:
        raise ValueError("invalid MoE sizes")
    ws = _workspace(gpu, nbytes)
    N.call("kq_moe_forward", N.ACT_SITU if activation == "situ" else N.ACT_SWIGLU,
           float(beta), float(linear_beta), N.ptr(xb), hidden, tokens, hidden, N.ptr(ids),
           N.ptr(rw), topk, experts, inter, N.ptr(w13q), N.ptr(w13s), N.ptr(w2q), N.ptr(w2s),
           N.DTYPE_CODES[out_dtype], N.ptr(out), N.ptr(ws), ws.numel(), 0, N.stream(gpu))
    return out if host is None else out.to(host)
