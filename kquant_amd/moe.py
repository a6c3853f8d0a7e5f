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

from dataclasses import dataclass

import torch

from . import _native as N
from .io.mxfp4 import dequant
from .linear import mxfp4_linear
from .source_weights import PackedMXFP4Matrix
from .tp_simulator import situ, swiglu

_WORKSPACES: dict[torch.device, torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    buf = _WORKSPACES.get(device)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORKSPACES[device] = buf
    return buf


@dataclass(frozen=True)
class MXFP4Experts:
    """Expert weights prepared for ``grouped_expert_forward``: the MXFP4 bytes
    of w13 and w2 repacked once into the MFMA-tiled layout
    (``kq_mx_tile_weights``: 1 KiB tiles of 16 rows x 128 columns, one E8M0
    byte per row and 32-column block alongside).  Same bytes, permuted; the
    role of the external kernel's ``prepare_weights`` step
    (scripts/closure_exl3_layer.py:412-443)."""

    w13_tiles: torch.Tensor
    w13_scale_tiles: torch.Tensor
    w2_tiles: torch.Tensor
    w2_scale_tiles: torch.Tensor
    experts: int
    hidden: int
    inter: int


def _tile(q: torch.Tensor, s: torch.Tensor, rows: int, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    experts = q.shape[0]
    qt = torch.empty(experts, rows // 16, k // 128, 1024, dtype=torch.uint8, device=q.device)
    st = torch.empty(experts, rows // 16, k // 128, 64, dtype=torch.uint8, device=q.device)
    N.call("kq_mx_tile_weights", N.ptr(q), N.ptr(s), experts, rows, k, N.ptr(qt), N.ptr(st),
           N.stream(q.device))
    return qt, st


def prepare_expert_weights(
    w13_packed: torch.Tensor,
    w13_scale: torch.Tensor,
    w2_packed: torch.Tensor,
    w2_scale: torch.Tensor,
) -> MXFP4Experts:
    """Validate checkpoint-layout MXFP4 expert weights and repack them once
    for ``grouped_expert_forward`` (on the GPU; CPU inputs are moved)."""

    for t in (w13_packed, w13_scale, w2_packed, w2_scale):
        if t.dtype != torch.uint8:
            raise TypeError(f"expected uint8 packed weights and scales, got {t.dtype}")
    if w13_packed.ndim != 3 or w2_packed.ndim != 3:
        raise ValueError("expert weights must be stacked [experts, rows, packed columns]")
    experts = w13_packed.shape[0]
    inter = w13_packed.shape[1] // 2
    hidden = w13_packed.shape[2] * 2
    if w13_packed.shape != (experts, 2 * inter, hidden // 2):
        raise ValueError(f"w13_packed shape {tuple(w13_packed.shape)} != {(experts, 2 * inter, hidden // 2)}")
    if w13_scale.shape != (experts, 2 * inter, hidden // 32):
        raise ValueError("w13_scale shape does not match w13_packed")
    if w2_packed.shape != (experts, hidden, inter // 2):
        raise ValueError(f"w2_packed shape {tuple(w2_packed.shape)} != {(experts, hidden, inter // 2)}")
    if w2_scale.shape != (experts, hidden, inter // 32):
        raise ValueError("w2_scale shape does not match w2_packed")
    if hidden % 512 or inter % 512:
        raise ValueError("hidden and intermediate sizes must be multiples of 512")
    (w13q, w13s, w2q, w2s), gpu, _ = N.to_gpu([w13_packed, w13_scale, w2_packed, w2_scale])
    w13q, w13s, w2q, w2s = (N.aligned(t) for t in (w13q, w13s, w2q, w2s))
    w13t, w13st = _tile(w13q, w13s, 2 * inter, hidden)
    w2t, w2st = _tile(w2q, w2s, hidden, inter)
    return MXFP4Experts(w13t, w13st, w2t, w2st, experts, hidden, inter)


def expert_output(
    inputs: torch.Tensor,
    w1: tuple[torch.Tensor, torch.Tensor],
    w3: tuple[torch.Tensor, torch.Tensor],
    w2: tuple[torch.Tensor, torch.Tensor],
    *,
    activation: str = "situ",
    beta: float = 4.0,
    linear_beta: float = 25.0,
) -> torch.Tensor:
    """One expert's MLP over its MXFP4 matrices, in fp32.

    kquant/pack/qsrt_validation.py:240-258 (``official_expert_output``):
    gate = x W1^T, up = x W3^T, middle = situ(gate, up), out = middle W2^T,
    every product an fp32 ``F.linear`` over the dequantized official
    matrix.  Here each matrix stays packed (``(packed, scale)`` or a
    ``PackedMXFP4Matrix``) and the products run in ``kq_mx_linear_f32``
    (fp32 activations split exactly into bf16 terms, fp32 accumulation);
    the activation runs in ``kq_expert_activation``.  Output fp32 [rows, H].
    """

    if activation not in ("situ", "swiglu"):
        raise ValueError(f"unsupported activation {activation!r}")
    act_flags = {"bf16": 0, "mxfp8": N.MOE_ACT_MXFP8, "mxfp4": N.MOE_ACT_MXFP4}
    if activation_format not in act_flags:
        raise ValueError(f"activation_format must be bf16, mxfp8 or mxfp4, got {activation_format!r}")
    if register_staged and activation_format != "bf16":
        raise ValueError("register_staged applies to the bf16-activation mode only")
    if inputs.ndim != 2:
        raise ValueError("expert inputs must be two-dimensional")
    (p1, s1), (p3, s3), (p2, s2) = (_pair(w) for w in (w1, w3, w2))
    x = inputs.float()
    gate = mxfp4_linear(x, p1, s1, out_dtype=torch.float32)
    up = mxfp4_linear(x, p3, s3, out_dtype=torch.float32)
    if activation == "situ":
        middle = situ(gate, up, beta=beta, linear_beta=linear_beta)
    else:
        middle = swiglu(gate, up)
    return mxfp4_linear(middle, p2, s2, out_dtype=torch.float32)


def _pair(w) -> tuple[torch.Tensor, torch.Tensor]:
    if isinstance(w, PackedMXFP4Matrix):
        return w.packed, w.scale
    packed, scale = w
    return packed, scale


def reconstruct_source(
    raw: dict[str, dict[str, torch.Tensor]],
    device: torch.device | str,
    *,
    scale_byte_max: int | None = None,
) -> dict[str, torch.Tensor]:
    """bf16 expert matrices from their MXFP4 parts, optionally clamping the
    E8M0 bytes to ``scale_byte_max`` first
    (scripts/closure_exl3_layer.py:143-161, ``_reconstruct_source``).
    ``raw[matrix]`` holds ``"packed"`` and ``"scale"``."""

    result = {}
    for matrix, value in raw.items():
        scale = value["scale"].view(torch.uint8)
        if scale_byte_max is not None:
            scale = scale.clamp(max=scale_byte_max)
        result[matrix] = dequant(value["packed"], scale, dtype=torch.bfloat16).to(device=device)
    return result


_reconstruct_source = reconstruct_source


def grouped_expert_forward(
    x: torch.Tensor,
    route_ids: torch.Tensor,
    route_weights: torch.Tensor,
    w13_packed: torch.Tensor | MXFP4Experts,
    w13_scale: torch.Tensor | None = None,
    w2_packed: torch.Tensor | None = None,
    w2_scale: torch.Tensor | None = None,
    *,
    activation: str = "situ",
    beta: float = 4.0,
    linear_beta: float = 25.0,
    out_dtype: torch.dtype = torch.float32,
    register_staged: bool = False,
    activation_format: str = "bf16",
) -> torch.Tensor:
    """Route-weighted expert outputs ``[T, H]`` (fp32 by default, as the
    reference's accumulator is).

    The weights are either an ``MXFP4Experts`` from
    ``prepare_expert_weights`` (serving: prepare once per layer) or the four
    checkpoint-layout tensors, which are then prepared on every call.
    ``register_staged`` runs the grouped GEMMs on the register-staged kernel
    (taken anyway when a buffer exceeds 4 GiB) instead of the direct-to-LDS
    one; both meet the same error bound and differ only by fp32 rounding.

    ``activation_format`` "mxfp8" / "mxfp4" selects the activation-quantized
    modes (W4A8 / W4A4, no kquant counterpart): the tokens and the bf16
    intermediates are MX-quantized per row (the ``mxfp8_quantize`` /
    ``mxfp4_quantize`` rule) and every GEMM runs on the block-scaled fp8/fp4
    MFMA.  The result is an fp32 GEMM over the dequantized operands up to
    summation order; it is not the bf16-activation result.
    """

    if activation not in ("situ", "swiglu"):
        raise ValueError(f"unsupported activation {activation!r}")
    act_flags = {"bf16": 0, "mxfp8": N.MOE_ACT_MXFP8, "mxfp4": N.MOE_ACT_MXFP4}
    if activation_format not in act_flags:
        raise ValueError(f"activation_format must be bf16, mxfp8 or mxfp4, got {activation_format!r}")
    if register_staged and activation_format != "bf16":
        raise ValueError("register_staged applies to the bf16-activation mode only")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("out_dtype must be float32 or bfloat16")
    if x.ndim != 2:
        raise ValueError("x must be [tokens, hidden]")
    if route_ids.shape != route_weights.shape or route_ids.ndim != 2 or route_ids.shape[0] != x.shape[0]:
        raise ValueError("route_ids and route_weights must both be [tokens, topk]")
    if isinstance(w13_packed, MXFP4Experts):
        prepared = w13_packed
    else:
        if w13_scale is None or w2_packed is None or w2_scale is None:
            raise ValueError("pass MXFP4Experts or all four packed weight tensors")
        prepared = prepare_expert_weights(w13_packed, w13_scale, w2_packed, w2_scale)
    tokens, hidden = x.shape
    if hidden != prepared.hidden:
        raise ValueError(f"x hidden size {hidden} != expert hidden size {prepared.hidden}")
    topk = route_ids.shape[1]
    xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
    ids = route_ids.to(torch.int32)
    rw = route_weights.to(torch.float32)
    gpu = prepared.w13_tiles.device
    host = None if xb.is_cuda else xb.device
    xb, ids, rw = (N.aligned(t.to(gpu)) for t in (xb, ids, rw))
    out = torch.empty(tokens, hidden, dtype=out_dtype, device=gpu)
    lib = N.library()
    nbytes = int(lib.kq_moe_workspace_size(tokens, topk, prepared.experts, hidden, prepared.inter))
    if nbytes < 0:
        raise ValueError("invalid MoE sizes")
    ws = _workspace(gpu, nbytes)
    N.call("kq_moe_forward", N.ACT_SITU if activation == "situ" else N.ACT_SWIGLU,
           float(beta), float(linear_beta), N.ptr(xb), hidden, tokens, hidden, N.ptr(ids),
           N.ptr(rw), topk, prepared.experts, prepared.inter, N.ptr(prepared.w13_tiles),
           N.ptr(prepared.w13_scale_tiles), N.ptr(prepared.w2_tiles), N.ptr(prepared.w2_scale_tiles),
           N.DTYPE_CODES[out_dtype], N.ptr(out), N.ptr(ws), ws.numel(),
           (N.MOE_REGISTER_STAGED if register_staged else 0) | act_flags[activation_format], N.stream(gpu))
    return out if host is None else out.to(host)
