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
from .x4t import pack_x4t_scale_components_batched, x4t_fixed_bytes, x4t_tile_index

_WORKSPACES: dict[tuple[torch.device, int], torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The forward's workspace, one per (device, stream): calls on one stream
    serialize, calls on different streams must not share it."""
    key = (device, torch.cuda.current_stream(device).stream_id)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


@dataclass(frozen=True)
class X4TScalePlanes:
    """One expert matrix kind's E8M0 scale planes [experts, rows, columns],
    X4T-coded and resident on the GPU, as kquant's X4T container keeps them
    (kquant/x4t.py:594-602): ``fixed`` uint8 [experts, fixed_bytes],
    ``exceptions`` uint32 words (matrix-local positions), ``exception_offsets``
    int64 [experts + 1]; plus ``tile_index`` uint32 [experts * rows/16 + 1]
    (``x4t_tile_index``), which lets the forward expand a routed expert's
    scales without searching."""

    fixed: torch.Tensor
    exceptions: torch.Tensor
    exception_offsets: torch.Tensor
    tile_index: torch.Tensor
    rows: int
    columns: int


def x4t_scale_planes(
    fixed: torch.Tensor,
    exceptions: torch.Tensor,
    exception_offsets: torch.Tensor,
    *,
    rows: int,
    columns: int,
    device: torch.device | str | None = None,
) -> X4TScalePlanes:
    """Move one matrix kind's X4T scale components to the GPU and build their
    tile index.  The components must be a valid X4T encoding (as
    ``decode_scale_components`` accepts, which kquant's container reader
    checks); the forward expands them without validation."""

    experts = int(exception_offsets.numel()) - 1
    if experts < 1 or exception_offsets.dtype != torch.int64:
        raise ValueError("X4T exception offsets must be int64 [experts + 1]")
    if fixed.dtype != torch.uint8 or fixed.numel() != experts * x4t_fixed_bytes(rows, columns):
        raise ValueError("X4T fixed scale tensor has invalid geometry")
    if exceptions.dtype != torch.uint32 or exceptions.ndim != 1:
        raise ValueError("X4T exception tensor must be one-dimensional uint32")
    gpu = torch.device(device) if device is not None else None
    if gpu is None:
        _, gpu, _ = N.to_gpu([fixed])
    f = N.aligned(fixed.reshape(experts, -1).to(gpu))
    e = exceptions.to(gpu)
    e = N.aligned(e, 4) if e.numel() else torch.zeros(1, dtype=torch.uint32, device=gpu)
    o = N.aligned(exception_offsets.to(gpu), 8)
    index = x4t_tile_index(exceptions.to(gpu), o, rows=rows, columns=columns)
    return X4TScalePlanes(f, e, o, index, rows, columns)


@dataclass(frozen=True)
class MXFP4Experts:
    """Expert weights prepared for ``grouped_expert_forward``: the MXFP4 bytes
    of w13 and w2 repacked once into the MFMA-tiled layout
    (``kq_mx_tile_weights``: 1 KiB tiles of 16 rows x 128 columns, one E8M0
    byte per row and 32-column block alongside).  Same bytes, permuted; the
    role of the external kernel's ``prepare_weights`` step
    (scripts/closure_exl3_layer.py:412-443).

    With X4T scales (``scale_format="x4t"`` or
    ``prepare_expert_weights_x4t``) the scale tiles are None and the w1, w3
    and w2 scale planes stay X4T-coded on the GPU; every forward expands only
    the routed experts' scales (docs/qsrt-technical-brief.md:446-474)."""

    w13_tiles: torch.Tensor
    w13_scale_tiles: torch.Tensor | None
    w2_tiles: torch.Tensor
    w2_scale_tiles: torch.Tensor | None
    experts: int
    hidden: int
    inter: int
    w1_scale_x4t: X4TScalePlanes | None = None
    w3_scale_x4t: X4TScalePlanes | None = None
    w2_scale_x4t: X4TScalePlanes | None = None

    @property
    def scale_format(self) -> str:
        return "x4t" if self.w1_scale_x4t is not None else "tiled"


def _tile(q: torch.Tensor, s: torch.Tensor | None, rows: int, k: int) -> tuple[torch.Tensor, torch.Tensor | None]:
    experts = q.shape[0]
    qt = torch.empty(experts, rows // 16, k // 128, 1024, dtype=torch.uint8, device=q.device)
    st = None
    if s is not None:
        st = torch.empty(experts, rows // 16, k // 128, 64, dtype=torch.uint8, device=q.device)
    N.call("kq_mx_tile_weights", N.ptr(q), None if s is None else N.ptr(s), experts, rows, k, N.ptr(qt),
           None if st is None else N.ptr(st), N.stream(q.device))
    return qt, st


def _expert_shapes(w13_packed: torch.Tensor, w2_packed: torch.Tensor) -> tuple[int, int, int]:
    if w13_packed.dtype != torch.uint8 or w2_packed.dtype != torch.uint8:
        raise TypeError("expected uint8 packed weights and scales")
    if w13_packed.ndim != 3 or w2_packed.ndim != 3:
        raise ValueError("expert weights must be stacked [experts, rows, packed columns]")
    experts = w13_packed.shape[0]
    inter = w13_packed.shape[1] // 2
    hidden = w13_packed.shape[2] * 2
    if w13_packed.shape != (experts, 2 * inter, hidden // 2):
        raise ValueError(f"w13_packed shape {tuple(w13_packed.shape)} != {(experts, 2 * inter, hidden // 2)}")
    if w2_packed.shape != (experts, hidden, inter // 2):
        raise ValueError(f"w2_packed shape {tuple(w2_packed.shape)} != {(experts, hidden, inter // 2)}")
    # prefill-sized batches need inter % 512 (the grouped GEMMs' tiles); a
    # decode batch with bf16 activations takes inter % 256 (the library checks)
    if hidden % 512 or inter % 256:
        raise ValueError("hidden must be a multiple of 512 and the intermediate size of 256 "
                         "(512 outside bf16-activation decode batches)")
    return experts, hidden, inter


def _x4t_limits(hidden: int, inter: int) -> None:
    if hidden // 32 > 255 or inter // 32 > 255:
        raise ValueError("X4T scale planes have at most 255 columns (hidden and intermediate <= 8160)")


def prepare_expert_weights(
    w13_packed: torch.Tensor,
    w13_scale: torch.Tensor,
    w2_packed: torch.Tensor,
    w2_scale: torch.Tensor,
    *,
    scale_format: str = "tiled",
) -> MXFP4Experts:
    """Validate checkpoint-layout MXFP4 expert weights and repack them once
    for ``grouped_expert_forward`` (on the GPU; CPU inputs are moved).

    ``scale_format="x4t"`` keeps the scales X4T-coded instead (w1 = the gate
    rows of w13_scale, w3 = the up rows, w2): the coding runs on the GPU
    (``pack_x4t_scale_components_batched``) and the forward expands the
    routed experts' scales on every call."""

    if scale_format not in ("tiled", "x4t"):
        raise ValueError(f"scale_format must be 'tiled' or 'x4t', got {scale_format!r}")
    if w13_scale.dtype != torch.uint8 or w2_scale.dtype != torch.uint8:
        raise TypeError(f"expected uint8 packed weights and scales, got {w13_scale.dtype} / {w2_scale.dtype}")
    experts, hidden, inter = _expert_shapes(w13_packed, w2_packed)
    if w13_scale.shape != (experts, 2 * inter, hidden // 32):
        raise ValueError("w13_scale shape does not match w13_packed")
    if w2_scale.shape != (experts, hidden, inter // 32):
        raise ValueError("w2_scale shape does not match w2_packed")
    (w13q, w13s, w2q, w2s), gpu, _ = N.to_gpu([w13_packed, w13_scale, w2_packed, w2_scale])
    w13q, w13s, w2q, w2s = (N.aligned(t) for t in (w13q, w13s, w2q, w2s))
    if scale_format == "x4t":
        _x4t_limits(hidden, inter)
        planes = []
        for plane, rows, cols in ((w13s[:, :inter], inter, hidden // 32), (w13s[:, inter:], inter, hidden // 32),
                                  (w2s, hidden, inter // 32)):
            fixed, exc, offsets = pack_x4t_scale_components_batched(plane.contiguous())
            planes.append(x4t_scale_planes(fixed, exc, offsets, rows=rows, columns=cols, device=gpu))
        w13t, _ = _tile(w13q, None, 2 * inter, hidden)
        w2t, _ = _tile(w2q, None, hidden, inter)
        return MXFP4Experts(w13t, None, w2t, None, experts, hidden, inter, *planes)
    w13t, w13st = _tile(w13q, w13s, 2 * inter, hidden)
    w2t, w2st = _tile(w2q, w2s, hidden, inter)
    return MXFP4Experts(w13t, w13st, w2t, w2st, experts, hidden, inter)


def prepare_expert_weights_x4t(
    w13_packed: torch.Tensor,
    w2_packed: torch.Tensor,
    w1_scale: X4TScalePlanes | tuple[torch.Tensor, torch.Tensor, torch.Tensor],
    w3_scale: X4TScalePlanes | tuple[torch.Tensor, torch.Tensor, torch.Tensor],
    w2_scale: X4TScalePlanes | tuple[torch.Tensor, torch.Tensor, torch.Tensor],
) -> MXFP4Experts:
    """Expert weights whose scales arrive X4T-coded, as kquant's X4T layer
    container stores them per matrix kind: (fixed [experts, fixed_bytes],
    exceptions uint32, exception_offsets int64 [experts + 1]) for w1, w3 and
    w2, or ``X4TScalePlanes``.  The packed weights are in checkpoint layout
    (gate-first w13 [E, 2I, H/2], w2 [E, H, I/2]) and are tiled once; the
    scales stay coded on the GPU."""

    experts, hidden, inter = _expert_shapes(w13_packed, w2_packed)
    _x4t_limits(hidden, inter)
    (w13q, w2q), gpu, _ = N.to_gpu([w13_packed, w2_packed])
    planes = []
    for given, rows, cols in ((w1_scale, inter, hidden // 32), (w3_scale, inter, hidden // 32),
                              (w2_scale, hidden, inter // 32)):
        if isinstance(given, X4TScalePlanes):
            if (given.rows, given.columns) != (rows, cols):
                raise ValueError(f"X4T plane is [{given.rows}, {given.columns}], expected [{rows}, {cols}]")
            planes.append(given)
        else:
            planes.append(x4t_scale_planes(*given, rows=rows, columns=cols, device=gpu))
        if int(planes[-1].exception_offsets.numel()) != experts + 1:
            raise ValueError("X4T exception offsets do not cover every expert")
    w13t, _ = _tile(N.aligned(w13q), None, 2 * inter, hidden)
    w2t, _ = _tile(N.aligned(w2q), None, hidden, inter)
    return MXFP4Experts(w13t, None, w2t, None, experts, hidden, inter, *planes)


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
    x4t = prepared.scale_format == "x4t"
    size_fn = lib.kq_moe_x4t_workspace_size if x4t else lib.kq_moe_workspace_size
    nbytes = int(size_fn(tokens, topk, prepared.experts, hidden, prepared.inter))
    if nbytes < 0:
        raise ValueError("invalid MoE sizes")
    ws = _workspace(gpu, nbytes)
    act_code = N.ACT_SITU if activation == "situ" else N.ACT_SWIGLU
    flags = (N.MOE_REGISTER_STAGED if register_staged else 0) | act_flags[activation_format]
    head = (act_code, float(beta), float(linear_beta), N.ptr(xb), hidden, tokens, hidden, N.ptr(ids),
            N.ptr(rw), topk, prepared.experts, prepared.inter)
    tail = (N.DTYPE_CODES[out_dtype], N.ptr(out), N.ptr(ws), ws.numel(), flags, N.stream(gpu))
    if x4t:
        planes = []
        for p in (prepared.w1_scale_x4t, prepared.w3_scale_x4t, prepared.w2_scale_x4t):
            planes += [N.ptr(p.fixed), N.ptr(p.exceptions), N.ptr(p.tile_index)]
        N.call("kq_moe_forward_x4t", *head, N.ptr(prepared.w13_tiles), N.ptr(prepared.w2_tiles), *planes,
               *tail)
    else:
        N.call("kq_moe_forward", *head, N.ptr(prepared.w13_tiles), N.ptr(prepared.w13_scale_tiles),
               N.ptr(prepared.w2_tiles), N.ptr(prepared.w2_scale_tiles), *tail)
    return out if host is None else out.to(host)
