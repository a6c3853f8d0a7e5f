"""Dequant-fused block-scaled linear layers (bf16 activations x MX weights).

``mxfp8_linear`` / ``mxfp4_linear`` compute ``source @ dequant(weight).T`` with
fp32 accumulation in one HIP kernel (``kq_mx_linear``).  They replace the
dequantize-then-matmul fp32 oracle of kquant's closures
(scripts/closure_mxfp8_mlp.py:146-160, kquant/pack/qsrt_validation.py:249-258)
and the external ``mxfp8_linear.mm`` kernel call
(scripts/closure_mxfp8_mlp.py:172-177) with an A16 kernel: activations stay
bf16, weights are expanded exactly to bf16 inside the kernel.

fp32 sources take ``kq_mx_linear_f32``: the source is split exactly into
three bf16 terms and all three products accumulate in fp32 in one launch, so
the result has fp32-GEMM accuracy, as the reference's fp32 ``F.linear``
(kquant/pack/qsrt_validation.py:240-258) does.

``mxfp8_linear_mm`` is the production form of the MXFP8 linear
(scripts/closure_mxfp8_mlp.py:163-187): the input rows are quantized to
MXFP8 with the ``mxfp8_quantize`` rule (``block_fp8_linear.quantize_input``,
:155) and both MXFP8 operands are multiplied as they are on the block-scaled
fp8 matrix cores (``kq_mx_linear_mm``); ``mxfp8_linear_mx`` takes input rows
that are already quantized (``kq_mx_linear_mx``).  Its oracle is
``_reference_from_packed`` (:146-160): dequantize both operands, fp32 product.
"""

from __future__ import annotations

import torch

from . import _native as N


def _linear(fmt: int, source: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
            out_dtype: torch.dtype | None) -> torch.Tensor:
    if out_dtype is None:
        out_dtype = torch.float32 if source.dtype == torch.float32 else torch.bfloat16
    if source.ndim < 1:
        raise ValueError("source must have a feature dimension")
    if scale.dtype != torch.uint8:
        raise TypeError(f"scales must be uint8 E8M0, got {scale.dtype}")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("out_dtype must be bfloat16 or float32")
    k = source.shape[-1]
    n = weight.shape[0]
    packed_k = k if fmt == N.FMT_MXFP8_E4M3 else k // 2
    if weight.ndim != 2 or weight.shape[1] != packed_k:
        raise ValueError(f"weight shape {tuple(weight.shape)} does not match K={k}")
    if tuple(scale.shape) != (n, k // 32):
        raise ValueError(f"scale shape {tuple(scale.shape)} != {(n, k // 32)}")
    if k % 64:
        raise ValueError(f"K={k} must be a multiple of 64")
    lead = source.shape[:-1]
    a = source.reshape(-1, k)
    exact_f32 = a.dtype == torch.float32
    if not exact_f32 and a.dtype != torch.bfloat16:
        a = a.to(torch.bfloat16)
    (a, w, s), gpu, host = N.to_gpu([a, weight.view(torch.uint8), scale])
    a, w, s = N.aligned(a), N.aligned(w), N.aligned(s)
    m = a.shape[0]
    if exact_f32:
        out = torch.empty(m, n, dtype=torch.float32, device=gpu)
        ws = torch.empty(max(int(N.library().kq_mx_linear_f32_workspace_size(m, k)), 16),
                         dtype=torch.uint8, device=gpu)
        N.call("kq_mx_linear_f32", fmt, N.ptr(a), k, N.ptr(w), N.ptr(s), m, n, k, N.ptr(out), n,
               N.ptr(ws), ws.numel(), N.stream(gpu))
        out = out.to(out_dtype)
    else:
        out = torch.empty(m, n, dtype=out_dtype, device=gpu)
        N.call("kq_mx_linear", fmt, N.ptr(a), k, N.ptr(w), N.ptr(s), m, n, k,
               N.DTYPE_CODES[out_dtype], N.ptr(out), n, N.stream(gpu))
    out = out.reshape(*lead, n)
    return out if host is None else out.to(host)


def mxfp8_linear(source: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, *,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``source [..., K] @ dequant(weight E4M3 [N, K], scale [N, K/32]).T``.

    Output dtype defaults to fp32 for fp32 sources and bf16 otherwise.
    """
    if weight.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError(f"MXFP8 weight must be float8_e4m3fn, got {weight.dtype}")
    return _linear(N.FMT_MXFP8_E4M3, source, weight, scale, out_dtype)


def mxfp4_linear(source: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, *,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``source [..., K] @ dequant(packed [N, K/2], scale [N, K/32]).T``.

    Output dtype defaults to fp32 for fp32 sources and bf16 otherwise.
    """
    if packed.dtype != torch.uint8:
        raise TypeError(f"expected uint8, got {packed.dtype}")
    return _linear(N.FMT_MXFP4_E2M1, source, packed, scale, out_dtype)


MX_LINEAR_K_ALIGN = 128  # the MXFP8 x MXFP8 kernel's K granule


def _pad_k(t: torch.Tensor, width: int, value: int = 0) -> torch.Tensor:
    """Zero-pad the last dimension (the reference pads the source to the packed
    weight's padded_in_features, scripts/closure_mxfp8_mlp.py:136-143)."""
    if t.shape[-1] == width:
        return t
    return torch.nn.functional.pad(t, (0, width - t.shape[-1]), value=value)


def _mx_weight(weight: torch.Tensor, scale: torch.Tensor, k: int):
    if weight.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError(f"MXFP8 weight must be float8_e4m3fn, got {weight.dtype}")
    if scale.dtype != torch.uint8:
        raise TypeError(f"scales must be uint8 E8M0, got {scale.dtype}")
    if weight.ndim != 2 or weight.shape[1] != k:
        raise ValueError(f"weight shape {tuple(weight.shape)} does not match K={k}")
    if tuple(scale.shape) != (weight.shape[0], k // 32):
        raise ValueError(f"scale shape {tuple(scale.shape)} != {(weight.shape[0], k // 32)}")
    kp = -(-k // MX_LINEAR_K_ALIGN) * MX_LINEAR_K_ALIGN
    # padded weight columns are zero codes, so they add nothing whatever their scale
    return _pad_k(weight.view(torch.uint8), kp), _pad_k(scale, kp // 32, 127), kp


def mxfp8_linear_mm(source: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, *,
                    out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``mxfp8_linear.mm(source, packed)`` of the reference's production MXFP8
    linear: ``source [..., K]`` (bf16, fp16 or fp32) is quantized per row to
    MXFP8 (the ``mxfp8_quantize`` rule, 32-element blocks along K), then
    multiplied by the MXFP8 weight (E4M3 [N, K], scale [N, K/32]) on the
    block-scaled fp8 matrix cores with fp32 accumulation.  Equals
    ``dequant(quantize(source)) @ dequant(weight).T`` (the reference's
    operand-exact oracle) up to the matrix cores' summation.  K is padded to
    a multiple of 128 with zeros when needed (a per-call copy of the weight;
    pad it once to skip that)."""
    if source.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("source must be bfloat16, float16 or float32")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("out_dtype must be bfloat16 or float32")
    k = source.shape[-1]
    if k % 32:
        raise ValueError(f"K={k} must be a multiple of 32 (the MX block)")
    lead = source.shape[:-1]
    (a, w, s), gpu, host = N.to_gpu([source.reshape(-1, k), weight.view(torch.uint8), scale])
    w, s, kp = _mx_weight(w, s, k)
    a = _pad_k(a, kp)
    a = a if a.stride(-1) == 1 and a.stride(0) % 8 == 0 else a.contiguous()
    a, w, s = N.aligned(a), N.aligned(w), N.aligned(s, 4)
    m, n = a.shape[0], w.shape[0]
    out = torch.empty(m, n, dtype=out_dtype, device=gpu)
    ws = torch.empty(max(int(N.library().kq_mx_linear_mm_workspace_size(m, n, kp)), 256), dtype=torch.uint8,
                     device=gpu)
    N.call("kq_mx_linear_mm", N.FMT_MXFP8_E4M3, N.ptr(a), N.DTYPE_CODES[a.dtype], a.stride(0), N.ptr(w), N.ptr(s),
           m, n, kp, N.DTYPE_CODES[out_dtype], N.ptr(out), n, N.ptr(ws), ws.numel(), N.stream(gpu))
    out = out.reshape(*lead, n)
    return out if host is None else out.to(host)


def mxfp8_linear_mx(source_q: torch.Tensor, source_scale: torch.Tensor, weight: torch.Tensor,
                    scale: torch.Tensor, *, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``dequant(source_q, source_scale) @ dequant(weight, scale).T`` for input
    rows already in MXFP8 (E4M3 [M, K], E8M0 [M, K/32], e.g. from
    ``mxfp8_quantize``), on the block-scaled fp8 matrix cores."""
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("out_dtype must be bfloat16 or float32")
    if source_q.ndim != 2:
        raise ValueError("source_q must be [M, K]")
    k = source_q.shape[1]
    if k % 32:
        raise ValueError(f"K={k} must be a multiple of 32 (the MX block)")
    if source_scale.dtype != torch.uint8 or tuple(source_scale.shape) != (source_q.shape[0], k // 32):
        raise ValueError(f"source_scale must be uint8 [{source_q.shape[0]}, {k // 32}]")
    (aq, as_, w, s), gpu, host = N.to_gpu([source_q.view(torch.uint8), source_scale, weight.view(torch.uint8), scale])
    w, s, kp = _mx_weight(w, s, k)
    aq, as_ = _pad_k(aq, kp).contiguous(), _pad_k(as_, kp // 32, 127).contiguous()
    aq, as_, w, s = N.aligned(aq), N.aligned(as_, 4), N.aligned(w), N.aligned(s, 4)
    m, n = aq.shape[0], w.shape[0]
    out = torch.empty(m, n, dtype=out_dtype, device=gpu)
    ws = torch.empty(max(int(N.library().kq_mx_linear_mx_workspace_size(m, n, kp)), 256), dtype=torch.uint8,
                     device=gpu)
    N.call("kq_mx_linear_mx", N.FMT_MXFP8_E4M3, N.ptr(aq), N.ptr(as_), kp, N.FMT_MXFP8_E4M3, N.ptr(w), N.ptr(s),
           m, n, kp, N.DTYPE_CODES[out_dtype], N.ptr(out), n, N.ptr(ws), ws.numel(), N.stream(gpu))
    return out if host is None else out.to(host)
