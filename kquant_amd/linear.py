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
