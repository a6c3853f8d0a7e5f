"""vLLM's serialized MXFP8 dense-weight format (E4M3 values, per-32 E8M0).

Drop-in for ``kquant/mxfp8.py``: ``mxfp8_quantize_cpu`` and
``mxfp8_dequantize_cpu`` keep the reference's names, validation, layouts and
CPU-resident results, but compute on the GPU with the HIP codec kernels.
``mxfp8_quantize`` / ``mxfp8_dequantize`` are the same operations returning on
the input's device.
"""

from __future__ import annotations

import torch

from . import _native as N

MXFP8_BLOCK_SIZE = 32
MXFP8_E4M3_MAX = 448.0


def _validate_weight(weight: torch.Tensor) -> None:
    # kquant/mxfp8.py:21-34
    if weight.ndim != 2:
        raise ValueError(
            f"MXFP8 requires a rank-2 weight, got shape={tuple(weight.shape)}"
        )
    if not weight.dtype.is_floating_point:
        raise TypeError(f"MXFP8 requires a floating-point weight, got {weight.dtype}")
    if weight.shape[1] % MXFP8_BLOCK_SIZE:
        raise ValueError(
            "MXFP8 input dimension must be divisible by "
            f"{MXFP8_BLOCK_SIZE}, got {weight.shape[1]}"
        )


def mxfp8_quantize(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize a rank-2 weight to (float8_e4m3fn [out, in], uint8 [out, in/32])
    on the weight's device, with kquant's rule (kquant/mxfp8.py:41-50):
    e = clamp(ceil(log2(max(amax,1e-30)/448)), -127, 128), byte = e + 127,
    q = e4m3(clamp(x / 2^e, +-448)).
    """

    _validate_weight(weight)
    out_features, in_features = weight.shape
    w = weight.detach()
    if w.dtype not in N.DTYPE_CODES:
        w = w.float()
    (w,), gpu, host = N.to_gpu([w])
    ld = w.stride(0) if w.stride(1) == 1 else None
    if ld is None or ld < in_features or (ld * w.element_size()) % 16 or w.data_ptr() % 16:
        w = N.aligned(w)
        ld = in_features
    q = torch.empty(out_features, in_features, dtype=torch.uint8, device=gpu)
    scale = torch.empty(out_features, in_features // MXFP8_BLOCK_SIZE, dtype=torch.uint8, device=gpu)
    if out_features and in_features:
        N.call("kq_mx_quantize", N.FMT_MXFP8_E4M3, N.DTYPE_CODES[w.dtype], N.ptr(w), ld,
               out_features, in_features, N.ptr(q), N.ptr(scale), 0, N.stream(gpu))
    q = q.view(torch.float8_e4m3fn)
    if host is not None:
        q, scale = q.to(host), scale.to(host)
    return q, scale


def mxfp8_quantize_cpu(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize a rank-2 weight to E4M3 values and per-32 E8M0 scales.

    kquant/mxfp8.py:11-51.  The returned layout is the one consumed by vLLM's
    serialized MXFP8 linear method: ``weight`` remains ``[out_features,
    in_features]`` and ``weight_scale`` is ``uint8[out_features, in_features /
    32]``; both are returned on the CPU as the reference does.  The
    arithmetic runs on the GPU.
    """

    q, scale = mxfp8_quantize(weight)
    return q.cpu(), scale.cpu()


def _validate_pair(weight: torch.Tensor, scale: torch.Tensor) -> None:
    # kquant/mxfp8.py:62-76
    if weight.ndim != 2:
        raise ValueError(
            f"MXFP8 requires a rank-2 weight, got shape={tuple(weight.shape)}"
        )
    out_features, in_features = weight.shape
    expected_scale_shape = (out_features, in_features // MXFP8_BLOCK_SIZE)
    if in_features % MXFP8_BLOCK_SIZE or tuple(scale.shape) != expected_scale_shape:
        raise ValueError(
            f"invalid MXFP8 scale shape {tuple(scale.shape)} for weight "
            f"shape {tuple(weight.shape)}; expected {expected_scale_shape}"
        )
    if scale.dtype != torch.uint8:
        raise TypeError(f"MXFP8 scales must be uint8, got {scale.dtype}")
    if weight.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError(f"MXFP8 weight must be float8_e4m3fn, got {weight.dtype}")


def mxfp8_dequantize(
    weight: torch.Tensor, scale: torch.Tensor, *, dtype: torch.dtype = torch.float32
) -> torch.Tensor:
    """E4M3 values x 2^(scale-127) on the input's device (kquant/mxfp8.py:79-84)."""

    _validate_pair(weight, scale)
    out_features, in_features = weight.shape
    (w, s), gpu, host = N.to_gpu([weight.view(torch.uint8), scale])
    w, s = N.aligned(w), N.aligned(s)
    kernel_dtype = dtype if dtype in N.DTYPE_CODES else torch.float32
    out = torch.empty(out_features, in_features, dtype=kernel_dtype, device=gpu)
    if out_features and in_features:
        N.call("kq_mx_dequant", N.FMT_MXFP8_E4M3, N.ptr(w), N.ptr(s), out_features, in_features,
               N.DTYPE_CODES[kernel_dtype], N.ptr(out), 0, N.stream(gpu))
    if kernel_dtype != dtype:
        out = out.to(dtype)
    return out if host is None else out.to(host)


def mxfp8_dequantize_cpu(
    weight: torch.Tensor,
    scale: torch.Tensor,
    *,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Dequantize the serialized MXFP8 layout (kquant/mxfp8.py:54-84).

    The result is returned on the CPU as the reference does.
    """

    return mxfp8_dequantize(weight, scale, dtype=dtype).cpu()
