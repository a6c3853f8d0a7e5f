"""MXFP4 (E2M1 + E8M0, 32-element blocks) quantizer.

kquant has no MXFP4 quantizer: its MXFP4 weights arrive pre-quantized in the
compressed-tensors ``mxfp4-pack-quantized`` layout (kquant/io/mxfp4.py:1-8).
This module freezes one rule for producing that layout: kquant's own MXFP8
rule (kquant/mxfp8.py:41-50) with (E4M3, 448) replaced by (E2M1, 6.0):

    e     = clamp(ceil(log2(max(amax, 1e-30) / 6)), -127, 128)
    scale = uint8(e + 127)
    code  = E2M1 round-to-nearest-even of clamp(x / 2^e, -6, 6), sign kept
            (negative values that round to zero give code 8, -0)

and packs codes with kquant's ``pack_codes`` convention (low nibble = even K).
"""

from __future__ import annotations

import torch

from . import _native as N
from .constants import MXFP4_BLOCK

MXFP4_E2M1_MAX = 6.0


def mxfp4_quantize(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize ``[..., K]`` floating weights to (packed uint8 [..., K/2],
    E8M0 scale uint8 [..., K/32]) on the input's device.

    Validation mirrors ``mxfp8_quantize_cpu`` (kquant/mxfp8.py:21-34), except
    that leading batch dimensions (stacked experts) are accepted.
    """

    if weight.ndim < 2:
        raise ValueError(
            f"MXFP4 requires a rank>=2 weight, got shape={tuple(weight.shape)}"
        )
    if not weight.dtype.is_floating_point:
        raise TypeError(f"MXFP4 requires a floating-point weight, got {weight.dtype}")
    k = weight.shape[-1]
    if k % MXFP4_BLOCK:
        raise ValueError(
            f"MXFP4 input dimension must be divisible by {MXFP4_BLOCK}, got {k}"
        )
    w = weight.detach()
    if w.dtype not in N.DTYPE_CODES:
        w = w.float()
    (w,), gpu, host = N.to_gpu([w])
    w = N.aligned(w)
    rows = w.numel() // k if k else 0
    packed = torch.empty(*weight.shape[:-1], k // 2, dtype=torch.uint8, device=gpu)
    scale = torch.empty(*weight.shape[:-1], k // MXFP4_BLOCK, dtype=torch.uint8, device=gpu)
    if rows and k:
        N.call("kq_mx_quantize", N.FMT_MXFP4_E2M1, N.DTYPE_CODES[w.dtype], N.ptr(w), k, rows, k,
               N.ptr(packed), N.ptr(scale), 0, N.stream(gpu))
    if host is not None:
        packed, scale = packed.to(host), scale.to(host)
    return packed, scale
