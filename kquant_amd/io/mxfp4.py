"""Codec for compressed-tensors ``mxfp4-pack-quantized`` expert weights.

Drop-in for ``kquant/io/mxfp4.py`` (same names, arguments, layouts, errors).

Storage:
  weight_packed: uint8 [out, K/2], two E2M1 codes per byte, low nibble = even
                 K index (compressed-tensors pack_fp4 convention);
  weight_scale:  uint8 [out, K/32], E8M0 exponent (value = 2^(byte-127)),
                 one scale per 32 consecutive K elements.

Every function runs a HIP kernel of ``libkquant_amd.so`` on the GPU.  CPU
inputs are processed on the current GPU and the result is returned on the
input's device.
"""

from __future__ import annotations

import torch

from .. import _native as N
from .. import constants as C

E2M1_VALUES = torch.tensor(C.E2M1_LUT, dtype=torch.float32)


def _finish(out: torch.Tensor, host: torch.device | None) -> torch.Tensor:
    return out if host is None else out.to(host)


def unpack_codes(packed: torch.Tensor) -> torch.Tensor:
    """uint8 [..., K/2] -> uint8 codes [..., K] (values 0..15).

    kquant/io/mxfp4.py:19-29.
    """
    if packed.dtype != torch.uint8:
        raise TypeError(f"expected uint8, got {packed.dtype}")
    (p,), gpu, host = N.to_gpu([packed])
    p = N.aligned(p)
    out = torch.empty(*packed.shape[:-1], packed.shape[-1] * 2, dtype=torch.uint8, device=gpu)
    N.call("kq_unpack_codes", N.ptr(p), p.numel(), N.ptr(out), N.stream(gpu))
    return _finish(out, host)


def pack_codes(codes: torch.Tensor) -> torch.Tensor:
    """uint8 codes [..., K] -> uint8 [..., K/2] (inverse of unpack_codes).

    kquant/io/mxfp4.py:32-38: byte = codes[0::2] | codes[1::2] << 4 (mod 256).
    """
    if codes.shape[-1] % 2:
        raise ValueError("K must be even")
    if codes.dtype != torch.uint8:
        # the reference ORs the operands in their own dtype before the uint8
        # cast; the kernel works on bytes
        codes = codes.to(torch.uint8)
    (c,), gpu, host = N.to_gpu([codes])
    c = N.aligned(c)
    out = torch.empty(*codes.shape[:-1], codes.shape[-1] // 2, dtype=torch.uint8, device=gpu)
    N.call("kq_pack_codes", N.ptr(c), c.numel(), N.ptr(out), N.stream(gpu))
    return _finish(out, host)


def _decode(table: int, values: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    (v,), gpu, host = N.to_gpu([values])
    v = N.aligned(v)
    out = torch.empty(values.shape, dtype=dtype, device=gpu)
    N.call("kq_decode_bytes", table, N.ptr(v), v.numel(), N.DTYPE_CODES[dtype], N.ptr(out),
           N.stream(gpu))
    return _finish(out, host)


def scale_factors(scale: torch.Tensor) -> torch.Tensor:
    """uint8 E8M0 [..., K/32] -> float32 2^(e-127).  kquant/io/mxfp4.py:41-43."""
    if scale.dtype != torch.uint8:
        raise TypeError(f"expected uint8 E8M0 scales, got {scale.dtype}")
    return _decode(N.TABLE_E8M0, scale)


def code_values(codes: torch.Tensor) -> torch.Tensor:
    """uint8 codes -> float32 E2M1 values (unscaled).  kquant/io/mxfp4.py:46-49."""
    if codes.dtype != torch.uint8:
        codes = codes.to(torch.uint8)
    if codes.numel() and int(codes.max()) >= 16:
        raise IndexError("E2M1 code out of range (codes must be 0..15)")
    return _decode(N.TABLE_E2M1, codes)


def _check_scale_blocks(packed: torch.Tensor, scale: torch.Tensor) -> int:
    k = packed.shape[-1] * 2
    if scale.shape[-1] * C.MXFP4_BLOCK != k:
        raise ValueError(
            f"scale blocks {scale.shape[-1]} do not cover K={k} at block {C.MXFP4_BLOCK}"
        )
    if scale.dtype != torch.uint8:
        raise TypeError(f"expected uint8 E8M0 scales, got {scale.dtype}")
    return k


def dequant(packed: torch.Tensor, scale: torch.Tensor, *, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Packed codes + E8M0 scales -> float32 weights [..., K].

    kquant/io/mxfp4.py:52-64.  ``dtype`` (bf16/fp16/fp32) is an extension: the
    fp32 result rounded to nearest even in the kernel, as
    scripts/closure_exl3_layer.py:157 does with ``.to(torch.bfloat16)``.
    """
    if packed.dtype != torch.uint8:
        raise TypeError(f"expected uint8, got {packed.dtype}")
    k = _check_scale_blocks(packed, scale)
    lead = torch.broadcast_shapes(packed.shape[:-1], scale.shape[:-1])
    packed = packed.expand(*lead, packed.shape[-1])
    scale = scale.expand(*lead, scale.shape[-1])
    (p, s), gpu, host = N.to_gpu([packed, scale])
    p, s = N.aligned(p), N.aligned(s)
    rows = p.numel() // max(p.shape[-1], 1) if p.shape[-1] else 0
    out = torch.empty(*lead, k, dtype=dtype, device=gpu)
    if k:
        N.call("kq_mx_dequant", N.FMT_MXFP4_E2M1, N.ptr(p), N.ptr(s), rows, k,
               N.DTYPE_CODES[dtype], N.ptr(out), 0, N.stream(gpu))
    return _finish(out, host)


def dequant_blocked(packed: torch.Tensor, scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Return (code_values [..., nb, 32] float32, scale_factors [..., nb]).

    kquant/io/mxfp4.py:67-79.
    """
    if packed.dtype != torch.uint8:
        raise TypeError(f"expected uint8, got {packed.dtype}")
    codes = unpack_codes(packed)
    vals = _decode(N.TABLE_E2M1, codes)
    s = scale_factors(scale)
    nb = s.shape[-1]
    vals = vals.view(*vals.shape[:-1], nb, C.MXFP4_BLOCK)
    return vals, s
