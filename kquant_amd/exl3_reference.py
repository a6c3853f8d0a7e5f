"""The QSRT/EXL3 trellis decode of ``kquant/exl3_reference.py``, on the GPU.

Same names, arguments and results as the reference's pure-PyTorch
operations:

  ``reconstruct_trellis_states(edge_symbols, bits)`` (:37-61)
      cyclic 16-bit states of K-bit edges (``kq_trellis_pack`` then
      ``kq_trellis_unpack``: the packed stream holds exactly the edges);
  ``tensor_core_permutation(device)`` (:88-108);
  ``decode_regularized_weight`` (:110-147), ``decode_qsrt_regularized_weight``
  (:149-192), ``decode_exl3_weight`` (:243-267), ``decode_qsrt_weight``
  (:270-295), ``normalized_hadamard`` (:195-212)
      one launch per matrix (``kq_qsrt_decode_states``): labels, the
      tensor-core order, the [K, N] layout and, for the full decodes, the
      blockwise Hadamard rotation with suh / svh in LDS.

Decodes run on the GPU with the states' device kept for the result; the
codebook must be one of the named SQG tables, or a custom table whose values
are all E4M3 numbers (as ``sqg_e4m3_codebook`` tables are).  K and N must be
multiples of 128 for the rotated decodes, of 16 otherwise.
"""

from __future__ import annotations

import math

import torch

from . import _native as N
from .qsrt import pack_trellis_edges, unpack_trellis_states
from .sqg_e4m3 import (
    SQG_CHEB,
    SQG_CHEB_NORMAL_E4M3,
    SQG_NORMAL_E4M3,
    SQG_XOR_CHEB_T12,
    sqg_codebook_bytes,
)

TILE_VALUES = 256
HADAMARD_BLOCK = 128
CODEBOOK_SQG_NORMAL_E4M3 = SQG_NORMAL_E4M3
CODEBOOK_SQG_XOR_CHEB_T12 = SQG_XOR_CHEB_T12
CODEBOOK_SQG_CHEB_NORMAL_E4M3 = SQG_CHEB_NORMAL_E4M3
CODEBOOK_SQG_CHEB = SQG_CHEB
QSRT_CODEBOOKS = (
    CODEBOOK_SQG_XOR_CHEB_T12,
    CODEBOOK_SQG_NORMAL_E4M3,
    CODEBOOK_SQG_CHEB_NORMAL_E4M3,
    CODEBOOK_SQG_CHEB,
)


def _validate_bits(bits: int) -> None:
    if isinstance(bits, bool) or not isinstance(bits, int) or bits not in (2, 3, 4):
        raise ValueError("the QSRT reference supports K=2, K=3, or K=4")


def reconstruct_trellis_states(edge_symbols: torch.Tensor, bits: int) -> torch.Tensor:
    """Recover cyclic 16-bit trellis states from their stored K-bit edges."""

    _validate_bits(bits)
    if edge_symbols.ndim < 1 or edge_symbols.shape[-1] != TILE_VALUES:
        raise ValueError("edge_symbols must have a final dimension of 256")
    if edge_symbols.dtype == torch.bool or edge_symbols.is_floating_point():
        raise TypeError("edge_symbols must use an integer dtype")
    return unpack_trellis_states(pack_trellis_edges(edge_symbols, bits), bits)


def tensor_core_permutation(device: torch.device | str = "cpu") -> torch.Tensor:
    """The native EXL 16x16 row-major -> tensor-core element order."""

    t = torch.arange(TILE_VALUES, dtype=torch.long, device=device)
    thread, j = t // 8, t % 8
    row0 = (thread % 4) * 2
    rsel = j % 4
    rows = row0 + (rsel % 2) + 8 * (rsel // 2)
    return rows * 16 + thread // 4 + 8 * (j // 4)


def normalized_hadamard(*, device: torch.device | str, dtype: torch.dtype = torch.float32,
                        size: int = HADAMARD_BLOCK) -> torch.Tensor:
    if size <= 0 or size & (size - 1):
        raise ValueError("Hadamard size must be a positive power of two")
    i = torch.arange(size, device=device)
    bits = torch.bitwise_and(i[:, None], i[None, :])
    parity = torch.zeros_like(bits)
    for shift in range(int(math.log2(size)) + 1):
        parity ^= (bits >> shift) & 1
    return (1 - 2 * parity).to(dtype) * (1.0 / math.sqrt(size))


def _labels(codebook: str, bits_needed, rate_axis, codebook_values, device) -> torch.Tensor:
    """uint8 [3, 65536] labels for K2..K4 on ``device`` (only the rates in use are built)."""
    table = torch.zeros(3, 1 << 16, dtype=torch.uint8, device=device)
    if codebook_values is not None:
        if codebook_values.ndim != 1 or codebook_values.numel() != 1 << 16:
            raise ValueError("custom codebook must contain exactly 65,536 values")
        if not codebook_values.is_floating_point():
            raise TypeError("custom codebook must be floating point")
        if not bool(torch.isfinite(codebook_values).all()):
            raise ValueError("custom codebook must be finite")
        values = codebook_values.to(device=device, dtype=torch.float32)
        raw = values.to(torch.float8_e4m3fn)
        if not torch.equal(raw.float(), values):
            raise ValueError("custom codebook values must be E4M3 numbers for the GPU decoder")
        table[:] = raw.view(torch.uint8)
        return table
    if codebook not in QSRT_CODEBOOKS:
        raise ValueError(f"unsupported QSRT codebook {codebook!r}; expected one of {QSRT_CODEBOOKS}")
    for bits in sorted(set(bits_needed)):
        table[bits - 2] = sqg_codebook_bytes(bits, codebook, rate_axis=rate_axis, device=device)
    return table


def _decode(states: torch.Tensor, tile_bits, rate_axis: str, codebook: str, codebook_values,
            suh=None, svh=None) -> torch.Tensor:
    if states.ndim != 3 or states.shape[-1] != TILE_VALUES:
        raise ValueError("states must have shape [K/16, N/16, 256]")
    k_tiles, n_tiles, _ = states.shape
    (s,), gpu, host = N.to_gpu([states])
    s = N.aligned((s.to(torch.int64) & 0xFFFF).to(torch.int16) if s.dtype != torch.int16 else s, 2)
    rotate = suh is not None
    pad_k = (-k_tiles) % 8
    pad_n = (-n_tiles) % 8
    if rotate and (pad_k or pad_n):
        raise ValueError("EXL K and N dimensions must be divisible by 128")
    if pad_k or pad_n:  # the kernel decodes 128 x 128 blocks; padding tiles decode to values dropped below
        s = torch.nn.functional.pad(s, (0, 0, 0, pad_n, 0, pad_k))
    rate_tiles = s.shape[0] if rate_axis == "k" else s.shape[1]
    bits = list(tile_bits) + [tile_bits[-1]] * (rate_tiles - len(tile_bits))
    tb = torch.tensor(bits, dtype=torch.uint8, device=gpu)
    labels = _labels(codebook, tile_bits, rate_axis, codebook_values, gpu)
    kt, nt = s.shape[0], s.shape[1]
    out = torch.empty(kt * 16, nt * 16, dtype=torch.float32, device=gpu)
    su = sv = None
    if rotate:
        su = N.aligned(suh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
        sv = N.aligned(svh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
    N.call("kq_qsrt_decode_states", N.ptr(s), kt, nt, 0 if rate_axis == "k" else 1, N.ptr(tb), N.ptr(labels),
           N.ptr(su), N.ptr(sv), N.DT_F32, N.ptr(out), nt * 16, 0, N.stream(gpu))
    out = out[: k_tiles * 16, : n_tiles * 16].contiguous()
    return out if host is None else out.to(host)


def decode_regularized_weight(states: torch.Tensor, *, codebook: str = CODEBOOK_SQG_XOR_CHEB_T12,
                              codebook_values: torch.Tensor | None = None, bits: int | None = None) -> torch.Tensor:
    """Decode ``[K/16, N/16, 256]`` states to transformed ``[K, N]``."""

    if states.ndim != 3 or states.shape[-1] != TILE_VALUES:
        raise ValueError("states must have shape [K/16, N/16, 256]")
    if codebook_values is None:
        if codebook not in QSRT_CODEBOOKS:
            raise ValueError(f"unsupported QSRT codebook {codebook!r}; expected one of {QSRT_CODEBOOKS}")
        if bits is None:
            raise ValueError("SQG reconstruction requires an explicit trellis rate")
        _validate_bits(bits)
        return _decode(states, (bits,) * states.shape[0], "k", codebook, None)
    return _decode(states, (2,) * states.shape[0], "k", codebook, codebook_values)


def _tile_bits(states: torch.Tensor, rate_axis: str, tile_bits) -> tuple[int, ...]:
    if states.ndim != 3 or states.shape[-1] != TILE_VALUES:
        raise ValueError("states must have shape [K/16, N/16, 256]")
    if rate_axis not in ("k", "n"):
        raise ValueError("rate_axis must be 'k' or 'n'")
    axis = 0 if rate_axis == "k" else 1
    if len(tile_bits) != states.shape[axis]:
        raise ValueError("tile_bits length does not match the selected rate axis")
    if any(isinstance(v, bool) or not isinstance(v, int) or v not in (2, 3, 4) for v in tile_bits):
        raise ValueError("tile_bits must contain only integer K2, K3, or K4")
    return tuple(tile_bits)


def decode_qsrt_regularized_weight(states: torch.Tensor, *, rate_axis: str, tile_bits: tuple[int, ...],
                                   codebook: str) -> torch.Tensor:
    """Decode a K2/K3/K4 tile map to transformed ``[K, N]`` weights."""

    bits = _tile_bits(states, rate_axis, tile_bits)
    if codebook not in QSRT_CODEBOOKS:
        raise ValueError(f"unsupported QSRT codebook: {codebook}")
    return _decode(states, bits, rate_axis, codebook, None)


def _scales(weight_shape, suh, svh):
    if suh.ndim != 1 or suh.numel() != weight_shape[0]:
        raise ValueError("suh length does not match the EXL K dimension")
    if svh.ndim != 1 or svh.numel() != weight_shape[1]:
        raise ValueError("svh length does not match the EXL N dimension")


def decode_exl3_weight(states: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, *,
                       codebook: str = CODEBOOK_SQG_XOR_CHEB_T12, codebook_values: torch.Tensor | None = None,
                       bits: int | None = None) -> torch.Tensor:
    """Decode stored states/scales to an EXL-oriented ``[K, N]`` weight."""

    if states.ndim != 3 or states.shape[-1] != TILE_VALUES:
        raise ValueError("states must have shape [K/16, N/16, 256]")
    _scales((states.shape[0] * 16, states.shape[1] * 16), suh, svh)
    if codebook_values is None:
        if bits is None:
            raise ValueError("SQG reconstruction requires an explicit trellis rate")
        _validate_bits(bits)
        return _decode(states, (bits,) * states.shape[0], "k", codebook, None, suh, svh)
    return _decode(states, (2,) * states.shape[0], "k", codebook, codebook_values, suh, svh)


def decode_qsrt_weight(states: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, *, rate_axis: str,
                       tile_bits: tuple[int, ...], codebook: str = CODEBOOK_SQG_XOR_CHEB_T12) -> torch.Tensor:
    """Decode stored QSRT states and scales to an EXL ``[K, N]`` weight."""

    bits = _tile_bits(states, rate_axis, tile_bits)
    if codebook not in QSRT_CODEBOOKS:
        raise ValueError(f"unsupported QSRT codebook: {codebook}")
    _scales((states.shape[0] * 16, states.shape[1] * 16), suh, svh)
    return _decode(states, bits, rate_axis, codebook, None, suh, svh)
