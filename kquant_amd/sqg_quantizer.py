"""SQG trellis quantizer on the GPU (the reference's one native kernel).

``kquant/sqg_quantizer.py`` builds ``kquant/csrc/sqg_quantize.cu`` as a torch
extension and patches an EXL encoder module's ``quantize_tiles`` to run the
SQG Viterbi search.  Here the search is ``kq_sqg_quantize_tiles`` in
``libkquant_amd.so`` (same fp16 arithmetic, decision packing and tie order,
so the same states and values) and:

  ``quantize_tiles_sqg(tiles, lut, bits, tailbite_context)``
      the extension call (``quantize_tiles_sqg``, sqg_quantize.cu:165-342):
      fp32 tiles [N, 256] and 65,536 E4M3 state labels -> (values fp32
      [N, 256], states int16 [N, 256]);
  ``install_sqg_quantizer(quantizer_module)`` (sqg_quantizer.py:64-164)
      the same patch, with the same argument checks and messages, routing the
      SQG laws to that kernel and a ``None`` entry of ``sqg_e4m3_luts_by_bits``
      to the MCG control;
  ``quantize_tiles_procedural(tiles, bits, codebook, tailbite_context)``
      the extension call ``quantize_tiles_procedural`` (sqg_quantize.cu:
      261-330): the same search against the procedural EXL3 codebooks,
      1 = MCG, 2 = MUL1 (kquant/csrc/exl3_compat/quant/codebook.cuh:27-92),
      whose labels the kernel computes per state.
"""

from __future__ import annotations

from collections.abc import Mapping

import torch

from . import _native as N
from .sqg_e4m3 import sqg_e4m3_bytes

_WORKSPACES: dict[tuple[torch.device, int, int], torch.Tensor] = {}


def _workgroups(device: torch.device) -> int:
    return torch.cuda.get_device_properties(device).multi_processor_count


def quantize_tiles_sqg(tiles: torch.Tensor, lut: torch.Tensor, bits: int,
                       tailbite_context: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Trellis-quantize fp32 tiles [N, 256] against SQG E4M3 labels."""

    if not tiles.is_cuda:
        raise ValueError("input_tiles must be CUDA")
    if tiles.dtype != torch.float32:
        raise ValueError("input_tiles must be FP32")
    if tiles.ndim != 2 or tiles.shape[1] != 256:
        raise ValueError("input_tiles must have shape [tiles, 256]")
    if bits not in (2, 3, 4):
        raise ValueError("SQG validation kernel supports K2--K4")
    if not 1 <= tailbite_context <= 128:
        raise ValueError("tailbite_context must be in 1..128")
    if lut.dtype != torch.uint8 or lut.numel() != 65536:
        raise ValueError("codebook must contain 65,536 uint8 E4M3 values")
    device = tiles.device
    x = N.aligned(tiles.contiguous(), 4)
    table = N.aligned(lut.to(device=device).contiguous(), 16)
    out = torch.empty_like(x)
    states = torch.empty(x.shape, dtype=torch.int16, device=device)
    ws = _workspace(device, bits)
    N.call("kq_sqg_quantize_tiles", N.ptr(x), x.shape[0], N.ptr(table), bits, int(tailbite_context), N.ptr(out),
           N.ptr(states), N.ptr(ws), ws.numel(), _workgroups(device), N.stream(device))
    return out, states


def _workspace(device: torch.device, bits: int) -> torch.Tensor:
    """Decision workspace, one per (device, stream, rate)."""
    need = int(N.library().kq_sqg_quantize_workspace_size(bits, _workgroups(device)))
    key = (device, torch.cuda.current_stream(device).stream_id, bits)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def quantize_tiles_procedural(tiles: torch.Tensor, bits: int, codebook: int,
                              tailbite_context: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Trellis-quantize fp32 tiles [N, 256] against the MCG (1) or MUL1 (2)
    procedural codebook."""

    if not tiles.is_cuda:
        raise ValueError("input_tiles must be CUDA")
    if tiles.dtype != torch.float32:
        raise ValueError("input_tiles must be FP32")
    if tiles.ndim != 2 or tiles.shape[1] != 256:
        raise ValueError("input_tiles must have shape [tiles, 256]")
    if bits not in (2, 3, 4):
        raise ValueError("procedural control supports K2--K4")
    if codebook not in (1, 2):
        raise ValueError("procedural codebook must be 1 (MCG) or 2 (MUL1)")
    if not 1 <= tailbite_context <= 128:
        raise ValueError("tailbite_context must be in 1..128")
    device = tiles.device
    x = N.aligned(tiles.contiguous(), 4)
    out = torch.empty_like(x)
    states = torch.empty(x.shape, dtype=torch.int16, device=device)
    ws = _workspace(device, bits)
    N.call("kq_sqg_quantize_tiles_procedural", N.ptr(x), x.shape[0], bits, codebook, int(tailbite_context),
           N.ptr(out), N.ptr(states), N.ptr(ws), ws.numel(), _workgroups(device), N.stream(device))
    return out, states


def install_sqg_quantizer(quantizer_module) -> None:
    """Teach a loaded EXL encoder module to consume ``sqg_e4m3_lut``
    (kquant/sqg_quantizer.py:64-164); process-local, idempotent."""

    if getattr(quantizer_module, "_kquant_sqg_installed", False):
        return
    original = quantizer_module.quantize_tiles
    device_luts: dict[tuple[str, int, str], torch.Tensor] = {}

    def quantize_tiles(tiles: torch.Tensor, quant_args: dict):
        codebook = quant_args.get("sqg_e4m3_lut")
        rate_codebooks = quant_args.get("sqg_e4m3_luts_by_bits")
        mode = quant_args.get("sqg_e4m3_mode")
        if codebook is None and rate_codebooks is None and mode is None:
            return original(tiles, quant_args)
        if len(quant_args["devices"]) != 1:
            raise ValueError("the SQG validation hook currently requires one CUDA device")
        tiles = tiles.contiguous()
        if tiles.dtype != torch.float32 or tiles.ndim != 2 or tiles.shape[1] != 256:
            raise ValueError("SQG tiles must be contiguous FP32 [N, 256]")
        bits = int(quant_args["K"])
        if rate_codebooks is not None:
            if codebook is not None or mode is not None:
                raise ValueError("rate-specific SQG LUTs cannot be combined with another SQG law")
            if not isinstance(rate_codebooks, Mapping):
                raise TypeError("sqg_e4m3_luts_by_bits must be a mapping")
            if set(rate_codebooks) - {2, 3, 4}:
                raise ValueError("rate-specific SQG LUT keys must be K2, K3, or K4")
            try:
                codebook = rate_codebooks[bits]
            except KeyError as exc:
                raise ValueError(f"missing rate-specific SQG K{bits} LUT") from exc
            if codebook is None:  # the MCG control
                return quantize_tiles_procedural(tiles, bits, 1, int(quant_args.get("tailbite_context", 128)))
        elif codebook is None:
            if mode != "normal":
                raise ValueError("the supported R44 mode is 'normal'")
            key = (str(tiles.device), bits, mode)
            codebook = device_luts.get(key)
            if codebook is None:
                codebook = sqg_e4m3_bytes(bits, mode, device=tiles.device)
                device_luts[key] = codebook
        lut = codebook.to(device=tiles.device, dtype=torch.uint8).contiguous()
        return quantize_tiles_sqg(tiles, lut, bits, int(quant_args.get("tailbite_context", 128)))

    quantizer_module.quantize_tiles = quantize_tiles
    quantizer_module._kquant_sqg_installed = True
