"""Packed official MXFP4 matrices and their device dequantization.

``PackedMXFP4Matrix`` and ``dequant_packed_matrix`` mirror
kquant/source_weights.py:35-40 and :139-150
(``OfficialMXFP4Store._dequant_packed_matrix``): the compact codes and E8M0
scales of one matrix, expanded to a contiguous fp32 matrix on the target
device.  The expansion is the ``kq_mx_dequant`` kernel; a CPU target is
computed on the GPU and copied back.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .io.mxfp4 import dequant


@dataclass(frozen=True)
class PackedMXFP4Matrix:
    """One official matrix in its original code-and-scale representation."""

    packed: torch.Tensor
    scale: torch.Tensor


def dequant_packed_matrix(
    raw: PackedMXFP4Matrix,
    *,
    device: torch.device | str | None = None,
) -> torch.Tensor:
    """fp32 [out, in] matrix of ``raw`` on ``device`` (default: the CPU)."""

    target = torch.device("cpu") if device is None else torch.device(device)
    if target.type == "cpu":
        return dequant(raw.packed, raw.scale)
    packed = raw.packed.to(device=target, non_blocking=True)
    scale = raw.scale.to(device=target, non_blocking=True)
    return dequant(packed, scale).contiguous()
