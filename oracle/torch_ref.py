"""TEST INFRASTRUCTURE ONLY — torch-CPU restatements of the reference's CPU
formulas, used as the timed CPU baseline of bench.py and as checkers.

These follow the reference's own op sequences on torch's CPU kernels (the
reference's path is torch on CPU), so their timing is what the reference's
CPU path costs on the same host:
  mxfp8_quantize_cpu   kquant/mxfp8.py:34-50
  dequant_mxfp4        kquant/io/mxfp4.py:52-64
  weighted_covariance  kquant/candidate_hessian.py:92-107 (chunked fp32 addmm_)
"""

from __future__ import annotations

import torch

E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def mxfp8_quantize_cpu(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    out_features, in_features = weight.shape
    values = weight.detach().to(device="cpu", dtype=torch.float32).contiguous()
    blocks = values.view(out_features, in_features // 32, 32)
    amax = blocks.abs().amax(dim=-1)
    exponent = torch.ceil(torch.log2(amax.clamp(min=1e-30) / 448.0)).clamp(min=-127, max=128)
    scale = (exponent + 127.0).to(torch.uint8)
    quantized = (
        blocks.div(torch.exp2(exponent).unsqueeze(-1))
        .clamp(-448.0, 448.0)
        .view(out_features, in_features)
        .to(torch.float8_e4m3fn)
    )
    return quantized, scale


def dequant_mxfp4(packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    lo = packed & 0x0F
    hi = packed >> 4
    codes = torch.empty(*packed.shape[:-1], packed.shape[-1] * 2, dtype=torch.uint8)
    codes[..., 0::2] = lo
    codes[..., 1::2] = hi
    vals = E2M1[codes.long()]
    s = torch.exp2(scale.to(torch.float32) - 127)
    k = vals.shape[-1]
    vals = vals.view(*vals.shape[:-1], s.shape[-1], 32)
    return (vals * s.unsqueeze(-1)).view(*vals.shape[:-2], k)


def weighted_covariance(rows: torch.Tensor, weights: torch.Tensor, chunk_rows: int = 256) -> torch.Tensor:
    dimension = int(rows.shape[1])
    accumulator = torch.zeros((dimension, dimension), dtype=torch.float32)
    denominator = float(weights.double().sum())
    for begin in range(0, int(rows.shape[0]), chunk_rows):
        values = rows[begin : begin + chunk_rows].to(dtype=torch.float32)
        local_weights = weights[begin : begin + chunk_rows].to(dtype=torch.float32)
        accumulator.addmm_(values.T, values * local_weights[:, None])
    covariance = accumulator.div_(denominator)
    return ((covariance + covariance.T) * 0.5).contiguous()
