"""TEST INFRASTRUCTURE ONLY — torch-CPU restatements of the reference's CPU
formulas, used as the timed CPU baseline of bench.py and as checkers.

These follow the reference's own op sequences on torch's CPU kernels (the
reference's path is torch on CPU), so their timing is what the reference's
CPU path costs on the same host:
  mxfp8_quantize_cpu   kquant/mxfp8.py:34-50
  dequant_mxfp4        kquant/io/mxfp4.py:52-64
  weighted_covariance  kquant/candidate_hessian.py:92-107 (chunked fp32 addmm_)
  mxfp8_dequantize_cpu kquant/mxfp8.py:79-84
  reference_rank       scripts/closure_exl3_layer.py:557-598 (fp32 operands)
  mxfp4_quantize_cpu   no reference exists: the frozen MXFP4 rule (kquant/mxfp8.py:
                       41-50 with E2M1 and 6.0) on the same torch CPU ops
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


# E2M1 magnitudes, the midpoints between neighbours, and for each midpoint
# whether a tie goes to the lower code (the even one)
_E2M1_MAG = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
_E2M1_MID = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
_E2M1_TIE_LOWER = torch.tensor([True, False, True, False, True, False, True])


def mxfp4_quantize_cpu(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """packed u8 [N, K/2] (low nibble = even k) and E8M0 u8 [N, K/32]: the
    MXFP8 rule with E2M1 (max 6.0), nearest code with ties to the even code."""
    out_features, in_features = weight.shape
    values = weight.detach().to(device="cpu", dtype=torch.float32).contiguous()
    blocks = values.view(out_features, in_features // 32, 32)
    amax = blocks.abs().amax(dim=-1)
    exponent = torch.ceil(torch.log2(amax.clamp(min=1e-30) / 6.0)).clamp(min=-127, max=128)
    scale = (exponent + 127.0).to(torch.uint8)
    y = blocks.div(torch.exp2(exponent).unsqueeze(-1)).clamp(-6.0, 6.0).view(out_features, in_features)
    a = y.abs()
    code = torch.bucketize(a, _E2M1_MID, right=True)  # ties to the upper code here
    tie = (code > 0) & (a == _E2M1_MID[(code - 1).clamp(min=0)]) & _E2M1_TIE_LOWER[(code - 1).clamp(min=0)]
    code = (code - tie.to(code.dtype)).to(torch.uint8) | (torch.signbit(y).to(torch.uint8) << 3)
    packed = code[:, 0::2] | (code[:, 1::2] << 4)
    return packed, scale


def mxfp8_dequantize_cpu(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    values = q.to(torch.float32)
    n, k = values.shape
    s = torch.exp2(scale.to(torch.float32) - 127.0)
    return (values.view(n, k // 32, 32) * s.unsqueeze(-1)).view(n, k)


def situ(gate: torch.Tensor, up: torch.Tensor, beta: float = 4.0, linear_beta: float = 25.0) -> torch.Tensor:
    gate_value = beta * torch.tanh(gate.float() / beta) * torch.sigmoid(gate.float())
    up_value = linear_beta * torch.tanh(up.float() / linear_beta)
    return (gate_value * up_value).to(gate.dtype)


def reference_rank(x: torch.Tensor, route_ids: torch.Tensor, route_weights: torch.Tensor,
                   weights: dict[int, tuple[torch.Tensor, torch.Tensor]]) -> torch.Tensor:
    """The routed-expert loop of _reference_rank (tp 1) over the experts in
    ``weights`` (expert id -> (w13 [2I, H] gate rows first, w2 [H, I]),
    dequantized), fp32 operands; other experts are skipped."""
    output = torch.zeros(x.shape[0], next(iter(weights.values()))[1].shape[0], dtype=torch.float32)
    for expert, (w13, w2) in weights.items():
        selected = (route_ids == expert).nonzero(as_tuple=False)
        if selected.numel() == 0:
            continue
        token_ids = selected[:, 0]
        inter = w13.shape[0] // 2
        rows = x[token_ids]
        gate = torch.nn.functional.linear(rows, w13[:inter])
        up = torch.nn.functional.linear(rows, w13[inter:])
        partial = torch.nn.functional.linear(situ(gate, up), w2)
        output.index_add_(0, token_ids, route_weights[token_ids, selected[:, 1]].unsqueeze(1) * partial)
    return output
