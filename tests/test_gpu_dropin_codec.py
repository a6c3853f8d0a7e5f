"""The drop-in Python surface (kquant names) on the GPU, checked against the
oracle and the reference's own known answers (tests/test_mxfp4.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import constants as C
from kquant_amd import mxfp4 as kq_mxfp4
from kquant_amd import mxfp8
from kquant_amd.io import mxfp4

pytestmark = pytest.mark.gpu


def test_reference_mxfp4_known_answers_on_gpu(gpu):
    # tests/test_mxfp4.py:7-40 with the same seeded inputs
    g = torch.Generator().manual_seed(0)
    codes = torch.randint(0, 16, (7, 64), dtype=torch.uint8, generator=g)
    assert torch.equal(mxfp4.unpack_codes(mxfp4.pack_codes(codes)), codes)
    assert mxfp4.unpack_codes(torch.tensor([[0x21]], dtype=torch.uint8)).tolist() == [[1, 2]]
    codes = torch.zeros(1, 32, dtype=torch.uint8)
    codes[0, 0], codes[0, 1] = 7, 15
    w = mxfp4.dequant(mxfp4.pack_codes(codes), torch.full((1, 1), C.E8M0_BIAS + 1, dtype=torch.uint8))
    assert w.device.type == "cpu" and w.dtype == torch.float32
    assert w[0, 0].item() == 12.0 and w[0, 1].item() == -12.0 and w[0, 2].item() == 0.0
    g = torch.Generator().manual_seed(1)
    codes = torch.randint(0, 16, (3, 5, 96), dtype=torch.uint8, generator=g)
    packed = mxfp4.pack_codes(codes)
    scale = torch.randint(100, 140, (3, 5, 3), dtype=torch.uint8, generator=g)
    w1 = mxfp4.dequant(packed, scale)
    vals, s = mxfp4.dequant_blocked(packed, scale)
    assert torch.equal(w1, (vals * s.unsqueeze(-1)).reshape(w1.shape))


def test_gpu_tensors_stay_on_gpu(gpu):
    packed = torch.randint(0, 256, (16, 64), dtype=torch.uint8, device=gpu)
    scale = torch.randint(100, 140, (16, 4), dtype=torch.uint8, device=gpu)
    w = mxfp4.dequant(packed, scale)
    assert w.is_cuda
    ref = oracle.mx_dequant("mxfp4", packed.cpu().numpy(), scale.cpu().numpy())
    assert np.array_equal(w.cpu().numpy(), ref)
    assert torch.equal(mxfp4.scale_factors(scale).cpu(), torch.exp2(scale.cpu().float() - 127))
    codes = mxfp4.unpack_codes(packed)
    assert torch.equal(mxfp4.code_values(codes).cpu(), torch.tensor(C.E2M1_LUT)[codes.cpu().long()])


def test_mxfp8_quantize_cpu_contract(gpu):
    w = (torch.randn(64, 256, generator=torch.Generator().manual_seed(3)) * 0.02).to(torch.bfloat16)
    q, s = mxfp8.mxfp8_quantize_cpu(w)
    assert q.device.type == "cpu" and q.dtype == torch.float8_e4m3fn and q.shape == (64, 256)
    assert s.device.type == "cpu" and s.dtype == torch.uint8 and s.shape == (64, 8)
    rq, rs = oracle.mx_quantize("mxfp8", w.view(torch.int16).numpy().view(np.uint16), "bf16")
    assert np.array_equal(q.view(torch.uint8).numpy(), rq) and np.array_equal(s.numpy(), rs)
    d = mxfp8.mxfp8_dequantize_cpu(q, s)
    assert d.device.type == "cpu" and np.array_equal(d.numpy(), oracle.mx_dequant("mxfp8", rq, rs))
    d16 = mxfp8.mxfp8_dequantize_cpu(q, s, dtype=torch.bfloat16)
    assert torch.equal(d16, d.to(torch.bfloat16))


def test_mxfp4_quantize_stacked_experts(gpu):
    w = (torch.randn(3, 64, 256, generator=torch.Generator().manual_seed(4)) * 0.02).to(torch.bfloat16)
    packed, scale = kq_mxfp4.mxfp4_quantize(w.to(gpu))
    assert packed.shape == (3, 64, 128) and scale.shape == (3, 64, 8) and packed.is_cuda
    rq, rs = oracle.mx_quantize("mxfp4", w.reshape(192, 256).view(torch.int16).numpy().view(np.uint16), "bf16")
    assert np.array_equal(packed.reshape(192, 128).cpu().numpy(), rq)
    assert np.array_equal(scale.reshape(192, 8).cpu().numpy(), rs)
