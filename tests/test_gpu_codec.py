"""GPU parity of the MX codec kernels against the CPU oracle (bit-exact).

Both conversion paths of the kernels are covered: the gfx950 scaled convert
instructions (default) and the bit-level software rounding
(KQ_FLAG_SOFTWARE_CVT).  Inputs: every finite bf16 value under a sweep of
block scales, random blocks with planted ties and zeros, the benchmark
configurations at full size, fp16/fp32 inputs and strided rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from kquant_amd import _native as N
from kquant_amd import workloads
from tests import codec_cases as cases

pytestmark = pytest.mark.gpu

FMTS = {"mxfp8": N.FMT_MXFP8_E4M3, "mxfp4": N.FMT_MXFP4_E2M1}


def _quantize(fmt: str, x: torch.Tensor, flags: int = 0, ld: int | None = None, k: int | None = None):
    rows = x.shape[0]
    k = k if k is not None else x.shape[1]
    ld = ld if ld is not None else x.stride(0)
    q = torch.empty(rows, k if fmt == "mxfp8" else k // 2, dtype=torch.uint8, device=x.device)
    s = torch.empty(rows, k // 32, dtype=torch.uint8, device=x.device)
    N.call("kq_mx_quantize", FMTS[fmt], N.DTYPE_CODES[x.dtype], N.ptr(x), ld, rows, k,
           N.ptr(q), N.ptr(s), flags, N.stream(x.device))
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def _dequant(fmt: str, q: torch.Tensor, s: torch.Tensor, k: int, dtype, flags: int = 0):
    rows = q.shape[0]
    out = torch.empty(rows, k, dtype=dtype, device=q.device)
    N.call("kq_mx_dequant", FMTS[fmt], N.ptr(q), N.ptr(s), rows, k, N.DTYPE_CODES[dtype],
           N.ptr(out), flags, N.stream(q.device))
    torch.cuda.synchronize()
    return out.cpu()


def _bits_tensor(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


@pytest.mark.parametrize("flags", [0, N.FLAG_SOFTWARE_CVT], ids=["hw", "sw"])
@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_quantize_exhaustive_bf16(gpu, fmt, flags):
    span = (8, 12) if fmt == "mxfp8" else (2, 4)
    qmax = 448.0 if fmt == "mxfp8" else 6.0
    bits = np.concatenate([cases.exhaustive_scale_blocks(qmax, *span), cases.random_blocks_bf16(30_000)])
    pad = (-bits.shape[0]) % 8
    bits = np.concatenate([bits, np.zeros((pad, 32), np.uint16)]).reshape(-1, 256)
    print(f"case quantize {fmt} flags={flags} blocks={bits.size // 32}", flush=True)
    q, s = _quantize(fmt, _bits_tensor(bits, gpu), flags)
    rq, rs = oracle.mx_quantize(fmt, bits, "bf16")
    assert np.array_equal(s, rs), f"scale mismatches: {np.count_nonzero(s != rs)}"
    assert np.array_equal(q, rq), f"code mismatches: {np.count_nonzero(q != rq)}"


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_scale_of_every_finite_amax(gpu, fmt, dtype):
    """Every finite bf16 / fp16 value (both signs) as the largest magnitude of
    a block of its own: the block exponent is derived from the value's bits
    (no division) and must match the oracle's fl(amax / qmax) exponent on each
    one, including the values whose significand equals, or sits one step
    above or below, that of qmax."""
    if dtype == "bf16":
        mags = cases.finite_bf16_patterns()
        mags = mags[mags < 0x8000]
    else:
        mags = np.arange(0x7C00, dtype=np.uint16)  # +0 .. largest finite fp16
    vals = np.concatenate([mags, mags | 0x8000])
    blocks = np.zeros((vals.size, 32), np.uint16)
    blocks[:, 0] = vals
    blocks[:, 1] = ((vals & 0x7FFF) >> 1) | (vals & 0x8000)  # a second value of smaller magnitude
    pad = (-blocks.shape[0]) % 8
    blocks = np.concatenate([blocks, np.zeros((pad, 32), np.uint16)]).reshape(-1, 256)
    print(f"case scale-of-every-amax {fmt} {dtype} blocks={blocks.size // 32}", flush=True)
    if dtype == "bf16":
        x = _bits_tensor(blocks, gpu)
        rq, rs = oracle.mx_quantize(fmt, blocks, "bf16")
    else:
        h = blocks.view(np.float16)
        x = torch.from_numpy(h.copy()).to(gpu)
        rq, rs = oracle.mx_quantize(fmt, h, "f16")
    q, s = _quantize(fmt, x)
    assert np.array_equal(s, rs), f"scale mismatches: {np.count_nonzero(s != rs)}"
    assert np.array_equal(q, rq), f"code mismatches: {np.count_nonzero(q != rq)}"


@pytest.mark.parametrize("flags", [0, N.FLAG_SOFTWARE_CVT], ids=["hw", "sw"])
def test_cfg1_mxfp4_roundtrip_bit_exact(gpu, flags):
    w = workloads.cfg1_weight()
    bits = w.view(torch.int16).numpy().view(np.uint16)
    q, s = _quantize("mxfp4", w.to(gpu), flags)
    rq, rs = oracle.mx_quantize("mxfp4", bits, "bf16")
    assert np.array_equal(s, rs) and np.array_equal(q, rq)
    deq = _dequant("mxfp4", torch.from_numpy(q).to(gpu), torch.from_numpy(s).to(gpu), 2048, torch.float32, flags)
    assert np.array_equal(deq.numpy(), oracle.mx_dequant("mxfp4", rq, rs))
    deq16 = _dequant("mxfp4", torch.from_numpy(q).to(gpu), torch.from_numpy(s).to(gpu), 2048, torch.bfloat16, flags)
    assert torch.equal(deq16, deq.to(torch.bfloat16))


def test_cfg2_mxfp8_full_size_bit_exact(gpu):
    w = workloads.cfg2_weight()
    bits = w.view(torch.int16).numpy().view(np.uint16)
    q, s = _quantize("mxfp8", w.to(gpu))
    rq, rs = oracle.mx_quantize("mxfp8", bits, "bf16")
    assert np.array_equal(s, rs)
    assert np.array_equal(q, rq)


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_quantize_f16_f32_inputs(gpu, fmt, dtype):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(96, 512, generator=g) * torch.exp2(torch.randint(-8, 8, (96, 1), generator=g).float())
    x[3] = 0.0
    x[5, :32] = -0.0
    x = x.to(dtype)
    for flags in (0, N.FLAG_SOFTWARE_CVT):
        q, s = _quantize(fmt, x.to(gpu), flags)
        rq, rs = oracle.mx_quantize(fmt, x.numpy(), "f16" if dtype == torch.float16 else "f32")
        assert np.array_equal(s, rs) and np.array_equal(q, rq)


def test_quantize_strided_rows(gpu):
    base = workloads.cfg1_weight(64, 1024).to(gpu)
    view = base[:, 256:768]  # ld = 1024, k = 512
    q, s = _quantize("mxfp8", view, ld=1024, k=512)
    bits = base[:, 256:768].contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    rq, rs = oracle.mx_quantize("mxfp8", bits, "bf16")
    assert np.array_equal(q, rq) and np.array_equal(s, rs)


@pytest.mark.parametrize("flags", [0, N.FLAG_SOFTWARE_CVT], ids=["hw", "sw"])
@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dequant_exhaustive(gpu, fmt, dtype, flags):
    # every code byte under every scale byte
    k = 256 if fmt == "mxfp8" else 512  # one row holds all 256 code bytes
    scales = np.repeat(np.arange(256, dtype=np.uint8), k // 32).reshape(256, k // 32)
    q = np.tile(np.arange(256, dtype=np.uint8), (256, 1))
    out = _dequant(fmt, torch.from_numpy(q).to(gpu), torch.from_numpy(scales).to(gpu), k, dtype, flags)
    ref = torch.from_numpy(oracle.mx_dequant(fmt, q, scales))
    if dtype == torch.float32:
        # NaN == NaN positions, values equal elsewhere (bitwise incl. signed zeros)
        assert torch.equal(torch.isnan(out), torch.isnan(ref))
        m = ~torch.isnan(ref)
        assert torch.equal(out[m].view(torch.int32), ref[m].view(torch.int32))
    else:
        r = ref.to(dtype)
        assert torch.equal(torch.isnan(out), torch.isnan(r))
        m = ~torch.isnan(r)
        assert torch.equal(out[m].view(torch.int16), r[m].view(torch.int16))


@pytest.mark.parametrize("n", [0, 1, 2, 3, 4, 5, 7, 1000, 4096, 1 << 20])
def test_pack_unpack(gpu, n):
    rng = np.random.default_rng(n)
    packed = rng.integers(0, 256, n, dtype=np.uint8)
    codes = torch.empty(2 * n, dtype=torch.uint8, device=gpu)
    p = torch.from_numpy(packed).to(gpu)
    N.call("kq_unpack_codes", N.ptr(p), n, N.ptr(codes), N.stream(gpu))
    assert np.array_equal(codes.cpu().numpy(), oracle.unpack_codes(packed))
    wide = rng.integers(0, 256, 2 * n, dtype=np.uint8)  # whole bytes OR-ed as the reference does
    back = torch.empty(n, dtype=torch.uint8, device=gpu)
    w = torch.from_numpy(wide).to(gpu)
    N.call("kq_pack_codes", N.ptr(w), 2 * n, N.ptr(back), N.stream(gpu))
    assert np.array_equal(back.cpu().numpy(), oracle.pack_codes(wide))


@pytest.mark.parametrize("table", [N.TABLE_E8M0, N.TABLE_E2M1, N.TABLE_E4M3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_decode_bytes_tables(gpu, table, dtype):
    b = torch.arange(256, dtype=torch.uint8)
    out = torch.empty(256, dtype=dtype, device=gpu)
    bd = b.to(gpu)
    N.call("kq_decode_bytes", table, N.ptr(bd), 256, N.DTYPE_CODES[dtype], N.ptr(out), N.stream(gpu))
    if table == N.TABLE_E8M0:
        ref = torch.exp2(b.float() - 127)  # kquant/io/mxfp4.py:43
    elif table == N.TABLE_E2M1:
        ref = torch.full((256,), float("nan"))
        ref[:16] = torch.tensor(oracle.E2M1_LUT)
    else:
        ref = b.view(torch.float8_e4m3fn).float()
    ref = ref.to(dtype)
    out = out.cpu()
    assert torch.equal(torch.isnan(out), torch.isnan(ref))
    m = ~torch.isnan(ref)
    assert torch.equal(out[m].view(torch.int16 if dtype != torch.float32 else torch.int32),
                       ref[m].view(torch.int16 if dtype != torch.float32 else torch.int32))


def test_repeat_runs_are_identical(gpu):
    w = workloads.cfg1_weight(1024, 2048).to(gpu)
    a = _quantize("mxfp4", w)
    b = _quantize("mxfp4", w)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
