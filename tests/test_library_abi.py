"""The C-ABI library loads and exports every entry point that
include/kquant_amd.h declares (no GPU needed: nothing is launched)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from kquant_amd import _build, _native

HEADER = Path(__file__).resolve().parent.parent / "include" / "kquant_amd.h"


def declared_symbols() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(kq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "kq_mx_quantize" in syms and "kq_moe_forward" in syms and "kq_syrk_accumulate" in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_build.LIB_PATH))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"missing exports: {missing}"


def test_python_binding_covers_every_entry_point():
    lib = _native.library()
    assert lib.kq_version() >> 16 == 1
    bound = set(_native.SIGNATURES) | {"kq_version", "kq_last_error", "kq_moe_workspace_size",
                                        "kq_moe_x4t_workspace_size", "kq_mx_linear_f32_workspace_size",
                                        "kq_cholesky_workspace_size", "kq_block_ldl_workspace_size",
                                        "kq_sqg_quantize_workspace_size", "kq_qsrt_linear_workspace_size",
                                        "kq_qsrt_moe_workspace_size",
                                        "kq_route_sort_workspace_size", "kq_syrk_accumulate_workspace_size",
                                        "kq_mx_linear_mm_workspace_size", "kq_mx_linear_mx_workspace_size"}
    assert set(declared_symbols()) <= bound


def test_argument_errors_need_no_gpu():
    lib = _native.library()
    rc = lib.kq_mx_quantize(0, 0, None, 100, 4, 100, None, None, 0, None)  # k % 32 != 0
    assert rc == _native.KQ_ERR_INVALID
    assert b"k % 32" in lib.kq_last_error()
    assert lib.kq_moe_workspace_size(8, 8, 384, 7168, 2048) > 8 * 8 * 7168 * 4


def test_linear_a8_argument_errors_need_no_gpu():
    lib = _native.library()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    e4m3, e2m1 = _native.FMT_MXFP8_E4M3, _native.FMT_MXFP4_E2M1
    args = [e4m3, fake, fake, 256, e4m3, fake, fake, 8, 8, 256, _native.DT_BF16, fake, 8, fake, 1 << 20, None]
    bad = list(args)
    bad[4] = e2m1
    assert lib.kq_mx_linear_mx(*bad) == _native.KQ_ERR_INVALID and b"only MXFP8" in lib.kq_last_error()
    bad = list(args)
    bad[9] = 192  # k % 128 != 0
    assert lib.kq_mx_linear_mx(*bad) == _native.KQ_ERR_INVALID and b"k % 128" in lib.kq_last_error()
    bad = list(args)
    bad[3] = 264  # lda % 16 != 0
    assert lib.kq_mx_linear_mx(*bad) == _native.KQ_ERR_INVALID and b"lda % 16" in lib.kq_last_error()
    bad = list(args)
    bad[1] = ctypes.c_void_p(264)
    assert lib.kq_mx_linear_mx(*bad) == _native.KQ_ERR_INVALID and b"16-byte aligned" in lib.kq_last_error()
    bad = list(args)
    bad[14] = 16
    assert lib.kq_mx_linear_mx(*bad) == _native.KQ_ERR_INVALID and b"workspace needs" in lib.kq_last_error()
    assert lib.kq_mx_linear_mx_workspace_size(4096, 12288, 7168) >= (4096 + 12288) * 224
    assert lib.kq_mx_linear_mm_workspace_size(4096, 12288, 7168) >= 4096 * 7168 + (2 * 4096 + 12288) * 224
    mm = [e4m3, fake, _native.DT_BF16, 256, fake, fake, 8, 8, 256, _native.DT_BF16, fake, 8, fake, 16, None]
    assert lib.kq_mx_linear_mm(*mm) == _native.KQ_ERR_INVALID and b"workspace needs" in lib.kq_last_error()
    bad = list(mm)
    bad[2] = 9
    assert lib.kq_mx_linear_mm(*bad) == _native.KQ_ERR_INVALID and b"input dtype" in lib.kq_last_error()


def test_x4t_moe_argument_errors_need_no_gpu():
    lib = _native.library()
    per_expert = 2 * 2048 * 7168 // 32 + 7168 * 2048 // 32  # w13 and w2 scale bytes
    # decoding (<= 256 pairs): the GEMVs decode X4T scales themselves, no slots
    base = lib.kq_moe_workspace_size(4, 8, 384, 7168, 2048)
    assert base <= lib.kq_moe_x4t_workspace_size(4, 8, 384, 7168, 2048) < base + per_expert
    # otherwise one slot per possible grouped-GEMM expert: min(pairs / 17, experts)
    base = lib.kq_moe_workspace_size(64, 8, 384, 7168, 2048)
    assert lib.kq_moe_x4t_workspace_size(64, 8, 384, 7168, 2048) >= base + 30 * per_expert
    base = lib.kq_moe_workspace_size(8192, 8, 384, 7168, 2048)
    assert lib.kq_moe_x4t_workspace_size(8192, 8, 384, 7168, 2048) >= base + 384 * per_expert
    assert lib.kq_moe_x4t_workspace_size(4, 0, 384, 7168, 2048) == -1
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    planes = [fake] * 9
    rc = lib.kq_moe_forward_x4t(_native.ACT_SITU, 4.0, 25.0, fake, 8192, 1, 8192, fake, fake, 8, 384,
                                2048, fake, fake, *planes, _native.DT_F32, fake, fake, 1 << 30, 0, None)
    assert rc == _native.KQ_ERR_LIMIT and b"X4T geometry" in lib.kq_last_error()
    planes[4] = None
    rc = lib.kq_moe_forward_x4t(_native.ACT_SITU, 4.0, 25.0, fake, 7168, 1, 7168, fake, fake, 8, 384,
                                2048, fake, fake, *planes, _native.DT_F32, fake, fake, 1 << 30, 0, None)
    assert rc == _native.KQ_ERR_INVALID and b"null X4T component" in lib.kq_last_error()
    rc = lib.kq_x4t_tile_index(fake, 0, None, 1, 32, 300, fake, None)
    assert rc != 0


def test_ldl_argument_errors_need_no_gpu():
    lib = _native.library()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    # two 64 x 64 fp32 inverse slots per matrix, then one int counter per matrix (256-byte granules)
    assert lib.kq_cholesky_workspace_size(7168, 1) == 2 * 64 * 64 * 4 + 256
    assert lib.kq_cholesky_workspace_size(7168, 65) == 65 * 2 * 64 * 64 * 4 + 512
    assert lib.kq_block_ldl_workspace_size(2048, 16, 3) == 3 * 2048 * 16 * 4
    rc = lib.kq_cholesky(fake, 0, 0, fake, 0, 0, 0, 1, fake, fake, 1 << 20, None)
    assert rc == _native.KQ_ERR_INVALID
    rc = lib.kq_cholesky(fake, 64, 4096, ctypes.c_void_p(512), 64, 4096, 64, 2, fake, fake, 1 << 20, None)
    assert rc == _native.KQ_ERR_INVALID and b"overlap" in lib.kq_last_error()
    rc = lib.kq_block_ldl(fake, 96, 0, 96, 3, 1, 0, fake, 1 << 20, None)
    assert rc == _native.KQ_ERR_INVALID and b"power of two" in lib.kq_last_error()
    rc = lib.kq_blockwise_hadamard(fake, 100, 128, 128, 1, 0, 1, None, None, None)
    assert rc == _native.KQ_ERR_INVALID and b"multiple of 128" in lib.kq_last_error()
    rc = lib.kq_h_regularize(fake, 10, 10, -1.0, 0.025, None, fake, None)
    assert rc == _native.KQ_ERR_INVALID


def test_qsrt_linear_argument_errors_need_no_gpu():
    lib = _native.library()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    bits = bytes([3] * 2)
    assert lib.kq_qsrt_linear_workspace_size(1, 12, 16) == 0  # K not a multiple of 128
    args = [fake, _native.DT_BF16, 1, 256, fake, 2 * 8 * 16 * 16 * 3, 16, 16, 1, bits, fake, None, None,
            _native.DT_F32, fake, 256, None, 0, None]
    bad_axis = list(args)
    bad_axis[8] = 2
    assert lib.kq_qsrt_linear(*bad_axis) == _native.KQ_ERR_INVALID and b"rate_axis" in lib.kq_last_error()
    bad_words = list(args)
    bad_words[5] -= 1
    assert lib.kq_qsrt_linear(*bad_words) == _native.KQ_ERR_INVALID and b"payload has" in lib.kq_last_error()
    bad_rate = list(args)
    bad_rate[9] = bytes([3, 5])
    assert lib.kq_qsrt_linear(*bad_rate) == _native.KQ_ERR_INVALID and b"rate 5" in lib.kq_last_error()
    odd = list(args)
    odd[4] = ctypes.c_void_p(260)  # 4 bytes past a 16-byte boundary: the direct loads need 16
    assert lib.kq_qsrt_linear(*odd) == _native.KQ_ERR_INVALID and b"16-byte aligned" in lib.kq_last_error()
    half = list(args)
    half[11] = fake
    assert lib.kq_qsrt_linear(*half) == _native.KQ_ERR_INVALID and b"suh and svh" in lib.kq_last_error()
    narrow = list(args)
    narrow[3] = 100
    assert lib.kq_qsrt_linear(*narrow) == _native.KQ_ERR_INVALID and b"ldx" in lib.kq_last_error()


def test_qsrt_moe_argument_errors_need_no_gpu():
    lib = _native.library()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    assert lib.kq_qsrt_moe_workspace_size(1, 16, 224, 12) == 0  # I not a multiple of 128
    args = [_native.ACT_SITU, 4.0, 25.0, fake, _native.DT_BF16, 1, 3584, fake, fake, 16, fake, 896, 224, 16, 1, 0,
            fake, _native.DT_BF16, fake, 3584, fake, 1 << 20, None]
    bad = list(args)
    bad[0] = 7
    assert lib.kq_qsrt_moe_decode(*bad) == _native.KQ_ERR_INVALID and b"activation" in lib.kq_last_error()
    bad = list(args)
    bad[13] = 12
    assert lib.kq_qsrt_moe_decode(*bad) == _native.KQ_ERR_INVALID and b"multiples of 128" in lib.kq_last_error()
    bad = list(args)
    bad[15] = 2
    assert lib.kq_qsrt_moe_decode(*bad) == _native.KQ_ERR_INVALID and b"rate axes" in lib.kq_last_error()
    bad = list(args)
    bad[1] = 0.0
    assert lib.kq_qsrt_moe_decode(*bad) == _native.KQ_ERR_INVALID and b"betas" in lib.kq_last_error()
    bad = list(args)
    bad[19] = 100
    assert lib.kq_qsrt_moe_decode(*bad) == _native.KQ_ERR_INVALID and b"ldo" in lib.kq_last_error()
    bad = list(args)
    bad[16] = ctypes.c_void_p(260)  # the label table is staged by 16-byte direct loads
    assert lib.kq_qsrt_moe_decode(*bad) == _native.KQ_ERR_INVALID and b"labels must be 16-byte" in lib.kq_last_error()
