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
                                        "kq_mx_linear_f32_workspace_size",
                                        "kq_route_sort_workspace_size"}
    assert set(declared_symbols()) <= bound


def test_argument_errors_need_no_gpu():
    lib = _native.library()
    rc = lib.kq_mx_quantize(0, 0, None, 100, 4, 100, None, None, 0, None)  # k % 32 != 0
    assert rc == _native.KQ_ERR_INVALID
    assert b"k % 32" in lib.kq_last_error()
    assert lib.kq_moe_workspace_size(8, 8, 384, 7168, 2048) > 8 * 8 * 7168 * 4
