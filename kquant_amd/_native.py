"""ctypes binding of ``libkquant_amd.so`` (the C ABI in include/kquant_amd.h).

The product path always runs the HIP kernels.  There is no CPU fallback: when
the library is missing or no GPU is visible the calls raise RuntimeError.
CPU tensors handed to the public functions are copied to the current GPU,
processed there, and the results copied back, so callers that keep weights
on the host (as kquant's CPU helpers do) still run the GPU path.
"""

from __future__ import annotations

import ctypes
from collections.abc import Iterable

import torch

from ._build import LIB_PATH

# enums of include/kquant_amd.h
KQ_OK = 0
KQ_ERR_INVALID = -1
KQ_ERR_HIP = -2
KQ_ERR_LIMIT = -3
FMT_MXFP8_E4M3 = 0
FMT_MXFP4_E2M1 = 1
DT_BF16 = 0
DT_F16 = 1
DT_F32 = 2
QSRT_OUT_E4M3 = 3  # kq_qsrt_decode_weight's E4M3 label-byte output (KQ_QSRT_OUT_E4M3)
FLAG_SOFTWARE_CVT = 1
TABLE_E8M0 = 0
TABLE_E2M1 = 1
TABLE_E4M3 = 2
SYRK_OVERWRITE = 1
SYRK_SQUARE_WEIGHTS = 2
SUM_SQUARE_F64 = 4
MOE_REGISTER_STAGED = 1
MOE_ACT_MXFP8 = 2
MOE_ACT_MXFP4 = 4
ACT_SITU = 0
ACT_SWIGLU = 1
MOE_NOALLOC_SCRATCH_BYTES = 16 << 20  # KQ_MOE_NOALLOC_SCRATCH_BYTES

DTYPE_CODES = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32}

_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_U32 = ctypes.c_uint32
_F32 = ctypes.c_float
_F64 = ctypes.c_double

# name -> argtypes (every entry point returns int)
SIGNATURES: dict[str, list] = {
    "kq_mx_quantize": [_INT, _INT, _VP, _I64, _I64, _I64, _VP, _VP, _U32, _VP],
    "kq_mx_dequant": [_INT, _VP, _VP, _I64, _I64, _INT, _VP, _U32, _VP],
    "kq_mx_tile_weights": [_VP, _VP, _I64, _I64, _I64, _VP, _VP, _VP],
    "kq_unpack_codes": [_VP, _I64, _VP, _VP],
    "kq_pack_codes": [_VP, _I64, _VP, _VP],
    "kq_decode_bytes": [_INT, _VP, _I64, _INT, _VP, _VP],
    "kq_syrk_accumulate": [_INT, _VP, _I64, _I64, _I64, _VP, _VP, _I64, _U32, _VP],
    "kq_syrk_accumulate_ws": [_INT, _VP, _I64, _I64, _I64, _VP, _VP, _I64, _U32, _VP, _I64, _VP],
    "kq_syrk_finalize": [_VP, _I64, _I64, _F64, _F32, _VP, _I64, _VP],
    "kq_sym_lerp": [_VP, _F32, _VP, _I64, _F32, _VP, _VP],
    "kq_cov_stats": [_VP, _I64, _VP, _VP, _VP],
    "kq_mx_linear": [_INT, _VP, _I64, _VP, _VP, _I64, _I64, _I64, _INT, _VP, _I64, _VP],
    "kq_mx_linear_mx": [_INT, _VP, _VP, _I64, _INT, _VP, _VP, _I64, _I64, _I64, _INT, _VP, _I64, _VP, _I64, _VP],
    "kq_mx_linear_mm": [_INT, _VP, _INT, _I64, _VP, _VP, _I64, _I64, _I64, _INT, _VP, _I64, _VP, _I64, _VP],
    "kq_moe_forward": [_INT, _F32, _F32, _VP, _I64, _I64, _I64, _VP, _VP, _INT, _INT, _I64,
                       _VP, _VP, _VP, _VP, _INT, _VP, _VP, _I64, _U32, _VP],
    "kq_x4t_analyze": [_VP, _I64, _I64, _I64, _VP, _VP, _VP],
    "kq_x4t_emit_exceptions": [_VP, _I64, _I64, _I64, _VP, _VP, _VP, _VP],
    "kq_x4t_decode": [_VP, _VP, _I64, _VP, _I64, _I64, _I64, _VP, _VP, _VP],
    "kq_x4t_tile_index": [_VP, _I64, _VP, _I64, _I64, _I64, _VP, _VP],
    "kq_moe_forward_noalloc": [_INT, _F32, _F32, _VP, _I64, _I64, _I64, _VP, _VP, _INT, _INT, _I64,
                               _VP, _VP, _VP, _VP, _INT, _VP, _U32, _VP],
    "kq_moe_forward_x4t": [_INT, _F32, _F32, _VP, _I64, _I64, _I64, _VP, _VP, _INT, _INT, _I64,
                           _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _INT, _VP, _VP,
                           _I64, _U32, _VP],
    "kq_kqsc_measure": [_INT, _VP, _I64, _I64, _INT, _VP, _VP, _VP],
    "kq_kqsc_emit": [_INT, _VP, _I64, _I64, _INT, _VP, _VP, _VP, _VP],
    "kq_kqsc_decode": [_INT, _VP, _I64, _I64, _I64, _INT, _VP, _VP, _VP],
    "kq_kqsc_stats": [_VP, _I64, _I64, _I64, _INT, _VP, _VP, _VP],
    "kq_sqg_rank_permutation": [_INT, _INT, _INT, _VP, _VP],
    "kq_sqg_normal_rank_law": [_VP, _VP],
    "kq_sqg_finite_rank_lut": [_VP, _VP, _VP],
    "kq_sqg_check_rank_law": [_VP, _VP, _VP],
    "kq_sqg_modal_compress": [_VP, _VP, _VP],
    "kq_sqg_gather": [_VP, _I64, _INT, _VP, _I64, _VP, _VP, _VP],
    "kq_sqg_r44_bytes": [_INT, _VP, _VP, _VP],
    "kq_mx_linear_f32": [_INT, _VP, _I64, _VP, _VP, _I64, _I64, _I64, _VP, _I64, _VP, _I64, _VP],
    "kq_expert_activation": [_INT, _F32, _F32, _INT, _VP, _VP, _I64, _I64, _I64, _INT, _VP, _I64,
                             _VP],
    "kq_reduce_partials": [_VP, _I64, _I64, _I64, _INT, _VP, _VP],
    "kq_comparison_sums": [_INT, _VP, _INT, _VP, _I64, _VP, _VP, _VP],
    "kq_kimi_topk": [_INT, _VP, _I64, _VP, _I64, _INT, _INT, _F32, _VP, _VP, _VP],
    "kq_syrk_grouped": [_INT, _VP, _I64, _VP, _INT, _VP, _VP, _I64, _VP, _U32, _VP],
    "kq_segment_weight_sums": [_VP, _VP, _INT, _U32, _VP, _VP],
    "kq_syrk_finalize_grouped": [_VP, _I64, _INT, _VP, _VP, _VP],
    "kq_route_sort": [_VP, _I64, _INT, _INT, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _VP],
    "kq_covariance_comparison_sums": [_VP, _VP, _I64, _VP, _VP, _VP],
    "kq_h_regularize": [_VP, _I64, _I64, _F64, _F32, _VP, _VP, _VP],
    "kq_blockwise_hadamard": [_VP, _I64, _I64, _I64, _I64, _I64, _INT, _VP, _VP, _VP],
    "kq_cholesky": [_VP, _I64, _I64, _VP, _I64, _I64, _I64, _I64, _VP, _VP, _I64, _VP],
    "kq_block_ldl": [_VP, _I64, _I64, _I64, _INT, _I64, _U32, _VP, _I64, _VP],
    "kq_trellis_pack": [_VP, _I64, _INT, _VP, _VP],
    "kq_trellis_unpack": [_VP, _I64, _INT, _INT, _VP, _VP],
    "kq_qsrt_decode_weight": [_VP, _I64, _I64, _I64, _INT, _VP, _VP, _VP, _VP, _INT, _VP, _I64, _U32, _VP],
    "kq_qsrt_decode_states": [_VP, _I64, _I64, _INT, _VP, _VP, _VP, _VP, _INT, _VP, _I64, _U32, _VP],
    "kq_sqg_quantize_tiles": [_VP, _I64, _VP, _INT, _INT, _VP, _VP, _VP, _I64, _INT, _VP],
    "kq_sqg_quantize_tiles_procedural": [_VP, _I64, _INT, _INT, _INT, _VP, _VP, _VP, _I64, _INT, _VP],
    "kq_qsrt_moe_decode": [_INT, _F32, _F32, _VP, _INT, _I64, _I64, _VP, _VP, _INT, _VP, _INT, _I64, _I64, _INT,
                           _INT, _VP, _INT, _VP, _I64, _VP, _I64, _VP],
    "kq_qsrt_linear": [_VP, _INT, _I64, _I64, _VP, _I64, _I64, _I64, _INT, _VP, _VP, _VP, _VP, _INT, _VP, _I64,
                       _VP, _I64, _VP],
}
QSRT_TRANSPOSED = 1
LDL_ZERO_DIAGONAL = 1
SQG_RANK_XOR = 0
SQG_RANK_MIX = 1
SQG_RANK_K2_OCTILE = 2
COV_STATS_PARTS = 256

_lib: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Load the native library once; raise if it has not been built."""

    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"kquant_amd native library not found at {LIB_PATH}; "
                "build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.kq_version.restype = ctypes.c_int
        lib.kq_version.argtypes = []
        lib.kq_last_error.restype = ctypes.c_char_p
        lib.kq_last_error.argtypes = []
        lib.kq_moe_workspace_size.restype = ctypes.c_int64
        lib.kq_moe_workspace_size.argtypes = [_I64, _INT, _INT, _I64, _I64]
        lib.kq_moe_x4t_workspace_size.restype = ctypes.c_int64
        lib.kq_moe_x4t_workspace_size.argtypes = [_I64, _INT, _INT, _I64, _I64]
        lib.kq_mx_linear_f32_workspace_size.restype = ctypes.c_int64
        lib.kq_mx_linear_f32_workspace_size.argtypes = [_I64, _I64]
        lib.kq_mx_linear_mm_workspace_size.restype = ctypes.c_int64
        lib.kq_mx_linear_mm_workspace_size.argtypes = [_I64, _I64, _I64]
        lib.kq_mx_linear_mx_workspace_size.restype = ctypes.c_int64
        lib.kq_mx_linear_mx_workspace_size.argtypes = [_I64, _I64, _I64]
        lib.kq_cholesky_workspace_size.restype = ctypes.c_int64
        lib.kq_cholesky_workspace_size.argtypes = [_I64, _I64]
        lib.kq_block_ldl_workspace_size.restype = ctypes.c_int64
        lib.kq_block_ldl_workspace_size.argtypes = [_I64, _INT, _I64]
        lib.kq_sqg_quantize_workspace_size.restype = ctypes.c_int64
        lib.kq_sqg_quantize_workspace_size.argtypes = [_INT, _INT]
        lib.kq_qsrt_moe_workspace_size.restype = ctypes.c_int64
        lib.kq_qsrt_moe_workspace_size.argtypes = [_I64, _INT, _I64, _I64]
        lib.kq_qsrt_linear_workspace_size.restype = ctypes.c_int64
        lib.kq_qsrt_linear_workspace_size.argtypes = [_I64, _I64, _I64]
        lib.kq_syrk_accumulate_workspace_size.restype = ctypes.c_int64
        lib.kq_syrk_accumulate_workspace_size.argtypes = [_INT, _I64, _I64, _INT]
        lib.kq_route_sort_workspace_size.restype = ctypes.c_int64
        lib.kq_route_sort_workspace_size.argtypes = [_I64, _INT, _INT]
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call a C entry point and turn a non-zero status into RuntimeError."""

    lib = library()
    rc = getattr(lib, name)(*args)
    if rc != KQ_OK:
        message = lib.kq_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {message}")


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError(
            "kquant_amd runs its kernels on an MI355X GPU and no GPU is visible"
        )
    return torch.device("cuda", torch.cuda.current_device())


def to_gpu(tensors: Iterable[torch.Tensor | None]) -> tuple[list, torch.device, torch.device | None]:
    """Move tensors to one GPU; return (tensors, gpu, host device or None).

    The GPU is the device of the first GPU tensor, else the current device.
    ``host`` is the original device when the inputs came from the CPU, so the
    caller can return results where the reference would have produced them.
    """

    tensors = list(tensors)
    gpu = None
    for t in tensors:
        if t is not None and t.is_cuda:
            gpu = t.device
            break
    host = None
    if gpu is None:
        gpu = require_gpu()
        for t in tensors:
            if t is not None:
                host = t.device
                break
    else:
        library()
    moved = [None if t is None else t.to(gpu) for t in tensors]
    return moved, gpu, host


def aligned(t: torch.Tensor, align: int = 16) -> torch.Tensor:
    """Contiguous tensor whose data pointer is ``align``-byte aligned."""

    t = t.contiguous()
    if t.data_ptr() % align:
        t = t.clone()
    return t
