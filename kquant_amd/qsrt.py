"""QSRT trellis bitstream and the decode of packed QSRT matrices, on the GPU.

Drop-in for the bitstream functions of ``kquant/qsrt.py`` (same names,
arguments, dtypes and errors):

  ``pack_trellis_edges(indices, bits)``      (:811-833)  -> ``kq_trellis_pack``
  ``unpack_trellis_edges(packed, bits)``     (:836-857)  -> ``kq_trellis_unpack``
  ``unpack_trellis_states(packed, bits)``    (:860-863)  -> ``kq_trellis_unpack``

and, as the payload-level decode a serving loader needs (the role of
``decode_qsrt_exl3_weight``, :1107-1141, minus the mode tables of the
Kimi-K3 checkpoint schema), ``decode_qsrt_payload``: one launch from the
packed payload of 128-channel records to the EXL-oriented weight
(``kq_qsrt_decode_weight``).  ``qsrt_linear`` applies such a matrix to
activation rows without building the weight (``kq_qsrt_linear``): the
serving step of scripts/stream_k3_pytorch.py:771-775, which decodes the
dense weight and then runs the linear.  CPU inputs run on the current GPU
and come back on the CPU.
"""

from __future__ import annotations

import torch

from . import _native as N
from .sqg_e4m3 import SQG_XOR_CHEB_T12, sqg_codebook_bytes

TILE_CHANNELS = 16
TILE_VALUES = TILE_CHANNELS * TILE_CHANNELS
RECORD_CHANNELS = 128


def _validate_k(bits: int) -> None:
    if isinstance(bits, bool) or not isinstance(bits, int) or bits not in (2, 3, 4):
        raise ValueError("QSRT supports K=2, K=3, or K=4")


def _on_gpu(t: torch.Tensor) -> tuple[torch.Tensor, torch.device | None]:
    (g,), _, host = N.to_gpu([t])
    return g, host


def pack_trellis_edges(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack the low K bits of every index with the native word ordering."""

    _validate_k(bits)
    if indices.ndim < 1 or indices.shape[-1] != TILE_VALUES:
        raise ValueError("indices must have a final dimension of 256")
    if indices.dtype == torch.bool or indices.is_floating_point():
        raise TypeError("indices must use an integer dtype")
    g, host = _on_gpu(indices)
    sym = N.aligned((g & 0xFFFF).to(torch.int16) if g.dtype != torch.int16 else g, 2)
    tiles = sym.numel() // TILE_VALUES
    out = torch.empty(*indices.shape[:-1], TILE_CHANNELS * bits, dtype=torch.int16, device=g.device)
    N.call("kq_trellis_pack", N.ptr(sym), tiles, bits, N.ptr(out), N.stream(g.device))
    return out if host is None else out.to(host)


def _unpack(packed: torch.Tensor, bits: int, states: bool) -> torch.Tensor:
    _validate_k(bits)
    expected_words = TILE_CHANNELS * bits
    if packed.ndim < 1 or packed.shape[-1] != expected_words:
        raise ValueError(f"packed tiles must end in {expected_words} int16 words")
    if packed.dtype != torch.int16:
        raise TypeError("packed trellis words must use torch.int16")
    g, host = _on_gpu(packed)
    g = N.aligned(g, 2)
    tiles = g.numel() // expected_words
    out = torch.empty(*packed.shape[:-1], TILE_VALUES, dtype=torch.int16, device=g.device)
    N.call("kq_trellis_unpack", N.ptr(g), tiles, bits, 1 if states else 0, N.ptr(out), N.stream(g.device))
    return out if host is None else out.to(host)


def unpack_trellis_edges(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """Invert :func:`pack_trellis_edges` to the stored K-bit edge symbols."""

    return _unpack(packed, bits, False)


def unpack_trellis_states(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """Unpack native edge words and reconstruct every cyclic 16-bit state."""

    return _unpack(packed, bits, True)


# rows up to which kq_qsrt_linear runs the fused kernel (decode batches): it
# decodes the weight once per 16 rows, so past two row groups the library
# takes its prefill form (one decode to E4M3 label bytes and the MXFP8 MFMA
# linear between the two rotations)
FUSED_MAX_ROWS = 32

_LABELS: dict[tuple[str, str | None, torch.device], torch.Tensor] = {}
_LINEAR_WORKSPACES: dict[tuple, torch.Tensor] = {}


def rate_labels(codebook: str = SQG_XOR_CHEB_T12, *, rate_axis: str | None = None,
                device: torch.device | str | None = None) -> torch.Tensor:
    """The K2, K3 and K4 state labels of a codebook as one uint8 [3, 65536]
    device table (the layout the decode kernels read); built once per
    codebook, rate axis and device."""

    gpu = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if gpu.index is None:
        gpu = torch.device(gpu.type, torch.cuda.current_device())
    key = (codebook, rate_axis, gpu)
    table = _LABELS.get(key)
    if table is None:
        table = torch.stack([sqg_codebook_bytes(bits, codebook, rate_axis=rate_axis, device=gpu)
                             for bits in (2, 3, 4)]).contiguous()
        _LABELS[key] = table
    return table


def decode_qsrt_payload(
    payload: torch.Tensor,
    *,
    k_tiles: int,
    n_tiles: int,
    rate_axis: str,
    record_bits,
    suh: torch.Tensor | None = None,
    svh: torch.Tensor | None = None,
    codebook: str = SQG_XOR_CHEB_T12,
    out_dtype: torch.dtype = torch.float32,
    transposed: bool = False,
) -> torch.Tensor:
    """Decode a packed QSRT matrix (``pack_qsrt_trellis``'s payload,
    kquant/qsrt.py:983-1013) to its weight: ``[K, N]`` (EXL orientation) or,
    with ``transposed``, ``[N, K]``.  With ``suh`` / ``svh`` this is
    ``decode_qsrt_weight`` (kquant/exl3_reference.py:270-295); without, the
    regularized weight.  ``record_bits`` gives each 128-channel record's rate
    along ``rate_axis``."""

    if rate_axis not in ("k", "n"):
        raise ValueError("rate_axis must be 'k' or 'n'")
    if payload.dtype != torch.int16 or payload.ndim != 1:
        raise TypeError("QSRT trellis payload must be a one-dimensional torch.int16 tensor")
    if (suh is None) != (svh is None):
        raise ValueError("pass both suh and svh, or neither")
    bits = bytes(int(b) for b in record_bits)
    if any(b not in (2, 3, 4) for b in bits):
        raise ValueError("tile_bits must contain only integer K2, K3, or K4")
    g, host = _on_gpu(payload)
    g = N.aligned(g, 16)  # the fast decode stages 16-byte pieces by direct loads
    gpu = g.device
    k, n = k_tiles * TILE_CHANNELS, n_tiles * TILE_CHANNELS
    _check_record_count(bits, k_tiles, n_tiles, rate_axis)
    labels = rate_labels(codebook, rate_axis=rate_axis, device=gpu)
    su = sv = None
    if suh is not None:
        if suh.numel() != k or svh.numel() != n:
            raise ValueError("suh and svh must match the K and N dimensions")
        su = N.aligned(suh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
        sv = N.aligned(svh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
    shape = (n, k) if transposed else (k, n)
    out = torch.empty(shape, dtype=out_dtype, device=gpu)
    # record rates are a host array (bytes pass as a pointer to their buffer)
    N.call("kq_qsrt_decode_weight", N.ptr(g), g.numel(), k_tiles, n_tiles, 0 if rate_axis == "k" else 1,
           bits, N.ptr(labels), N.ptr(su), N.ptr(sv), N.DTYPE_CODES[out_dtype], N.ptr(out), shape[1],
           N.QSRT_TRANSPOSED if transposed else 0, N.stream(gpu))
    return out if host is None else out.to(host)


def _check_record_bits(record_bits) -> bytes:
    bits = bytes(int(b) for b in record_bits)
    if any(b not in (2, 3, 4) for b in bits):
        raise ValueError("tile_bits must contain only integer K2, K3, or K4")
    return bits


def _check_record_count(bits: bytes, k_tiles: int, n_tiles: int, rate_axis: str) -> None:
    """One rate per 128-channel record along the rate axis (the library reads
    that many bytes of the host array)."""
    if k_tiles <= 0 or n_tiles <= 0 or k_tiles % 8 or n_tiles % 8:
        raise ValueError("both dimensions must be positive multiples of 128")
    records = (k_tiles if rate_axis == "k" else n_tiles) // 8
    if len(bits) != records:
        raise ValueError(f"{len(bits)} record rates for {records} records along {rate_axis}")


def _workspace(cache: dict, key: tuple, nbytes: int, gpu: torch.device) -> torch.Tensor:
    """A zeroed workspace per (device, stream, geometry): the fused kernels'
    completion counters and polled partial sums return to zero after every
    call, but calls on two streams must not share them."""
    ws = cache.get(key)
    if ws is None:
        ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=gpu)
        cache[key] = ws
    return ws


def qsrt_linear_launcher(
    x: torch.Tensor,
    payload: torch.Tensor,
    out: torch.Tensor,
    *,
    k_tiles: int,
    n_tiles: int,
    rate_axis: str,
    record_bits,
    suh: torch.Tensor | None = None,
    svh: torch.Tensor | None = None,
    codebook: str = SQG_XOR_CHEB_T12,
):
    """A zero-argument callable that writes ``x @ W`` into ``out`` with fixed
    device buffers (x [m, K] and out [m, N] on the payload's GPU, row-major):
    every check, table and workspace is settled once, so the call allocates
    nothing and may be captured in a HIP graph.  Up to ``FUSED_MAX_ROWS`` rows
    a call is one launch (the fused kernel).  From ``FUSED_MAX_ROWS + 1`` rows
    it is the prefill form, four launches (five for fp32 / fp16 rows): the row
    rotation, the weight decode to E4M3 label bytes, the three-term split of
    fp32 rows, the MXFP8 MFMA product and the output rotation -- the weight is
    decoded again on every call."""

    if rate_axis not in ("k", "n"):
        raise ValueError("rate_axis must be 'k' or 'n'")
    if payload.dtype != torch.int16 or payload.ndim != 1 or not payload.is_cuda:
        raise TypeError("QSRT trellis payload must be a one-dimensional torch.int16 GPU tensor")
    if (suh is None) != (svh is None):
        raise ValueError("pass both suh and svh, or neither")
    if x.dtype not in N.DTYPE_CODES or out.dtype not in N.DTYPE_CODES:
        raise TypeError("x and out must be bfloat16, float16 or float32")
    k, n = k_tiles * TILE_CHANNELS, n_tiles * TILE_CHANNELS
    if x.ndim != 2 or x.shape[1] != k or x.stride(1) != 1:
        raise ValueError(f"x must be [m, {k}] with unit column stride")
    if out.shape != (x.shape[0], n) or out.stride(1) != 1:
        raise ValueError(f"out must be [{x.shape[0]}, {n}] with unit column stride")
    gpu = payload.device
    if x.device != gpu or out.device != gpu:
        raise ValueError("x, out and the payload must be on one GPU")
    if payload.data_ptr() % 16:
        raise ValueError("the payload must be 16-byte aligned")
    bits = _check_record_bits(record_bits)
    _check_record_count(bits, k_tiles, n_tiles, rate_axis)
    m = x.shape[0]
    labels = rate_labels(codebook, rate_axis=rate_axis, device=gpu)
    su = sv = None
    if suh is not None:
        if suh.numel() != k or svh.numel() != n:
            raise ValueError("suh and svh must match the K and N dimensions")
        su = N.aligned(suh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
        sv = N.aligned(svh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
    need = int(N.library().kq_qsrt_linear_workspace_size(max(m, 1), k_tiles, n_tiles)) if m else 0
    if need < 0:
        raise RuntimeError("kq_qsrt_linear_workspace_size: no HIP device")
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu) if need else None  # starts (and stays) zero
    args = (N.ptr(x), N.DTYPE_CODES[x.dtype], m, x.stride(0) if m else k, N.ptr(payload), payload.numel(),
            k_tiles, n_tiles, 0 if rate_axis == "k" else 1, bits, N.ptr(labels), N.ptr(su), N.ptr(sv),
            N.DTYPE_CODES[out.dtype], N.ptr(out), out.stride(0) if m else n, N.ptr(ws), need)
    keep = (x, payload, out, labels, su, sv, ws)  # the buffers the pointers refer to

    def run(_keep=keep) -> None:
        N.call("kq_qsrt_linear", *args, N.stream(gpu))

    return run


def qsrt_linear(
    x: torch.Tensor,
    payload: torch.Tensor,
    *,
    k_tiles: int,
    n_tiles: int,
    rate_axis: str,
    record_bits,
    suh: torch.Tensor | None = None,
    svh: torch.Tensor | None = None,
    codebook: str = SQG_XOR_CHEB_T12,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``x @ W`` for the packed QSRT matrix W of ``decode_qsrt_payload``
    (same arguments), computed from the trellis words directly: x [..., K]
    (bf16, fp16 or fp32) -> [..., N] in ``out_dtype`` (default x's dtype),
    fp32 arithmetic inside.  For the reference's dense path this is
    ``F.linear(x, decode_qsrt_exl3_weight(...).T)`` without the bf16 weight
    it materializes (scripts/stream_k3_pytorch.py:771-775).  Beyond
    ``FUSED_MAX_ROWS`` rows (prefill), where the fused kernel would decode
    the weight once per 16 rows, ``kq_qsrt_linear`` rotates the rows, decodes
    the regularized weight once to its exact E4M3 label bytes and runs the
    MXFP8 MFMA linear, then rotates the output: fp32 and fp16 rows keep fp32
    accuracy (exact three-term bf16 split); bf16 rows are rotated to bf16."""

    if rate_axis not in ("k", "n"):
        raise ValueError("rate_axis must be 'k' or 'n'")
    if payload.dtype != torch.int16 or payload.ndim != 1:
        raise TypeError("QSRT trellis payload must be a one-dimensional torch.int16 tensor")
    if (suh is None) != (svh is None):
        raise ValueError("pass both suh and svh, or neither")
    if x.dtype not in N.DTYPE_CODES:
        raise TypeError("x must be bfloat16, float16 or float32")
    k, n = k_tiles * TILE_CHANNELS, n_tiles * TILE_CHANNELS
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, the matrix has K = {k}")
    bits = _check_record_bits(record_bits)
    _check_record_count(bits, k_tiles, n_tiles, rate_axis)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    (g, xg), gpu, host = N.to_gpu([payload, x])
    g = N.aligned(g, 16)
    rows = xg.reshape(-1, k)
    rows = rows if rows.stride(-1) == 1 else rows.contiguous()
    m = rows.shape[0]
    labels = rate_labels(codebook, rate_axis=rate_axis, device=gpu)
    su = sv = None
    if suh is not None:
        if suh.numel() != k or svh.numel() != n:
            raise ValueError("suh and svh must match the K and N dimensions")
        su = N.aligned(suh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
        sv = N.aligned(svh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
    out = torch.empty(m, n, dtype=out_dtype, device=gpu)
    need = int(N.library().kq_qsrt_linear_workspace_size(max(m, 1), k_tiles, n_tiles)) if m else 0
    if need < 0:
        raise RuntimeError("kq_qsrt_linear_workspace_size: no HIP device")
    stream = N.stream(gpu)
    if not need:
        ws = None
    elif m <= FUSED_MAX_ROWS:
        # the fused kernel's counters and polled partials: zeroed once, back at zero after every call
        ws = _workspace(_LINEAR_WORKSPACES, (gpu, stream.value, m, k_tiles, n_tiles), need, gpu)
    else:
        # the prefill form keeps no state between calls: a buffer from torch's
        # caching allocator, released with this call, so prompts of many
        # lengths do not each pin a workspace of their own
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    N.call("kq_qsrt_linear", N.ptr(rows), N.DTYPE_CODES[rows.dtype], m, rows.stride(0) if m else k, N.ptr(g),
           g.numel(), k_tiles, n_tiles, 0 if rate_axis == "k" else 1, bits, N.ptr(labels), N.ptr(su), N.ptr(sv),
           N.DTYPE_CODES[out_dtype], N.ptr(out), n, N.ptr(ws) if need else None, need, stream)
    out = out.reshape(*x.shape[:-1], n)
    return out if host is None else out.to(host)


class QSRTExperts:
    """QSRT-coded routed experts on one GPU, as ``kq_qsrt_moe_decode`` reads
    them: per expert a w1, w3 (EXL [H, I], records along ``rate13_axis``,
    the reference's MATRIX_RATE_AXIS, kquant/qsrt.py:83-87) and w2 ([I, H],
    records along ``rate2_axis``), each given as ``(payload, record_bits,
    suh, svh)`` with the payload of ``pack_qsrt_trellis`` (int16 words).
    Every payload's length is checked against its record rates here, since
    the kernel reads the descriptors from device memory."""

    KINDS = ("w1", "w3", "w2")

    def __init__(self, w1, w3, w2, *, hidden: int, inter: int, rate13_axis: str = "n", rate2_axis: str = "k",
                 codebook: str = SQG_XOR_CHEB_T12, device: torch.device | str | None = None):
        if hidden % RECORD_CHANNELS or inter % RECORD_CHANNELS or hidden <= 0 or inter <= 0:
            raise ValueError("hidden and intermediate sizes must be positive multiples of 128")
        if rate13_axis not in ("k", "n") or rate2_axis not in ("k", "n"):
            raise ValueError("rate axes must be 'k' or 'n'")
        if not (len(w1) == len(w3) == len(w2)) or not w1:
            raise ValueError("w1, w3 and w2 must list the same, non-zero number of experts")
        gpu = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if gpu.index is None:
            gpu = torch.device(gpu.type, torch.cuda.current_device())
        self.device, self.hidden, self.inter = gpu, hidden, inter
        self.rate13_axis, self.rate2_axis, self.codebook = rate13_axis, rate2_axis, codebook
        self.experts = len(w1)
        self._keep = []
        rows = []
        for e in range(self.experts):
            row = []
            for kind, spec in zip(self.KINDS, (w1[e], w3[e], w2[e])):
                k, n = (hidden, inter) if kind != "w2" else (inter, hidden)
                axis = rate13_axis if kind != "w2" else rate2_axis
                payload, record_bits, suh, svh = spec
                bits = _check_record_bits(record_bits)
                records = (k if axis == "k" else n) // RECORD_CHANNELS
                if len(bits) != records:
                    raise ValueError(f"expert {e} {kind}: {len(bits)} record rates for {records} records")
                per_record = 8 * ((n if axis == "k" else k) // TILE_CHANNELS)  # tiles per record
                words = sum(per_record * TILE_CHANNELS * b for b in bits)
                if payload.dtype != torch.int16 or payload.ndim != 1 or payload.numel() != words:
                    raise ValueError(f"expert {e} {kind}: payload must be {words} int16 words")
                if suh.numel() != k or svh.numel() != n:
                    raise ValueError(f"expert {e} {kind}: suh / svh must have {k} / {n} values")
                p = N.aligned(payload.to(gpu), 16)  # the kernels stage 16-byte pieces by direct loads
                prefix = torch.tensor([0, *torch.tensor(list(bits)).cumsum(0).tolist()], dtype=torch.int32,
                                      device=gpu)
                su = N.aligned(suh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
                sv = N.aligned(svh.to(device=gpu, dtype=torch.float32).reshape(-1), 4)
                self._keep += [p, prefix, su, sv]
                row.append([p.data_ptr(), prefix.data_ptr(), su.data_ptr(), sv.data_ptr()])
            rows.append(row)
        self.descriptors = torch.tensor(rows, dtype=torch.int64, device=gpu).contiguous()  # [E, 3, 4]
        # K2..K4 labels for w1 / w3, then for w2 (a codebook may depend on the rate axis)
        self.labels = torch.cat([rate_labels(codebook, rate_axis=rate13_axis, device=gpu),
                                 rate_labels(codebook, rate_axis=rate2_axis, device=gpu)]).contiguous()


_MOE_WORKSPACES: dict[tuple, torch.Tensor] = {}


def qsrt_expert_forward(
    x: torch.Tensor,
    route_ids: torch.Tensor,
    route_weights: torch.Tensor,
    experts: QSRTExperts,
    *,
    activation: str = "situ",
    beta: float = 4.0,
    linear_beta: float = 25.0,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Routed expert forward of a decode batch on QSRT experts
    (``kq_qsrt_moe_decode``): out[t] = sum_s w[t, s] act(x_t W1_e, x_t W3_e)
    W2_e for e = route_ids[t, s] in [0, experts), computed from the trellis
    words in fp32 - the expert MLP of scripts/closure_exl3_layer.py:557-598
    without the dense bf16 weights scripts/stream_k3_pytorch.py:771-775
    decodes first.  x [tokens, H]; route_ids / route_weights [tokens, topk]."""

    if activation not in ("situ", "swiglu"):
        raise ValueError("activation must be 'situ' or 'swiglu'")
    if x.ndim != 2 or x.shape[1] != experts.hidden:
        raise ValueError(f"x must be [tokens, {experts.hidden}]")
    if route_ids.shape != route_weights.shape or route_ids.ndim != 2 or route_ids.shape[0] != x.shape[0]:
        raise ValueError("route_ids and route_weights must be [tokens, topk]")
    if x.dtype not in N.DTYPE_CODES:
        raise TypeError("x must be bfloat16, float16 or float32")
    gpu = experts.device
    out_dtype = x.dtype if out_dtype is None else out_dtype
    host = None if x.is_cuda else x.device
    xg = x.to(gpu)
    xg = xg if xg.stride(1) == 1 else xg.contiguous()
    ids = N.aligned(route_ids.to(device=gpu, dtype=torch.int32), 4)
    wts = N.aligned(route_weights.to(device=gpu, dtype=torch.float32), 4)
    tokens, topk = ids.shape
    out = torch.empty(tokens, experts.hidden, dtype=out_dtype, device=gpu)
    if tokens:
        h_tiles, i_tiles = experts.hidden // TILE_CHANNELS, experts.inter // TILE_CHANNELS
        need = int(N.library().kq_qsrt_moe_workspace_size(tokens, topk, h_tiles, i_tiles))
        if need < 0:
            raise RuntimeError("kq_qsrt_moe_workspace_size: no HIP device")
        stream = N.stream(gpu)
        ws = _workspace(_MOE_WORKSPACES, (gpu, stream.value, tokens, topk, h_tiles, i_tiles), need, gpu)
        act = N.ACT_SITU if activation == "situ" else N.ACT_SWIGLU
        N.call("kq_qsrt_moe_decode", act, float(beta), float(linear_beta), N.ptr(xg), N.DTYPE_CODES[xg.dtype],
               tokens, xg.stride(0), N.ptr(ids), N.ptr(wts), topk, N.ptr(experts.descriptors), experts.experts,
               h_tiles, i_tiles, 0 if experts.rate13_axis == "k" else 1, 0 if experts.rate2_axis == "k" else 1,
               N.ptr(experts.labels), N.DTYPE_CODES[out_dtype], N.ptr(out), experts.hidden, N.ptr(ws), need,
               stream)
    return out if host is None else out.to(host)
