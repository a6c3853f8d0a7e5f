"""Covariance / Hessian helpers of kquant's calibration (drop-in surface).

Same names, arguments, validation and return conventions as
``kquant/candidate_hessian.py``; the O(N K^2) accumulation runs in the bf16
MFMA SYRK kernel of libkquant_amd.so (``kq_syrk_accumulate``) and the
normalise / symmetrise / damp / shrink steps in HIP kernels as well.

Extensions that have no kquant counterpart:
  ``accumulate_hessian``  unnormalised accumulator (kquant/capture.py:713-730)
  ``damped_hessian``      sum(w x x^T)/sum(w) + damp*mean(diag)*I in one call
                          (the accumulation of candidate_hessian followed by
                          the damping of kquant/exl3_encoder_backend.py:1613-1625)
"""

from __future__ import annotations

import math

import torch

from . import _native as N


# ----------------------------------------------------------- validation --

def _validate_samples(rows: torch.Tensor, weights: torch.Tensor, chunk_rows: int) -> None:
    # kquant/candidate_hessian.py:80-89
    if rows.ndim != 2 or weights.ndim != 1 or rows.shape[0] != weights.shape[0]:
        raise ValueError("invalid covariance sample shapes")
    if not rows.shape[0] or not rows.shape[1]:
        raise ValueError("covariance samples must be nonempty")
    if chunk_rows <= 0:
        raise ValueError("chunk_rows must be positive")
    if not torch.all(torch.isfinite(rows)) or not torch.all(torch.isfinite(weights)):
        raise ValueError("covariance samples must be finite")
    if torch.any(weights < 0):
        raise ValueError("covariance weights must be nonnegative")


def _prepare_rows(rows: torch.Tensor, gpu: torch.device) -> tuple[torch.Tensor, int]:
    x = rows.detach().to(gpu)
    if x.dtype not in N.DTYPE_CODES:
        x = x.float()
    k = x.shape[1]
    if k % 8:
        # the kernel reads 8-feature groups; zero features add zero rows/cols
        x = torch.nn.functional.pad(x, (0, 8 - k % 8))
    x = N.aligned(x)
    return x, k


_SPLIT_WORKSPACES: dict[tuple[torch.device, int], torch.Tensor] = {}


def _split_workspace(gpu: torch.device, dtype_code: int, n: int, k: int, weighted: bool) -> torch.Tensor | None:
    """Partial-tile slots of the split launch (None when it does not pay),
    cached per device and stream: calls sharing slots must not overlap."""
    need = int(N.library().kq_syrk_accumulate_workspace_size(dtype_code, n, k, int(weighted)))
    if need <= 0:
        return None
    key = (gpu, torch.cuda.current_stream(gpu).stream_id)
    ws = _SPLIT_WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        _SPLIT_WORKSPACES[key] = ws
    return ws


def _syrk(x: torch.Tensor, weights: torch.Tensor | None, gpu: torch.device) -> torch.Tensor:
    """Upper-tile accumulator of X^T diag(w) X, [kp, kp] fp32 (kp = padded k)."""
    n, kp = x.shape
    acc = torch.empty(kp, kp, dtype=torch.float32, device=gpu)
    w = None
    if weights is not None:
        w = N.aligned(weights.detach().to(device=gpu, dtype=torch.float32))
    code = N.DTYPE_CODES[x.dtype]
    ws = _split_workspace(gpu, code, n, kp, w is not None)
    N.call("kq_syrk_accumulate_ws", code, N.ptr(x), kp, n, kp, N.ptr(w), N.ptr(acc), kp, N.SYRK_OVERWRITE,
           N.ptr(ws), 0 if ws is None else ws.numel(), N.stream(gpu))
    return acc


def _finalize(acc: torch.Tensor, denominator: float, damp: float, k: int) -> torch.Tensor:
    kp = acc.shape[0]
    out = torch.empty(kp, kp, dtype=torch.float32, device=acc.device)
    N.call("kq_syrk_finalize", N.ptr(acc), kp, kp, float(denominator), float(damp), N.ptr(out),
           kp, N.stream(acc.device))
    if kp != k:
        out = out[:k, :k].contiguous()
    return out


# ------------------------------------------------------------ public API --

def weighted_covariance(
    rows: torch.Tensor,
    weights: torch.Tensor,
    *,
    device: torch.device,
    chunk_rows: int = 256,
    return_cpu: bool = True,
) -> tuple[torch.Tensor, float]:
    """Return ``sum(w * x xT) / sum(w)`` as symmetric FP32.

    kquant/candidate_hessian.py:70-112.  The kernel streams all rows at once,
    so ``chunk_rows`` is validated but does not change the result's layout.
    The result lives on ``device`` (CPU when ``return_cpu``).
    """

    _validate_samples(rows, weights, chunk_rows)
    denominator = float(weights.double().sum())
    if not math.isfinite(denominator) or denominator <= 0:
        raise ValueError("covariance weights must have a positive finite sum")
    (gpu_rows,), gpu, _ = N.to_gpu([rows])
    x, k = _prepare_rows(gpu_rows, gpu)
    unit = bool(torch.all(weights == 1))
    acc = _syrk(x, None if unit else weights, gpu)
    covariance = _finalize(acc, denominator, 0.0, k)
    target = torch.device("cpu") if return_cpu else torch.device(device)
    covariance = covariance.to(target)
    if not torch.all(torch.isfinite(covariance)):
        raise ValueError("weighted covariance is non-finite")
    return covariance, denominator


def accumulate_hessian(
    rows: torch.Tensor,
    weights: torch.Tensor,
    *,
    device: torch.device,
    chunk_rows: int = 1024,
) -> tuple[torch.Tensor, float]:
    """Unnormalised accumulator ``sum(w x x^T)`` and ``sum(w)`` (f64).

    kquant/capture.py:713-730 (``_accumulate_hessian``).  The accumulator is
    returned exactly symmetric (the kernel computes one triangle).
    """

    if rows.ndim != 2 or weights.ndim != 1 or rows.shape[0] != weights.shape[0]:
        raise ValueError("invalid Hessian sample shapes")
    denominator = float(weights.double().sum())
    (gpu_rows,), gpu, _ = N.to_gpu([rows])
    x, k = _prepare_rows(gpu_rows, gpu)
    if rows.shape[0] == 0:
        return torch.zeros(k, k, dtype=torch.float32, device=device), 0.0
    acc = _syrk(x, weights, gpu)
    return _finalize(acc, 1.0, 0.0, k).to(device), denominator


def damped_hessian(
    rows: torch.Tensor,
    weights: torch.Tensor | None = None,
    *,
    damp: float = 0.01,
) -> tuple[torch.Tensor, float]:
    """``H = sum(w x x^T) / sum(w)`` symmetrised, then ``H.diag += damp *
    mean(diag(H))``, on the GPU.  ``weights=None`` means unit weights (the
    plain X^T X / N calibration Hessian)."""

    if rows.ndim != 2 or not rows.shape[0] or not rows.shape[1]:
        raise ValueError("covariance samples must be nonempty")
    (gpu_rows,), gpu, _ = N.to_gpu([rows])
    if weights is None:
        denominator = float(rows.shape[0])
    else:
        if weights.ndim != 1 or weights.shape[0] != rows.shape[0]:
            raise ValueError("invalid covariance sample shapes")
        denominator = float(weights.double().sum())
        if not math.isfinite(denominator) or denominator <= 0:
            raise ValueError("covariance weights must have a positive finite sum")
    x, k = _prepare_rows(gpu_rows, gpu)
    acc = _syrk(x, weights, gpu)
    return _finalize(acc, denominator, damp, k), denominator


def shrink_covariance(
    global_covariance: torch.Tensor,
    local_covariance: torch.Tensor,
    alpha: float,
) -> torch.Tensor:
    """Convexly shrink a low-support local covariance toward a global one.

    kquant/candidate_hessian.py:115-138: sym(lerp(global, local, alpha)).
    """

    alpha = float(alpha)
    if not math.isfinite(alpha) or not 0.0 <= alpha <= 1.0:
        raise ValueError("alpha must be finite and in [0, 1]")
    if (
        global_covariance.ndim != 2
        or global_covariance.shape[0] != global_covariance.shape[1]
        or local_covariance.shape != global_covariance.shape
    ):
        raise ValueError("global and local covariances must be equal-size squares")
    if not torch.all(torch.isfinite(global_covariance)) or not torch.all(
        torch.isfinite(local_covariance)
    ):
        raise ValueError("covariances must be finite")
    (g, l), gpu, host = N.to_gpu([global_covariance.float(), local_covariance.float()])
    g, l = g.contiguous(), l.contiguous()
    k = g.shape[0]
    out = torch.empty(k, k, dtype=torch.float32, device=gpu)
    N.call("kq_sym_lerp", N.ptr(g), 0.0, N.ptr(l), k, alpha, N.ptr(out), N.stream(gpu))
    return out if host is None else out.to(host)


def _weight_sums(w: torch.Tensor, offsets: torch.Tensor, groups: int, flags: int) -> torch.Tensor:
    out = torch.empty(groups, dtype=torch.float64, device=w.device if w is not None else offsets.device)
    N.call("kq_segment_weight_sums", N.ptr(w), N.ptr(offsets), groups, flags, N.ptr(out),
           N.stream(out.device))
    return out


def _single_group(n: int, gpu: torch.device) -> torch.Tensor:
    return torch.tensor([0, n], dtype=torch.int64, device=gpu)


def weighted_effective_sample_size(weights: torch.Tensor) -> float:
    """Kish effective sample size (kquant/candidate_hessian.py:141-153):
    (sum w)^2 / sum w^2 with both sums in f64 (``kq_segment_weight_sums``)."""

    if weights.ndim != 1 or not weights.numel():
        raise ValueError("weights must be a nonempty vector")
    (w,), gpu, _ = N.to_gpu([weights])
    if not torch.all(torch.isfinite(w)) or torch.any(w < 0):
        raise ValueError("weights must be finite and nonnegative")
    w = N.aligned(w.float(), 4)
    offsets = _single_group(w.numel(), gpu)
    total = float(_weight_sums(w, offsets, 1, 0).item())
    squared_total = float(_weight_sums(w, offsets, 1, N.SUM_SQUARE_F64).item())
    if total <= 0 or squared_total <= 0:
        raise ValueError("weights must have positive effective support")
    return total * total / squared_total


def adaptive_identity_shrinkage(
    local_covariance: torch.Tensor,
    weights: torch.Tensor,
    *,
    max_local_alpha: float = 0.75,
) -> tuple[torch.Tensor, dict[str, float]]:
    """Shrink a weighted local covariance toward its scaled identity.

    kquant/candidate_hessian.py:156-216 (Oracle Approximating Shrinkage with
    the Kish effective sample size; target trace(local)/dimension * I).  The
    f64 trace and sum of squares come from ``kq_cov_stats``; the blend runs in
    ``kq_sym_lerp``.
    """

    max_local_alpha = float(max_local_alpha)
    if not math.isfinite(max_local_alpha) or not 0.0 <= max_local_alpha <= 1.0:
        raise ValueError("max_local_alpha must be finite and in [0, 1]")
    if local_covariance.ndim != 2 or (local_covariance.shape[0] != local_covariance.shape[1]):
        raise ValueError("local covariance must be square")
    if not torch.all(torch.isfinite(local_covariance)):
        raise ValueError("local covariance must be finite")

    effective_rows = weighted_effective_sample_size(weights)
    dimension = int(local_covariance.shape[0])
    (local,), gpu, host = N.to_gpu([local_covariance.float()])
    local = local.contiguous()
    ws = torch.empty(2 * N.COV_STATS_PARTS, dtype=torch.float64, device=gpu)
    stats = torch.empty(2, dtype=torch.float64, device=gpu)
    N.call("kq_cov_stats", N.ptr(local), dimension, N.ptr(ws), N.ptr(stats), N.stream(gpu))
    local_trace, sum_sq = (float(v) for v in stats.cpu())
    if local_trace <= 0:
        raise ValueError("local covariance trace must be positive")

    mu = local_trace / dimension
    mean_square = sum_sq / (dimension * dimension)
    denominator = (effective_rows + 1.0) * (mean_square - mu * mu / dimension)
    if denominator <= 0:
        oas_shrinkage = 1.0
    else:
        oas_shrinkage = min(1.0, max(0.0, float((mean_square + mu * mu) / denominator)))
    local_alpha = min(max_local_alpha, 1.0 - oas_shrinkage)
    identity_scale = float(mu)
    out = torch.empty(dimension, dimension, dtype=torch.float32, device=gpu)
    # the reference builds eye(dimension) * fp32(identity_scale)
    N.call("kq_sym_lerp", N.ptr(None), float(torch.tensor(identity_scale, dtype=torch.float32)),
           N.ptr(local), dimension, local_alpha, N.ptr(out), N.stream(gpu))
    blended = out if host is None else out.to(host)
    return blended, {
        "effective_sample_size": effective_rows,
        "oas_shrinkage": oas_shrinkage,
        "local_alpha": local_alpha,
        "max_local_alpha": max_local_alpha,
        "identity_scale": identity_scale,
    }


def covariance_comparison(reference: torch.Tensor, candidate: torch.Tensor) -> dict[str, float]:
    """Compact scale/shape diagnostics (kquant/candidate_hessian.py:219-258).

    This is the parity metric itself: the relative Frobenius difference, trace
    ratio and diagonal cosine from f64 sums (``kq_covariance_comparison_sums``),
    and the candidate's largest asymmetry.
    """

    if reference.ndim != 2 or reference.shape[0] != reference.shape[1]:
        raise ValueError("reference covariance must be square")
    if candidate.shape != reference.shape:
        raise ValueError("candidate covariance shape differs")
    (r, c), gpu, _ = N.to_gpu([reference, candidate])
    r, c = r.float().contiguous(), c.float().contiguous()
    if not torch.all(torch.isfinite(r)) or not torch.all(torch.isfinite(c)):
        raise ValueError("covariances must be finite")
    k = r.shape[0]
    ws = torch.empty(256 * 8, dtype=torch.float64, device=gpu)
    out = torch.empty(8, dtype=torch.float64, device=gpu)
    N.call("kq_covariance_comparison_sums", N.ptr(r), N.ptr(c), k, N.ptr(ws), N.ptr(out),
           N.stream(gpu))
    s_dd, s_rr, tr_r, tr_c, d_rr, d_cc, d_rc, asym = (float(v) for v in out.cpu().tolist())
    reference_norm = math.sqrt(s_rr)
    diagonal_denominator = math.sqrt(d_rr) * math.sqrt(d_cc)
    return {
        "relative_frobenius_difference": math.sqrt(s_dd) / reference_norm
        if reference_norm > 0
        else math.inf,
        "trace_ratio": tr_c / tr_r if tr_r != 0 else math.inf,
        "diagonal_cosine_similarity": d_rc / diagonal_denominator
        if diagonal_denominator > 0
        else 0.0,
        "candidate_symmetry_max_abs": float(torch.tensor(asym, dtype=torch.float32)),
    }


# -------------------------------------------------------- per-expert Hessians --

def _grouped(x: torch.Tensor, k: int, offsets: torch.Tensor, groups: int, index, weights,
             flags: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Finalized [groups, k, k] covariances and f64 denominators [groups]."""
    gpu = x.device
    kp = x.shape[1]
    acc = torch.empty(groups, kp, kp, dtype=torch.float32, device=gpu)
    N.call("kq_syrk_grouped", N.DTYPE_CODES[x.dtype], N.ptr(x), kp, N.ptr(offsets), groups, N.ptr(index),
           N.ptr(weights), kp, N.ptr(acc), flags, N.stream(gpu))
    sq = N.SYRK_SQUARE_WEIGHTS if flags & N.SYRK_SQUARE_WEIGHTS else 0
    denominators = _weight_sums(weights, offsets, groups, sq)
    out = torch.empty_like(acc)
    N.call("kq_syrk_finalize_grouped", N.ptr(acc), kp, groups, N.ptr(denominators), N.ptr(out),
           N.stream(gpu))
    del acc
    if kp != k:
        out = out[:, :k, :k].contiguous()
    return out, denominators


def expert_hessians(
    inputs: torch.Tensor,
    route_ids: torch.Tensor,
    gates: torch.Tensor,
    experts: int,
    *,
    gate_square: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Every expert's gate^2-weighted covariance of the token rows routed to it.

    ``inputs`` [T, K]; ``route_ids`` / ``gates`` [T, topk].  Expert e gets
    sum(g^2 x x^T) / sum(g^2) over its routed rows in token order, exactly the
    ``weighted_covariance(rows_e, gates_e.square())`` that
    ``build_expert_hessians`` (kquant/qsrt_candidates.py:534-586) forms per
    expert, for all experts in one routing sort and one grouped SYRK launch.
    Returns (H [E, K, K] fp32, denominators [E] f64, row counts [E] int64);
    experts without rows get zeros and denominator 0.
    """

    if inputs.ndim != 2 or route_ids.ndim != 2 or route_ids.shape != gates.shape:
        raise ValueError("inputs must be [T, K] and route_ids / gates [T, topk]")
    if route_ids.shape[0] != inputs.shape[0]:
        raise ValueError("route_ids rows must match inputs")
    (x, ids, g), gpu, _ = N.to_gpu([inputs, route_ids, gates])
    x, k = _prepare_rows(x, gpu)
    tokens, topk = map(int, ids.shape)
    ids = N.aligned(ids.to(torch.int32), 4)
    g = N.aligned(g.float(), 4)
    lib = N.library()
    ws = torch.empty(max(int(lib.kq_route_sort_workspace_size(tokens, topk, experts)), 256),
                     dtype=torch.uint8, device=gpu)
    offsets = torch.empty(experts + 1, dtype=torch.int64, device=gpu)
    rows = torch.empty(max(tokens * topk, 1), dtype=torch.int32, device=gpu)
    sorted_w = torch.empty(max(tokens * topk, 1), dtype=torch.float32, device=gpu)
    N.call("kq_route_sort", N.ptr(ids), tokens, topk, experts, N.ptr(g), N.ptr(offsets), N.ptr(rows),
           None, N.ptr(sorted_w), N.ptr(ws), ws.numel(), N.stream(gpu))
    flags = N.SYRK_SQUARE_WEIGHTS if gate_square else 0
    h, denominators = _grouped(x, k, offsets, experts, rows, sorted_w, flags)
    return h, denominators, offsets[1:] - offsets[:-1]


def expert_hessians_from_rows(
    rows: torch.Tensor,
    offsets: torch.Tensor,
    weights: torch.Tensor | None = None,
    *,
    square_weights: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-group covariances of rows already grouped by expert.

    ``rows`` [P, K] with group g at rows [offsets[g], offsets[g+1]) (the
    per-expert post-SiTU rows of the H2 fit, kquant/qsrt_candidates.py:
    577-583), optional row ``weights`` [P] (squared first when
    ``square_weights``).  Returns (H [G, K, K], denominators [G] f64).
    """

    if rows.ndim != 2 or offsets.ndim != 1 or offsets.numel() < 2:
        raise ValueError("rows must be [P, K] and offsets [G + 1]")
    host_offsets = offsets.detach().to("cpu", torch.int64)
    if (int(host_offsets[0]) != 0 or bool((host_offsets[1:] < host_offsets[:-1]).any())
            or int(host_offsets[-1]) > rows.shape[0]):
        raise ValueError("offsets must rise from 0 to at most the number of rows")
    if weights is not None and (weights.ndim != 1 or weights.shape[0] < int(host_offsets[-1])):
        raise ValueError("weights must cover every grouped row")
    (x, o, w), gpu, _ = N.to_gpu([rows, offsets, weights])
    x, k = _prepare_rows(x, gpu)
    o = N.aligned(o.to(torch.int64), 8)
    if w is not None:
        w = N.aligned(w.float(), 4)
    flags = N.SYRK_SQUARE_WEIGHTS if square_weights else 0
    return _grouped(x, k, o, int(o.numel()) - 1, None, w, flags)


def build_expert_hessians(
    inputs: torch.Tensor,
    gates: torch.Tensor,
    source_middle: torch.Tensor,
    *,
    global_h13: torch.Tensor,
    global_h2: torch.Tensor,
    device: torch.device,
    h13_alpha: float = 0.0,
    h2_alpha: float | None = None,
    chunk_rows: int = 256,
    max_local_alpha: float = 0.75,
) -> tuple[torch.Tensor, torch.Tensor, dict[str, float | str]]:
    """H13 and support-aware post-SiTU H2 of one expert
    (kquant/qsrt_candidates.py:534-618; defaults are the reference's PHASE1
    constants kquant/qsrt.py:204-209: h13_alpha 0, H2 weighted OAS toward the
    scaled identity capped at 0.75).  Weights are gates^2."""

    if inputs.ndim != 2 or inputs.shape[0] != gates.shape[0]:
        raise ValueError("invalid expert input covariance samples")
    if source_middle.ndim != 2 or source_middle.shape[0] != inputs.shape[0]:
        raise ValueError("source middle rows do not match expert inputs")
    if global_h2.shape != (source_middle.shape[1], source_middle.shape[1]):
        raise ValueError("global H2 dimension does not match source middle rows")
    (g,), gpu, _ = N.to_gpu([gates])
    g = N.aligned(g.float().contiguous(), 4)
    offsets = _single_group(int(g.numel()), gpu)
    h13_weight = float(_weight_sums(g, offsets, 1, N.SYRK_SQUARE_WEIGHTS).item())
    global_h13 = global_h13.to(device=device, dtype=torch.float32)
    if h13_alpha == 0.0:
        h13 = global_h13
    else:
        local_h13, _ = expert_hessians_from_rows(inputs, offsets, g, square_weights=True)
        h13 = shrink_covariance(global_h13, local_h13[0], h13_alpha).to(device)
    local_h2, h2_den = expert_hessians_from_rows(source_middle, offsets, g, square_weights=True)
    h2_weight = float(h2_den[0].item())
    if not math.isclose(h13_weight, h2_weight, rel_tol=1e-9, abs_tol=1e-12):
        raise ValueError("H13 and H2 expert covariance weights differ")
    local_h2 = local_h2[0]
    if h2_alpha is None:
        square = (g * g).contiguous()
        h2, shrinkage = adaptive_identity_shrinkage(local_h2, square, max_local_alpha=max_local_alpha)
        evidence: dict[str, float | str] = {
            "h2_shrinkage_policy": "weighted_oas_scaled_identity",
            "h2_local_alpha": shrinkage["local_alpha"],
            "h2_local_alpha_cap": shrinkage["max_local_alpha"],
            "h2_effective_sample_size": shrinkage["effective_sample_size"],
            "h2_oas_shrinkage": shrinkage["oas_shrinkage"],
            "h2_identity_scale": shrinkage["identity_scale"],
        }
    else:
        dimension = local_h2.shape[0]
        ws = torch.empty(2 * N.COV_STATS_PARTS, dtype=torch.float64, device=gpu)
        stats = torch.empty(2, dtype=torch.float64, device=gpu)
        N.call("kq_cov_stats", N.ptr(local_h2), dimension, N.ptr(ws), N.ptr(stats), N.stream(gpu))
        identity_scale = float(torch.tensor(float(stats[0].item()), dtype=torch.float32)) / dimension
        h2 = torch.empty_like(local_h2)
        N.call("kq_sym_lerp", None, float(torch.tensor(identity_scale, dtype=torch.float32)),
               N.ptr(local_h2), dimension, float(h2_alpha), N.ptr(h2), N.stream(gpu))
        evidence = {
            "h2_shrinkage_policy": "fixed_alpha_scaled_identity",
            "h2_local_alpha": float(h2_alpha),
            "h2_local_alpha_cap": float(h2_alpha),
            "h2_identity_scale": identity_scale,
        }
    return h13, h2.to(device), {"gate_square_sum": h13_weight, "h13_local_alpha": float(h13_alpha),
                                **evidence}
