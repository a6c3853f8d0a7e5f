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


def _syrk(x: torch.Tensor, weights: torch.Tensor | None, gpu: torch.device) -> torch.Tensor:
    """Upper-tile accumulator of X^T diag(w) X, [kp, kp] fp32 (kp = padded k)."""
    n, kp = x.shape
    acc = torch.empty(kp, kp, dtype=torch.float32, device=gpu)
    w = None
    if weights is not None:
        w = N.aligned(weights.detach().to(device=gpu, dtype=torch.float32))
    N.call("kq_syrk_accumulate", N.DTYPE_CODES[x.dtype], N.ptr(x), kp, n, kp, N.ptr(w),
           N.ptr(acc), kp, N.SYRK_OVERWRITE, N.stream(gpu))
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


def weighted_effective_sample_size(weights: torch.Tensor) -> float:
    """Kish effective sample size (kquant/candidate_hessian.py:141-153)."""

    if weights.ndim != 1 or not weights.numel():
        raise ValueError("weights must be a nonempty vector")
    if not torch.all(torch.isfinite(weights)) or torch.any(weights < 0):
        raise ValueError("weights must be finite and nonnegative")
    weights64 = weights.double()
    total = weights64.sum()
    squared_total = weights64.square().sum()
    if total <= 0 or squared_total <= 0:
        raise ValueError("weights must have positive effective support")
    return float(total.square() / squared_total)


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

    This is the parity metric itself (relative Frobenius difference in f64);
    it is evaluated with torch on the tensors' device.
    """

    if reference.ndim != 2 or reference.shape[0] != reference.shape[1]:
        raise ValueError("reference covariance must be square")
    if candidate.shape != reference.shape:
        raise ValueError("candidate covariance shape differs")
    reference = reference.float()
    candidate = candidate.float().to(reference.device)
    if not torch.all(torch.isfinite(reference)) or not torch.all(torch.isfinite(candidate)):
        raise ValueError("covariances must be finite")
    reference_norm = torch.linalg.vector_norm(reference.double())
    reference_diagonal = torch.diagonal(reference).double()
    candidate_diagonal = torch.diagonal(candidate).double()
    diagonal_denominator = torch.linalg.vector_norm(reference_diagonal) * torch.linalg.vector_norm(
        candidate_diagonal
    )
    trace = torch.trace(reference.double())
    return {
        "relative_frobenius_difference": float(
            torch.linalg.vector_norm((candidate - reference).double()) / reference_norm
        )
        if reference_norm > 0
        else math.inf,
        "trace_ratio": float(torch.trace(candidate.double()) / trace) if trace != 0 else math.inf,
        "diagonal_cosine_similarity": float(
            torch.dot(reference_diagonal, candidate_diagonal) / diagonal_denominator
        )
        if diagonal_denominator > 0
        else 0.0,
        "candidate_symmetry_max_abs": float((candidate - candidate.T).abs().max()),
    }
