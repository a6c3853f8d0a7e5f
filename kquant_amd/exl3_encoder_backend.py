"""The Hessian finalize of kquant's trellis encoder, on the GPU.

Drop-in for these functions of ``kquant/exl3_encoder_backend.py`` (same
names, arguments, in-place behaviour and return values):

  ``blockwise_preapply_had_l_`` / ``blockwise_preapply_had_r_`` (:288-313)
      in-place blockwise Hadamard (``kq_blockwise_hadamard``; 128-wide
      Sylvester blocks, the ``had_k``/``had_n`` the encoder uses);
  ``block_ldl(H, b, quant_args, verbose)`` (:316-386)
      Cholesky with the reference's retry policy (on failure the diagonal
      grows by 2 * sigma_reg * mean(diag), at most 10 times), then the block
      LDL step; ``kq_cholesky`` + ``kq_block_ldl``.  Returns (L in H's
      device storage, H on the CPU) as the reference does;
  ``finalize_capture_H(H_data, quant_args, verbose)`` (:1588-1663)
      count division and diagonal regularization (``kq_h_regularize``),
      random sign flips su drawn exactly as the reference draws them
      (``torch.randn(k, device).sign()``), the two-sided rotation in one
      launch, block LDL with b = 16 and the zeroed diagonal.

``block_ldl_batched`` (no kquant counterpart) factors many experts' H2
matrices in one pass: every launch of the blocked Cholesky covers the whole
batch.  All work runs in ``libkquant_amd.so`` (fp32, as the reference);
without the library or a GPU every call raises.
"""

from __future__ import annotations

import threading

import torch

from . import _native as N

had_k, had_n = 128, 128
_MAX_CHOLESKY_RETRIES = 10


def _gpu_float_matrix(x: torch.Tensor, what: str) -> None:
    if x.dtype != torch.float32 or x.ndim != 2:
        raise ValueError(f"{what} must be a two-dimensional float32 tensor")
    if not x.is_cuda:
        raise ValueError(f"{what} must be a GPU tensor")
    if x.stride(1) != 1:
        raise ValueError(f"{what} rows must be contiguous")


def _hadamard_(x: torch.Tensor, had_dim: int, sides: int, rs=None, cs=None) -> None:
    if had_dim != had_k:
        raise ValueError(f"had_dim must be {had_k}")
    target = x if x.is_cuda else x.to(torch.cuda.current_device())
    _gpu_float_matrix(target, "x")
    rows, cols = target.shape
    N.call("kq_blockwise_hadamard", N.ptr(target), rows, cols, target.stride(0), 1, 0, sides,
           N.ptr(rs), N.ptr(cs), N.stream(target.device))
    if target is not x:
        x.copy_(target)


def blockwise_preapply_had_l_(x: torch.Tensor, had_dim):
    """x[blk, :] = had @ x[blk, :] for every 128-row block, in place."""
    k, n = x.shape
    assert k % had_dim == 0
    assert x.dtype == torch.float
    _hadamard_(x, had_dim, 1)


def blockwise_preapply_had_r_(x: torch.Tensor, had_dim):
    """x[:, blk] = x[:, blk] @ had for every 128-column block, in place."""
    k, n = x.shape
    assert n % had_dim == 0
    assert x.dtype == torch.float
    _hadamard_(x, had_dim, 2)


def _cholesky_(h: torch.Tensor, batch: int = 1) -> torch.Tensor:
    """In-place lower Cholesky of [batch, n, n] (or [n, n]); returns info."""
    n = h.shape[-1]
    ws = torch.empty(max(int(N.library().kq_cholesky_workspace_size(n, batch)), 256), dtype=torch.uint8,
                     device=h.device)
    info = torch.empty(batch, dtype=torch.int32, device=h.device)
    stride = n * h.stride(-2)
    N.call("kq_cholesky", N.ptr(h), h.stride(-2), stride, N.ptr(h), h.stride(-2), stride, n, batch,
           N.ptr(info), N.ptr(ws), ws.numel(), N.stream(h.device))
    return info


def _block_ldl_(lower: torch.Tensor, b: int, batch: int = 1, zero_diagonal: bool = False) -> None:
    n = lower.shape[-1]
    ws = torch.empty(max(int(N.library().kq_block_ldl_workspace_size(n, b, batch)), 256), dtype=torch.uint8,
                     device=lower.device)
    N.call("kq_block_ldl", N.ptr(lower), lower.stride(-2), n * lower.stride(-2), n, b, batch,
           N.LDL_ZERO_DIAGONAL if zero_diagonal else 0, N.ptr(ws), ws.numel(), N.stream(lower.device))


def _add_mean_diagonal_(h: torch.Tensor, sigma: float) -> None:
    """diag(h) += sigma * mean(diag(h)) in place (the retry damping)."""
    n = h.shape[0]
    mean = torch.empty(1, dtype=torch.float32, device=h.device)
    N.call("kq_h_regularize", N.ptr(h), n, h.stride(0), 0.0, float(sigma), None, N.ptr(mean), N.stream(h.device))


def block_ldl(H: torch.Tensor, b: int, quant_args: dict, verbose: bool):
    """Block LDL of a symmetric positive definite H (kquant/exl3_encoder_backend.py:316-386).

    Returns ``(L, H)``: L occupies H's device storage (unit block-lower, the
    b x b diagonal blocks identities) and H comes back as a CPU copy, as in
    the reference.  A failed factorization adds 2 * sigma_reg * mean(diag)
    to H's diagonal and retries, at most 10 times, then raises.
    """

    return _block_ldl_retrying(H, b, quant_args, zero_diagonal=False)


def _block_ldl_retrying(H: torch.Tensor, b: int, quant_args: dict, zero_diagonal: bool):
    _gpu_float_matrix(H, "H")
    n = H.shape[0]
    assert n % b == 0
    if H.shape != (n, n) or not H.is_contiguous():
        raise ValueError("H must be a contiguous square matrix")
    sigma_reg = quant_args.get("sigma_reg", 0.025)
    retries = 0
    while True:
        h_cpu = H.cpu()
        info = int(_cholesky_(H).item())
        if info == 0:
            break
        retries += 1
        if retries > _MAX_CHOLESKY_RETRIES:
            H.copy_(h_cpu)
            print(" ## Cholesky decomp. failed, number of retries exceeded")
            raise torch.linalg.LinAlgError(
                f"linalg.cholesky: The factorization could not be completed because the input is not "
                f"positive-definite (the leading minor of order {info} is not positive-definite).")
        print(f" !! Cholesky decomp. failed, increasing diagonal damping, attempt {retries}/10")
        H.copy_(h_cpu)
        _add_mean_diagonal_(H, 2.0 * sigma_reg)
    _block_ldl_(H, b, zero_diagonal=zero_diagonal)
    return H, h_cpu


def block_ldl_batched(H: torch.Tensor, b: int = 16) -> tuple[torch.Tensor, torch.Tensor]:
    """Block LDL of a stack of SPD matrices [E, n, n] in one pass (new API).

    Returns ``(L, info)``: L [E, n, n] (unit block-lower, identity diagonal
    blocks) and info int32 [E] (0, or the order of the first leading minor
    that is not positive definite, LAPACK's convention; that expert's L is
    then meaningless).  H is not modified.
    """

    if H.dtype != torch.float32 or H.ndim != 3 or H.shape[1] != H.shape[2] or not H.is_cuda:
        raise ValueError("H must be a float32 GPU tensor [experts, n, n]")
    experts, n, _ = H.shape
    if n % b:
        raise ValueError("n must be a multiple of b")
    lower = H.contiguous().clone()
    info = _cholesky_(lower, experts)
    _block_ldl_(lower, b, experts)
    return lower, info


finalize_capture_H_mutex = threading.Lock()


def finalize_capture_H(H_data: dict, quant_args: dict, verbose: bool):
    """kquant/exl3_encoder_backend.py:1588-1663 on the GPU.

    Returns ``(q_fallback, H, L, su, diag)`` and fills ``H_data`` as the
    reference does ("L", "finalized", "diag", "q_fallback", "su", "H")."""

    with finalize_capture_H_mutex:
        if H_data["H"].is_meta:
            H_data["L"] = None
            H_data["finalized"] = True
            H_data["diag"] = None
            H_data["q_fallback"] = True
            H = H_data["H"]
            k = H.shape[0]
            su = (torch.randn(k, device=H_data["device"]).sign() + 1e-5).sign().to(torch.float).unsqueeze(1)
            H_data["su"] = su
            return True, None, None, su, None

        if "H_swap_device" in H_data:
            H_data["H"] = H_data["H"].to(H_data["H_swap_device"])
            del H_data["H_swap_device"]

        H = H_data["H"]
        if H_data["finalized"]:
            return H_data["q_fallback"], H, H_data["L"], H_data["su"], H_data["diag"]
        _gpu_float_matrix(H, "H")
        if not H.is_contiguous():
            raise ValueError("H must be contiguous")
        k = H.shape[0]

        count = H_data["count"]
        sigma_reg = quant_args.get("sigma_reg", 0.025)
        if count == 0:
            q_fallback = True
        else:
            mean = torch.empty(1, dtype=torch.float32, device=H.device)
            N.call("kq_h_regularize", N.ptr(H), k, H.stride(0), float(count), float(sigma_reg), None,
                   N.ptr(mean), N.stream(H.device))
            q_fallback = float(mean.item()) < 1e-20
        diag = H.diagonal().clone()

        if verbose:
            print(f"     - H min/max: {H.min().item():.6f}   {H.max().item():.6f}")
            print(f"     - H mean/std: {H.mean().item():.6f}   {H.std().item():.6f}")
            print(f"     - H diag min/max: {diag.min():.6f}   {diag.max():.6f} ")

        su = (torch.randn(k, device=H.device).sign() + 1e-5).sign().to(torch.float).unsqueeze(1)
        H_data["su"] = su
        if k % had_k:
            raise ValueError(f"H dimension must be a multiple of {had_k}")
        sv = su.reshape(-1).contiguous()
        N.call("kq_blockwise_hadamard", N.ptr(H), k, k, H.stride(0), 1, 0, 3, N.ptr(sv), N.ptr(sv),
               N.stream(H.device))

        if q_fallback:
            L = None
        else:
            # block_ldl(H, 16) followed by L[dr, dr] = 0, the zeroing done in the same kernel
            L, H = _block_ldl_retrying(H, 16, quant_args, zero_diagonal=True)

        H_data["L"] = L
        H = H.cpu()
        H_data["H"] = H.cpu()
        H_data["finalized"] = True
        H_data["diag"] = diag
        H_data["q_fallback"] = q_fallback
        return q_fallback, H, L, su, diag
