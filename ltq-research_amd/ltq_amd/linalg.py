"""Dense linear algebra of the matrix quantizer, arranged so that almost all flops land in large library GEMMs
(hipBLASLt / rocBLAS on MI355X) instead of the launch-bound panel kernels of an unblocked factorization.

  cholesky_lower   A = L L^T. On the device, matrices above `leaf` rows go to MAGMA's blocked hybrid potrf
                   (torch's magma backend; rocSOLVER's unblocked panels make its potrf launch-bound at these
                   sizes); otherwise, and where MAGMA is absent, recursive 2 x 2 blocking: L11 = chol(A11),
                   L21 = A21 L11^-T (trsm), L22 = chol(A22 - L21 L21^T), leaves to torch.linalg.cholesky_ex.
                   Used for src/liqk_v2.py:1079 (the flipped, damped Hessian) and for the SPD system of the
                   suh refit (src/liqk_v2.py:1163).
  tri_inv_lower    L^-1 for lower-triangular L, recursive: [[A, 0], [B, C]]^-1 = [[A^-1, 0], [-C^-1 B A^-1, C^-1]].
                   Replaces solve_triangular(L, I) (src/liqk_v2.py:1081) at a third of the flops.
  spd_solve        A x = b through cholesky_lower and two blocked substitutions; falls back to the LU solve
                   of src/liqk_v2.py:1163 when A is not numerically positive definite.

All results agree with the unblocked routines to fp32 rounding (the order of the sums differs, as it does
between any two BLAS libraries).
"""
from __future__ import annotations

from typing import Tuple

import torch


def _split(n: int) -> int:
    h = (n // 2) // 256 * 256
    return h if h > 0 else n // 2


_MAGMA = [None]


def _magma_cholesky(A: torch.Tensor):
    """torch.linalg.cholesky_ex through the magma backend, or None where the build has no MAGMA."""
    if _MAGMA[0] is False:
        return None
    prev = torch.backends.cuda.preferred_linalg_library()
    try:
        torch.backends.cuda.preferred_linalg_library("magma")
        L, info = torch.linalg.cholesky_ex(A)
        _MAGMA[0] = True
        return L, info.to(torch.int64)
    except RuntimeError:
        _MAGMA[0] = False
        return None
    finally:
        torch.backends.cuda.preferred_linalg_library(prev)


def cholesky_lower(A: torch.Tensor, leaf: int = 2048, magma: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """(L, info): lower Cholesky factor of symmetric A (only its lower triangle is read) and an int tensor that is
    0 when the factorization succeeded."""
    n = A.shape[0]
    if magma and A.is_cuda and n > leaf:
        r = _magma_cholesky(A)
        if r is not None:
            return r
    if n <= leaf:
        L, info = torch.linalg.cholesky_ex(A)
        return L, info.to(torch.int64)
    h = _split(n)
    L = torch.zeros_like(A)
    L11, i1 = cholesky_lower(A[:h, :h], leaf, False)
    L[:h, :h] = L11
    L21 = torch.linalg.solve_triangular(L11.T, A[h:, :h], upper=True, left=False)
    L[h:, :h] = L21
    S = torch.addmm(A[h:, h:], L21, L21.T, alpha=-1.0)
    L22, i2 = cholesky_lower(S, leaf, False)
    L[h:, h:] = L22
    return L, i1.abs() + i2.abs()


def tri_inv_lower(L: torch.Tensor, leaf: int = 1024) -> torch.Tensor:
    """Inverse of a lower-triangular matrix (its strict upper triangle must be zero)."""
    n = L.shape[0]
    if n <= leaf:
        return torch.linalg.solve_triangular(L, torch.eye(n, dtype=L.dtype, device=L.device), upper=False)
    h = _split(n)
    out = torch.zeros_like(L)
    Ai = tri_inv_lower(L[:h, :h], leaf)
    Ci = tri_inv_lower(L[h:, h:], leaf)
    out[:h, :h] = Ai
    out[h:, h:] = Ci
    out[h:, :h] = -(Ci @ (L[h:, :h] @ Ai))
    return out


def _solve_lower_vec(L: torch.Tensor, b: torch.Tensor, nb: int) -> torch.Tensor:
    n = L.shape[0]
    x = torch.empty_like(b)
    for i in range(0, n, nb):
        j = min(n, i + nb)
        r = b[i:j] - L[i:j, :i] @ x[:i] if i else b[i:j]
        x[i:j] = torch.linalg.solve_triangular(L[i:j, i:j], r.unsqueeze(1), upper=False).squeeze(1)
    return x


def _solve_upper_vec(Ut: torch.Tensor, b: torch.Tensor, nb: int) -> torch.Tensor:
    n = Ut.shape[0]
    x = torch.empty_like(b)
    for j in range(n, 0, -nb):
        i = max(0, j - nb)
        r = b[i:j] - Ut[i:j, j:] @ x[j:] if j < n else b[i:j]
        x[i:j] = torch.linalg.solve_triangular(Ut[i:j, i:j], r.unsqueeze(1), upper=True).squeeze(1)
    return x


def spd_solve(A: torch.Tensor, b: torch.Tensor, nb: int = 512) -> torch.Tensor:
    """x with A x = b for symmetric positive definite A [n, n], b [n]; LU solve when the Cholesky fails."""
    L, info = cholesky_lower(A)
    if int(info.item()) != 0:
        return torch.linalg.solve(A, b)
    y = _solve_lower_vec(L, b, nb)
    return _solve_upper_vec(L.T, y, nb)
