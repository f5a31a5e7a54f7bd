"""Dense linear algebra of the matrix quantizer, arranged so that almost all flops land in large library GEMMs
(hipBLASLt / rocBLAS on MI355X) instead of the launch-bound panel kernels of an unblocked factorization.

  cholesky_lower   A = L L^T. On the device, matrices above `leaf` rows go to MAGMA's blocked hybrid potrf
                   (torch's magma backend; rocSOLVER's unblocked panels make its potrf launch-bound at these
                   sizes); otherwise, and where MAGMA is absent, recursive 2 x 2 blocking: L11 = chol(A11),
                   L21 = A21 L11^-T (trsm), L22 = chol(A22 - L21 L21^T), leaves to torch.linalg.cholesky_ex.
                   Used for src/liqk_v2.py:1079 (the flipped, damped Hessian) and for the SPD system of the
                   suh refit (src/liqk_v2.py:1163).
  tri_inv_lower    L^-1 for lower-triangular L, recursive: [[A, 0], [B, C]]^-1 = [[A^-1, 0], [-C^-1 B A^-1, C^-1]],
                   the two products with triangular factors themselves recursive (n^3 / 3 flops in all).
                   Replaces solve_triangular(L, I) (src/liqk_v2.py:1081).
  spd_solve        A x = b through cholesky_lower and two blocked substitutions; falls back to the LU solve
                   of src/liqk_v2.py:1163 when A is not numerically positive definite.
  cholesky_many    the factors of a batch of matrices of up to `leaf` rows in one batched device call (MoE
                   experts: 128 factorizations of 2048 rows take 16 ms against 6 ms each one by one). The
                   device's batched potrf (MAGMA) gives each matrix the same bits whatever batch it is in (two or
                   more), but its single-matrix potrf is another algorithm; so a lone matrix up to `leaf` rows
                   is factored as a batch of two (itself twice), and a matrix factors to the same bits alone or
                   in a batch.

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


LEAF = 2048


def cholesky_many(A: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(L, info) [B, n, n], [B] for symmetric A [B, n, n] (lower triangles read), n <= LEAF: one batched call; on
    the device a batch of one goes as a batch of two, so each factor has the bits of the batched algorithm."""
    if A.is_cuda and A.shape[0] == 1:
        L, info = torch.linalg.cholesky_ex(A.expand(2, -1, -1).contiguous())
        return L[:1], info[:1].to(torch.int64)
    L, info = torch.linalg.cholesky_ex(A)
    return L, info.to(torch.int64)


def cholesky_lower(A: torch.Tensor, leaf: int = LEAF, magma: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """(L, info): lower Cholesky factor of symmetric A (only its lower triangle is read) and an int tensor that is
    0 when the factorization succeeded."""
    n = A.shape[0]
    if magma and A.is_cuda and n > leaf:
        r = _magma_cholesky(A)
        if r is not None:
            return r
    if A.is_cuda:
        # on the device the recursion has been measured correct with leaves of 1024 and 2048 rows (and 128) but
        # failing (info != 0) with leaves of 256 and of 512 at K = 14336, cause not found; keep leaves >= 1024
        leaf = max(leaf, 1024)
    if n <= leaf:
        L, info = cholesky_many(A.unsqueeze(0))
        return L[0], info[0]
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


def _trmm_right_lower(B: torch.Tensor, T: torch.Tensor, out: torch.Tensor, leaf: int) -> None:
    """out = B T for lower-triangular T [h, h] (strict upper triangle zero), B [m, h]:
    [B1 B2] [[T11, 0], [T21, T22]] = [B1 T11 + B2 T21, B2 T22], recursively, so the zero triangle costs no flops
    above the leaf size."""
    h = T.shape[0]
    if h <= leaf:
        out.addmm_(B, T, beta=0.0)
        return
    s = _split(h)
    _trmm_right_lower(B[:, :s], T[:s, :s], out[:, :s], leaf)
    out[:, :s].addmm_(B[:, s:], T[s:, :s])
    _trmm_right_lower(B[:, s:], T[s:, s:], out[:, s:], leaf)


def _trmm_left_lower(T: torch.Tensor, B: torch.Tensor, out: torch.Tensor, leaf: int) -> None:
    """out = T B for lower-triangular T [h, h], B [h, m]: [[T11, 0], [T21, T22]] [B1; B2] = [T11 B1; T21 B1 + T22 B2]."""
    h = T.shape[0]
    if h <= leaf:
        out.addmm_(T, B, beta=0.0)
        return
    s = _split(h)
    _trmm_left_lower(T[:s, :s], B[:s], out[:s], leaf)
    _trmm_left_lower(T[s:, s:], B[s:], out[s:], leaf)
    out[s:].addmm_(T[s:, :s], B[:s])


def tri_inv_lower(L: torch.Tensor, leaf: int = 1024) -> torch.Tensor:
    """Inverse of a lower-triangular matrix (its strict upper triangle must be zero). The off-diagonal block
    -C^-1 (B A^-1) is two triangular-times-full products, each done recursively on the triangle (half the flops of
    full GEMMs)."""
    n = L.shape[0]
    if n <= leaf:
        return torch.linalg.solve_triangular(L, torch.eye(n, dtype=L.dtype, device=L.device), upper=False)
    h = _split(n)
    out = torch.zeros_like(L)
    Ai = tri_inv_lower(L[:h, :h], leaf)
    Ci = tri_inv_lower(L[h:, h:], leaf)
    out[:h, :h] = Ai
    out[h:, h:] = Ci
    BA = torch.empty((n - h, h), dtype=L.dtype, device=L.device)
    _trmm_right_lower(L[h:, :h], Ai, BA, leaf)
    CBA = torch.empty_like(BA)
    _trmm_left_lower(Ci, BA, CBA, leaf)
    out[h:, :h] = CBA.neg_()
    return out


def _diag_block_inverses(L: torch.Tensor, nb: int) -> list:
    """Inverses of the nb x nb diagonal blocks of lower-triangular L (the last one ragged), full blocks in one
    batched triangular solve."""
    n = L.shape[0]
    nfull = n // nb
    out = []
    if nfull:
        blocks = torch.stack([L[i * nb:(i + 1) * nb, i * nb:(i + 1) * nb] for i in range(nfull)])
        eye = torch.eye(nb, dtype=L.dtype, device=L.device).expand(nfull, nb, nb)
        out = list(torch.linalg.solve_triangular(blocks, eye, upper=False).unbind(0))
    if n % nb:
        i = nfull * nb
        out.append(torch.linalg.solve_triangular(L[i:, i:], torch.eye(n - i, dtype=L.dtype, device=L.device),
                                                 upper=False))
    return out


def _solve_lower_vec(L: torch.Tensor, b: torch.Tensor, nb: int, Dinv=None) -> torch.Tensor:
    """L x = b, right-looking by nb-row blocks: x_i = L_ii^-1 r_i, then r[j:] -= L[j:, i:j] x_i (a tall matrix-
    vector product over the rows below the block)."""
    n = L.shape[0]
    Dinv = _diag_block_inverses(L, nb) if Dinv is None else Dinv
    x = b.clone()
    for k, i in enumerate(range(0, n, nb)):
        j = min(n, i + nb)
        x[i:j] = Dinv[k] @ x[i:j]
        if j < n:
            x[j:].addmv_(L[j:, i:j], x[i:j], alpha=-1.0)
    return x


def _solve_upper_vec(Ut: torch.Tensor, b: torch.Tensor, nb: int, Dinv=None) -> torch.Tensor:
    """Ut x = b for Ut = L^T (upper), from the last block up: x_i = (L_ii^-1)^T r_i, then r[:i] -= L[i:j, :i]^T
    x_i."""
    L = Ut.T
    n = L.shape[0]
    Dinv = _diag_block_inverses(L, nb) if Dinv is None else Dinv
    x = b.clone()
    starts = list(range(0, n, nb))
    for k in range(len(starts) - 1, -1, -1):
        i = starts[k]
        j = min(n, i + nb)
        x[i:j] = Dinv[k].T @ x[i:j]
        if i > 0:
            x[:i].addmv_(L[i:j, :i].T, x[i:j], alpha=-1.0)
    return x


def gram_lower(A: torch.Tensor, B: torch.Tensor, nb: int = 2048) -> torch.Tensor:
    """C = A^T B [n, n] for A, B [m, n] with C symmetric (B = diag(w) A or the like): only the block rows' parts
    on and left of the diagonal are multiplied (A[:, I]^T B[:, :end of I]); the strict upper triangle of C beyond
    them is zero."""
    n = A.shape[1]
    C = torch.zeros((n, n), dtype=A.dtype, device=A.device)
    for i in range(0, n, nb):
        j = min(n, i + nb)
        C[i:j, :j] = A[:, i:j].T @ B[:, :j]
    return C


def spd_solve(A: torch.Tensor, b: torch.Tensor, nb: int = 512) -> torch.Tensor:
    """x with A x = b for symmetric positive definite A [n, n] (only its lower triangle is read), b [n]; LU solve
    of the symmetric matrix when the Cholesky fails."""
    return spd_solve_factored(A, b, *cholesky_lower(A), nb=nb)


def spd_solve_factored(A: torch.Tensor, b: torch.Tensor, L: torch.Tensor, info: torch.Tensor,
                       nb: int = 512) -> torch.Tensor:
    """spd_solve with A's Cholesky factor (L, info) already computed (e.g. by cholesky_many)."""
    if int(info.item()) != 0:
        full = torch.tril(A) + torch.tril(A, -1).T
        return torch.linalg.solve(full, b)
    Dinv = _diag_block_inverses(L, nb)
    y = _solve_lower_vec(L, b, nb, Dinv)
    return _solve_upper_vec(L.T, y, nb, Dinv)
