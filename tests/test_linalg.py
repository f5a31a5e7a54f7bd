"""Blocked dense linear algebra of the matrix quantizer (ltq_amd.linalg) against float64 LAPACK: the recursive
Cholesky (src/liqk_v2.py:1079), the recursive triangular inverse that replaces solve_triangular(L, I)
(src/liqk_v2.py:1081) and the SPD solve of the suh refit (src/liqk_v2.py:1163), at sizes whose recursion
splits unevenly (not multiples of the leaf)."""
import pytest

torch = pytest.importorskip("torch")


def _spd(n, seed, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn((n // 2, n), generator=g, dtype=torch.float64)
    return (X.T @ X / n + 0.1 * torch.eye(n, dtype=torch.float64)).float().to(device)


def _check(n, leaf, nb, device):
    from ltq_amd import linalg
    A = _spd(n, n, device)
    L, info = linalg.cholesky_lower(A, leaf=leaf)
    assert int(info) == 0
    Lr = torch.linalg.cholesky(A.double().cpu())
    Lc = L.double().cpu()
    assert torch.equal(Lc, torch.tril(Lc))
    # backward error of a float32 Cholesky (of the order of sqrt(n) u |A| for any order of the sums; a wrong
    # update or solve gives O(|A|)), then the forward error against LAPACK in float64
    Ad = A.double().cpu()
    assert (Lc @ Lc.T - Ad).abs().max() <= 1e-5 * Ad.abs().max()
    assert (Lc - Lr).abs().max() <= 2e-6 * Lr.abs().max()
    Li = linalg.tri_inv_lower(L, leaf=leaf).double().cpu()
    assert torch.equal(Li, torch.tril(Li))
    assert (Li @ Lc - torch.eye(n, dtype=torch.float64)).abs().max() <= 1e-5
    b = torch.randn(n, generator=torch.Generator().manual_seed(1)).to(device)
    x = linalg.spd_solve(A, b, nb=nb).double().cpu()
    xr = torch.linalg.solve(A.double().cpu(), b.double().cpu())
    assert (x - xr).norm() <= 1e-5 * xr.norm()


@pytest.mark.parametrize("n,leaf,nb", [(300, 128, 64), (1100, 256, 200), (777, 2048, 512)])
def test_blocked_linalg_cpu(n, leaf, nb):
    _check(n, leaf, nb, "cpu")


def test_spd_solve_falls_back_to_lu_for_indefinite():
    from ltq_amd import linalg
    A = torch.diag(torch.tensor([2.0, -1.0, 3.0]))
    b = torch.tensor([2.0, 1.0, 3.0])
    assert torch.allclose(linalg.spd_solve(A, b), torch.tensor([1.0, -1.0, 1.0]))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [5000, 2304])
def test_blocked_linalg_gpu(n):
    print(f"blocked linalg n={n}", flush=True)
    _check(n, 2048 if n > 2304 else 512, 512, "cuda")


@pytest.mark.parametrize("m,n,nb", [(50, 300, 64), (33, 257, 100)])
def test_gram_lower_is_the_lower_triangle_of_the_product(m, n, nb):
    from ltq_amd import linalg
    g = torch.Generator().manual_seed(n)
    A = torch.randn((m, n), generator=g, dtype=torch.float64)
    B = A * torch.rand((m, 1), generator=g, dtype=torch.float64)  # diag(w) A: the product is symmetric
    C = linalg.gram_lower(A, B, nb=nb)
    full = A.T @ B
    assert torch.allclose(torch.tril(C), torch.tril(full), rtol=1e-12, atol=1e-12)
    # every block row is formed up to the end of its diagonal block, nothing to the right of it
    for i in range(0, n, nb):
        assert torch.all(C[i:i + nb, min(n, i + nb):] == 0)


def test_spd_solve_reads_only_the_lower_triangle():
    from ltq_amd import linalg
    A = _spd(300, 5)
    b = torch.randn(300, generator=torch.Generator().manual_seed(6))
    junk = A + torch.triu(torch.full_like(A, 7.0), 1)
    x = linalg.spd_solve(junk, b, nb=64).double()
    xr = torch.linalg.solve(A.double(), b.double())
    assert (x - xr).norm() <= 1e-5 * xr.norm()
    # indefinite: the LU fallback rebuilds the symmetric matrix from the lower triangle
    Ai = torch.tensor([[2.0, 99.0], [1.0, -1.0]])
    assert torch.allclose(linalg.spd_solve(Ai, torch.tensor([3.0, 0.0])), torch.tensor([1.0, 1.0]))


@pytest.mark.gpu
def test_recursive_cholesky_without_magma_gpu():
    """The recursive factorization the device falls back to without MAGMA (leaves of at least 1024 rows through
    the batched potrf, L21 by triangular solve, Schur complements by GEMM): info 0 and a float32 backward error."""
    from ltq_amd import linalg
    n = 5000
    A = _spd(n, 11, "cuda")
    print(f"recursive cholesky n={n}", flush=True)
    L, info = linalg.cholesky_lower(A, leaf=256, magma=False)  # leaves are kept at >= 1024 rows on the device
    assert int(info) == 0
    Lc, Ad = torch.tril(L).double().cpu(), A.double().cpu()
    assert (Lc @ Lc.T - Ad).abs().max() <= 1e-5 * Ad.abs().max()
