"""Input-covariance accumulation (src/liqk_v2.py:207-231): the oracle pinned on the CPU, the gfx950 kernel
(ltq_cov_accumulate / ltq_cov_finalize through ltq_amd.hessian.CovAccumulator) against it on the GPU.

Tolerance of the GPU path: within a batch of m rows the kernel sums exact products in fp32, so every entry of
the batch's X^T X is within gamma_m = m u / (1 - m u) (u = 2^-24) of the exact sum, relative to the entry of
|X|^T |X| (the textbook bound for any summation order); the fp64 running sum adds nothing measurable and get()
rounds once more to fp32 (half an ulp). Inputs whose partial sums are all exact in fp32 (small integers) must
match bit for bit."""
import numpy as np
import pytest
import torch

from oracle.cov_ref import CovAccumulatorRef, cov_loop

DEV = "cuda"
U32 = 2.0 ** -24


# ---- oracle pins (CPU) ------------------------------------------------------------------------------------

def test_oracle_matches_loop_on_tiny_inputs():
    rng = np.random.default_rng(3)
    for n, K in ((1, 1), (3, 4), (7, 5)):
        x = rng.standard_normal((n, K)).astype(np.float32)
        acc = CovAccumulatorRef()
        acc.add(x)
        np.testing.assert_allclose(acc.H, np.array(cov_loop(x)), rtol=1e-12, atol=1e-12)


def test_oracle_closed_forms():
    # one-hot rows: H = diag(row counts) / n
    idx = np.array([0, 2, 2, 5, 5, 5, 1])
    x = np.eye(6, dtype=np.float32)[idx]
    acc = CovAccumulatorRef()
    acc.add(x)
    np.testing.assert_array_equal(acc.get(), np.diag(np.bincount(idx, minlength=6) / len(idx)).astype(np.float32))
    # constant rows c: H = c^2 everywhere
    acc = CovAccumulatorRef()
    acc.add(np.full((10, 3), 1.5, dtype=np.float32))
    np.testing.assert_array_equal(acc.get(), np.full((3, 3), 2.25, dtype=np.float32))
    # rows a u and b v with u, v orthonormal: H = (sum a^2 u u^T + sum b^2 v v^T) / n
    u = np.array([0.6, 0.8, 0.0])
    v = np.array([0.0, 0.0, 1.0])
    x = np.stack([2 * u, -3 * v, 1 * u])
    acc = CovAccumulatorRef()
    acc.add(x)
    np.testing.assert_allclose(acc.H, 5 * np.outer(u, u) + 9 * np.outer(v, v), atol=1e-12)


def test_oracle_batching_and_leading_dims():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 6, 5))
    a, b = CovAccumulatorRef(), CovAccumulatorRef()
    a.add(x)
    b.add(x[0])
    b.add(x[1, :2])
    b.add(x[1, 2:])
    assert a.n == b.n == 12
    np.testing.assert_allclose(a.H, b.H, rtol=1e-13)


def test_oracle_get_scales_by_reciprocal_count():
    acc = CovAccumulatorRef()
    acc.add(np.ones((3, 1)))
    assert acc.get()[0, 0] == np.float32(3.0 * (1.0 / 3.0))
    empty = CovAccumulatorRef()
    empty.add(np.zeros((0, 2)))
    np.testing.assert_array_equal(empty.get(), np.zeros((2, 2), np.float32))


# ---- GPU parity -------------------------------------------------------------------------------------------

def _bound(ref: CovAccumulatorRef, batches, m_max: int):
    gamma = m_max * U32 / (1 - m_max * U32)
    scale = ref.abs_sum(batches) / max(ref.n, 1)
    return gamma * scale + U32 * np.abs(ref.H / max(ref.n, 1)) + 1e-30


def _run(batches, dtype):
    from ltq_amd.hessian import CovAccumulator
    acc, ref, host = CovAccumulator(), CovAccumulatorRef(), []
    for b in batches:
        xd = b.to(DEV, dtype)
        acc.add(xd)
        hb = xd.float().cpu().numpy()
        ref.add(hb)
        host.append(hb)
    out = acc.get()
    torch.cuda.synchronize()
    return acc, ref, host, out


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,K", [(64, 8), (512, 256), (512, 392)])
def test_gpu_cov_exact_on_small_integers(n, K, dtype):
    """Small-integer inputs: every partial sum is exact in fp32, so the result is the exact one, bit for bit
    (n is a power of two, so the reciprocal scaling is exact too)."""
    g = torch.Generator().manual_seed(n + K)
    x = torch.randint(-4, 5, (n, K), generator=g).float()
    print(f"cov exact n={n} K={K} {dtype}", flush=True)
    _, ref, _, out = _run([x], dtype)
    np.testing.assert_array_equal(out.cpu().numpy(), ref.get())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shapes", [
    [(1, 8)],                       # one row
    [(31, 100)],                    # K % 8 != 0: element loads, ragged last tile
    [(300, 200), (45, 200)],        # two batches, partial chunks
    [(1000, 1031)],                 # K not a multiple of 128 or 8
    [(2048, 768), (2048, 768)],     # C4 down_proj Hessian size
    [(4096, 2048)],
])
def test_gpu_cov_random_within_fp32_bound(shapes, dtype):
    g = torch.Generator().manual_seed(sum(n * 7 + K for n, K in shapes))
    batches = [torch.randn((n, K), generator=g) * 2.0 for n, K in shapes]
    print(f"cov random {shapes} {dtype}", flush=True)
    acc, ref, host, out = _run(batches, dtype)
    got = out.cpu().numpy().astype(np.float64)
    bound = _bound(ref, host, max(n for n, _ in shapes))
    err = np.abs(got - ref.H / max(ref.n, 1))
    assert (err <= bound).all(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.3f}"
    assert torch.equal(out, out.T)  # read from one triangle
    assert acc.n == sum(n for n, _ in shapes)


@pytest.mark.gpu
def test_gpu_cov_get_matches_torch_device_scaling():
    """get() is the reference's `(H / n).to(float32)` on the device, bit for bit, for the same fp64 sum."""
    from ltq_amd.hessian import CovAccumulator
    g = torch.Generator().manual_seed(11)
    acc = CovAccumulator()
    for n in (300, 77):  # 377 rows: the reciprocal is inexact
        acc.add(torch.randn((n, 520), generator=g).to(DEV, torch.bfloat16))
    low = torch.tril(acc.H)
    Hsym = low + torch.tril(low, -1).T
    want = (Hsym / max(acc.n, 1)).to(torch.float32)
    got = acc.get()
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.gpu
def test_gpu_cov_strided_and_batched_inputs():
    """[B, S, K] activations and row-strided views give the same sums as the contiguous rows."""
    from ltq_amd.hessian import CovAccumulator
    g = torch.Generator().manual_seed(12)
    wide = torch.randn((96, 400), generator=g).to(DEV, torch.bfloat16)
    a, b = CovAccumulator(), CovAccumulator()
    a.add(wide[:, :264])                   # row stride 400, 16-byte aligned rows
    a.add(wide[:, 8:272].view(8, 12, 264))  # offset view, 3-D
    a.add(wide[:, 1:265])                  # misaligned rows: element loads
    b.add(wide[:, :264].contiguous())
    b.add(wide[:, 8:272].contiguous())
    b.add(wide[:, 1:265].contiguous())
    torch.cuda.synchronize()
    assert a.n == b.n == 288
    assert torch.equal(a.get(), b.get())


@pytest.mark.gpu
def test_gpu_cov_fp32_batches_and_mixing():
    """fp32 batches take the reference's fp32 GEMM; mixed with bf16 batches the sums still agree with the
    oracle to fp32 rounding."""
    from ltq_amd.hessian import CovAccumulator
    g = torch.Generator().manual_seed(13)
    x1, x2 = torch.randn((200, 136), generator=g), torch.randn((50, 136), generator=g)
    acc, ref = CovAccumulator(), CovAccumulatorRef()
    acc.add(x1.to(DEV))
    acc.add(x2.to(DEV, torch.bfloat16))
    ref.add(x1.numpy())
    ref.add(x2.to(torch.bfloat16).float().numpy())
    got = acc.get().cpu().numpy()
    np.testing.assert_allclose(got, ref.get(), rtol=2e-5, atol=2e-5 * np.abs(ref.get()).max())


@pytest.mark.gpu
def test_gpu_cov_c3_size_against_fp64_gemm():
    """The benchmark's H (2048 N(0,1) bf16 rows, K = 14336) against an fp64 device GEMM of the same rows."""
    from ltq_amd.hessian import CovAccumulator
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn((2048, 14336), generator=g, device=DEV).to(torch.bfloat16)
    acc = CovAccumulator()
    print("cov C3 2048 x 14336", flush=True)
    acc.add(x)
    got = acc.get().double()
    xd = x.double()
    want = (xd.T @ xd) / 2048
    bound = (2048 * U32 * 1.001) * ((xd.abs().T @ xd.abs()) / 2048) + U32 * want.abs()
    del xd
    ok = bool(((got - want).abs() <= bound).all())
    torch.cuda.synchronize()
    assert ok
