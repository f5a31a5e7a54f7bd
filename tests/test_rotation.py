"""FWHT-256, Rademacher signs and suh (src/iqk_format.py:153-179, src/liqk_v2.py:409-441).

CPU: the oracle's FWHT against the reference's golden vectors (bit pattern of the butterfly tree) and
against the Sylvester-Hadamard matrix in float64 (closed form); the signs against the reference's draws.
GPU: the HIP kernels (rows with fused widening / divide / multiply, columns) bit-exact against the oracle.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")


def _hadamard(n):
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def test_oracle_fwht_matches_reference_golden(oracle, golden_dir):
    z = np.load(golden_dir / "fwht.npz")
    y = oracle.fwht256_ref(z["x"])
    assert np.array_equal(y.view(np.uint32), z["y"].view(np.uint32))


def test_oracle_fwht_closed_form_and_involution(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 512)).astype(np.float32)
    y = oracle.fwht256_ref(x)
    H = _hadamard(256) / 16.0  # normalized Sylvester matrix: the transform in natural (Hadamard) order
    ref = (x.reshape(-1, 256).astype(np.float64) @ H.T).reshape(x.shape)
    assert np.abs(y - ref).max() < 1e-5 * np.abs(ref).max()
    back = oracle.fwht256_ref(y)
    assert np.abs(back - x).max() < 1e-5

    # the closed form is sensitive to the plausible mistakes: a sign swapped in one stage, a stage skipped
    def butterflies(v, swap=-1, skip=-1):
        v = v.reshape(-1, 256).astype(np.float64).copy()
        h, k = 1, 0
        while h < 256:
            w = v.reshape(-1, 256 // (2 * h), 2, h)
            a, b = w[:, :, 0, :].copy(), w[:, :, 1, :].copy()
            if k != skip:
                w[:, :, 0, :], w[:, :, 1, :] = (a - b, a + b) if k == swap else (a + b, a - b)
            h, k = 2 * h, k + 1
        return (v / 16.0).reshape(x.shape)
    assert np.abs(butterflies(x) - ref).max() < 1e-9 * np.abs(ref).max()
    assert np.abs(butterflies(x, swap=3) - ref).max() > 0.1
    assert np.abs(butterflies(x, skip=7) - ref).max() > 0.1


def test_rademacher_signs_match_reference_draws(golden_dir):
    from ltq_amd.rotation import make_rademacher_signs
    z = np.load(golden_dir / "signs.npz")
    for key in z.files:
        dim, seed = map(int, key.split("_"))
        s = make_rademacher_signs(dim, seed, "cpu").numpy()
        assert set(np.unique(s)) <= {-1.0, 1.0}
        assert np.array_equal(np.packbits(s > 0), z[key]), key


# ---------------------------------------------------------------------------------------------- GPU
DEV = "cuda"


def _u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.gpu
def test_gpu_fwht_golden(golden_dir):
    from ltq_amd.rotation import fwht_inplace
    z = np.load(golden_dir / "fwht.npz")
    y = fwht_inplace(torch.tensor(z["x"], device=DEV))
    torch.cuda.synchronize()
    assert np.array_equal(_u32(y.cpu().numpy()), _u32(z["y"]))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_gpu_fwht_rows_fused_scale(oracle, dtype, mode):
    from ltq_amd.rotation import fwht_rows
    g = torch.Generator().manual_seed(5 + mode)
    rows, cols = 37, 1280
    x = (torch.randn((rows, cols), generator=g) * torch.logspace(-2, 2, cols)).to(dtype)
    s = (torch.rand(cols, generator=g) * 3 + 0.25) * (torch.randint(0, 2, (cols,), generator=g) * 2 - 1)
    s = s.to(torch.float16).float()
    print(f"fwht rows dtype={dtype} mode={mode} shape={rows}x{cols}", flush=True)
    y = fwht_rows(x.to(DEV), s.to(DEV), mode=mode)
    torch.cuda.synchronize()
    xf = x.float()
    pre = xf if mode == 0 else (xf / s if mode == 1 else xf * s)
    assert np.array_equal(_u32(y.cpu().numpy()), _u32(oracle.fwht256_ref(pre.numpy())))


@pytest.mark.gpu
@pytest.mark.parametrize("cols", [32, 77, 128, 300, 448])
@pytest.mark.parametrize("mode", [0, 2])
def test_gpu_fwht_cols_matches_transposed_rows(oracle, cols, mode):
    """fwht_cols(x, s) == fwht_inplace(x.T * s).T of the reference (the second side of H, liqk_v2.py:440)."""
    from ltq_amd.rotation import fwht_cols
    g = torch.Generator().manual_seed(cols)
    x = torch.randn((512, cols), generator=g)
    s = torch.rand(512, generator=g) + 0.5
    print(f"fwht cols mode={mode} shape=512x{cols}", flush=True)
    y = fwht_cols(x.to(DEV), s.to(DEV), mode=mode)
    torch.cuda.synchronize()
    pre = x.T.contiguous() * (s if mode else 1.0)
    ref = oracle.fwht256_ref(pre.numpy()).T
    assert np.array_equal(_u32(y.cpu().numpy()), _u32(ref))


@pytest.mark.gpu
def test_suh_ref_pins():
    """The oracle's suh: float64 definition (sign = Rademacher sign, |suh| the fp16 rounding of the clamped scale
    computed in float64 by torch), the clamp at 0.25 / 4, row weights, and flips against the reference's fp32
    text only on fp16 rounding boundaries (none expected at these sizes)."""
    from oracle import liqk_ref
    from ltq_amd.rotation import make_rademacher_signs
    g = torch.Generator().manual_seed(9)
    M, K = 96, 1024
    W = torch.randn((M, K), generator=g) * 0.02
    W[:, 5] *= 100      # clamps at 4
    W[:, 6] *= 1e-4     # clamps at 0.25
    X = torch.randn((300, K), generator=g)
    H = X.T @ X / 300
    s = liqk_ref.suh_ref(W, H, seed=1337)
    signs = make_rademacher_signs(K, 1337, "cpu").numpy()
    assert np.array_equal(np.sign(s), signs)
    cr = W.double().square().mean(0).sqrt()
    cr = cr / cr.mean()
    hs = H.double().diagonal().sqrt()
    hs = hs / hs.mean()
    sc = (cr.sqrt() * hs.pow(-0.25)).clamp(0.25, 4.0)
    assert np.array_equal(np.abs(s), sc.to(torch.float16).float().numpy())
    assert abs(s[5]) == 4.0 and abs(s[6]) == 0.25
    flips = int((torch.from_numpy(s) != liqk_ref.suh_torch_fp32(W, H)).sum())
    print(f"suh: {flips} of {K} differ from the fp32 torch text")
    assert flips <= K // 200
    # row weights: uniform weights give the unweighted scale; a weighted row moves the column rms
    assert np.array_equal(liqk_ref.suh_ref(W, H, row_weights=np.full(M, 3.0)), s)
    rw = np.ones(M)
    rw[0] = 100.0
    assert not np.array_equal(liqk_ref.suh_ref(W, H, row_weights=rw), s)


@pytest.mark.gpu
def test_gpu_compute_optimal_suh(oracle):
    """suh and the rotated W / H of the reference recipe, with H rotated on both sides by the kernels."""
    from ltq_amd.rotation import compute_optimal_suh, make_rademacher_signs
    g = torch.Generator().manual_seed(9)
    M, K = 64, 512
    W = (torch.randn((M, K), generator=g) * 0.02).to(torch.bfloat16)
    X = torch.randn((300, K), generator=g)
    H = X.T @ X / 300
    W_rot, H_rot, suh = compute_optimal_suh(W.to(DEV), H.to(DEV), seed=1337)
    torch.cuda.synchronize()
    from oracle import liqk_ref
    suh_c = suh.cpu()
    signs = make_rademacher_signs(K, 1337, "cpu")
    assert torch.equal(torch.sign(suh_c), signs)
    assert np.array_equal(_u32(suh_c.numpy()), _u32(liqk_ref.suh_ref(W, H, seed=1337)))  # bit-exact
    # given the device's suh, the rotations are exact
    Wr = oracle.fwht256_ref((W.float() / suh_c).numpy())
    assert np.array_equal(_u32(W_rot.cpu().numpy()), _u32(Wr))
    Ht = oracle.fwht256_ref((H * suh_c).numpy())
    Hr = oracle.fwht256_ref((torch.tensor(Ht).T.contiguous() * suh_c).numpy()).T
    assert np.array_equal(_u32(H_rot.cpu().numpy()), _u32(Hr))
