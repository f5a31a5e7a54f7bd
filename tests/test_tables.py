"""Table training for extended-label formats (src/universal_bench.py:85-116): the closed-form start and the Lloyd
step on the GPU Viterbi.

CPU: the start is the N(0, spread^2) quantile grid in the reference's subset-major layout (pinned against
scipy's normal quantiles and the layout rule: subset j holds points j, j + nl, ...).
GPU: one Lloyd step against the C oracle's Viterbi and a float64 centroid update (codes bit-exact; the table to
the rounding of the device's fp32 index_add sums), and a short training run on the C4 format (K=3 D4, 16
subsets, h=3 with 4 gain candidates) that must lower the quantization error of the closed-form start.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

C4_MASKS = (40, 475)  # extra masks of the 16-subset K=3 D4 format of the MoE config (primary 359)


def test_closed_form_table_is_the_quantile_grid():
    from scipy.stats import norm
    from ltq_amd.tables import closed_form_table
    for K, me in ((3, C4_MASKS), (2, ()), (4, (241,))):
        nl, U = 4 << len(me), 1 << (K - 1)
        n = nl * U
        tab = closed_form_table(K, me, spread=1.3, device="cpu").numpy()
        grid = (1.3 * norm.ppf((np.arange(n) + 0.5) / n)).astype(np.float32)
        for j in range(nl):
            assert np.allclose(tab[j * U:(j + 1) * U], grid[j::nl], rtol=1e-6, atol=1e-6)
        assert np.all(np.diff(tab.reshape(nl, U), axis=1) > 0)


def _lloyd_ref(x, tab, gains, K, m_extra, n_cand, pp):
    from oracle import ref
    nl, U = 4 << len(m_extra), 1 << (K - 1)
    _, gi, lev = ref.viterbi_ub_cuda_ref(x, tab, K, 10, 359, gains, sub=16, n_cand=n_cand, tail_biting=True,
                                         m_extra=m_extra, pair_parity=pp, return_code=True)
    j, gv, xf = lev.reshape(-1).astype(np.int64), gains[gi.reshape(-1)].astype(np.float64), x.reshape(-1)
    num = np.zeros(tab.size)
    den = np.zeros(tab.size)
    np.add.at(num, j, gv * xf)
    np.add.at(den, j, gv * gv)
    new = np.where(den > 0, num / np.maximum(den, 1e-12), tab)
    return np.sort(new.reshape(nl, U), axis=1).reshape(-1), (gi.astype(np.int64) << 16) | lev


@pytest.mark.gpu
def test_gpu_lloyd_step_vs_oracle():
    from ltq_amd.tables import closed_form_table, lloyd_step
    from ltq_amd.tcq_proto import make_gains
    K, me, h, pp = 3, C4_MASKS, 3, 2
    rng = np.random.default_rng(5)
    x = rng.standard_normal((96, 256)).astype(np.float32)
    x /= np.sqrt(np.square(x).mean(axis=1, keepdims=True))
    tab = closed_form_table(K, me, device="cpu").numpy()
    gains = make_gains(h, 0.15, "cpu").numpy()
    print("lloyd step C4 format", flush=True)
    new, codes = lloyd_step(torch.from_numpy(x).cuda(), torch.from_numpy(tab).cuda(), torch.from_numpy(gains).cuda(),
                            K, me, 4, pp=pp)
    torch.cuda.synchronize()
    want_tab, want_codes = _lloyd_ref(x, tab, gains, K, me, 4, pp)
    assert np.array_equal(codes.cpu().numpy().astype(np.int64), want_codes)
    assert np.allclose(new.cpu().numpy(), want_tab, rtol=2e-5, atol=1e-6)


@pytest.mark.gpu
def test_gpu_train_tcq_x_lowers_error():
    from ltq_amd.tables import closed_form_table, train_tcq_x
    from ltq_amd.tcq_proto import make_gains, viterbi_ub_cuda
    K, me, h, pp = 3, C4_MASKS, 3, 2
    print("train_tcq_x C4 format, 3 iterations", flush=True)
    tab, gains, n_cand = train_tcq_x(K, h, 0.15, me, iters=3, n_tiles=512, pp=pp)
    assert n_cand == 4 and tab.numel() == 64 and gains.numel() == 8
    x = torch.randn((256, 256), generator=torch.Generator(device="cuda").manual_seed(77), device="cuda")
    x = x / x.square().mean(dim=1, keepdim=True).sqrt()

    def mse(t):
        rec = viterbi_ub_cuda(x, t, K, 10, 359, gains, sub=16, n_cand=n_cand, tail_biting=True, m_extra=me,
                              pair_parity=pp)
        return float((rec - x).square().mean())

    e0, e1 = mse(closed_form_table(K, me)), mse(tab)
    torch.cuda.synchronize()
    assert e1 < e0, (e0, e1)
