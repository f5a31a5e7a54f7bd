"""lut_subs_quant, the second export of the reference C ABI (src/cuda/tcq_viterbi.cu:768-811; caller
src/liqk_v2.py:497-500 via src/tcq_proto.py:537-548).

No reference fixture records the CUDA kernel's outputs, so the oracle (oracle/ltq_oracle.c) is pinned by what
the definition fixes: the float64 argmin of the weighted error (apart from near-ties), agreement with the
reference's torch path quantize_subs_lut_chunked (src/liqk_v2.py:445-466, restated below) apart from near-ties,
the first-minimum tie rule, the per-position weights, round-half-to-even buckets and the clamp. The HIP kernel
must equal the oracle bit for bit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

NB = 8192


def _case(S, seed):
    rng = np.random.default_rng(seed)
    max_g = 3.0
    inv_step = (NB - 1) / (2.0 * max_g)
    half_b = (NB - 1) * 0.5
    centers = (np.arange(NB) - half_b) / inv_step
    lut = (centers[:, None] + rng.normal(0, 0.05, (NB, 64))).astype(np.float32)
    xs = rng.normal(0, 1.0, (S, 16)).astype(np.float32)
    dh = rng.uniform(0.1, 2.0, (S, 16)).astype(np.float32)
    return xs, dh, lut, np.float32(inv_step), np.float32(half_b)


def _torch_path(xs, dh, lut, inv_step, half_b):
    """src/liqk_v2.py:445-466 (quantize_subs_lut_chunked): separate multiply and add, torch's sum order."""
    x = torch.from_numpy(xs)
    b = (x * float(inv_step) + float(half_b)).round().long().clamp(0, NB - 1)
    g = torch.from_numpy(lut)[b]
    bc = ((x.unsqueeze(-1) - g).square() * torch.from_numpy(dh).unsqueeze(-1)).sum(dim=1).argmin(dim=-1)
    return g[torch.arange(x.shape[0]), :, bc].numpy()


def _err64(xs, dh, lut, inv_step, half_b):
    # bucket of a fused multiply-add rounded once to fp32 (x * inv_step is exact in float64)
    fma32 = (xs.astype(np.float64) * np.float64(inv_step) + np.float64(half_b)).astype(np.float32)
    b = np.clip(np.rint(fma32), 0, NB - 1).astype(np.int64)
    g = lut[b].astype(np.float64)  # [S, 16, 64]
    return ((xs[..., None] - g) ** 2 * dh[..., None]).sum(axis=1), b


def _chosen(out, lut, b):
    """candidate index whose values are out (first match)."""
    g = lut[b]  # [S, 16, 64]
    eq = (g == out[..., None]).all(axis=1)
    return eq.argmax(axis=1)


def test_oracle_is_the_weighted_argmin():
    from oracle import ref
    xs, dh, lut, inv, hb = _case(4000, 1)
    out = ref.lut_subs_ref(xs, dh, lut, inv, hb)
    e64, b = _err64(xs, dh, lut, inv, hb)
    c = _chosen(out, lut, b)
    best = e64.min(axis=1)
    assert np.all(e64[np.arange(len(c)), c] <= best * (1 + 1e-5) + 1e-12)
    exact = e64.argmin(axis=1) == c
    assert exact.mean() > 0.99


def test_oracle_agrees_with_reference_torch_path():
    from oracle import ref
    xs, dh, lut, inv, hb = _case(4000, 2)
    out = ref.lut_subs_ref(xs, dh, lut, inv, hb)
    tp = _torch_path(xs, dh, lut, inv, hb)
    same = (out == tp).all(axis=1)
    assert same.mean() > 0.995
    e64, b = _err64(xs, dh, lut, inv, hb)
    for i in np.nonzero(~same)[0]:  # only near-ties (or a bucket flip at a rounding boundary) may differ
        ea = ((xs[i].astype(np.float64) - out[i]) ** 2 * dh[i]).sum()
        eb = ((xs[i].astype(np.float64) - tp[i]) ** 2 * dh[i]).sum()
        assert abs(ea - eb) <= 1e-4 * max(ea, eb)


def test_oracle_ties_weights_rounding_and_clamp():
    from oracle import ref
    inv, hb = np.float32(2.0), np.float32(4.0)
    lut = np.tile(np.arange(64, dtype=np.float32) * 0.01, (9, 1))
    lut[:, 7] = lut[:, 3] = -5.0  # a tie between candidates 3 and 7: the first wins
    xs = np.full((5, 16), -5.0, np.float32)
    dh = np.ones((5, 16), np.float32)
    xs[1] = 0.05  # nearest value is candidate 5
    xs[2, :8], xs[2, 8:] = 0.05, 0.62  # equal weights: candidate ~33; weights on the first half only: 5
    dh[2, 8:] = 0.0
    xs[3] = 0.25  # 0.25 * 2 + 4 = 4.5 -> bucket 4 (half to even)
    xs[4] = 1e30  # clamps to the last bucket
    out = ref.lut_subs_ref(xs, dh, lut, inv, hb)
    assert np.all(out[0] == -5.0) and np.all(out[1] == lut[0, 5]) and np.all(out[2] == lut[0, 5])
    lut2 = lut.copy()
    lut2[4] += 100.0  # bucket 4 stands out: a row of x = 0.25 must read it (not bucket 5)
    assert np.all(np.isin(ref.lut_subs_ref(xs[3:4], dh[3:4], lut2, inv, hb), lut2[4]))
    lut3 = lut.copy()
    lut3[8] += 200.0
    # the last bucket; every error overflows to inf, so the strict '<' scan keeps candidate 0
    assert np.all(ref.lut_subs_ref(xs[4:5], dh[4:5], lut3, inv, hb) == lut3[8, 0])


# ---------------------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
def test_gpu_lut_subs_matches_oracle():
    from oracle import ref
    from ltq_amd.tcq_proto import lut_subs_quant_cuda
    xs, dh, lut, inv, hb = _case(20001, 3)
    xs[5, 3] = np.nan  # a NaN weight position: every error of the sub-block is NaN -> candidate 0
    xs[6, 0] = np.inf
    xs[7] = 1e30
    xs[8] = -1e30
    lut[:, 9] = lut[:, 2]  # ties everywhere between candidates 2 and 9
    dh[10] = 0.0  # all-zero weights: every error 0 -> candidate 0
    print("lut_subs_quant S=20001", flush=True)
    out = lut_subs_quant_cuda(torch.from_numpy(xs).cuda(), torch.from_numpy(dh).cuda(), torch.from_numpy(lut).cuda(),
                              float(inv), float(hb)).cpu().numpy()
    torch.cuda.synchronize()
    want = ref.lut_subs_ref(xs, dh, lut, inv, hb)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_gpu_lut_subs_argument_checks():
    from ltq_amd import _lib
    x = torch.zeros((4, 16), device="cuda")
    t = torch.zeros((8, 64), device="cuda")
    L, st = _lib.lib(), _lib.stream_ptr()
    # no sub-blocks: the reference's zero-block launch error (9), on which its caller raises
    assert L.lut_subs_quant(x.data_ptr(), x.data_ptr(), t.data_ptr(), x.data_ptr(), 0, 1.0, 0.0, 8, st) == 9
    assert L.lut_subs_quant(x.data_ptr(), x.data_ptr(), t.data_ptr(), x.data_ptr(), -1, 1.0, 0.0, 8, st) == -1
    assert L.lut_subs_quant(x.data_ptr(), x.data_ptr(), t.data_ptr(), x.data_ptr(), 4, 1.0, 0.0, 0, st) == -1
    torch.cuda.synchronize()
