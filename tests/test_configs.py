"""BASELINE configs as parity cases at reduced sizes (the bench runs C3; C2 / C3 formats run through the matrix
path in tests/test_liqk.py, C5 rings in tests/test_rings.py).

C1 (Gaussian rig, K=2, 4 subsets, h=2 gain per 16, FWHT-256 rows, no Hessian; the reference's trained table
results/universal_gaussian.json["tcq_K2_h2"], committed as tests/golden/c1_tcq_K2_h2.json): the free-start
Viterbi of the reference's CPU rig bit-exact against the oracle, and the tail-biting run packed into .ltq tiles
that decode bit-exactly to the quantizer's values.
C4 (MoE experts, K=3 D4 with 16 subsets, h=3 with 4 gain candidates; no trained table exists, so the closed-form
start of src/universal_bench.py:91-94): the matrix path's two-pass tail-biting Viterbi with per-position weights
bit-exact against the oracle.
"""
import json

import numpy as np
import pytest

torch = pytest.importorskip("torch")


def _c1_format(golden_dir):
    from ltq_amd.formats import LtqFormat
    from ltq_amd.tcq_proto import make_gains
    d = json.loads((golden_dir / "c1_tcq_K2_h2.json").read_text())
    return LtqFormat("C1_K2_h2", 2, 0, (359,), 2, float(d["step"]), 16, np.asarray(d["tab"], np.float32),
                     make_gains(2, float(d["step"]), "cpu").numpy())


def test_c1_table_fixture_shape(golden_dir):
    f = _c1_format(golden_dir)
    assert f.lut.shape == (8,) and f.gain_tab.shape == (4,) and f.n_labels == 4 and f.U == 2


@pytest.mark.gpu
def test_gpu_c1_gaussian_rig(golden_dir):
    from oracle import pack, ref
    from ltq_amd import rotation
    from ltq_amd.ltq_file import pack_slice
    from ltq_amd.tcq_proto import viterbi_ub_cuda
    f = _c1_format(golden_dir)
    W = torch.randn((64, 1024), generator=torch.Generator().manual_seed(0))
    print("C1 rig 64 x 1024", flush=True)
    Wr = rotation.fwht_rows(W.cuda())
    Wr_ref = ref.fwht256_ref(W.numpy())
    assert np.array_equal(Wr.cpu().numpy().view(np.uint32), Wr_ref.view(np.uint32))
    lut, gains = torch.from_numpy(f.lut).cuda(), torch.from_numpy(f.gain_tab).cuda()
    # the reference CPU rig: free start over 256-value rows
    x = Wr.reshape(-1, 256)
    rec, gi, idx = viterbi_ub_cuda(x, lut, 2, 10, 359, gains, sub=16, return_code=True)
    r_ref, g_ref, i_ref = ref.viterbi_ub_cuda_ref(Wr_ref.reshape(-1, 256), f.lut, 2, 10, 359, f.gain_tab, sub=16,
                                                  return_code=True)
    assert np.array_equal(rec.cpu().numpy().view(np.uint32), np.asarray(r_ref, np.float32).view(np.uint32))
    assert np.array_equal(gi.cpu().numpy(), g_ref) and np.array_equal(idx.cpu().numpy(), i_ref)
    # packed tiles: tail-biting 16 x 16 tiles of the rotated matrix -> .ltq slice -> decode
    t = pack.tiles(Wr.cpu().numpy())
    rec_t, gi_t, ix_t = viterbi_ub_cuda(torch.from_numpy(t).cuda(), lut, 2, 10, 359, gains, sub=16,
                                        return_code=True, tail_biting=True)
    torch.cuda.synchronize()
    R, Kc = Wr.shape
    idx_m = pack.untiles(ix_t.cpu().numpy(), R, Kc)
    gi_m = pack.untiles(gi_t.cpu().numpy(), R, Kc)
    b = pack_slice(torch.from_numpy(idx_m.astype(np.int16)).cuda(), torch.from_numpy(gi_m.astype(np.uint8)).cuda(), f)
    dec = pack.decode_slice(b, R, Kc, f.K, f.frac, f.h, f.sub, f.masks, f.lut, f.gain_tab)
    want = pack.untiles(rec_t.cpu().numpy(), R, Kc)
    assert np.array_equal(dec.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_gpu_c4_sixteen_subset_d4_candidates():
    from oracle import ref
    from ltq_amd.tables import closed_form_table
    from ltq_amd.tcq_proto import make_gains, viterbi_ub_cuda
    K, me, h, pp = 3, (40, 475), 3, 2
    tab = closed_form_table(K, me, device="cpu").numpy()
    gains = make_gains(h, 0.15, "cpu").numpy()
    rng = np.random.default_rng(4)
    x = (rng.standard_t(5, size=(48, 256)) * 0.9).astype(np.float32)  # one expert's 768 rows: 48 tiles
    w = np.tile(rng.uniform(0.3, 2.0, 16).astype(np.float32), 16)
    print("C4 16-subset D4 with candidates, 48 tiles", flush=True)
    out = viterbi_ub_cuda(torch.from_numpy(x).cuda(), torch.from_numpy(tab).cuda(), K, 10, 359,
                          torch.from_numpy(gains).cuda(), sub=16, wts=torch.from_numpy(w).cuda(), n_cand=4,
                          tail_biting=True, tb_window=32, m_extra=me, pair_parity=pp, return_code=True)
    torch.cuda.synchronize()
    want = ref.viterbi_ub_cuda_ref(x, tab, K, 10, 359, gains, sub=16, wts=w, n_cand=4, tail_biting=True,
                                   tb_window=32, m_extra=me, pair_parity=pp, return_code=True)
    for got, exp in zip(out, want):
        assert np.array_equal(got.cpu().numpy().astype(np.int64) if got.dtype != torch.float32 else
                              got.cpu().numpy().view(np.uint32),
                              np.asarray(exp).astype(np.int64) if got.dtype != torch.float32 else
                              np.asarray(exp, np.float32).view(np.uint32))
