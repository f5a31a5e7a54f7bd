"""The torch restatement of the reference's CPU Viterbi (oracle/torch_viterbi.py), timed as bench.py's CPU
baseline: it must reproduce the reference's own viterbi_ub outputs (tests/golden/viterbi_ub.npz, incl. the
tie-heavy cases) and the C oracle's two-pass tail-biting results for the production modes bit for bit."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")


def test_torch_restatement_matches_viterbi_ub_goldens(golden_dir):
    from oracle import torch_viterbi
    z = np.load(golden_dir / "viterbi_ub.npz")
    names = sorted({k.split(".")[0] for k in z.files})
    assert len(names) >= 10
    for name in names:
        g = {k.split(".", 1)[1]: z[k] for k in z.files if k.startswith(name + ".")}
        gains = g["gains"] if int(g["h"]) > 0 else None
        wts = g["wts"] if g["wts"].size else None
        rec, lab, u, gidx = torch_viterbi.viterbi_ub_torch(g["x"], g["small"], int(g["K"]), int(g["nu"]), 359, gains,
                                                           sub=int(g["sub"]), wts=wts)
        assert np.array_equal(lab, g["labels"]), name
        assert np.array_equal(u, g["u"]), name
        if gains is not None:
            assert np.array_equal(gidx, g["gidx"]), name
        assert np.array_equal(rec.view(np.uint32), g["rec"].view(np.uint32)), name


@pytest.mark.parametrize("spec", ["TCQ275X2", "TCQ3X3", "TCQ275Y3", "TCQ375X"])
def test_torch_restatement_matches_oracle_tail_biting(oracle, spec):
    from oracle import torch_viterbi
    from ltq_amd.formats import TCQ_CONFIG, make_format
    cfg, f = TCQ_CONFIG[spec], make_format(spec)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((6, 256)) * 1.1).astype(np.float32)
    w = (rng.random(256) + 0.5).astype(np.float32)
    kw = dict(sub=16, wts=w, n_cand=cfg.get("n_cand", 0), tail_biting=True, tb_window=32, m_extra=f.masks[1:],
              pair_parity=int(cfg.get("pp", 0)))
    r_o, g_o, i_o = oracle.viterbi_ub_cuda_ref(x, f.lut, f.K, 10, 359, f.gain_tab, return_code=True, **kw)
    r_t, g_t, i_t = torch_viterbi.viterbi_ub_cuda_torch(x, f.lut, f.K, 10, 359, f.gain_tab, **kw)
    assert np.array_equal(np.asarray(g_o), g_t) and np.array_equal(np.asarray(i_o), i_t)
    assert np.array_equal(np.asarray(r_o, np.float32).view(np.uint32), r_t.view(np.uint32))
