"""Pins the CPU oracle's Viterbi before anything is checked against it.

- golden vectors of the reference's torch viterbi_ub (src/tcq_proto.py:363-419), incl. tie-heavy inputs;
- exhaustive search on tiny tiles (oracle/ltq_brute.c) for integer, D2, D4 and EQ modes, free and
  given start, tail-biting end, extended labels, several gains;
- the label closed form (src/cuda/tcq_viterbi.cu:85-95) against a direct bit-parity evaluation;
- a planted mistake (a transposed tie rule) must fail the tie-heavy golden case.
"""
import numpy as np
import pytest


def _golden(golden_dir):
    z = np.load(golden_dir / "viterbi_ub.npz")
    names = sorted({k.split(".")[0] for k in z.files})
    return z, names


def test_oracle_matches_viterbi_ub_golden(oracle, golden_dir):
    z, names = _golden(golden_dir)
    assert len(names) >= 10
    for name in names:
        g = {k.split(".", 1)[1]: z[k] for k in z.files if k.startswith(name + ".")}
        K, nu, sub = int(g["K"]), int(g["nu"]), int(g["sub"])
        gains = g["gains"] if int(g["h"]) > 0 else None
        wts = g["wts"] if g["wts"].size else None
        rec, lab, u, gidx = oracle.viterbi_ub_ref(g["x"], g["small"], K, nu, 359, gains, sub=sub, wts=wts)
        assert np.array_equal(lab, g["labels"]), name
        assert np.array_equal(u, g["u"]), name
        if gains is not None:
            assert np.array_equal(gidx, g["gidx"]), name
        assert np.array_equal(rec.view(np.uint32), g["rec"].view(np.uint32)), name


def test_planted_tie_mistake_is_caught(oracle, golden_dir):
    """With the predecessor tie rule transposed (p1 wins ties) the oracle must fail the tie-heavy golden case."""
    import ctypes
    z, _ = _golden(golden_dir)
    plant = ctypes.c_int.in_dll(oracle.lib(), "ltq_oracle_plant")
    for name in ("k2_ties_h0", "k4_ties_h2"):  # unit / power-of-two-grid metrics: many exact ties
        g = {k.split(".", 1)[1]: z[k] for k in z.files if k.startswith(name + ".")}
        gains = g["gains"] if int(g["h"]) > 0 else None
        wts = g["wts"] if g["wts"].size else None
        plant.value = 1
        try:
            rec, lab, u, gidx = oracle.viterbi_ub_ref(g["x"], g["small"], int(g["K"]), int(g["nu"]), 359, gains,
                                                      sub=16, wts=wts)
        finally:
            plant.value = 0
        assert not np.array_equal(lab, g["labels"]), name


def _path_cost(E, lab, par, gsl, sub):
    T = lab.shape[0]
    return sum(float(E[t, gsl[t // sub], lab[t], par[t]]) for t in range(T))


CASES = [  # S, nl masks, G, sub, pp, init, tail, T
    dict(S=256, m_extra=(), G=1, sub=4, pp=0, init=-1, tail=False, T=12, U=4),
    dict(S=256, m_extra=(), G=2, sub=4, pp=0, init=-1, tail=False, T=12, U=4),
    dict(S=1024, m_extra=(), G=2, sub=8, pp=0, init=613, tail=True, T=16, U=4),
    dict(S=1024, m_extra=(241,), G=2, sub=8, pp=0, init=77, tail=False, T=16, U=4),
    dict(S=1024, m_extra=(241,), G=2, sub=8, pp=1, init=901, tail=True, T=16, U=4),
    dict(S=1024, m_extra=(241,), G=2, sub=8, pp=2, init=5, tail=True, T=16, U=4),
    dict(S=1024, m_extra=(40, 475), G=1, sub=8, pp=2, init=300, tail=False, T=16, U=4),
    dict(S=1024, m_extra=(), G=2, sub=8, pp=3, init=999, tail=True, T=16, U=8),
    dict(S=1024, m_extra=(211, 397), G=3, sub=4, pp=2, init=1, tail=True, T=12, U=4),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_oracle_equals_brute_force(oracle, case):
    c = CASES[case]
    rng = np.random.default_rng(100 + case)
    nl = 4 << len(c["m_extra"])
    U = c["U"]
    tab = np.sort(rng.standard_normal(nl * U)).astype(np.float32).reshape(U, nl).T.copy().reshape(-1)
    gains = (2.0 ** ((np.arange(c["G"]) - (c["G"] - 1) / 2) * 0.3)).astype(np.float32)
    ok = 0
    for rep in range(3):
        x = rng.standard_normal((1, c["T"])).astype(np.float32) * 1.3
        w = (rng.random((1, c["T"])) + 0.5).astype(np.float32)
        r = oracle.tcq_viterbi(x, w, tab, gains, init_st=[c["init"]] if c["init"] >= 0 else None, tail=c["tail"],
                               S=c["S"], U=U, m=359, sub=c["sub"], m_extra=c["m_extra"], pp=c["pp"])
        code = r["code"][0]
        lab = (code & 0xFFFF) // U
        uu = (code & 0xFFFF) % U
        gsl = (code >> 16)[:: c["sub"]]
        par = (uu & 1) if c["pp"] else np.zeros_like(uu)
        E = oracle.step_metrics(x[0], w[0], tab, gains, U, nl, c["pp"])
        cost_o = _path_cost(E, lab, par, gsl, c["sub"])
        cost_b, st_b, g_b, low_b = oracle.brute_force(x[0], w[0], tab, gains, S=c["S"], U=U, m=359,
                                                        m_extra=c["m_extra"], sub=c["sub"], pp=c["pp"],
                                                        init=c["init"], tail=c["tail"])
        assert cost_o >= cost_b - 1e-9 * abs(cost_b) - 1e-12
        assert abs(cost_o - cost_b) <= 1e-5 * abs(cost_b) + 1e-9, (cost_o, cost_b)
        labs = oracle.labels_ref(c["S"], 359, c["m_extra"])
        if np.array_equal(labs[st_b], lab) and np.array_equal(g_b, gsl):
            ok += 1
            if c["pp"]:
                assert np.array_equal(low_b, par)
        # the oracle's labels must come from one trellis path consistent with the start / end rules
        if c["tail"]:
            assert r["best"][0] % c["S"] == c["init"]
    assert ok >= 2


def test_labels_closed_form(oracle):
    for masks in ((), (241,), (40, 475), (211, 397, 58)):
        s = np.arange(1024)
        got = oracle.labels_ref(1024, 359, masks)
        exp = s & 1
        for i, mk in enumerate((359,) + masks):
            v = (s >> 1) & mk
            p = np.array([bin(int(a)).count("1") & 1 for a in v])
            exp = exp | (p << (i + 1))
        assert np.array_equal(got, exp)


def test_oracle_rejects_invalid_configs(oracle):
    x = np.zeros((1, 32), np.float32)
    tab = np.zeros(16, np.float32)
    for kw in (dict(sub=3), dict(pp=1, S=256), dict(pp=2, sub=6), dict(m_extra=(1, 2, 3, 4))):
        with pytest.raises(Exception):
            oracle.tcq_viterbi(x, np.ones_like(x), tab, np.ones(1, np.float32), **kw)
    with pytest.raises(RuntimeError):  # G = 5 is not a supported gain count
        oracle.tcq_viterbi(x, np.ones_like(x), tab, np.ones(5, np.float32))
