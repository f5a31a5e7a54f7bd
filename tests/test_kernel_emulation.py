"""The gfx950 kernel source (ltq-research_amd/csrc/tcq_trellis.h) compiled for the host and run with one
thread per lane (tests/emu) must match the oracle bit for bit: pins the register layout, decision-word
format and traceback indexing on the CPU, for every parity mode, before any GPU run."""
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent / "emu"))

CASES = [
    dict(pp=0, ext=(), G=1, T=32),
    dict(pp=0, ext=(), G=4, T=64),
    dict(pp=0, ext=(241,), G=2, T=64, init=True, tail=True),
    dict(pp=0, ext=(), G=2, T=64, S=256),
    dict(pp=0, ext=(), G=3, T=48, S=256, init=True, tail=True),
    dict(pp=1, ext=(241,), G=2, T=64),
    dict(pp=2, ext=(241,), G=4, T=64),
    dict(pp=2, ext=(241,), G=2, T=64, init=True, tail=True),
    dict(pp=3, ext=(), G=2, T=64, U=8),
    dict(pp=2, ext=(241,), G=2, T=64, n_cand=2, Gfull=4),
    dict(pp=2, ext=(241,), G=4, T=32, ld=64, steps=32, rot=16, mid_t=16),
    dict(pp=0, ext=(), G=2, T=36, sub=6),
    dict(pp=0, ext=(40, 475), G=2, T=64, mix=16),
    dict(pp=2, ext=(211, 397), G=1, T=32),
    # 8 gain slots (8 states per lane, 2 wavefronts per slot), every mode
    dict(pp=0, ext=(), G=8, T=48, init=True, tail=True),
    dict(pp=1, ext=(241,), G=8, T=64),
    dict(pp=2, ext=(241,), G=8, T=32, sub=8),
    dict(pp=3, ext=(), G=8, T=32, U=8),
    # partial last chunks, odd mid positions, more label counts, candidates in integer mode
    dict(pp=0, ext=(), G=2, T=20, sub=10, mid_t=7),
    dict(pp=1, ext=(), G=2, T=40, sub=8, mid_t=13, ld=48, rot=5),
    dict(pp=1, ext=(241,), G=3, T=34, sub=2),
    dict(pp=2, ext=(241,), G=4, T=20, sub=4, mid_t=10),
    dict(pp=3, ext=(40,), G=2, T=36, sub=12, U=8, init=True, tail=True),
    dict(pp=2, ext=(40, 475, 211), G=2, T=32),
    dict(pp=0, ext=(40, 475, 211), G=4, T=32, n_cand=4, Gfull=8),
    dict(pp=0, ext=(), G=1, T=64, S=256, mid_t=33),
    # sub-blocks of 32 through the streamlined walk (a merge at every other chunk), also with a mid-state pass
    dict(pp=0, ext=(241,), G=2, T=64, sub=32),
    dict(pp=1, ext=(241,), G=4, T=64, sub=32, mid_t=40),
    dict(pp=2, ext=(241,), G=2, T=96, sub=32, init=True, tail=True),
    # the straight-line metric table (one entry per thread: D4 / EQ with 8 labels, D2 with 4; U = 2 and 4)
    dict(pp=2, ext=(241,), G=4, T=32, U=2),
    dict(pp=1, ext=(), G=2, T=64, U=2),
    dict(pp=1, ext=(), G=4, T=64, U=4),
    dict(pp=3, ext=(241,), G=2, T=32, U=2),
    # the reference's limits: the longest tile (MAX_T = 512) in D4, and the largest metric table (sub G nl = 4096)
    dict(pp=2, ext=(241,), G=4, T=512, sub=32),
    dict(pp=0, ext=(211, 397, 58), G=4, T=64, sub=32),
]


@pytest.mark.parametrize("ci", range(len(CASES)))
def test_emulated_kernel_matches_oracle(oracle, ci):
    import emu
    c = CASES[ci]
    rng = np.random.default_rng(ci)
    nl = 4 << len(c["ext"])
    U = c.get("U", 4)
    S = c.get("S", 1024)
    Gf = c.get("Gfull", c["G"])
    N = 2
    ld = c.get("ld", c["T"])
    tab = rng.standard_normal(nl * U).astype(np.float32)
    gains = (2.0 ** ((np.arange(Gf) - (Gf - 1) / 2) * 0.22)).astype(np.float32)
    x = (rng.standard_normal((N, ld)) * 1.2).astype(np.float32)
    w = (rng.random((N, ld)) + 0.5).astype(np.float32)
    init = rng.integers(0, S, size=N).astype(np.int32) if c.get("init") else None
    tab_hi = rng.standard_normal(nl * 2 * U).astype(np.float32) if c.get("mix") else None
    gains_hi = (gains * 1.1).astype(np.float32) if c.get("mix") else None
    kw = dict(init_st=init, tail=c.get("tail", False), S=S, U=U, sub=c.get("sub", 16), m_extra=c["ext"], pp=c["pp"],
              n_cand=c.get("n_cand", 0), steps=c.get("steps", 0), rot=c.get("rot", 0), mid_t=c.get("mid_t", 0),
              tab_hi=tab_hi, gains_hi=gains_hi, mix=c.get("mix", 0))
    o = oracle.tcq_viterbi(x, w, tab, gains, want_end=True, **kw)
    e = emu.tcq_viterbi(x, w, tab, gains, **kw)
    assert np.array_equal(o["best"], e["best"])
    if kw["mid_t"]:
        assert np.array_equal(o["mid"], e["mid"])
    else:
        assert np.array_equal(o["code"], e["code"])
        assert np.array_equal(o["rec"].view(np.uint32), e["rec"].view(np.uint32))
    if o["gcand"] is not None:
        assert np.array_equal(o["gcand"], e["gcand"])


TB_CASES = [
    dict(pp=2, ext=(241,), G=4, T=256, window=32),          # the matrix path (TCQ275X2)
    dict(pp=2, ext=(), G=4, T=64, window=0, U=8),           # whole-tile pass 1
    dict(pp=1, ext=(241,), G=2, T=128, window=16),          # D2
    dict(pp=3, ext=(), G=2, T=64, window=16),               # EQ
    dict(pp=0, ext=(241, 40), G=4, Gfull=8, T=128, window=32, n_cand=4),  # candidates
    dict(pp=0, ext=(), G=8, T=64, window=16),               # G = 8: the general walker
]


@pytest.mark.parametrize("ci", range(len(TB_CASES)))
def test_emulated_fused_tail_biting_matches_two_pass_driver(ci):
    """Both passes in one launch (tcq_tile_tb) against the oracle's two-pass driver (src/tcq_proto.py:584-609)."""
    import emu
    from oracle import ref
    c = TB_CASES[ci]
    rng = np.random.default_rng(100 + ci)
    nl = 4 << len(c["ext"])
    U = c.get("U", 4)
    Gf = c.get("Gfull", c["G"])
    N, T = 2, c["T"]
    tab = rng.standard_normal(nl * U).astype(np.float32)
    gains = (2.0 ** ((np.arange(Gf) - (Gf - 1) / 2) * 0.22)).astype(np.float32)
    x = (rng.standard_normal((N, T)) * 1.2).astype(np.float32)
    w = (rng.random((N, T)) + 0.5).astype(np.float32)
    e = emu.tcq_viterbi_tb(x, w, tab, gains, n_cand=c.get("n_cand", 0), m_extra=c["ext"], pp=c["pp"],
                           window=c["window"])
    rec, gi, ix = ref.viterbi_ub_cuda_ref(x, tab, int(np.log2(U)) + 1, 10, 359, gains, sub=16, wts=w,
                                          n_cand=c.get("n_cand", 0), tail_biting=True, tb_window=c["window"],
                                          m_extra=c["ext"], pair_parity=c["pp"], return_code=True)
    assert np.array_equal(e["rec"].view(np.uint32), np.asarray(rec, np.float32).view(np.uint32))
    assert np.array_equal(e["code"], (np.asarray(gi, np.int64) << 16 | np.asarray(ix, np.int64)).astype(np.int32))


COMPACT_CASES = [
    dict(pp=2, ext=(241,), G=4, T=256, N=3),                         # TCQ275X2 closing pass: whole chunks
    dict(pp=2, ext=(241,), G=4, T=64, N=3, ld=256, rot=96, mid_t=32),  # its first pass (window 32)
    dict(pp=0, ext=(241,), G=4, Gfull=8, n_cand=4, T=64, N=2),        # candidates: gcand beside the words
    dict(pp=1, ext=(241,), G=2, T=40, N=2, sub=8),                   # partial last chunk (general walker)
    dict(pp=0, ext=(), G=8, T=48, N=2),                              # G = 8
]


@pytest.mark.parametrize("ci", range(len(COMPACT_CASES)))
def test_emulated_compact_scratch_window(oracle, ci):
    """The decision-scratch layout of tcq_viterbi_static (each tile's words in a window of its needed words
    rounded up to 64, nothing else) gives the oracle's results and writes nothing past the last window."""
    import emu
    c = COMPACT_CASES[ci]
    rng = np.random.default_rng(300 + ci)
    nl = 4 << len(c["ext"])
    U, Gf, N = 4, c.get("Gfull", c["G"]), c["N"]
    ld = c.get("ld", c["T"])
    tab = rng.standard_normal(nl * U).astype(np.float32)
    gains = (2.0 ** ((np.arange(Gf) - (Gf - 1) / 2) * 0.22)).astype(np.float32)
    x = (rng.standard_normal((N, ld)) * 1.2).astype(np.float32)
    w = (rng.random((N, ld)) + 0.5).astype(np.float32)
    kw = dict(sub=c.get("sub", 16), m_extra=c["ext"], pp=c["pp"], n_cand=c.get("n_cand", 0),
              steps=c["T"] if ld != c["T"] else 0, rot=c.get("rot", 0), mid_t=c.get("mid_t", 0))
    o = oracle.tcq_viterbi(x, w, tab, gains, want_end=True, **kw)
    e, guard_ok = emu.tcq_viterbi_compact(x, w, tab, gains, **kw)
    assert guard_ok
    assert np.array_equal(o["best"], e["best"])
    if kw["mid_t"]:
        assert np.array_equal(o["mid"], e["mid"])
    else:
        assert np.array_equal(o["code"], e["code"])
        assert np.array_equal(o["rec"].view(np.uint32), e["rec"].view(np.uint32))
