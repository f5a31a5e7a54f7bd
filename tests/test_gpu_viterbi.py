"""GPU parity of the gfx950 TCQ Viterbi (libltq_hip.so through ltq_amd.tcq_proto) against the CPU oracle and
the reference's golden viterbi_ub vectors. Bar: bit-exact rec, code (gain index, label * U + u), best, mid."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def tp():
    from ltq_amd import tcq_proto
    return tcq_proto


def test_golden_viterbi_ub_on_gpu(tp, golden_dir):
    """The HIP path reproduces the reference torch viterbi_ub outputs (free start, all gains, 4 subsets)."""
    z = np.load(golden_dir / "viterbi_ub.npz")
    names = sorted({k.split(".")[0] for k in z.files})
    for name in names:
        g = {k.split(".", 1)[1]: z[k] for k in z.files if k.startswith(name + ".")}
        K, nu, sub = int(g["K"]), int(g["nu"]), int(g["sub"])
        gains = torch.tensor(g["gains"], device=DEV) if int(g["h"]) > 0 else None
        wts = torch.tensor(g["wts"], device=DEV) if g["wts"].size else None
        x = torch.tensor(g["x"], device=DEV)
        print(f"golden case {name} K={K} nu={nu} shape={tuple(x.shape)}", flush=True)
        rec, gi, idx = tp.viterbi_ub_cuda(x, torch.tensor(g["small"], device=DEV), K, nu, 359, gains, sub=sub, wts=wts,
                                          return_code=True)
        torch.cuda.synchronize()
        U = 1 << (K - 1)
        idx = idx.cpu().numpy()
        assert np.array_equal(idx // U, g["labels"]), name
        assert np.array_equal(idx % U, g["u"]), name
        if gains is not None:
            assert np.array_equal(gi.cpu().numpy()[:, ::sub], g["gidx"]), name
        assert np.array_equal(_u32(rec.cpu().numpy()), _u32(g["rec"])), name


SINGLE = [  # kwargs of one kernel call (reference ABI semantics)
    dict(nu=10, nl_ext=(), G=1, T=32, U=4, pp=0),
    dict(nu=10, nl_ext=(), G=4, T=256, U=4, pp=0),
    dict(nu=10, nl_ext=(241,), G=2, T=256, U=4, pp=0, init=True, tail=True),
    dict(nu=10, nl_ext=(40, 475), G=3, T=128, U=4, pp=0, init=True),
    dict(nu=10, nl_ext=(211, 397, 58), G=2, T=64, U=4, pp=0),
    dict(nu=8, nl_ext=(), G=2, T=64, U=4, pp=0),
    dict(nu=8, nl_ext=(), G=8, T=96, U=8, pp=0, init=True, tail=True),
    dict(nu=10, nl_ext=(241,), G=2, T=256, U=4, pp=1),
    dict(nu=10, nl_ext=(241,), G=4, T=256, U=4, pp=2),
    dict(nu=10, nl_ext=(241,), G=4, T=256, U=4, pp=2, init=True, tail=True),
    dict(nu=10, nl_ext=(), G=2, T=256, U=8, pp=3),
    dict(nu=10, nl_ext=(241,), G=2, T=256, U=4, pp=2, n_cand=2, Gfull=4),
    dict(nu=10, nl_ext=(241,), G=4, T=256, U=4, pp=2, n_cand=4, Gfull=8),
    dict(nu=10, nl_ext=(241,), G=4, T=64, U=4, pp=2, steps=64, ld=256, rot=96, mid_t=32),
    dict(nu=10, nl_ext=(), G=2, T=36, U=4, pp=0, sub=6),
    dict(nu=10, nl_ext=(), G=4, T=512, U=16, pp=0, sub=32),
    dict(nu=10, nl_ext=(), G=2, T=128, U=4, pp=0, mix=16),
    dict(nu=10, nl_ext=(40,), G=8, T=128, U=4, pp=2),
    # the straight-line metric table with 2 levels per label and D2 / EQ shapes
    dict(nu=10, nl_ext=(241,), G=4, T=256, U=2, pp=2),
    dict(nu=10, nl_ext=(), G=2, T=256, U=2, pp=1),
    dict(nu=10, nl_ext=(), G=4, T=256, U=4, pp=1),
    dict(nu=10, nl_ext=(241,), G=2, T=256, U=2, pp=3),
    # the reference's limits: the longest tile (MAX_T = 512) in D4, and the largest metric table (sub G nl = 4096)
    dict(nu=10, nl_ext=(241,), G=4, T=512, U=4, pp=2, sub=32),
    dict(nu=10, nl_ext=(211, 397, 58), G=4, T=64, U=4, pp=0, sub=32),
]


@pytest.mark.parametrize("ci", range(len(SINGLE)))
def test_single_pass_matches_oracle(oracle, ci):
    from ltq_amd import _lib
    c = dict(SINGLE[ci])
    rng = np.random.default_rng(1000 + ci)
    nu, T = c["nu"], c["T"]
    S = 1 << nu
    nl = 4 << len(c["nl_ext"])
    U = c["U"]
    Gf = c.get("Gfull", c["G"])
    N = 48
    ld = c.get("ld", T)
    tab = rng.standard_normal(nl * U).astype(np.float32)
    gains = (2.0 ** ((np.arange(Gf) - (Gf - 1) / 2) * 0.22)).astype(np.float32)
    x = (rng.standard_normal((N, ld)) * 1.3).astype(np.float32)
    w = (rng.random((N, ld)) + 0.5).astype(np.float32)
    init = rng.integers(0, S, size=N).astype(np.int32) if c.get("init") else None
    tab_hi = gains_hi = None
    if c.get("mix"):
        tab_hi = rng.standard_normal(nl * 2 * U).astype(np.float32)
        gains_hi = (gains * 1.1).astype(np.float32)
    kw = dict(init_st=init, tail=c.get("tail", False), S=S, U=U, sub=c.get("sub", 16), m_extra=c["nl_ext"],
              pp=c["pp"], n_cand=c.get("n_cand", 0), steps=c.get("steps", 0), rot=c.get("rot", 0),
              mid_t=c.get("mid_t", 0), tab_hi=tab_hi, gains_hi=gains_hi, mix=c.get("mix", 0))
    print(f"single-pass case {ci}: {c}", flush=True)
    o = oracle.tcq_viterbi(x, w, tab, gains, want_end=True, **kw)

    # same call through the C ABI on the GPU
    t = lambda a, dt=torch.float32: None if a is None else torch.tensor(a, dtype=dt, device=DEV)
    Tn = kw["steps"] or ld
    G = c["G"]
    xd, wd, tabd, gd = t(x), t(w), t(tab), t(gains)
    tabhd = t(tab_hi) if tab_hi is not None else tabd
    ghd = t(gains_hi) if gains_hi is not None else gd
    rec = torch.empty((N, ld), device=DEV)
    bp = torch.empty((N, Tn, G, S // 32), dtype=torch.int32, device=DEV)
    gsel = torch.empty((N, Tn // kw["sub"], S), dtype=torch.uint8, device=DEV)
    initd = t(init, torch.int32)
    end = torch.empty(N, dtype=torch.int32, device=DEV)
    cand = torch.empty((N, Tn // kw["sub"], G), dtype=torch.uint8, device=DEV) if G < Gf else None
    best = torch.empty(N, dtype=torch.int32, device=DEV)
    code = torch.empty((N, ld), dtype=torch.int32, device=DEV)
    mid = torch.empty(N, dtype=torch.int32, device=DEV) if kw["mid_t"] else None
    pp = c["pp"]
    pbits = (torch.empty((N, Tn // 4, G, 9, S // 32), dtype=torch.int32, device=DEV) if pp >= 2 else
             torch.empty((N, Tn // 2, G, S // 32), dtype=torch.int32, device=DEV) if pp == 1 else None)
    me = (list(c["nl_ext"]) + [0, 0, 0])[:3]
    p = _lib.ptr
    rc = _lib.lib().tcq_viterbi(p(xd), p(wd), p(tabd), p(gd), p(rec), p(bp), p(gsel), p(initd), p(end), p(tabhd), p(ghd),
                                p(cand), p(best), p(code), p(mid), kw["mid_t"], int(kw["tail"]), N, Tn, S, U, G, Gf, 359,
                                kw["sub"], tabhd.numel() // nl, kw["mix"], me[0], me[1], me[2], nl, ld, kw["rot"],
                                p(pbits), pp, _lib.stream_ptr())
    assert rc == 0
    torch.cuda.synchronize()
    assert np.array_equal(best.cpu().numpy(), o["best"])
    assert np.array_equal(end.cpu().numpy(), o["end"])
    if cand is not None:
        assert np.array_equal(cand.cpu().numpy(), o["gcand"])
    if kw["mid_t"]:
        assert np.array_equal(mid.cpu().numpy(), o["mid"])
    else:
        assert np.array_equal(code.cpu().numpy(), o["code"])
        assert np.array_equal(_u32(rec.cpu().numpy()), _u32(o["rec"]))


FORMATS = ["TCQ275X2", "TCQ275X", "TCQ375X", "TCQ25X", "TCQ3X3", "TCQ4X", "TCQ2X0", "TCQ3W2", "TCQ5X", "TCQ3X16",
           "TCQ225X", "TCQ45X"]


@pytest.mark.parametrize("name", FORMATS)
@pytest.mark.parametrize("tb_window", [32, 0])
def test_tail_biting_driver_matches_oracle(tp, oracle, name, tb_window):
    """Every production format through the two-pass tail-biting driver, as _quantize_rows_tcq_ldlq calls it
    (src/liqk_v2.py:917-919), on Student-t tiles with per-position weights."""
    from ltq_amd.formats import TCQ_CONFIG, make_format
    cfg = TCQ_CONFIG[name]
    f = make_format(name)
    rng = np.random.default_rng(7)
    N = 64
    x = (rng.standard_t(5, size=(N, 256)) * 0.9).astype(np.float32)
    w = (rng.random(16) * 2 + 0.2).astype(np.float32)
    wts = np.tile(w, 16)
    n_cand = cfg.get("n_cand", 0)
    print(f"format {name} window {tb_window}", flush=True)
    rec, gi, idx = tp.viterbi_ub_cuda(torch.tensor(x, device=DEV), torch.tensor(f.lut, device=DEV), f.K, 10, 359,
                                      torch.tensor(f.gain_tab, device=DEV), sub=f.sub, wts=torch.tensor(wts, device=DEV),
                                      n_cand=n_cand, tail_biting=True, tb_window=tb_window, m_extra=f.masks[1:],
                                      pair_parity=int(cfg.get("pp", 0)), return_code=True)
    torch.cuda.synchronize()
    r_rec, r_gi, r_idx = oracle.viterbi_ub_cuda_ref(x, f.lut, f.K, 10, 359, f.gain_tab, sub=f.sub, wts=wts,
                                                    n_cand=n_cand, tail_biting=True, tb_window=tb_window,
                                                    m_extra=f.masks[1:], pair_parity=int(cfg.get("pp", 0)),
                                                    return_code=True)
    assert np.array_equal(gi.cpu().numpy(), r_gi)
    assert np.array_equal(idx.cpu().numpy(), r_idx)
    assert np.array_equal(_u32(rec.cpu().numpy()), _u32(r_rec))


@pytest.mark.parametrize("name,tb_window", [("TCQ4X", 0), ("TCQ2X", 32), ("TCQ3X3", 0)])
def test_integer_launch_with_two_workgroups_per_cu_matches_oracle(tp, oracle, name, tb_window):
    """Integer-mode launches with at least two tiles per CU run the two-workgroups-per-CU build of the kernel
    (half the LDS, 64 VGPRs): bit-exact against the oracle like the one-workgroup build."""
    from ltq_amd.formats import TCQ_CONFIG, make_format
    cfg, f = TCQ_CONFIG[name], make_format(name)
    N = 2 * torch.cuda.get_device_properties(0).multi_processor_count + 37
    rng = np.random.default_rng(11)
    x = (rng.standard_t(5, size=(N, 256)) * 0.9).astype(np.float32)
    wts = np.tile((rng.random(16) * 2 + 0.2).astype(np.float32), 16)
    n_cand = cfg.get("n_cand", 0)
    print(f"two workgroups per CU: {name} N={N} window {tb_window}", flush=True)
    rec, gi, idx = tp.viterbi_ub_cuda(torch.tensor(x, device=DEV), torch.tensor(f.lut, device=DEV), f.K, 10, 359,
                                      torch.tensor(f.gain_tab, device=DEV), sub=f.sub, wts=torch.tensor(wts, device=DEV),
                                      n_cand=n_cand, tail_biting=True, tb_window=tb_window, m_extra=f.masks[1:],
                                      pair_parity=int(cfg.get("pp", 0)), return_code=True)
    torch.cuda.synchronize()
    r_rec, r_gi, r_idx = oracle.viterbi_ub_cuda_ref(x, f.lut, f.K, 10, 359, f.gain_tab, sub=f.sub, wts=wts,
                                                    n_cand=n_cand, tail_biting=True, tb_window=tb_window,
                                                    m_extra=f.masks[1:], pair_parity=int(cfg.get("pp", 0)),
                                                    return_code=True)
    assert np.array_equal(gi.cpu().numpy(), r_gi)
    assert np.array_equal(idx.cpu().numpy(), r_idx)
    assert np.array_equal(_u32(rec.cpu().numpy()), _u32(r_rec))


def test_rejected_configs_raise(tp):
    x = torch.zeros((2, 32), device=DEV)
    with pytest.raises(RuntimeError):
        tp.viterbi_ub_cuda(x, torch.zeros(16, device=DEV), 3, 10, 359, torch.ones(5, device=DEV))  # G = 5
    with pytest.raises(RuntimeError):
        tp.viterbi_ub_cuda(x, torch.zeros(16, device=DEV), 3, 10, 359, None, sub=3)


@pytest.mark.gpu
@pytest.mark.parametrize("name,window", [("TCQ275X2", 32), ("TCQ25X", 0), ("TCQ3X3", 32), ("TCQ4X", 16)])
def test_gpu_fused_tail_biting_equals_two_launches(name, window):
    """The fused two-pass launch (tcq_viterbi_tb) gives exactly the two separate launches' results."""
    from ltq_amd.formats import TCQ_CONFIG, make_format
    from ltq_amd.tcq_proto import viterbi_ub_cuda
    f, cfg = make_format(name), TCQ_CONFIG[name]
    g = torch.Generator().manual_seed(9)
    x = (torch.randn((300, 256), generator=g) * 1.1).cuda()
    w = (torch.rand((300, 256), generator=g) + 0.5).cuda()
    kw = dict(sub=f.sub, wts=w, n_cand=cfg.get("n_cand", 0), tail_biting=True, tb_window=window,
              m_extra=f.masks[1:], pair_parity=f.frac, return_code=True)
    lut, gains = torch.tensor(f.lut).cuda(), torch.tensor(f.gain_tab).cuda()
    print(f"fused vs two launches {name} w={window}", flush=True)
    a = viterbi_ub_cuda(x, lut, f.K, 10, f.masks[0], gains, _fuse=True, **kw)
    b = viterbi_ub_cuda(x, lut, f.K, 10, f.masks[0], gains, _fuse=False, **kw)
    torch.cuda.synchronize()
    assert torch.equal(a[0].view(torch.int32), b[0].view(torch.int32))
    assert torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])


def test_gpu_timing_hook_keeps_results_and_times_the_launches(tp):
    """The benchmark's timing hook (events handed to the launches through ltq_viterbi_timing) leaves the results
    bit-identical, stamps both events, and a later call without the hook is not stamped."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import bench
    g = torch.Generator().manual_seed(5)
    x = (torch.randn((64, 256), generator=g) * 1.3).to(DEV)
    w = (torch.rand((256,), generator=g) + 0.5).to(DEV)
    lut = torch.randn(32, generator=g).to(DEV)
    gains = tp.make_gains(2, 0.22, DEV)
    kw = dict(sub=16, wts=w, tail_biting=True, tb_window=32, m_extra=(241,), pair_parity=2, return_code=True)
    ref = tp.viterbi_ub_cuda(x, lut, 3, 10, 359, gains, **kw)
    tp.LAUNCH_EVENTS, tp.LAUNCH_SAMPLE, tp._launch_count, tp.EVENT_FACTORY = [], 1, 0, bench.DeviceEvent
    try:
        out = tp.viterbi_ub_cuda(x, lut, 3, 10, 359, gains, **kw)
        recs = tp.LAUNCH_EVENTS
    finally:
        tp.LAUNCH_EVENTS, tp.EVENT_FACTORY = None, None
    again = tp.viterbi_ub_cuda(x, lut, 3, 10, 359, gains, **kw)
    torch.cuda.synchronize()
    for a, b, c in zip(ref, out, again):
        assert torch.equal(a, b) and torch.equal(a, c)
    assert len(recs) == 1 and recs[0]["launches"] == [(64, 4), (256, 4)]
    assert len(recs[0]["ev"]) == 2  # one event pair per launch
    ms = [e0.elapsed_time(e1) for e0, e1 in recs[0]["ev"]]
    print(f"pass 1 / pass 2 over 64 tiles: {ms[0] * 1e3:.1f} / {ms[1] * 1e3:.1f} us", flush=True)
    assert all(0.0 < t < 50.0 for t in ms) and ms[0] < ms[1]


@pytest.mark.gpu
def test_gpu_empty_inputs_behave_like_the_reference(tp):
    """Empty inputs: the FWHT of no rows is an empty tensor, as torch's transform gives (src/iqk_format.py:153-170);
    a Viterbi call over no tiles and a LUT call over no sub-blocks raise, as the reference's callers raise on the
    error 9 of its zero-block launches (src/tcq_proto.py:544-547 and the tcq_viterbi return-code check)."""
    from ltq_amd.rotation import fwht_cols, fwht_rows
    print("empty inputs", flush=True)
    assert fwht_rows(torch.zeros((0, 512), device=DEV)).shape == (0, 512)
    assert fwht_cols(torch.zeros((0, 64), device=DEV)).shape == (0, 64)
    with pytest.raises(RuntimeError, match="9"):
        tp.viterbi_ub_cuda(torch.zeros((0, 32), device=DEV), torch.zeros(16, device=DEV), 3, 10, 359)
    with pytest.raises(RuntimeError, match="9"):
        tp.lut_subs_quant_cuda(torch.zeros((0, 16), device=DEV), torch.zeros((0, 16), device=DEV),
                               torch.zeros((8, 64), device=DEV), 1.0, 4.0)
    torch.cuda.synchronize()
