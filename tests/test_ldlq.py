"""The LDLQ block error feedback (src/liqk_v2.py:948-980) and its pins.

CPU, the oracle (oracle/liqk_ref.py over oracle/ldlq_oracle.c):
  - its sums are the ascending fma chains (exact rational arithmetic on a few outputs);
  - its loop satisfies the loop's defining identity W_rot - W_hat = E U (E_j = (fed_j - W_hat_j) U_jj^-1) to a
    few units of roundoff, and its Viterbi inputs are exactly fl(fed * fl(1 / d)); a planted wrong sign, factor
    slice or feedback index fails one of the two;
  - with H = I (no feedback) every weight is fed as it is, and the reconstruction is d times the Viterbi's.
GPU, the HIP kernels against the oracle, bit for bit:
  - ltq_ldlq_err / ltq_ldlq_update (fp32 MFMA) and ltq_ldlq_sub;
  - the whole row quantizer for the C2 / C3 formats: codes, gain indices, tile values, reconstruction, fed
    values and scales equal (so the reconstruction MSE is the same number);
  - at the full C3 shape (4096 x 14336, TCQ275X2) the GPU loop satisfies the identity.
"""
from fractions import Fraction

import numpy as np
import pytest

torch = pytest.importorskip("torch")

DEV = "cuda"
ULP = 2.0 ** -24


def _ptr(a):
    return None if a is None else a.ctypes.data


def _synthetic(M, K, n_act=300, seed=0, outliers=0):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((M, K), generator=g)
    chi2 = sum(torch.randn((M, K), generator=g).square() for _ in range(5))
    W = (z / (chi2 / 5).sqrt()) * 0.02
    if outliers:
        W[:, torch.randperm(K, generator=g)[:outliers]] *= 20
    X = torch.randn((n_act, K), generator=g)
    return W, X.T @ X / n_act


def _fma_chain(a, b):
    """float32 result of acc = fma(a[k], b[k], acc) for k ascending from acc = 0, in exact arithmetic."""
    acc = Fraction(0)
    for x, y in zip(a, b):
        acc = Fraction(float(np.float32(acc + Fraction(float(x)) * Fraction(float(y)))))
    return np.float32(float(acc))


def test_oracle_ldlq_sums_are_ascending_fma_chains(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(1)
    M, N = 16, 256
    E = (rng.standard_normal((M, 256)) * 2.0 ** rng.integers(-8, 8, (M, 256))).astype(np.float32)
    U = (rng.standard_normal((256, N)) * 2.0 ** rng.integers(-8, 8, (256, N))).astype(np.float32)
    W = rng.standard_normal((M, N)).astype(np.float32)
    W0 = W.copy()
    L.ltq_oracle_ldlq_update(_ptr(W), N, _ptr(E), 256, _ptr(U), N, M, N)
    for i, j in ((0, 0), (3, 17), (15, 255), (7, 128)):
        assert W[i, j] == np.float32(W0[i, j] - _fma_chain(E[i], U[:, j]))
    # the reversed chain differs somewhere: the order is what the oracle fixes
    diff = [W[i, j] != np.float32(W0[i, j] - _fma_chain(E[i][::-1], U[::-1, j])) for i in range(4) for j in range(8)]
    assert any(diff)
    ws = rng.standard_normal((M, 256)).astype(np.float32)
    G = rng.standard_normal((M, 256)).astype(np.float32)
    d = (rng.random(M) + 0.5).astype(np.float32)
    Ui = np.triu(rng.standard_normal((256, 256))).astype(np.float32)
    Eo = np.empty((M, 256), np.float32)
    wh = np.empty((M, 256), np.float32)
    L.ltq_oracle_ldlq_err(_ptr(ws), 256, _ptr(G), 256, _ptr(d), 1, _ptr(Ui), 256, _ptr(Eo), 256, _ptr(wh), 256, M)
    assert np.array_equal(wh, d[:, None] * G)
    a = ws - wh
    for i, j in ((0, 0), (5, 100), (15, 255)):
        assert Eo[i, j] == _fma_chain(a[i], Ui[:, j])


def _oracle_case(M, K, spec, seed=0, identity_h=False):
    from oracle import liqk_ref
    from ltq_amd.formats import TCQ_CONFIG, make_format
    W, H = _synthetic(M, K, seed=seed)
    if identity_h:
        H = torch.eye(K)
    U, dw, Ubi = liqk_ref.factor_hessian_ref(H, 0.2)
    return W, U, dw, Ubi, TCQ_CONFIG[spec], make_format(spec)


@pytest.mark.parametrize("spec", ["TCQ275X2", "TCQ3X3"])
def test_oracle_ldlq_loop_identity_and_tiles(spec):
    from oracle import liqk_ref
    W, U, dw, Ubi, cfg, f = _oracle_case(64, 768, spec)
    _, _, _, d_all = liqk_ref.row_scale_ref(W, cfg)
    inv = (np.float32(1) / np.maximum(d_all, np.float32(1e-8))).astype(np.float32)

    def run(mistake):
        tr = {}
        _, Wh, _, fed = liqk_ref.quantize_rows_ref(W, U, Ubi, dw, cfg, f.gain_tab, mistake=mistake, trace=tr)
        R, B = liqk_ref.ldlq_identity_residual(W.numpy(), Wh, fed, U.numpy(), Ubi.numpy())
        tiles = (fed.reshape(64, 3, 256) * inv[:, :, None]).reshape(64, 768)
        return float(np.max(np.abs(R) / B)), np.array_equal(tr["x"].view(np.uint32), tiles.view(np.uint32))

    rel, tiles_ok = run("")
    print(f"{spec}: identity residual {rel / ULP:.1f} ulp of |W_rot| + |E||U|")
    assert rel <= 64 * ULP and tiles_ok
    for mistake in ("sign", "slice"):
        rel_m, _ = run(mistake)
        assert rel_m > 1e-3, mistake
    assert not run("index")[1]


def test_oracle_ldlq_without_feedback_is_plain_quantization():
    """H = I: U is a multiple of I, every update adds exact zeros, each weight is fed unchanged and the
    reconstruction is fl(d * Viterbi(fl(w * fl(1 / d))))."""
    from oracle import liqk_ref, ref
    W, U, dw, Ubi, cfg, f = _oracle_case(32, 512, "TCQ275X2", identity_h=True)
    d_full, Wh, codes, fed = liqk_ref.quantize_rows_ref(W, U, Ubi, dw, cfg, f.gain_tab)
    Wn = W.numpy()
    assert np.array_equal(fed.view(np.uint32), Wn.view(np.uint32))
    _, _, _, d_all = liqk_ref.row_scale_ref(W, cfg)
    for b in range(2):
        d = d_all[:, b]
        for j in range(16):
            c = 256 * b + 16 * j
            x = (Wn[:, c:c + 16] * (np.float32(1) / d)[:, None]).reshape(2, 256)
            rec, _, _ = ref.viterbi_ub_cuda_ref(x, f.lut, 3, 10, 359, f.gain_tab, wts=np.tile(dw[c:c + 16].numpy(), 16),
                                                tail_biting=True, tb_window=32, m_extra=f.masks[1:], pair_parity=2,
                                                return_code=True)
            assert np.array_equal(Wh[:, c:c + 16], d[:, None] * np.asarray(rec, np.float32).reshape(32, 16))


def test_oracle_carried_state_threads_through_sub_blocks():
    """H = I (no feedback): a carried-state format (TCQ3R) quantizes the sub-blocks of each row group in order,
    every tile starting from the end state of the same rows' previous tile, across 256-column blocks too
    (src/liqk_v2.py:926-929); starting every tile free gives a different reconstruction."""
    from oracle import liqk_ref, ref
    from ltq_amd.formats import TCQ_CONFIG
    cfg = TCQ_CONFIG["TCQ3R"]
    W, H = _synthetic(32, 512, seed=4)
    U, dw, Ubi = liqk_ref.factor_hessian_ref(torch.eye(512), 0.2)
    gains, _, _ = _oracle_tables(cfg)
    d_full, Wh, codes, fed = liqk_ref.quantize_rows_ref(W, U, Ubi, dw, cfg, gains)
    assert codes is None
    Wn, lut = W.numpy(), np.asarray(cfg["lut"], np.float32)
    _, _, _, d_all = liqk_ref.row_scale_ref(W, cfg)
    carry = None
    free = np.empty_like(Wn)
    for b in range(2):
        d = np.maximum(d_all[:, b], np.float32(1e-8))
        for j in range(16):
            c = 256 * b + 16 * j
            x = (Wn[:, c:c + 16] * (np.float32(1) / d)[:, None]).reshape(2, 256)
            wts = np.tile(dw[c:c + 16].numpy(), 16)
            rec, carry = ref.viterbi_ub_cuda_ref(x, lut, 3, 10, 359, gains, wts=wts, init_state=carry,
                                                 return_end_state=True)
            assert np.array_equal(Wh[:, c:c + 16], d[:, None] * np.asarray(rec, np.float32).reshape(32, 16))
            rec0 = ref.viterbi_ub_cuda_ref(x, lut, 3, 10, 359, gains, wts=wts)
            free[:, c:c + 16] = d[:, None] * np.asarray(rec0, np.float32).reshape(32, 16)
    assert not np.array_equal(free, Wh)


def test_oracle_half_integer_rows_use_their_tables():
    """TCQ25R (H = I): even rows of every 16-row group take TCQ2R's tables, odd rows TCQ3R's, each premultiplied
    by its format's scale (src/liqk_v2.py:887-892): every reconstructed value / d is a product gain x level of
    its row's tables, and the odd rows use levels only the higher table has."""
    from oracle import liqk_ref
    from ltq_amd.formats import TCQ_CONFIG
    cfg = TCQ_CONFIG["TCQ25R"]
    W, _ = _synthetic(32, 512, seed=5)
    U, dw, Ubi = liqk_ref.factor_hessian_ref(torch.eye(512), 0.2)
    gains, lut, hi = _oracle_tables(cfg)
    _, Wh, _, _ = liqk_ref.quantize_rows_ref(W, U, Ubi, dw, cfg, gains, lut=lut, hi=hi)
    _, _, _, d_all = liqk_ref.row_scale_ref(W, cfg)
    lo_vals = np.unique(np.float32(gains)[:, None] * np.float32(lut)[None, :])
    hi_vals = np.unique(np.float32(hi["gains_hi"])[:, None] * np.float32(hi["small_hi"])[None, :])
    d = np.maximum(d_all, np.float32(1e-8))
    only_hi = 0
    for i in range(32):
        vals = hi_vals if i % 2 else lo_vals
        for b in range(2):
            allowed = set((d[i, b] * vals).tolist())  # W_hat = fl(d fl(gain level))
            row = Wh[i, 256 * b:256 * (b + 1)]
            assert all(float(v) in allowed for v in row), (i, b)
            if i % 2:
                only_hi += sum(float(v) not in set((d[i, b] * lo_vals).tolist()) for v in row)
    assert only_hi > 0


def test_oracle_dcand_branch_pins():
    """The branch without row scale (TCQ3, src/liqk_v2.py:982-1016) with H = I (U = c I, so the whitened
    products are the raw ones over c): the first d_cand is fp16 of the block's rms times the format's scale,
    each pass's d_refit is fp16 of the least-squares ratio <w, G> / <G, G> of that pass, the next pass starts from
    it, and every row keeps the (scale, pass) of least |w - d G|^2, the earlier on ties; the reconstruction is
    fl(d G) of that choice. Keeping d_cand (no refit) changes the result."""
    from oracle import liqk_ref
    from ltq_amd.formats import TCQ_CONFIG
    cfg = TCQ_CONFIG["TCQ3"]
    W, _ = _synthetic(32, 512, seed=6)
    U, dw, Ubi = liqk_ref.factor_hessian_ref(torch.eye(512), 0.2)
    gains, _, _ = _oracle_tables(cfg)
    tr = {}
    d_full, Wh = liqk_ref.quantize_rows_dcand_ref(W, U, Ubi, dw, cfg, gains, trace=tr)
    Wn = W.numpy()
    f16 = lambda a: np.maximum(np.asarray(a, np.float32).astype(np.float16).astype(np.float32), np.float32(1e-8))
    for b, passes in enumerate(tr["blocks"]):
        w = Wn[:, 256 * b:256 * (b + 1)].astype(np.float64)
        assert np.array_equal(tr["start"][b], Wn[:, 256 * b:256 * (b + 1)])  # H = I: no feedback between blocks
        rms = np.sqrt(np.mean(w * w, axis=1)).astype(np.float32)
        assert np.array_equal(passes[0][0], f16(rms * np.float32(cfg["scale"])))
        tries = []
        for p, (d_c, G, d_r) in enumerate(passes):
            g = G.astype(np.float64)
            ls = f16(np.sum(w * g, axis=1) / np.sum(g * g, axis=1))
            assert np.mean(ls == d_r) >= 0.99 and np.all(np.abs(ls - d_r) <= np.abs(d_r) * 2.0 ** -10)
            if p > 0:
                assert np.array_equal(d_c, passes[p - 1][2])
            tries += [(d_c, G), (d_r, G)]
        loss = np.stack([np.sum((w - d.astype(np.float64)[:, None] * G.astype(np.float64)) ** 2, axis=1)
                         for d, G in tries])
        pick = np.argmin(loss, axis=0)  # first minimum
        for i in range(32):
            d, G = tries[pick[i]]
            assert np.array_equal(Wh[i, 256 * b:256 * (b + 1)], d[i] * G[i]), (b, i)
            assert d_full[i, b] == np.float16(d[i])
    _, Wh_nr = liqk_ref.quantize_rows_dcand_ref(W, U, Ubi, dw, cfg, gains, mistake="no_refit")
    assert not np.array_equal(Wh_nr, Wh)


# ---------------------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("M,N", [(64, 256), (256, 1024), (4096, 512)])
def test_gpu_ldlq_err_and_update_bit_exact(oracle, M, N):
    """ltq_ldlq_err and ltq_ldlq_update (fp32 MFMA) equal the oracle's fma chains bit for bit, with the
    reconstruction, the next block's working copy and its first tiles."""
    from ltq_amd import _lib
    L = oracle.lib()
    rng = np.random.default_rng(M + N)
    ws = (rng.standard_normal((M, 256)) * 0.05).astype(np.float32)
    G = rng.standard_normal((M, 256)).astype(np.float32)
    d = (rng.random(M) * 0.02 + 0.01).astype(np.float32)
    Ui = np.triu(rng.standard_normal((256, 256)) * 0.3 + 4 * np.eye(256)).astype(np.float32)
    Up = (rng.standard_normal((256, N)) * 0.1).astype(np.float32)
    W = (rng.standard_normal((M, N)) * 0.05).astype(np.float32)
    dn = (rng.random(M) * 0.02 + 0.01).astype(np.float32)
    Eo = np.empty((M, 256), np.float32)
    who = np.empty((M, 256), np.float32)
    L.ltq_oracle_ldlq_err(_ptr(ws), 256, _ptr(G), 256, _ptr(d), 1, _ptr(Ui), 256, _ptr(Eo), 256, _ptr(who), 256, M)
    Wo = W.copy()
    L.ltq_oracle_ldlq_update(_ptr(Wo), N, _ptr(Eo), 256, _ptr(Up), N, M, N)
    t = {k: torch.from_numpy(v).to(DEV) for k, v in dict(ws=ws, G=G, d=d, Ui=Ui, Up=Up, W=W, dn=dn).items()}
    Et = torch.empty((256, M), device=DEV)
    wh = torch.empty((M, 256), device=DEV)
    wsub = torch.empty((M, 256), device=DEV)
    xn = torch.empty((M // 16, 256), device=DEV)
    lib, st = _lib.lib(), _lib.stream_ptr()
    print(f"ldlq err / update M={M} N={N}", flush=True)
    assert lib.ltq_ldlq_err(t["ws"].data_ptr(), 256, t["G"].data_ptr(), 256, t["d"].data_ptr(), 1, t["Ui"].data_ptr(),
                            256, Et.data_ptr(), M, wh.data_ptr(), 256, M, 0, 0, st) == 0
    assert lib.ltq_ldlq_update(t["W"].data_ptr(), N, Et.data_ptr(), M, t["Up"].data_ptr(), N, M, N, wsub.data_ptr(),
                               256, xn.data_ptr(), t["dn"].data_ptr(), 1, 0, 0, st) == 0
    torch.cuda.synchronize()
    u32 = lambda a: np.ascontiguousarray(a).view(np.uint32)
    assert np.array_equal(u32(wh.cpu().numpy()), u32(who))
    assert np.array_equal(u32(Et.cpu().numpy().T), u32(Eo))
    assert np.array_equal(u32(t["W"].cpu().numpy()), u32(Wo))
    assert np.array_equal(u32(wsub.cpu().numpy()), u32(Wo[:, :256]))
    xr = (Wo[:, :16] * (np.float32(1) / dn)[:, None]).reshape(M // 16, 256)
    assert np.array_equal(u32(xn.cpu().numpy()), u32(xr))


@pytest.mark.gpu
def test_gpu_ldlq_sub_bit_exact(oracle):
    from ltq_amd import _lib
    L = oracle.lib()
    g = torch.Generator().manual_seed(4)
    M = 64
    wk = torch.randn((M, 256), generator=g)
    rec = torch.randn((M // 16, 256), generator=g)
    d = torch.rand(M, generator=g) + 0.5
    U = torch.triu(torch.randn((256, 256), generator=g) * 0.1) + torch.eye(256)
    Ui = torch.linalg.inv(U).contiguous()
    for ib in (0, 7, 15):
        s0, s1 = 16 * ib, 16 * ib + 16
        wk_d, G, fed = wk.to(DEV).clone(), torch.zeros((M, 256), device=DEV), torch.zeros((M, 256), device=DEV)
        xn = torch.zeros((M // 16, 256), device=DEV)
        rec_d, d_d, Ui_d, U_d = rec.to(DEV), d.to(DEV), Ui.to(DEV), U.to(DEV)
        print(f"ldlq_sub ib={ib}", flush=True)
        code = torch.randint(0, 1 << 19, (M // 16, 256), generator=g, dtype=torch.int32)
        code_d = code.to(DEV)
        idx = torch.full((M, 512), -1, dtype=torch.int16, device=DEV)
        gi = torch.full((M, 512), 255, dtype=torch.uint8, device=DEV)
        rc = _lib.lib().ltq_ldlq_sub(wk_d.data_ptr(), 256, rec_d.data_ptr(), d_d.data_ptr(), 1, Ui_d.data_ptr(), 256,
                                     U_d.data_ptr(), 256, ib, G.data_ptr(), 256, xn.data_ptr(), M, code_d.data_ptr(),
                                     idx[:, 256:].data_ptr(), 512, gi[:, 256:].data_ptr(), 512, fed.data_ptr(), 256,
                                     0, 0, 0, _lib.stream_ptr())
        assert rc == 0
        torch.cuda.synchronize()
        cv = code.view(M, 16)
        assert torch.equal(idx.cpu()[:, 256 + s0:256 + s1], (cv & 0xFFFF).to(torch.int16))
        assert torch.equal(gi.cpu()[:, 256 + s0:256 + s1], (cv >> 16).to(torch.uint8))
        assert int((idx.cpu() != -1).sum()) == M * 16
        wo, Go, fo = wk.numpy().copy(), np.zeros((M, 256), np.float32), np.zeros((M, 256), np.float32)
        xo = np.zeros((M // 16, 256), np.float32)
        L.ltq_oracle_ldlq_sub(_ptr(wo), 256, _ptr(rec.numpy()), _ptr(d.numpy()), 1, _ptr(Ui.numpy()), 256,
                              _ptr(U.numpy()), 256, ib, _ptr(Go), 256, _ptr(xo) if s1 < 256 else None, M, _ptr(fo), 256)
        u32 = lambda a: np.ascontiguousarray(a).view(np.uint32)
        assert np.array_equal(u32(wk_d.cpu().numpy()), u32(wo))
        assert np.array_equal(u32(G.cpu().numpy()), u32(Go))
        assert np.array_equal(u32(fed.cpu().numpy()[:, s0:s1]), u32(fo[:, s0:s1]))
        if s1 < 256:
            assert np.array_equal(u32(xn.cpu().numpy()), u32(xo))


ROW_CASES = [("TCQ275X2", 64, 768, False), ("TCQ275X", 64, 768, False), ("TCQ25X", 64, 768, False),
             ("TCQ375X", 64, 768, False), ("TCQ3X3", 64, 768, True), ("TCQ275X2", 256, 2048, False),
             ("TCQ3R", 64, 768, False), ("TCQ4RH3", 64, 768, False), ("TCQ25R", 64, 768, False),
             ("TCQ35R", 48, 512, False), ("TCQ3", 64, 768, False), ("TCQ4", 48, 512, False)]


def _oracle_tables(cfg):
    """(gains, lut, hi) for quantize_rows_ref: a half-integer format's tables premultiplied by their formats'
    scales (src/liqk_v2.py:887-892), gains evaluated on the CPU as the quantizer's are."""
    from ltq_amd.formats import TCQ_CONFIG
    from ltq_amd.tcq_proto import make_gains
    if "K_hi" not in cfg:
        return make_gains(cfg["h"], cfg["step"], "cpu").numpy(), None, None
    lo, hi = TCQ_CONFIG[cfg["lo"]], TCQ_CONFIG[cfg["hi"]]
    lut = np.asarray(lo["lut"], np.float32) * np.float32(lo["scale"])
    return (make_gains(lo["h"], lo["step"], "cpu").numpy(), lut,
            {"small_hi": np.asarray(hi["lut"], np.float32) * np.float32(hi["scale"]),
             "gains_hi": make_gains(hi["h"], hi["step"], "cpu").numpy()})


@pytest.mark.gpu
@pytest.mark.parametrize("spec,M,K,identity_h", ROW_CASES)
def test_gpu_quantize_rows_bit_exact(spec, M, K, identity_h):
    """The GPU row quantizer against the oracle on the same rotated rows and factors: codes, gain indices, tile
    values, reconstruction, fed values and block scales bit for bit (C3 formats with a real Hessian and outlier
    columns; C2's TCQ3X3 with gain candidates and H = I; carried-state formats, with gain candidates and
    half-integer tables)."""
    from oracle import liqk_ref
    from ltq_amd import liqk, rotation
    from ltq_amd.formats import TCQ_CONFIG
    cfg = TCQ_CONFIG[spec]
    tb = bool(cfg.get("tb"))
    W, H = _synthetic(M, K, outliers=max(1, K // 100))
    if identity_h:
        H = torch.eye(K)
    W_rot, H_rot, _ = rotation.compute_optimal_suh(W.to(DEV), H.to(DEV), seed=1337)
    U, diag_w, Ub_inv = liqk.factor_hessian(H_rot, 0.2)
    fed = torch.empty((M, K), device=DEV) if cfg.get("row_scale") else None  # the d_cand branch has no single fed
    print(f"quantize rows {M} x {K} {spec}", flush=True)
    liqk.PACK = {"groups": []} if tb else None  # .ltq fields exist for the tail-biting formats
    try:
        d_full, W_hat = liqk._quantize_rows_tcq_ldlq(W_rot, U, Ub_inv, diag_w, spec, fed=fed)
        grp = liqk.PACK["groups"].pop() if tb else None
    finally:
        liqk.PACK = None
    torch.cuda.synchronize()
    gains, lut, hi = _oracle_tables(cfg)
    d_ref, Wh_ref, codes, fed_ref = liqk_ref.quantize_rows_ref(W_rot.cpu(), U.cpu(), Ub_inv.cpu(), diag_w.cpu(), cfg,
                                                               gains, lut=lut, hi=hi)
    u32 = lambda a: np.ascontiguousarray(a).view(np.uint32)
    n_idx = int((grp["idx"].cpu().numpy() != codes["idx"]).sum()) if tb else 0
    n_gi = int((grp["gi"].cpu().numpy() != codes["gi"]).sum()) if tb else 0
    Wr = W_rot.cpu().numpy().astype(np.float64)
    mse_gpu = float(np.mean((Wr - W_hat.cpu().numpy()) ** 2))
    mse_ref = float(np.mean((Wr - Wh_ref) ** 2))
    print(f"{spec} {M}x{K}: code mismatches {n_idx}, gain index mismatches {n_gi}, MSE gpu {mse_gpu:.6e} "
          f"oracle {mse_ref:.6e} (relative difference {abs(mse_gpu - mse_ref) / mse_ref:.1e})", flush=True)
    assert n_idx == 0 and n_gi == 0
    if fed is not None:
        assert np.array_equal(u32(fed.cpu().numpy()), u32(fed_ref))
    assert np.array_equal(u32(W_hat.cpu().numpy()), u32(Wh_ref))
    assert np.array_equal(d_full.cpu().numpy().view(np.uint16), d_ref.view(np.uint16))
    assert abs(mse_gpu - mse_ref) <= 1e-6 * mse_ref


@pytest.mark.gpu
def test_gpu_ldlq_identity_at_c3_shape():
    """The full C3 shape (4096 x 14336, TCQ275X2, H from 2048 activation rows): the GPU loop satisfies
    W_rot - W_hat = E U (float64 on the device) to a few units of roundoff."""
    from ltq_amd import liqk, rotation
    M, K = 4096, 14336
    g = torch.Generator(device=DEV).manual_seed(0)
    W = torch.randn((M, K), generator=g, device=DEV) * 0.02
    X = torch.randn((2048, K), generator=g, device=DEV)
    H = X.T @ X / 2048
    del X
    print("quantize rows 4096 x 14336 TCQ275X2 with fed values", flush=True)
    W_rot, H_rot, _ = rotation.compute_optimal_suh(W, H, seed=1337)
    del H
    U, diag_w, Ub_inv = liqk.factor_hessian(H_rot, 0.2)
    del H_rot
    fed = torch.empty((M, K), device=DEV)
    _, W_hat = liqk._quantize_rows_tcq_ldlq(W_rot, U, Ub_inv, diag_w, "TCQ275X2", fed=fed)
    torch.cuda.synchronize()
    print("identity check in float64", flush=True)
    Ud = U.double()
    E = torch.empty((M, K), dtype=torch.float64, device=DEV)
    for c0 in range(0, K, 16):
        b, s0 = c0 // 256, c0 % 256
        Uinv_jj = Ub_inv[b, s0:s0 + 16, s0:s0 + 16].double()
        E[:, c0:c0 + 16] = (fed[:, c0:c0 + 16].double() - W_hat[:, c0:c0 + 16].double()) @ Uinv_jj
    R = (W_rot.double() - W_hat.double()) - E @ Ud
    B = W_rot.double().abs() + E.abs() @ Ud.abs()
    rel = float((R.abs() / B).max())
    print(f"C3 identity residual: {rel / ULP:.1f} ulp", flush=True)
    assert rel <= 64 * ULP
