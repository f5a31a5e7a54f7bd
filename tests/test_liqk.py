"""The matrix path around the Viterbi: Hessian factorization, row scale, LDLQ error feedback, PACK and refit
(src/liqk_v2.py:877-1200).

CPU: the oracle's torch restatement of the row scale against its float64 definition, and of the factors
against their defining identities (U^T U = H^-1 after damping, block inverses).
GPU: the HIP row scale against the oracle's definition bit for bit; the c_row / suh refit against its closed
forms and float64 recomputations; PACK -> .ltq bytes -> decode equal to the quantizer's fields. The LDLQ loop
is pinned in tests/test_ldlq.py.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

DEV = "cuda"


def _synthetic(M, K, n_act=300, seed=0):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((M, K), generator=g)
    chi2 = sum(torch.randn((M, K), generator=g).square() for _ in range(5))
    W = (z / (chi2 / 5).sqrt()) * 0.02
    X = torch.randn((n_act, K), generator=g)
    return W, X.T @ X / n_act


def test_row_scale_ref_matches_float64_definition():
    from oracle import liqk_ref
    from ltq_amd.formats import TCQ_CONFIG
    cfg = TCQ_CONFIG["TCQ275X2"]
    W, _ = _synthetic(48, 1024)
    W[3, 256:512] *= 40  # an outlier block
    rms, d_row, e, d = liqk_ref.row_scale_ref(W, cfg)
    w64 = W.double().view(48, 4, 256)
    rms64 = w64.square().mean(dim=2).sqrt().clamp(min=1e-10) * cfg.get("scale", 1.0)
    # the fixed-order fp32 block sums are sums of 256 positive terms: within 9 ulp (log2(64) + 3 roundings)
    assert np.all(np.abs(rms / rms64.numpy() - 1) < 10 * 2.0 ** -24)
    d64 = torch.exp(torch.log(torch.from_numpy(rms).double()).mean(dim=1))
    assert torch.allclose(torch.from_numpy(d_row).double(), d64, rtol=2 ** -11)  # the nearest fp16
    e64 = (torch.log2(torch.from_numpy(rms).double() / torch.from_numpy(d_row).double().unsqueeze(1)) / 0.25)
    assert torch.all((torch.from_numpy(e).double() - e64.clamp(-16, 15)).abs() <= 0.5 + 1e-6)
    assert int(e[3, 1]) == 15  # the outlier block saturates the 5-bit exponent
    tab = liqk_ref._exp2_table(0.25, 5)
    assert np.array_equal(d, np.maximum(d_row[:, None] * tab[e.astype(np.int64) + 16], np.float32(1e-8)))


def test_exp2_table_is_torch_exp2():
    """The shared block-exponent table equals the reference's torch.exp2(0.25 e) (float32, CPU) entry for entry,
    and the product side (formats.exp2_table) is the same table."""
    from oracle import liqk_ref
    from ltq_amd.formats import exp2_table
    e = torch.arange(-16, 16, dtype=torch.float32)
    ref = torch.exp2(0.25 * e).numpy()
    assert np.array_equal(exp2_table().view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(liqk_ref._exp2_table(0.25, 5).view(np.uint32), ref.view(np.uint32))


def test_row_scale_ref_flips_vs_torch_fp32():
    """The exact definition against the reference's fp32 torch text on C2/C3-like rows: they differ only where
    an fp32 reduction or function lands d_row / e on the other side of an fp16 / half-step boundary. Where d_row
    and e agree, d is the same bits."""
    from oracle import liqk_ref
    from ltq_amd.formats import TCQ_CONFIG
    cfg = TCQ_CONFIG["TCQ275X2"]
    W, _ = _synthetic(512, 2048, seed=3)
    W[:, 77] *= 20
    _, d_row, e, d = liqk_ref.row_scale_ref(W, cfg)
    _, d_t, e_t, d_all_t = liqk_ref.row_scale_torch_fp32(W, cfg)
    flip_d = float((torch.from_numpy(d_row) != d_t).float().mean())
    flip_e = float((torch.from_numpy(e).float() != e_t).float().mean())
    print(f"row scale vs torch fp32: d_row flips {flip_d:.4%}, e flips {flip_e:.4%}")
    assert flip_d <= 0.01 and flip_e <= 0.005
    ok = (torch.from_numpy(d_row) == d_t).unsqueeze(1) & (torch.from_numpy(e).float() == e_t)
    assert torch.equal(torch.from_numpy(d)[ok], d_all_t.clamp(min=1e-8)[ok])


def test_factor_ref_identities():
    from oracle import liqk_ref
    _, H = _synthetic(16, 512)
    U, diag_w, Ub_inv = liqk_ref.factor_hessian_ref(H, 0.2)
    Hd = H.double().clone()
    Hd.diagonal().add_(0.2 * Hd.diagonal().mean())
    assert torch.allclose((U.double().T @ U.double()) @ Hd, torch.eye(512, dtype=torch.float64), atol=1e-3)
    assert torch.allclose(diag_w, 1.0 / torch.diagonal(U) ** 2)
    for b in range(2):
        blk = U[b * 256:(b + 1) * 256, b * 256:(b + 1) * 256].double()
        assert torch.allclose(blk @ Ub_inv[b].double(), torch.eye(256, dtype=torch.float64), atol=1e-3)


# ---------------------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("M,K,seed", [(256, 2048, 0), (4096, 14336, 5)])
def test_gpu_row_scale(M, K, seed):
    """The HIP row scale equals the oracle's definition bit for bit: d_row, e and d (no flips), including the
    C3 shape with outlier columns and an all-zero row (the 1e-10 / 1e-8 clamps)."""
    from oracle import liqk_ref
    from ltq_amd import liqk
    from ltq_amd.formats import TCQ_CONFIG
    cfg = TCQ_CONFIG["TCQ275X2"]
    g = torch.Generator().manual_seed(seed)
    W = torch.randn((M, K), generator=g) * 0.02
    W[:, torch.randperm(K, generator=g)[:max(1, K // 100)]] *= 20
    W[7] = 0.0
    print(f"row scale {M} x {K}", flush=True)
    d_row, e, d = liqk.row_scale(W.to(DEV), cfg)
    torch.cuda.synchronize()
    _, d_ref, e_ref, d_all_ref = liqk_ref.row_scale_ref(W, cfg)
    n_d = int((d_row.cpu().numpy() != d_ref).sum())
    n_e = int((e.cpu().numpy() != e_ref).sum())
    print(f"row scale {M} x {K}: d_row differs in {n_d} rows, e in {n_e} blocks", flush=True)
    assert n_d == 0 and n_e == 0
    assert np.array_equal(d.cpu().numpy().view(np.uint32), d_all_ref.view(np.uint32))


def _refit_inputs(M=64, K=512, seed=11, identity_h=False):
    g = torch.Generator().manual_seed(seed)
    W, H = _synthetic(M, K, seed=seed)
    if identity_h:
        H = torch.eye(K)
    suh = ((torch.rand(K, generator=g) * 1.5 + 0.5) * torch.sign(torch.randn(K, generator=g))).half().float()
    noise = 1 + 0.1 * torch.randn((M, K), generator=g)
    W_hat = W * noise
    W_hat[0] = W[0] * 0.8     # c_row = 1.25
    W_hat[1] = W[1] * 3.0     # c_row ~ 1/3: outside (0.5, 2), replaced by 1
    W_hat[2] = W[2] * 0.25    # c_row ~ 4: replaced by 1
    U_base = W_hat / suh
    d = (torch.rand((M, K // 256), generator=g) * 0.02 + 0.01).half()
    rw = (torch.rand(M, generator=g) + 0.5)
    return W, H, U_base, suh, d, rw


@pytest.mark.gpu
@pytest.mark.parametrize("weighted", [False, True])
def test_gpu_refit_pins(weighted):
    """refit_scales against what fixes it: c_row is the per-row ratio <W_hat, W H> / <W_hat, W_hat H> (float64)
    with the (0.5, 2) rule, d_new = fp16(d c_row) exactly, the normal equations (A, b) equal their float64
    definition, the solve's output satisfies them to fp32 backward error, the candidate follows the fp16 /
    validity rule exactly, and the two losses and the acceptance agree with their float64 recomputation."""
    from ltq_amd import liqk, rotation
    W, H, U_base, suh, d, rw = _refit_inputs()
    rw_n = rotation.normalized_row_weights(rw.to(DEV)).float() if weighted else None
    Wd, Hd = W.to(DEV), H.to(DEV)
    HW = Wd @ Hd
    print(f"refit pins weighted={weighted}", flush=True)
    rec, W_hat_out, HQ_out = liqk.refit_scales(Wd, Hd, HW, U_base.to(DEV), suh.to(DEV), d.to(DEV), rw_n, keep=True)
    torch.cuda.synchronize()
    W64, H64, Ub64, s64 = W.double(), H.double(), U_base.double(), suh.double()
    Wh64 = Ub64 * s64
    c64 = (Wh64 * (W64 @ H64)).sum(1) / (Wh64 * (Wh64 @ H64)).sum(1)
    c_raw = rec.c_raw.cpu().double()
    assert torch.allclose(c_raw, c64, rtol=2e-4), float(((c_raw - c64) / c64).abs().max())
    assert abs(float(c_raw[0]) - 1.25) < 1e-4 and float(rec.c_row[1]) == 1.0 and float(rec.c_row[2]) == 1.0
    ok = torch.isfinite(rec.c_raw) & (rec.c_raw > 0.5) & (rec.c_raw < 2.0)
    assert torch.equal(rec.c_row, torch.where(ok, rec.c_raw, torch.ones_like(rec.c_raw)))
    assert torch.equal(rec.d_new.cpu(), (d.float() * rec.c_row.cpu().unsqueeze(1)).half())
    assert torch.allclose(rec.c_eff.cpu().double(), (rec.d_new.cpu().double() / d.double()).mean(1), rtol=1e-6)
    # normal equations
    Us = Ub64 * rec.c_eff.cpu().double().unsqueeze(1)
    Uw = Us if rw_n is None else Us * rw_n.cpu().double().unsqueeze(1)
    A64 = (Uw.T @ Us) * H64
    A64.diagonal().add_(1e-3 * A64.diagonal().mean())
    b64 = (Uw * (W64 @ H64)).sum(0)
    A_low = torch.tril(rec.A.cpu().double())
    assert float((A_low - torch.tril(A64)).abs().max()) <= 1e-4 * float(A64.abs().max())
    assert torch.allclose(rec.b.cpu().double(), b64, rtol=1e-3, atol=1e-4 * float(b64.abs().max()))
    A_sys = A_low + torch.tril(A_low, -1).T            # the system the solver was handed
    sv = rec.s_solved.cpu().double()
    resid = float((A_sys @ sv - rec.b.cpu().double()).abs().max())
    scale = float(A_sys.abs().sum(1).max() * sv.abs().max())
    print(f"refit solve: residual {resid / scale:.2e} of ||A|| ||s||", flush=True)
    assert resid <= 1e-5 * scale
    s16 = rec.s_solved.half().float()
    good = torch.isfinite(s16) & (s16.abs() > 0.05) & (s16.abs() < 10.0)
    assert torch.equal(rec.suh_cand, torch.where(good, s16, suh.to(DEV)))
    # losses in float64 and the acceptance
    wt = torch.ones(W.shape[0], dtype=torch.float64) if rw_n is None else rw_n.cpu().double()
    loss_b = float((((W64 - Wh64) @ H64 * (W64 - Wh64)).sum(1) * wt).sum())
    Wc = Us * rec.suh_cand.cpu().double()
    loss_c = float((((W64 - Wc) @ H64 * (W64 - Wc)).sum(1) * wt).sum())
    tol = 1e-3 * max(abs(loss_b), abs(loss_c))
    assert abs(rec.loss_base - loss_b) <= tol and abs(rec.loss_cand - loss_c) <= tol
    if abs(loss_b - loss_c) > 2 * tol:
        assert rec.accepted == (loss_c < loss_b)
    assert rec.accepted == (rec.loss_cand < rec.loss_base)
    chosen = (Us.float() * rec.suh_cand.cpu()) if rec.accepted else (U_base * suh)
    assert torch.allclose(W_hat_out.cpu(), chosen, rtol=1e-6, atol=1e-9)


@pytest.mark.gpu
def test_gpu_refit_column_scale_closed_form():
    """With H = I the normal matrix is diagonal: s_j = <U_w[:, j], W[:, j]> / (<U_w[:, j], U_s[:, j]> + ridge),
    ridge = 1e-3 mean of the diagonal."""
    from ltq_amd import liqk
    W, H, U_base, suh, d, _ = _refit_inputs(identity_h=True, seed=12)
    Wd, Hd = W.to(DEV), H.to(DEV)
    rec, _, _ = liqk.refit_scales(Wd, Hd, Wd @ Hd, U_base.to(DEV), suh.to(DEV), d.to(DEV), None)
    torch.cuda.synchronize()
    Us = U_base.double() * rec.c_eff.cpu().double().unsqueeze(1)
    n = (Us * Us).sum(0)
    s = (Us * W.double()).sum(0) / (n + 1e-3 * n.mean())
    assert torch.allclose(rec.s_solved.cpu().double(), s, rtol=1e-5, atol=1e-6)


@pytest.mark.gpu
def test_gpu_quantize_matrix_pack_decodes_to_fields():
    """quantize_matrix_liqk_v2 with PACK: the packed .ltq slice decodes (oracle decoder) to exactly the tile
    values G of the PACK fields, and the proxy loss is that of a working quantizer."""
    from oracle import pack
    from ltq_amd import liqk
    from ltq_amd.formats import make_format
    from ltq_amd.ltq_file import pack_slice
    M, K = 64, 512
    W, H = _synthetic(M, K, seed=1)
    print("quantize matrix 64 x 512 TCQ275X2 with PACK", flush=True)
    liqk.PACK = {}
    try:
        q, W_hat, rel = liqk.quantize_matrix_liqk_v2(W.to(DEV), H.to(DEV), "TCQ275X2", damp=0.02)
        pm = liqk.PACK["matrix"]
    finally:
        liqk.PACK = None
    torch.cuda.synchronize()
    assert 0.0 < rel < 0.2, rel
    f = make_format("TCQ275X2")
    b = pack_slice(pm["idx"], pm["gi"], f)
    dec = pack.decode_slice(b, M, K, f.K, f.frac, f.h, f.sub, f.masks, f.lut, f.gain_tab)
    assert np.array_equal(dec.view(np.uint32), pm["G"].cpu().numpy().view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("spec", ["TCQ3R", "TCQ25R", "TCQ3", ((0, 32, "TCQ3R"), (32, 64, "TCQ275X2"))])
def test_gpu_quantize_matrix_other_branches(spec):
    """The matrix driver over the carried-state, half-integer and d_cand (no row scale) branches, and a matrix
    whose row slices mix a carried-state and a tail-biting format: the reconstruction is finite, the proxy loss
    is the one its definition gives for the returned W_hat, and it is below that of the all-zero reconstruction."""
    from ltq_amd import liqk
    M, K = 64, 512
    W, H = _synthetic(M, K, seed=2)
    Wd, Hd = W.to(DEV), H.to(DEV)
    print(f"quantize matrix {spec}", flush=True)
    q, W_hat, rel = liqk.quantize_matrix_liqk_v2(Wd, Hd, spec)
    torch.cuda.synchronize()
    assert torch.isfinite(W_hat).all() and q["d"].shape == (M, K // 256)
    dW = (Wd - W_hat).double()
    expect = float(torch.trace(dW @ Hd.double() @ dW.T) / torch.trace(Wd.double() @ Hd.double() @ Wd.double().T))
    print(f"{spec}: relative proxy loss {rel:.4f} (recomputed {expect:.4f})", flush=True)
    assert abs(rel - expect) <= 1e-3 * expect and rel < 0.5
