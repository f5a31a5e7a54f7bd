"""The matrix path around the Viterbi: Hessian factorization, row scale, LDLQ error feedback, PACK and refit
(src/liqk_v2.py:877-1200).

CPU: the oracle's torch restatement of the row scale against its float64 definition, and of the factors
against their defining identities (U^T U = H^-1 after damping, block inverses).
GPU: the HIP row scale and LDLQ kernels against the restatement, the whole TCQ275X2 row quantizer against the
CPU oracle driving the C Viterbi oracle, and PACK -> .ltq bytes -> decode equal to the quantizer's fields.
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


@pytest.mark.gpu
def test_gpu_ldlq_sub_matches_float64():
    from ltq_amd import _lib
    g = torch.Generator().manual_seed(4)
    M = 64
    wk = torch.randn((M, 256), generator=g)
    rec = torch.randn((M // 16, 256), generator=g)
    d = torch.rand(M, generator=g) + 0.5
    U = torch.triu(torch.randn((256, 256), generator=g) * 0.1) + torch.eye(256)
    Ui = torch.linalg.inv(U).contiguous()  # LAPACK may return column-major strides
    for ib in (0, 7, 15):
        s0, s1 = 16 * ib, 16 * ib + 16
        wk_d, G = wk.to(DEV).clone(), torch.zeros((M, 256), device=DEV)
        xn = torch.zeros((M // 16, 256), device=DEV)
        rec_d, d_d, Ui_d, U_d = rec.to(DEV), d.to(DEV), Ui.to(DEV), U.to(DEV)  # alive across the call
        print(f"ldlq_sub ib={ib}", flush=True)
        code = torch.randint(0, 1 << 19, (M // 16, 256), generator=g, dtype=torch.int32)
        code_d = code.to(DEV)
        idx = torch.full((M, 512), -1, dtype=torch.int16, device=DEV)
        gi = torch.full((M, 512), 255, dtype=torch.uint8, device=DEV)
        rc = _lib.lib().ltq_ldlq_sub(wk_d.data_ptr(), 256, rec_d.data_ptr(), d_d.data_ptr(), 1, Ui_d.data_ptr(), 256,
                                     U_d.data_ptr(), 256, ib, G.data_ptr(), 256, xn.data_ptr(), M, code_d.data_ptr(),
                                     idx[:, 256:].data_ptr(), 512, gi[:, 256:].data_ptr(), 512, _lib.stream_ptr())
        assert rc == 0
        torch.cuda.synchronize()
        cv = code.view(M, 16)
        assert torch.equal(idx.cpu()[:, 256 + s0:256 + s1], (cv & 0xFFFF).to(torch.int16))
        assert torch.equal(gi.cpu()[:, 256 + s0:256 + s1], (cv >> 16).to(torch.uint8))
        assert int((idx.cpu() != -1).sum()) == M * 16 and int((gi.cpu() != 255).sum()) <= M * 16
        g_sub = rec.view(M, 16).double()
        err = (wk[:, s0:s1].double() - d.double().unsqueeze(1) * g_sub) @ Ui.double()[s0:s1, s0:s1]
        ref = wk.double().clone()
        ref[:, s1:] -= err @ U.double()[s0:s1, s1:]
        assert torch.allclose(wk_d.cpu().double(), ref, rtol=1e-5, atol=1e-5)
        assert torch.equal(G.cpu()[:, s0:s1], rec.view(M, 16))
        if s1 < 256:
            xr = (wk_d.cpu()[:, s1:s1 + 16] * (1.0 / d).unsqueeze(1)).contiguous().view(M // 16, 256)
            assert torch.equal(xn.cpu(), xr)  # the same fp32 products as the reference's w * inv_d


@pytest.mark.gpu
@pytest.mark.parametrize("spec,identity_h", [("TCQ275X2", False), ("TCQ275X", False), ("TCQ25X", False),
                                             ("TCQ375X", False), ("TCQ3X3", True)])
def test_gpu_quantize_rows_vs_oracle(spec, identity_h):
    """Rows [64, 512] (C3 formats with a real Hessian; C2's TCQ3X3 with gain candidates and H = I): the GPU
    quantizer against the CPU oracle on the same row scale. The first sub-block's inputs are identical, so its
    codes are bit-exact; afterwards the error feedback sums round differently (FMA vs the oracle's torch
    matmul), so codes may differ at near-ties only."""
    from oracle import liqk_ref
    from ltq_amd import liqk, rotation
    from ltq_amd.formats import TCQ_CONFIG, make_format
    cfg = TCQ_CONFIG[spec]
    M, K = 64, 512
    W, H = _synthetic(M, K)
    if identity_h:
        H = torch.eye(K)
    Wd, Hd = W.to(DEV), H.to(DEV)
    W_rot, H_rot, _ = rotation.compute_optimal_suh(Wd, Hd, seed=1337)
    U, diag_w, Ub_inv = liqk.factor_hessian(H_rot, 0.2)
    print(f"quantize rows 64 x 512 {spec}", flush=True)
    liqk.PACK = {"groups": []}
    try:
        d_full, W_hat = liqk._quantize_rows_tcq_ldlq(W_rot, U, Ub_inv, diag_w, spec)
        grp = liqk.PACK["groups"].pop()
    finally:
        liqk.PACK = None
    torch.cuda.synchronize()
    _, _, d_dev = liqk.row_scale(W_rot, cfg)
    f = make_format(spec)
    dr, Wh_ref, codes, _ = liqk_ref.quantize_rows_ref(W_rot.cpu(), U.cpu(), Ub_inv.cpu(), diag_w.cpu(), cfg,
                                                      f.gain_tab, d_rb_all=d_dev.cpu())
    idx, gi = grp["idx"].cpu(), grp["gi"].cpu()
    assert torch.equal(idx[:, :16], codes["idx"][:, :16]) and torch.equal(gi[:, :16], codes["gi"][:, :16])
    agree = (idx == codes["idx"]).float().mean().item()
    assert agree >= 0.98, agree
    Wr = W_rot.cpu()
    mse_gpu = (Wr - W_hat.cpu()).square().mean().item()
    mse_ref = (Wr - Wh_ref).square().mean().item()
    assert abs(mse_gpu - mse_ref) <= 0.02 * mse_ref, (mse_gpu, mse_ref)
    assert torch.equal(d_full.cpu(), dr)


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
