"""The MoE expert batch (K=3 D4, 16-subset labels, 3-bit gains over 4 candidates, per-expert
Hessians from 256 activation rows, damping 0.2): src/streaming_quant.py:262-276 quantizes every expert alone.

CPU: the C4 format's table is the closed-form training start (tables.closed_form_table, pinned against
scipy's quantiles in tests/test_tables.py) and its .ltq tile size.
GPU: quantize_experts gives every expert exactly what its own quantize_matrix_liqk_v2 call gives (W_hat, scales,
PACK fields, loss), and the shared row loop of two down_proj-shaped experts [2048, 768] equals the CPU oracle's
loop on each expert bit for bit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

DEV = "cuda"


def test_c4_format_is_the_closed_form_start():
    from ltq_amd.formats import TCQ_CONFIG, make_format
    from ltq_amd.tables import closed_form_table
    c = TCQ_CONFIG["TCQ275Y3"]
    assert (c["K"], c["pp"], tuple(c["m_extra"]), c["h"], c["n_cand"], c["sub"]) == (3, 2, (40, 475), 3, 4, 16)
    t = closed_form_table(3, (40, 475), device="cpu").numpy()
    assert np.array_equal(np.asarray(c["lut"], np.float32).view(np.uint32), t.view(np.uint32))
    f = make_format("TCQ275Y3")
    # codes 16 + planes 16 + lsb 12 (D4: 3 of every 4) + gains 3 (16 sub-blocks x 3 bits) words of 16 bits
    assert f.tile_bytes() == 2 * (16 + 16 + 12 + 3) and f.n_labels == 16


def _experts(n, R, K, seed):
    g = torch.Generator().manual_seed(seed)
    Ws, Hs = [], []
    for _ in range(n):
        z = torch.randn((R, K), generator=g)
        chi2 = sum(torch.randn((R, K), generator=g).square() for _ in range(5))
        Ws.append(((z / (chi2 / 5).sqrt()) * 0.02).to(torch.bfloat16))
        X = torch.randn((256, K), generator=g)
        Hs.append(X.T @ X / 256)
    return Ws, Hs


@pytest.mark.gpu
def test_gpu_expert_batch_equals_single_calls():
    from ltq_amd import liqk, moe
    Ws, Hs = _experts(3, 256, 512, seed=1)
    Wd, Hd = [w.to(DEV) for w in Ws], [h.to(DEV) for h in Hs]
    seeds = [moe.expert_seed(3, f"gu{e}") for e in range(3)]
    print("expert batch: 3 experts 256 x 512 TCQ275Y3", flush=True)
    liqk.PACK = {}
    try:
        outs, fields = moe.quantize_experts(Wd, Hd, "TCQ275Y3", seeds, damp=0.02)
        for e in range(3):
            q, W_hat, rel = liqk.quantize_matrix_liqk_v2(Wd[e], Hd[e], "TCQ275Y3", seed=seeds[e], damp=0.02)
            pm = liqk.PACK["matrix"]
            qb, W_hat_b, rel_b = outs[e]
            assert torch.equal(W_hat_b.view(torch.int32), W_hat.view(torch.int32)), e
            assert torch.equal(qb["d"], q["d"]) and torch.equal(qb["suh"], q["suh"]) and rel_b == rel
            for k in ("idx", "gi", "G", "d_row", "e", "suh"):
                assert torch.equal(fields[e][k], pm[k]), (e, k)
    finally:
        liqk.PACK = None


@pytest.mark.gpu
def test_gpu_expert_rows_vs_oracle():
    """Two down_proj-shaped experts [2048, 768] stacked through the shared LDLQ loop against the oracle's loop on
    each expert with that expert's factors: codes, gain indices and reconstruction bit for bit."""
    from oracle import liqk_ref
    from ltq_amd import liqk
    from ltq_amd.formats import TCQ_CONFIG, make_format
    spec = "TCQ275Y3"
    cfg, f = TCQ_CONFIG[spec], make_format(spec)
    Ws, Hs = _experts(2, 2048, 768, seed=2)
    jobs = []
    for e in range(2):
        j = liqk._MatrixJob(Ws[e].to(DEV), Hs[e].to(DEV), [(0, 2048, spec)], 100 + e, 0.02, None)
        j.rotate_and_factor()
        jobs.append(j)
    print("expert rows: 2 experts 2048 x 768 TCQ275Y3", flush=True)
    liqk.PACK = {"groups": []}
    try:
        _, W_hat = liqk._ldlq_rows(torch.cat([j.W_rot for j in jobs]), torch.stack([j.U for j in jobs]),
                                   torch.stack([j.U_blks_inv for j in jobs]), torch.stack([j.diag_w for j in jobs]),
                                   spec)
        grp = liqk.PACK["groups"].pop()
    finally:
        liqk.PACK = None
    torch.cuda.synchronize()
    for e, j in enumerate(jobs):
        rows = slice(2048 * e, 2048 * (e + 1))
        _, Wh_ref, codes, _ = liqk_ref.quantize_rows_ref(j.W_rot.cpu(), j.U.cpu(), j.U_blks_inv.cpu(),
                                                         j.diag_w.cpu(), cfg, f.gain_tab)
        n_idx = int((grp["idx"][rows].cpu().numpy() != codes["idx"]).sum())
        n_gi = int((grp["gi"][rows].cpu().numpy() != codes["gi"]).sum())
        print(f"expert {e}: code mismatches {n_idx}, gain index mismatches {n_gi}", flush=True)
        assert n_idx == 0 and n_gi == 0
        assert np.array_equal(W_hat[rows].cpu().numpy().view(np.uint32), Wh_ref.view(np.uint32))
