"""The TCQ matrix quantizer on the GPU: Hessian factorization, row scale, LDLQ error feedback around the Viterbi,
PACK fields and the c_row / suh refit.

Mirrors (same names, argument meaning, results and the module-level PACK switch):
  PACK                        src/liqk_v2.py:74       (dict -> the matrix's .ltq fields are collected)
  factor_hessian              src/liqk_v2.py:1066-1088 (damping, Cholesky of the flipped H, U, diag_w, U_blks_inv)
  row_scale                   src/liqk_v2.py:938-946  (HIP kernel ltq_row_scale)
  _quantize_rows_tcq_ldlq     src/liqk_v2.py:877-1021 (the row-scale branch: every tail-biting / R format;
                                                       HIP kernels ltq_ldlq_prep / ltq_ldlq_sub per sub-block,
                                                       tcq_viterbi two-pass tail-biting, library GEMM across blocks)
  quantize_matrix_liqk_v2     src/liqk_v2.py:1029-1200 (single TCQ spec or TCQ row slices; refit and PACK tail)

The dense linear algebra (Cholesky, triangular inverse and solves, the inter-block error GEMM, the refit
products) runs on the device through ltq_amd.linalg and torch, i.e. as large hipBLASLt / rocBLAS GEMMs.
"""
from __future__ import annotations

import os
from typing import Dict, List, Optional, Tuple

import torch

from . import _lib, linalg, rotation
from .formats import QK_K, SUBBLOCK_SIZE, TCQ_CONFIG
from .tcq_proto import make_gains, viterbi_ub_cuda

PACK: Optional[dict] = None
# timing hook (off by default): a list receives (stage name, torch.cuda.Event) at every stage boundary of
# quantize_matrix_liqk_v2, recorded on the stream the kernels run on
STAGE_EVENTS: Optional[list] = None
NUM_SUBBLOCKS = QK_K // SUBBLOCK_SIZE


def _mark(name: str) -> None:
    if STAGE_EVENTS is not None:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(torch.cuda.current_stream())
        STAGE_EVENTS.append((name, ev))


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: HIP error code {rc}" if rc > 0 else f"{what}: rejected arguments")


@torch.no_grad()
def factor_hessian(H_rot: torch.Tensor, damp: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(U, diag_w, U_blks_inv): U upper Cholesky factor of H^-1 (U^T U = H^-1) from one factorization of the
    flipped, damped H and one triangular inversion; diag_w = 1 / diag(U)^2; inverses of U's 256 x 256 diagonal
    blocks."""
    K = H_rot.shape[0]
    nblocks = K // QK_K
    H_reg = H_rot.float().clone()
    diag_mean = H_reg.diagonal().mean().clamp(min=1e-8)
    H_reg.diagonal().add_(damp * diag_mean)
    L_flip, info = linalg.cholesky_lower(H_reg.flip(0, 1).contiguous())
    del H_reg
    if int(info.item()) != 0:
        raise torch.linalg.LinAlgError("factor_hessian: the damped Hessian is not positive definite")
    U = linalg.tri_inv_lower(L_flip).flip(0, 1).contiguous()  # the kernels take row-major factors
    diag_w = 1.0 / (torch.diagonal(U) ** 2).clamp(min=1e-12)
    # U = J L'^-1 J (J reverses the order), so U's diagonal block b is J (L'_cc)^-1 J with c = nblocks - 1 - b
    # and its inverse is J L'_cc J: the flipped diagonal blocks of the factor (src/liqk_v2.py:1086-1088 inverts
    # them numerically)
    U_blks_inv = torch.stack([L_flip[c * QK_K:(c + 1) * QK_K, c * QK_K:(c + 1) * QK_K]
                              for c in range(nblocks - 1, -1, -1)]).flip(1, 2).contiguous()
    del L_flip
    return U, diag_w, U_blks_inv


@torch.no_grad()
def row_scale(W_rot: torch.Tensor, cfg: dict) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(d_row [M] fp32 holding fp16 values, e [M, K/256] int8, d [M, K/256] = max(d_row 2^(e_step e), 1e-8))."""
    _lib.require_device(W_rot)
    W = W_rot.float()
    if W.stride(1) != 1 or W.stride(0) % 4 or W.data_ptr() % 16:
        W = W.contiguous()
    M, K = W.shape
    nblk = K // QK_K
    d_row = torch.empty(M, dtype=torch.float32, device=W.device)
    e = torch.empty((M, nblk), dtype=torch.int8, device=W.device)
    d = torch.empty((M, nblk), dtype=torch.float32, device=W.device)
    _check(_lib.lib().ltq_row_scale(W.data_ptr(), M, K, W.stride(0), float(cfg.get("scale", 1.0)),
                                    float(cfg.get("e_step", 0.25)), int(cfg.get("e_bits", 5)), d_row.data_ptr(),
                                    e.data_ptr(), nblk, d.data_ptr(), nblk, _lib.stream_ptr()), "ltq_row_scale")
    return d_row, e, d


@torch.no_grad()
def _quantize_rows_tcq_ldlq(W_rot: torch.Tensor, U: torch.Tensor, U_blks_inv: torch.Tensor, diag_w: torch.Tensor,
                            spec_name: str) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block16-LDLQ with every 16-column sub-block quantized in 16 x 16 tiles by the TCQ Viterbi. Returns
    (d_full [M, K/256] fp16, W_hat_rot [M, K])."""
    cfg = TCQ_CONFIG[spec_name]
    if not cfg.get("row_scale") or "K_hi" in cfg or (cfg.get("carry") and not cfg.get("tb")):
        raise NotImplementedError(f"{spec_name}: the GPU path serves the tail-biting row-scale formats")
    device = W_rot.device
    lut = torch.tensor(cfg["lut"], dtype=torch.float32, device=device)
    gains = make_gains(cfg["h"], cfg["step"], device)
    M, K = W_rot.shape
    assert M % 16 == 0, "TCQ: number of rows must be divisible by 16"
    nt = M // 16
    nblocks = K // QK_K
    n_cand = int(os.environ.get("TCQ_NCAND", cfg.get("n_cand", 0)))
    tb_window = int(os.environ.get("TCQ_TB_WIN", "32"))
    sub = cfg.get("sub", SUBBLOCK_SIZE)
    W_work = W_rot.float().clone()
    W_hat_rot = torch.empty_like(W_work)
    d_full = torch.empty((M, nblocks), dtype=torch.float16, device=device)
    pk = None
    if PACK is not None:
        assert cfg.get("tb") and cfg.get("row_scale"), f"{spec_name}: only formats with tail-biting and d_row are written to .ltq"
        pk = {"idx": torch.empty((M, K), dtype=torch.int16, device=device),
              "gi": torch.empty((M, K), dtype=torch.uint8, device=device),
              "G": torch.empty((M, K), dtype=torch.float32, device=device)}
    if U.stride(1) != 1:
        U = U.contiguous()
    if U_blks_inv.stride(2) != 1:
        U_blks_inv = U_blks_inv.contiguous()
    d_row, e_rb, d_rb_all = row_scale(W_rot, cfg)
    lib = _lib.lib()
    stream = _lib.stream_ptr()
    x_cur = torch.empty((nt, QK_K), dtype=torch.float32, device=device)
    x_nxt = torch.empty_like(x_cur)
    G_buf = torch.empty((M, QK_K), dtype=torch.float32, device=device) if pk is None else None
    for ibl in range(nblocks):
        c0, c1 = ibl * QK_K, (ibl + 1) * QK_K
        w_blk_start = W_work[:, c0:c1].clone()
        w_sub_work = w_blk_start.clone()
        U_blk = U[c0:c1, c0:c1]
        U_blk_inv = U_blks_inv[ibl]
        diag_w_blk = diag_w[c0:c1]
        d_rb = d_rb_all[:, ibl]
        # per-position weights of every sub-block's tiles (t = 16 r + c -> diag_w[s0 + c]), once per block
        wts_blk = diag_w_blk.view(NUM_SUBBLOCKS, 1, 1, SUBBLOCK_SIZE).expand(NUM_SUBBLOCKS, nt, 16, SUBBLOCK_SIZE)
        wts_blk = wts_blk.reshape(NUM_SUBBLOCKS, nt, 16 * SUBBLOCK_SIZE)
        G_pass = G_buf if pk is None else pk["G"][:, c0:c1]
        codes = (pk["idx"][:, c0:], pk["idx"].stride(0), pk["gi"][:, c0:], pk["gi"].stride(0)) if pk else None
        _check(lib.ltq_ldlq_prep(w_sub_work.data_ptr(), QK_K, d_rb.data_ptr(), nblocks, x_cur.data_ptr(), M, stream),
               "ltq_ldlq_prep")
        for ib in range(NUM_SUBBLOCKS):
            s0, s1 = ib * SUBBLOCK_SIZE, (ib + 1) * SUBBLOCK_SIZE
            out = viterbi_ub_cuda(x_cur, lut, cfg["K"], cfg["nu"], cfg["m"], gains, sub=sub, wts=wts_blk[ib],
                                  n_cand=n_cand, tail_biting=True, tb_window=tb_window,
                                  m_extra=cfg.get("m_extra", ()), pair_parity=cfg.get("pp", False),
                                  return_code=pk is not None, _raw_code=True)
            rec, code = out if pk is not None else (out, None)
            # G, the error feedback, the next sub-block's tiles and (PACK) the code / gain index scatter
            _check(lib.ltq_ldlq_sub(w_sub_work.data_ptr(), QK_K, rec.data_ptr(), d_rb.data_ptr(), nblocks,
                                    U_blk_inv.data_ptr(), U_blk_inv.stride(0), U_blk.data_ptr(), U_blk.stride(0), ib,
                                    G_pass.data_ptr(), G_pass.stride(0), x_nxt.data_ptr() if s1 < QK_K else None, M,
                                    code.data_ptr() if code is not None else None,
                                    codes[0].data_ptr() if codes else None, codes[1] if codes else 0,
                                    codes[2].data_ptr() if codes else None, codes[3] if codes else 0, stream),
                   "ltq_ldlq_sub")
            x_cur, x_nxt = x_nxt, x_cur
        best_what_row = d_rb.unsqueeze(1) * G_pass
        W_hat_rot[:, c0:c1] = best_what_row
        d_full[:, ibl] = d_rb.to(torch.float16)
        if c1 < K:
            err_blk = (w_blk_start - best_what_row) @ U_blk_inv
            W_work[:, c1:].addmm_(err_blk, U[c0:c1, c1:], alpha=-1.0)
    if pk is not None:
        PACK["groups"].append({"spec": spec_name, "d_row": d_row, "e": e_rb, "idx": pk["idx"], "gi": pk["gi"],
                               "G": pk["G"]})
    return d_full, W_hat_rot


def _fwht_rows(X: torch.Tensor) -> torch.Tensor:
    """Block normalized FWHT-256 along the first dimension."""
    return rotation.fwht_cols(X.float())


@torch.no_grad()
def quantize_matrix_liqk_v2(W: torch.Tensor, H: torch.Tensor, spec_or_row_specs, seed: int = 1337, damp: float = 0.02,
                            row_weights: Optional[torch.Tensor] = None, cd_sweeps: int = 2,
                            out_rot: bool = False) -> Tuple[Dict[str, torch.Tensor], torch.Tensor, float]:
    """W [M, K] with input Hessian H [K, K] -> (qdata {d, suh, row_slices}, W_hat_eff, relative proxy loss),
    for TCQ specs (one for the whole matrix or [(r0, r1, spec), ...] row slices)."""
    if out_rot:
        s_out = rotation.make_rademacher_signs(W.shape[0], seed=seed + 7919, device=W.device)
        rw = None
        if row_weights is not None:
            rw = row_weights.float().view(-1, QK_K).mean(dim=1, keepdim=True).expand(-1, QK_K).reshape(-1)
        q_res, w_hat_r, rel = quantize_matrix_liqk_v2(_fwht_rows(W.float() * s_out.unsqueeze(1)), H, spec_or_row_specs,
                                                      seed=seed, damp=damp, row_weights=rw, cd_sweeps=cd_sweeps)
        q_res["s_out"] = s_out.to(torch.int8)
        return q_res, _fwht_rows(w_hat_r) * s_out.unsqueeze(1), rel

    W_f32 = W.float()
    H_f32 = H.float()
    M, K = W_f32.shape
    nblocks = K // QK_K
    specs_used = [spec_or_row_specs] if isinstance(spec_or_row_specs, str) else [sp for _, _, sp in spec_or_row_specs]
    for sp in specs_used:
        if sp not in TCQ_CONFIG:
            raise NotImplementedError(f"{sp}: only TCQ formats are quantized on the GPU path")
    damp *= float(os.environ.get("TCQ_DAMP_MULT", "10"))

    _mark("start")
    W_rot, H_rot, suh = rotation.compute_optimal_suh(W_f32, H_f32, seed=seed, row_weights=row_weights)
    _mark("rotation")
    U, diag_w, U_blks_inv = factor_hessian(H_rot, damp)
    del H_rot
    _mark("factor")

    row_slices = [(0, M, spec_or_row_specs)] if isinstance(spec_or_row_specs, str) else spec_or_row_specs
    by_spec: Dict[str, List[Tuple[int, int]]] = {}
    for r0, r1, sp in row_slices:
        by_spec.setdefault(sp, []).append((r0, r1))

    W_hat_rot = torch.empty_like(W_rot)
    d_full = torch.empty((M, nblocks), dtype=torch.float16, device=W.device)
    if PACK is not None:
        PACK["groups"] = []
        pm = {"idx": torch.empty((M, K), dtype=torch.int16, device=W.device),
              "gi": torch.empty((M, K), dtype=torch.uint8, device=W.device),
              "G": torch.empty((M, K), dtype=torch.float32, device=W.device),
              "d_row": torch.empty(M, device=W.device),
              "e": torch.empty((M, nblocks), dtype=torch.int8, device=W.device)}
    for sp, ranges in by_spec.items():
        rows_idx = torch.cat([torch.arange(r0, r1, device=W.device) for r0, r1 in ranges], dim=0)
        d_sub, Wh_sub = _quantize_rows_tcq_ldlq(W_rot[rows_idx], U, U_blks_inv, diag_w, sp)
        W_hat_rot[rows_idx] = Wh_sub
        d_full[rows_idx] = d_sub
        if PACK is not None:
            g = PACK["groups"].pop()
            for k in ("idx", "gi", "G", "d_row", "e"):
                pm[k][rows_idx] = g[k].to(pm[k].dtype)
    _mark("rows")

    # ---- c_row / suh refit (src/liqk_v2.py:1139-1180) ----------------------------------------------------
    U_base = rotation.fwht_inplace(W_hat_rot.clone(), block_size=QK_K)
    W_hat_eff = U_base * suh.unsqueeze(0)
    c_pack = torch.ones((M,), dtype=torch.float32, device=W.device)
    HW = W_f32 @ H_f32
    HQ = W_hat_eff @ H_f32
    c_row = (W_hat_eff * HW).sum(dim=1) / (W_hat_eff * HQ).sum(dim=1).clamp(min=1e-12)
    c_row = torch.where(torch.isfinite(c_row) & (c_row > 0.5) & (c_row < 2.0), c_row, torch.ones_like(c_row))
    d_new = (d_full.float() * c_row.unsqueeze(1)).to(torch.float16)
    c_eff = (d_new.float() / d_full.float().clamp(min=1e-12)).mean(dim=1, keepdim=True)
    U_scaled = U_base * c_eff
    if row_weights is not None:
        rw = row_weights.float().clamp(min=float(row_weights.mean().item()) * 0.1)
        rw = (rw / rw.mean().clamp(min=1e-12)).clamp(0.25, 4.0)
        U_w = U_scaled * rw.unsqueeze(1)
    else:
        rw = torch.ones((M,), dtype=torch.float32, device=W.device)
        U_w = U_scaled
    # A_in = (U_w^T U_scaled) * H is symmetric (U_w = diag(rw) U_scaled): only its lower triangle is formed, which
    # is all the Cholesky of spd_solve reads
    A_in = linalg.gram_lower(U_w, U_scaled).mul_(H_f32)
    b_in = (U_w * HW).sum(dim=0)
    A_in.diagonal().add_(1e-3 * A_in.diagonal().mean().clamp(min=1e-12))
    try:
        suh_cand = linalg.spd_solve(A_in, b_in).to(torch.float16).to(torch.float32)
        valid_s = torch.isfinite(suh_cand) & (suh_cand.abs() > 0.05) & (suh_cand.abs() < 10.0)
        suh_cand = torch.where(valid_s, suh_cand, suh)
        W_hat_cand = U_scaled * suh_cand.unsqueeze(0)
        HQ_cand = W_hat_cand @ H_f32
        diff_base = W_f32 - W_hat_eff
        diff_cand = W_f32 - W_hat_cand
        loss_base = float((((HW - HQ) * diff_base).sum(dim=1) * rw).sum().item())
        loss_cand = float((((HW - HQ_cand) * diff_cand).sum(dim=1) * rw).sum().item())
        if loss_cand < loss_base:
            W_hat_eff = W_hat_cand
            d_full = d_new
            suh = suh_cand
            HQ = HQ_cand
            c_pack = c_eff.squeeze(1)
    except RuntimeError:
        pass
    del A_in

    if PACK is not None:  # the matrix exactly from the file fields
        d_row_p = (pm["d_row"] * c_pack).to(torch.float16)
        suh_p = suh.to(torch.float16)
        scale = d_row_p.float().unsqueeze(1) * torch.exp2(0.25 * pm["e"].float())
        Wq_rot = (scale.unsqueeze(2) * pm["G"].view(M, nblocks, QK_K)).view(M, K)
        W_hat_eff = rotation.fwht_inplace(Wq_rot, block_size=QK_K) * suh_p.float().unsqueeze(0)
        # the rebuilt matrix is the refit's W_hat_eff with row r scaled by rho_r = d_row_p / (d_row c_pack) (same
        # tile values, same fp16 suh), so its product with H is HQ scaled by row, equal to the reference's
        # W_hat_eff @ H up to fp32 rounding; rows whose block scale hit the 1e-8 clamp of the row-scale fit (where
        # the identity does not hold) are multiplied out
        rho = d_row_p.float() / (pm["d_row"] * c_pack)
        HQ = HQ * rho.unsqueeze(1)
        clamped = ((pm["d_row"].unsqueeze(1) * torch.exp2(0.25 * pm["e"].float())) < 1e-8).any(dim=1)
        if bool(clamped.any()):
            HQ[clamped] = W_hat_eff[clamped] @ H_f32
        PACK["matrix"] = {"row_slices": row_slices, "idx": pm["idx"], "gi": pm["gi"], "G": pm["G"], "d_row": d_row_p,
                          "e": pm["e"], "suh": suh_p}

    diff = W_f32 - W_hat_eff
    num_loss = float(((HW - HQ) * diff).sum().item())
    den_loss = float((HW * W_f32).sum().clamp(min=1e-12).item())
    rel_loss = num_loss / den_loss
    qdata_out = {"d": d_full, "suh": suh.to(torch.float16), "row_slices": row_slices}
    _mark("refit")
    return qdata_out, W_hat_eff, rel_loss
