"""TEST INFRASTRUCTURE ONLY -- CPU restatement of the TCQ matrix quantizer around the Viterbi (the checker
for ltq_amd.liqk). Only tests/ import it.

Reference anchors (torch on the CPU, float32, the reference's order of operations):
  row_scale_ref          src/liqk_v2.py:938-946
  factor_hessian_ref     src/liqk_v2.py:1066-1088
  quantize_rows_ref      src/liqk_v2.py:877-1021, row-scale branch with tail-biting formats (quant_sub at
                         :913-921 via the C oracle's two-pass tail-biting driver)
"""
from __future__ import annotations

import numpy as np
import torch

from . import ref

QK_K = 256
SUB = 16


def row_scale_ref(W_rot: torch.Tensor, cfg: dict):
    M, K = W_rot.shape
    nblocks = K // QK_K
    rms_rb = W_rot.float().view(M, nblocks, QK_K).square().mean(dim=2).sqrt().clamp(min=1e-10) * cfg.get("scale", 1.0)
    d_row = torch.exp(torch.log(rms_rb).mean(dim=1)).to(torch.float16).to(torch.float32).clamp(min=1e-8)
    e_step, e_max = cfg.get("e_step", 0.25), 1 << (cfg.get("e_bits", 5) - 1)
    e_rb = torch.round(torch.log2(rms_rb / d_row.unsqueeze(1)) / e_step).clamp(-e_max, e_max - 1)
    d_rb_all = d_row.unsqueeze(1) * torch.exp2(e_step * e_rb)
    return rms_rb, d_row, e_rb, d_rb_all


def factor_hessian_ref(H_rot: torch.Tensor, damp: float):
    K = H_rot.shape[0]
    nblocks = K // QK_K
    H_reg = H_rot.double().clone()
    H_reg.diagonal().add_(damp * H_reg.diagonal().mean().clamp(min=1e-8))
    L_flip = torch.linalg.cholesky(H_reg.flip(0, 1))
    U = torch.linalg.solve_triangular(L_flip, torch.eye(K, dtype=L_flip.dtype), upper=False).flip(0, 1)
    diag_w = 1.0 / (torch.diagonal(U) ** 2).clamp(min=1e-12)
    U_blks = torch.stack([U[b * QK_K:(b + 1) * QK_K, b * QK_K:(b + 1) * QK_K] for b in range(nblocks)])
    U_blks_inv = torch.linalg.solve_triangular(U_blks, torch.eye(QK_K, dtype=U.dtype).expand(nblocks, -1, -1), upper=True)
    return U.float(), diag_w.float(), U_blks_inv.float()


def quantize_rows_ref(W_rot: torch.Tensor, U: torch.Tensor, U_blks_inv: torch.Tensor, diag_w: torch.Tensor, cfg: dict,
                      gains: np.ndarray, tb_window: int = 32, n_cand: int | None = None, d_rb_all=None):
    """(d_full fp16 [M, nblk], W_hat_rot [M, K], codes {idx int16 [M, K], gi uint8 [M, K]}, first-sub-block
    Viterbi inputs [nt, 256]). d_rb_all may be given (the device's row scale) to compare the LDLQ loop alone."""
    M, K = W_rot.shape
    nt, nblocks = M // 16, K // QK_K
    n_cand = cfg.get("n_cand", 0) if n_cand is None else n_cand
    lut = np.asarray(cfg["lut"], np.float32)
    m_extra = tuple(cfg.get("m_extra", ()))
    W_work = W_rot.float().clone()
    W_hat_rot = torch.empty_like(W_work)
    d_full = torch.empty((M, nblocks), dtype=torch.float16)
    idx = torch.empty((M, K), dtype=torch.int16)
    gim = torch.empty((M, K), dtype=torch.uint8)
    if d_rb_all is None:
        _, _, _, d_rb_all = row_scale_ref(W_rot, cfg)
    first_x = None
    for ibl in range(nblocks):
        c0, c1 = ibl * QK_K, (ibl + 1) * QK_K
        w_blk_start = W_work[:, c0:c1].clone()
        U_blk = U[c0:c1, c0:c1]
        U_blk_inv = U_blks_inv[ibl]
        diag_w_blk = diag_w[c0:c1]
        d_rb = d_rb_all[:, ibl].clamp(min=1e-8)
        w_sub_work = w_blk_start.clone()
        G_pass = torch.empty((M, QK_K), dtype=torch.float32)
        inv_d = 1.0 / d_rb.unsqueeze(1)
        for ib in range(QK_K // SUB):
            s0, s1 = ib * SUB, (ib + 1) * SUB
            w_sub_orig = w_sub_work[:, s0:s1]
            xs = (w_sub_orig * inv_d).contiguous().view(nt, 256).numpy()
            if first_x is None:
                first_x = xs.copy()
            wts = np.tile(diag_w_blk[s0:s1].numpy(), 16)
            rec, gi, ix = ref.viterbi_ub_cuda_ref(xs, lut, cfg["K"], 10, cfg["m"], gains, sub=cfg.get("sub", 16),
                                                  wts=wts, n_cand=n_cand, tail_biting=True, tb_window=tb_window,
                                                  m_extra=m_extra, pair_parity=int(cfg.get("pp", 0)),
                                                  return_code=True)
            g_sub = torch.tensor(rec).view(M, SUB)
            idx[:, c0 + s0:c0 + s1] = torch.tensor(ix).view(M, SUB).to(torch.int16)
            gim[:, c0 + s0:c0 + s1] = torch.tensor(gi).view(M, SUB).to(torch.uint8)
            G_pass[:, s0:s1] = g_sub
            if s1 < QK_K:
                err_sub = (w_sub_orig - d_rb.unsqueeze(1) * g_sub) @ U_blk_inv[s0:s1, s0:s1]
                w_sub_work[:, s1:] -= err_sub @ U_blk[s0:s1, s1:]
        best_what_row = d_rb.unsqueeze(1) * G_pass
        W_hat_rot[:, c0:c1] = best_what_row
        d_full[:, ibl] = d_rb.to(torch.float16)
        if c1 < K:
            err_blk = (w_blk_start - best_what_row) @ U_blk_inv
            W_work[:, c1:] -= err_blk @ U[c0:c1, c1:]
    return d_full, W_hat_rot, {"idx": idx, "gi": gim}, first_x
