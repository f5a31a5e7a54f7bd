"""MoE expert batches: every expert of a layer quantized as quantize_matrix_liqk_v2 would quantize it alone, with
the Viterbi work of all experts in shared launches.

The reference quantizes the experts one by one (src/streaming_quant.py:262-276: gate_up_proj [2 I, H] with the
expert's input Hessian, down_proj [H, I] with the Hessian of its intermediate activations, each a full
quantize_matrix_liqk_v2 call with seed _seed(layer, name), src/streaming_quant.py:116-117, 130-133). Here the
per-expert stages that are matrix-sized linear algebra (rotation, refit, PACK fields) run per expert through
the same code as a single matrix, with the Cholesky factorizations of all experts (the Hessians' and the refits'
SPD systems) each in one batched call, which factors every matrix to the bits it gets alone
(liqk.factor_hessians, liqk.refit_jobs, linalg.cholesky_many). The row quantizer's LDLQ loop runs once for all
same-shaped experts stacked along rows: one two-pass Viterbi launch per 16-column sub-block covers the tiles of
every expert, and the LDLQ kernels read each tile's own expert factors (ltq_ldlq_* with matrix strides). Rows
are independent in that loop, so every expert's codes, scales and reconstruction equal those of its own call.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from . import liqk
from .formats import TCQ_CONFIG


def expert_seed(layer: int, name: str) -> int:
    """The reference's per-matrix rotation seed (src/streaming_quant.py:116-117)."""
    return 1000 + layer * 1009 + (sum(map(ord, name)) * 31) % 997


@torch.no_grad()
def quantize_experts(Ws: Sequence[torch.Tensor], Hs: Sequence[torch.Tensor], spec: str, seeds: Sequence[int],
                     damp: float = 0.02) -> Tuple[List[Tuple[dict, torch.Tensor, float]], Optional[List[dict]]]:
    """Experts W_e [R, K] (all the same shape) with Hessians H_e [K, K] in one format. Returns ([(qdata, W_hat,
    relative proxy loss)] per expert, as quantize_matrix_liqk_v2 returns them, and, when liqk.PACK is set, each
    expert's PACK["matrix"] fields (else None)."""
    if spec not in TCQ_CONFIG:
        raise NotImplementedError(f"{spec}: only TCQ formats are quantized on the GPU path")
    n = len(Ws)
    if n == 0:
        return [], None
    R, K = Ws[0].shape
    if any(W.shape != (R, K) for W in Ws) or any(H.shape != (K, K) for H in Hs) or len(Hs) != n or len(seeds) != n:
        raise ValueError("quantize_experts: experts must share one shape [R, K] with Hessians [K, K]")
    if R % 128 and n > 1:
        raise ValueError("quantize_experts: rows per expert must be a multiple of 128 to share launches")
    packing = liqk.PACK is not None
    liqk._mark("start")
    jobs, H_rots = [], []
    for W, H, seed in zip(Ws, Hs, seeds):
        job = liqk._MatrixJob(W, H, [(0, R, spec)], seed, damp, None)
        H_rots.append(job.rotate())
        jobs.append(job)
    # the experts' factorizations in one batched call (bit-identical to factoring each alone)
    for job, (U, dw, Ubi) in zip(jobs, liqk.factor_hessians(H_rots, jobs[0].damp)):
        job.U, job.diag_w, job.U_blks_inv = U, dw, Ubi
    del H_rots
    liqk._mark("factor")
    # the rows stage of all experts at once
    W_rot = torch.cat([j.W_rot for j in jobs], dim=0)
    U = torch.stack([j.U for j in jobs])
    U_bi = torch.stack([j.U_blks_inv for j in jobs])
    dw = torch.stack([j.diag_w for j in jobs])
    for j in jobs:
        del j.U, j.U_blks_inv
    if packing:
        liqk.PACK["groups"] = []
    d_all, W_hat_all = liqk._ldlq_rows(W_rot, U, U_bi, dw, spec)
    del U, U_bi, W_rot
    grp = liqk.PACK["groups"].pop() if packing else None
    liqk._mark("rows")
    out, fields = [], ([] if packing else None)
    for e, job in enumerate(jobs):
        rows = slice(e * R, (e + 1) * R)
        job.W_hat_rot = W_hat_all[rows]
        job.d = d_all[rows]
        job.fields = None
        if packing:
            job.fields = {"idx": grp["idx"][rows], "gi": grp["gi"][rows], "G": grp["G"][rows],
                          "d_row": grp["d_row"][rows], "e": grp["e"][rows]}
    liqk.refit_jobs(jobs)  # the refits' SPD systems factored in one batched call
    for e, job in enumerate(jobs):
        if packing:
            job.write_fields()
            fields.append(liqk.PACK.pop("matrix"))
        out.append(({"d": job.d, "suh": job.suh.to(torch.float16), "row_slices": job.row_slices}, job.W_hat,
                    job.relative_loss()))
    liqk._mark("refit")
    return out, fields
