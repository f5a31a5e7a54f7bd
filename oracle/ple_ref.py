"""TEST INFRASTRUCTURE ONLY -- CPU restatement of the ring quantizer of row tables (the checker for
ltq_amd.ple_quant). Only tests/ import it.

Reference anchor: src/ple_quant.py:28-67 (`hadamard_signs`, `quantize_rings`), torch on the CPU in the
reference's order of operations, oracle/ref.fwht256_ref for the rotation and the C oracle's two-pass tail-biting
Viterbi (tb_window 0) for `viterbi_ub_cuda`.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ref

RING = 256


def hadamard_signs_ref(seed: int = 4242) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(0, 2, (RING,), generator=g) * 2 - 1).float()


def quantize_rings_ref(W: torch.Tensor, cfg: dict, fmt, rot: bool, scales=(0.9, 1.0, 1.12)):
    """(table [rows, n*256] in W's dtype, chosen fp16 scale per ring, codes int32 [n_rings, 256] (gi << 16 | idx)
    of the chosen scale, unscaled values [n_rings, 256] of the chosen scale)."""
    signs = hadamard_signs_ref()
    x = W.reshape(-1, RING).float()
    if rot:
        x = torch.from_numpy(ref.fwht256_ref((x * signs).numpy()))
    rms = x.square().mean(dim=1, keepdim=True).sqrt().clamp(min=1e-8) * cfg.get("scale", 1.0)
    best = best_err = best_code = best_d = best_u = None
    for sc in scales:
        d = (rms * sc).half().float()
        xs = (x / d).numpy()
        rec, gi, ix = ref.viterbi_ub_cuda_ref(xs, np.asarray(fmt.lut, np.float32), fmt.K, 10, fmt.masks[0],
                                              np.asarray(fmt.gain_tab, np.float32), sub=fmt.sub, tail_biting=True,
                                              tb_window=0, m_extra=tuple(fmt.masks[1:]), pair_parity=int(fmt.frac),
                                              n_cand=cfg.get("n_cand", 0), return_code=True)
        u = torch.from_numpy(np.asarray(rec, np.float32)).reshape(x.shape)
        code = torch.from_numpy((np.asarray(gi, np.int64) << 16 | np.asarray(ix, np.int64)).astype(np.int32)).reshape(x.shape)
        r = u * d
        err = (r - x).square().sum(dim=1)
        if best is None:
            best, best_err, best_code, best_d, best_u = r, err, code, d, u
        else:
            better = err < best_err
            best = torch.where(better.unsqueeze(1), r, best)
            best_err = torch.where(better, err, best_err)
            best_code = torch.where(better.unsqueeze(1), code, best_code)
            best_d = torch.where(better.unsqueeze(1), d, best_d)
            best_u = torch.where(better.unsqueeze(1), u, best_u)
    if rot:
        best = torch.from_numpy(ref.fwht256_ref(best.contiguous().numpy())) * signs
    return best.to(W.dtype).view_as(W), best_d.squeeze(1).half(), best_code, best_u
