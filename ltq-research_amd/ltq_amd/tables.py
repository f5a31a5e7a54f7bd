"""Trellis tables for TCQ formats with extended labels: the closed-form start and the Lloyd training loop, on
the GPU Viterbi.

Mirrors src/universal_bench.py:85-116 (`train_tcq_x`, same arguments and results): nl = 4 << len(m_extra)
subsets of U = 2^(K-1) levels, table [nl * U] in kernel layout (subset-major). The start is the N(0, spread^2)
quantile grid at nl * U points, subset j taking points j, j + nl, ... Each iteration quantizes n_tiles
rms-normalized N(0, 1) tiles with the tail-biting Viterbi (codes returned), moves every level to the
gain-weighted centroid of the values coded with it (sum g x / sum g^2, levels never used keep their value), and
sorts each subset (or, with `additive`, fits tab[lb, u] = base[u] + off[lb] by weighted least squares).
The centroid sums run as torch index_add on the device.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .tcq_proto import make_gains, viterbi_ub_cuda

NU, MASK, SUB, T = 10, 359, 16, 256


def closed_form_table(K: int, m_extra: tuple, spread: float = 1.0, device="cuda") -> torch.Tensor:
    """The training start (src/universal_bench.py:91-94): quantiles of N(0, spread^2) at nl * U points."""
    nl, U = 4 << len(m_extra), 1 << (K - 1)
    n = nl * U
    q = (spread * torch.special.ndtri((torch.arange(n, dtype=torch.float64) + 0.5) / n)).float().to(device)
    return q.view(U, nl).T.contiguous().flatten()


@torch.no_grad()
def lloyd_step(x: torch.Tensor, tab: torch.Tensor, gains: torch.Tensor, K: int, m_extra: tuple, n_cand: int,
               sub: int = SUB, pp=False, additive: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """One training iteration on tiles x [n, T] (already rms-normalized): (new table, codes (gain index << 16 |
    level index) of the tiles under the old table)."""
    nl, U = 4 << len(m_extra), 1 << (K - 1)
    _, gi, lev = viterbi_ub_cuda(x, tab, K, NU, MASK, gains, sub=sub, n_cand=n_cand, return_code=True,
                                 tail_biting=True, m_extra=m_extra, pair_parity=pp)
    j, gv, xf = lev.flatten().long(), gains[gi.flatten().long()], x.flatten()
    num = torch.zeros_like(tab).index_add_(0, j, gv * xf)
    den = torch.zeros_like(tab).index_add_(0, j, gv * gv)
    new = torch.where(den > 0, num / den.clamp(min=1e-12), tab)
    if additive:
        c, wgt = new.view(nl, U), den.view(nl, U) + 1e-6
        off = torch.zeros(nl, device=new.device)
        for _ in range(20):
            base = ((c - off[:, None]) * wgt).sum(0) / wgt.sum(0)
            off = ((c - base[None, :]) * wgt).sum(1) / wgt.sum(1)
        new = (base[None, :] + off[:, None]).flatten()
    else:
        new = new.view(nl, U).sort(dim=1).values.flatten()
    return new, (gi.to(torch.int32) << 16) | lev.to(torch.int32)


@torch.no_grad()
def train_tcq_x(K: int, h: int, step: float, m_extra: tuple, iters: int = 16, n_tiles: int = 4096, seed: int = 0,
                spread: float = 1.0, additive: bool = False, sub: int = SUB, pp: bool = False):
    """(table [nl * U], gains [2^h], n_cand): n_cand = 4 when there are more than 4 gains (the candidate search
    of the quantizer), else 0."""
    dev = torch.device("cuda")
    tab = closed_form_table(K, m_extra, spread, dev)
    gains = make_gains(h, step, dev) if h > 0 else torch.ones(1, device=dev)
    g = torch.Generator(device=dev).manual_seed(seed + 1)
    n_cand = 4 if gains.numel() > 4 else 0
    for _ in range(iters):
        x = torch.randn((n_tiles, T), generator=g, device=dev)
        x = x / x.square().mean(dim=1, keepdim=True).sqrt()
        tab, _ = lloyd_step(x, tab, gains, K, m_extra, n_cand, sub=sub, pp=pp, additive=additive)
    return tab, gains, n_cand
