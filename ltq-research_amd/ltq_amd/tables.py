"""Trellis tables for TCQ formats with extended labels, trained by Lloyd iterations on the GPU Viterbi.

Same function, arguments and results as src/universal_bench.py:85-116 (`train_tcq_x`): a table of nl = 4 <<
len(m_extra) subsets of U = 2^(K-1) levels in the kernel's subset-major layout (entry lb * U + u), the gain table
make_gains(h, step) (or [1] for h = 0) and n_cand = 4 when there are more than 4 gains.

Training, as a small state machine (TableTrainer):
  start   levels = the N(0, spread^2) quantiles at the nl * U midpoints (k + 1/2) / (nl U), dealt round-robin to
          the subsets: subset lb gets quantiles lb, lb + nl, lb + 2 nl, ... (so every subset spans the range);
  sample  n_tiles tiles of N(0, 1) from a device generator seeded with seed + 1, each scaled to unit rms;
  step    the tail-biting Viterbi codes the tiles with the current table; each level moves to the gain-weighted
          centroid sum(g x) / sum(g^2) of the values coded with it (unused levels stay), then either every
          subset is sorted or, with `additive`, the table is fitted as base[u] + off[lb] by 20 sweeps of
          alternating weighted least squares (weights: the centroid denominators + 1e-6).
"""
from __future__ import annotations

from typing import Tuple

import torch

from .tcq_proto import make_gains, viterbi_ub_cuda

NU, MASK, SUB, T = 10, 359, 16, 256


def _shape(K: int, m_extra: tuple) -> Tuple[int, int]:
    return 4 << len(m_extra), 1 << (K - 1)


def closed_form_table(K: int, m_extra: tuple, spread: float = 1.0, device="cuda") -> torch.Tensor:
    """The start of training (src/universal_bench.py:91-94): [nl * U] float32, entry lb * U + u = the
    (u * nl + lb)-th of the nl * U midpoint quantiles of N(0, spread^2), computed in float64."""
    nl, U = _shape(K, m_extra)
    n = nl * U
    mid = (torch.arange(n, dtype=torch.float64) + 0.5) / n
    grid = (spread * torch.special.ndtri(mid)).to(torch.float32)
    lb, u = torch.meshgrid(torch.arange(nl), torch.arange(U), indexing="ij")
    return grid[(u * nl + lb).flatten()].to(device)


def _centroids(tab: torch.Tensor, level: torch.Tensor, g: torch.Tensor, x: torch.Tensor):
    """(new levels, denominators): per level j, sum(g x) / sum(g^2) over the positions coded with it; levels no
    position uses keep their value."""
    n = tab.numel()
    num = torch.zeros(n, dtype=tab.dtype, device=tab.device).index_add_(0, level, g * x)
    den = torch.zeros(n, dtype=tab.dtype, device=tab.device).index_add_(0, level, g * g)
    used = den > 0
    return torch.where(used, num / den.clamp(min=1e-12), tab), den


def _additive_fit(c: torch.Tensor, wgt: torch.Tensor, sweeps: int = 20) -> torch.Tensor:
    """Weighted least squares c[lb, u] ~ base[u] + off[lb] by alternating exact minimizations, off starting at
    0; returns base[None, :] + off[:, None]."""
    off = torch.zeros(c.shape[0], dtype=c.dtype, device=c.device)
    w_u, w_lb = wgt.sum(dim=0), wgt.sum(dim=1)
    for _ in range(sweeps):
        base = ((c - off.unsqueeze(1)) * wgt).sum(dim=0) / w_u
        off = ((c - base.unsqueeze(0)) * wgt).sum(dim=1) / w_lb
    return base.unsqueeze(0) + off.unsqueeze(1)


@torch.no_grad()
def lloyd_step(x: torch.Tensor, tab: torch.Tensor, gains: torch.Tensor, K: int, m_extra: tuple, n_cand: int,
               sub: int = SUB, pp=False, additive: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """One Lloyd iteration on unit-rms tiles x [n, T]: (the next table, the codes (gain index << 16 | level
    index) the current table gave the tiles)."""
    nl, U = _shape(K, m_extra)
    _, gi, lev = viterbi_ub_cuda(x, tab, K, NU, MASK, gains, sub=sub, n_cand=n_cand, return_code=True,
                                 tail_biting=True, m_extra=m_extra, pair_parity=pp)
    level = lev.reshape(-1).long()
    moved, den = _centroids(tab, level, gains[gi.reshape(-1).long()], x.reshape(-1))
    if additive:
        nxt = _additive_fit(moved.view(nl, U), den.view(nl, U) + 1e-6).reshape(-1)
    else:
        nxt = torch.sort(moved.view(nl, U), dim=1).values.reshape(-1)
    return nxt, (gi.to(torch.int32) << 16) | lev.to(torch.int32)


class TableTrainer:
    """The training loop's state: table, gains, candidate count and the tile generator."""

    def __init__(self, K: int, h: int, step: float, m_extra: tuple, seed: int = 0, spread: float = 1.0,
                 sub: int = SUB, pp: bool = False, device="cuda"):
        self.K, self.m_extra, self.sub, self.pp = K, tuple(m_extra), sub, pp
        self.device = torch.device(device)
        self.tab = closed_form_table(K, self.m_extra, spread, self.device)
        self.gains = make_gains(h, step, self.device) if h > 0 else torch.ones(1, device=self.device)
        self.n_cand = 4 if self.gains.numel() > 4 else 0
        self.gen = torch.Generator(device=self.device).manual_seed(seed + 1)

    def sample(self, n_tiles: int) -> torch.Tensor:
        x = torch.randn((n_tiles, T), generator=self.gen, device=self.device)
        return x / x.square().mean(dim=1, keepdim=True).sqrt()

    def step(self, n_tiles: int, additive: bool = False) -> torch.Tensor:
        self.tab, codes = lloyd_step(self.sample(n_tiles), self.tab, self.gains, self.K, self.m_extra, self.n_cand,
                                     sub=self.sub, pp=self.pp, additive=additive)
        return codes


@torch.no_grad()
def train_tcq_x(K: int, h: int, step: float, m_extra: tuple, iters: int = 16, n_tiles: int = 4096, seed: int = 0,
                spread: float = 1.0, additive: bool = False, sub: int = SUB, pp: bool = False):
    """(table [nl * U], gains [2^h], n_cand) after `iters` Lloyd iterations on fresh tiles each."""
    tr = TableTrainer(K, h, step, m_extra, seed=seed, spread=spread, sub=sub, pp=pp)
    for _ in range(iters):
        tr.step(n_tiles, additive=additive)
    return tr.tab, tr.gains, tr.n_cand
