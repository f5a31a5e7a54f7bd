"""The TCQ matrix quantizer on the GPU: Hessian factorization, row scale, LDLQ error feedback around the Viterbi,
PACK fields and the c_row / suh refit.

Mirrors (same names, argument meaning, results and the module-level PACK switch):
  PACK                        src/liqk_v2.py:74       (dict -> the matrix's .ltq fields are collected)
  factor_hessian              src/liqk_v2.py:1066-1088 (damping, Cholesky of the flipped H, U, diag_w, U_blks_inv)
  row_scale                   src/liqk_v2.py:938-946  (HIP kernel ltq_row_scale)
  _quantize_rows_tcq_ldlq     src/liqk_v2.py:877-1021 (the row-scale branch: every tail-biting / R format;
                                                       HIP kernels ltq_ldlq_sub per sub-block, tcq_viterbi
                                                       two-pass tail-biting, ltq_ldlq_err / ltq_ldlq_update on
                                                       the matrix cores across blocks: fixed-order sums)
  refit_scales                src/liqk_v2.py:1139-1180 (the joint c_row / suh refit, as a record)
  quantize_matrix_liqk_v2     src/liqk_v2.py:1030-1198 (single TCQ spec or TCQ row slices; refit and PACK tail)

The factorization and the refit's products and solve run on the device through ltq_amd.linalg and torch (MAGMA,
hipBLASLt / rocBLAS).
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib, linalg, rotation
from .formats import E_BITS, E_STEP, QK_K, SUBBLOCK_SIZE, TCQ_CONFIG, exp2_table
from .tcq_proto import make_gains, viterbi_ub_cuda

PACK: Optional[dict] = None
# timing hook (off by default): a list receives (stage name, torch.cuda.Event) at every stage boundary of
# quantize_matrix_liqk_v2, recorded on the stream the kernels run on
STAGE_EVENTS: Optional[list] = None
# the refit record of the last quantize_matrix_liqk_v2 call (for inspection)
LAST_REFIT = None
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
def _damped_flip(H_rot: torch.Tensor, damp: float) -> torch.Tensor:
    """The matrix factor_hessian factors: H + damp mean(diag H) I, rows and columns reversed."""
    H_reg = H_rot.float().clone()
    diag_mean = H_reg.diagonal().mean().clamp(min=1e-8)
    H_reg.diagonal().add_(damp * diag_mean)
    return H_reg.flip(0, 1).contiguous()


def _factors_from(L_flip: torch.Tensor, info: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(U, diag_w, U_blks_inv) from the Cholesky factor of the flipped, damped H."""
    if int(info.item()) != 0:
        raise torch.linalg.LinAlgError("factor_hessian: the damped Hessian is not positive definite")
    nblocks = L_flip.shape[0] // QK_K
    U = linalg.tri_inv_lower(L_flip).flip(0, 1).contiguous()  # the kernels take row-major factors
    diag_w = 1.0 / (torch.diagonal(U) ** 2).clamp(min=1e-12)
    # U = J L'^-1 J (J reverses the order), so U's diagonal block b is J (L'_cc)^-1 J with c = nblocks - 1 - b
    # and its inverse is J L'_cc J: the flipped diagonal blocks of the factor (src/liqk_v2.py:1086-1088 inverts
    # them numerically)
    U_blks_inv = torch.stack([L_flip[c * QK_K:(c + 1) * QK_K, c * QK_K:(c + 1) * QK_K]
                              for c in range(nblocks - 1, -1, -1)]).flip(1, 2).contiguous()
    return U, diag_w, U_blks_inv


def factor_hessian(H_rot: torch.Tensor, damp: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(U, diag_w, U_blks_inv): U upper Cholesky factor of H^-1 (U^T U = H^-1) from one factorization of the
    flipped, damped H and one triangular inversion; diag_w = 1 / diag(U)^2; inverses of U's 256 x 256 diagonal
    blocks."""
    return _factors_from(*linalg.cholesky_lower(_damped_flip(H_rot, damp)))


def factor_hessians(H_rots: Sequence[torch.Tensor], damp: float) -> List[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
    """factor_hessian of each matrix, bit for bit; the factorizations of same-sized matrices of up to
    linalg.LEAF rows go through one batched call (linalg.cholesky_many)."""
    out: List = [None] * len(H_rots)
    by_size: Dict[int, List[int]] = {}
    for i, H in enumerate(H_rots):
        by_size.setdefault(H.shape[0], []).append(i)
    for K, idx in by_size.items():
        if K > linalg.LEAF or not H_rots[idx[0]].is_cuda:
            for i in idx:
                out[i] = factor_hessian(H_rots[i], damp)
            continue
        L, info = linalg.cholesky_many(torch.stack([_damped_flip(H_rots[i], damp) for i in idx]))
        for j, i in enumerate(idx):
            out[i] = _factors_from(L[j], info[j])
        del L
    return out


_EXP2_TABS: Dict[tuple, torch.Tensor] = {}


def exp2_table_device(device, e_step: float = E_STEP, e_bits: int = E_BITS) -> torch.Tensor:
    """formats.exp2_table on `device` (cached per device and exponent format)."""
    key = (str(torch.device(device)), float(e_step), int(e_bits))
    t = _EXP2_TABS.get(key)
    if t is None:
        t = _EXP2_TABS[key] = torch.from_numpy(exp2_table(e_step, e_bits)).to(device)
    return t


def block_scale(d_row: torch.Tensor, e: torch.Tensor, e_step: float = E_STEP, e_bits: int = E_BITS) -> torch.Tensor:
    """d_row[m] * 2^(e_step e[m, b]) [M, nblk] float32 through the shared exponent table (src/liqk_v2.py:946)."""
    tab = exp2_table_device(d_row.device, e_step, e_bits)
    return d_row.float().unsqueeze(1) * tab[e.long() + (1 << (e_bits - 1))]


@torch.no_grad()
def row_scale(W_rot: torch.Tensor, cfg: dict) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(d_row [M] fp32 holding fp16 values, e [M, K/256] int8, d [M, K/256] = max(d_row 2^(e_step e), 1e-8))."""
    _lib.require_device(W_rot)
    W = W_rot.float()
    if W.stride(1) != 1 or W.stride(0) % 4 or W.data_ptr() % 16:
        W = W.contiguous()
    M, K = W.shape
    nblk = K // QK_K
    e_step, e_bits = float(cfg.get("e_step", E_STEP)), int(cfg.get("e_bits", E_BITS))
    tab = exp2_table_device(W.device, e_step, e_bits)
    d_row = torch.empty(M, dtype=torch.float32, device=W.device)
    e = torch.empty((M, nblk), dtype=torch.int8, device=W.device)
    d = torch.empty((M, nblk), dtype=torch.float32, device=W.device)
    _check(_lib.lib().ltq_row_scale(W.data_ptr(), M, K, W.stride(0), float(cfg.get("scale", 1.0)), e_step, e_bits,
                                    tab.data_ptr(), d_row.data_ptr(), e.data_ptr(), nblk, d.data_ptr(), nblk,
                                    _lib.stream_ptr()), "ltq_row_scale")
    return d_row, e, d


@torch.no_grad()
def _format_tables(cfg: dict, device) -> Tuple[torch.Tensor, torch.Tensor, dict]:
    """(level table, gains, the half-integer keywords) of a format (src/liqk_v2.py:885-895): a K_hi format alternates
    its lower format's tables on even tile rows with the higher one's on odd rows, each table premultiplied by its
    format's scale (its d then carries no factor)."""
    if "K_hi" not in cfg:
        return (torch.tensor(cfg["lut"], dtype=torch.float32, device=device), make_gains(cfg["h"], cfg["step"], device),
                {})
    lo, hi = TCQ_CONFIG[cfg["lo"]], TCQ_CONFIG[cfg["hi"]]
    lut = torch.tensor(lo["lut"], dtype=torch.float32, device=device) * lo["scale"]
    hi_kw = {"small_hi": torch.tensor(hi["lut"], dtype=torch.float32, device=device) * hi["scale"],
             "gains_hi": make_gains(hi["h"], hi["step"], device), "mix": SUBBLOCK_SIZE}
    return lut, make_gains(lo["h"], lo["step"], device), hi_kw


def _quantize_rows_tcq_ldlq(W_rot: torch.Tensor, U: torch.Tensor, U_blks_inv: torch.Tensor, diag_w: torch.Tensor,
                            spec_name: str, n_pass: int = 2,
                            fed: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block16-LDLQ with every 16-column sub-block quantized in 16 x 16 tiles by the TCQ Viterbi
    (src/liqk_v2.py:877-1021, the row-scale branch: tail-biting tiles, tiles whose trellis state carries over from
    the previous sub-block of the same rows, half-integer formats; n_pass belongs to the branch without row scale
    and is unused).
    Returns (d_full [M, K/256] fp16, W_hat_rot [M, K]). If fed [M, K] fp32 is given, it receives the value of every
    weight at the moment its sub-block was quantized (the Viterbi input times d)."""
    return _ldlq_rows(W_rot, U.unsqueeze(0), U_blks_inv.unsqueeze(0), diag_w.unsqueeze(0), spec_name, fed=fed)


def _ldlq_rows(W_rot: torch.Tensor, U: torch.Tensor, U_blks_inv: torch.Tensor, diag_w: torch.Tensor, spec_name: str,
               fed: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """The LDLQ loop over n stacked matrices sharing a format and a shape: W_rot [n R, K] (matrix m = rows
    [m R, (m + 1) R)), U [n, K, K], U_blks_inv [n, K/256, 256, 256], diag_w [n, K]. Every matrix gets exactly the
    results of its own loop; the tiles of all of them go through one Viterbi launch per sub-block.

    Per 256-column block: 16 x (two-pass tail-biting Viterbi over the tiles, ltq_ldlq_sub: the sub-block's
    feedback into the block's working copy and the next tiles), then ltq_ldlq_err (the block's error E and its
    reconstruction) and ltq_ldlq_update (W[:, c1:] -= E U[c0:c1, c1:], which also writes the next block's working
    copy and first tiles). Every sum is a fixed-order fma chain, so the loop is a defined function of its inputs.
    With PACK, appends the group's fields to PACK["groups"]."""
    cfg = TCQ_CONFIG[spec_name]
    if not cfg.get("row_scale"):
        if U.shape[0] != 1 or fed is not None:
            raise NotImplementedError(f"{spec_name}: formats without row scale quantize one matrix at a time")
        return _ldlq_rows_dcand(W_rot, U[0], U_blks_inv[0], diag_w[0], cfg, spec_name)
    device = W_rot.device
    lut, gains, hi_kw = _format_tables(cfg, device)
    M, K = W_rot.shape
    n_mat = U.shape[0]
    R = M // n_mat
    assert M % 16 == 0, "TCQ: number of rows must be divisible by 16"
    assert R * n_mat == M and (n_mat == 1 or R % 128 == 0), "stacked matrices: rows per matrix a multiple of 128"
    nt, tiles_per_mat = M // 16, R // 16
    nblocks = K // QK_K
    n_cand = int(os.environ.get("TCQ_NCAND", cfg.get("n_cand", 0)))
    tb_window = int(os.environ.get("TCQ_TB_WIN", "32"))
    sub = cfg.get("sub", SUBBLOCK_SIZE)
    W_work = W_rot.float().clone()
    W_hat_rot = torch.empty_like(W_work)
    pk = None
    if PACK is not None:
        assert cfg.get("tb") and cfg.get("row_scale"), f"{spec_name}: only formats with tail-biting and d_row are written to .ltq"
        pk = {"idx": torch.empty((M, K), dtype=torch.int16, device=device),
              "gi": torch.empty((M, K), dtype=torch.uint8, device=device),
              "G": torch.empty((M, K), dtype=torch.float32, device=device)}
    U = U.contiguous()
    U_blks_inv = U_blks_inv.contiguous()
    if fed is not None:
        assert fed.shape == (M, K) and fed.dtype == torch.float32 and fed.stride(1) == 1
    stack = (R if n_mat > 1 else 0)
    u_ms, ubi_ms = (K * K, nblocks * QK_K * QK_K) if n_mat > 1 else (0, 0)
    d_row, e_rb, d_rb_all = row_scale(W_rot, cfg)
    d_full = d_rb_all.to(torch.float16)
    lib = _lib.lib()
    stream = _lib.stream_ptr()
    carry = None  # end states of the previous sub-block's tiles (carried-state formats), across blocks as well
    x_cur = torch.empty((nt, QK_K), dtype=torch.float32, device=device)
    x_nxt = torch.empty_like(x_cur)
    w_sub = W_work[:, :QK_K].clone()      # the working copy of the block being quantized
    E_t = torch.empty((QK_K, M), dtype=torch.float32, device=device)
    G_buf = torch.empty((M, QK_K), dtype=torch.float32, device=device) if pk is None else None
    _check(lib.ltq_ldlq_prep(w_sub.data_ptr(), QK_K, d_rb_all.data_ptr(), nblocks, x_cur.data_ptr(), M, stream),
           "ltq_ldlq_prep")
    for ibl in range(nblocks):
        c0, c1 = ibl * QK_K, (ibl + 1) * QK_K
        U_blk = U[0, c0:c1, c0:c1]
        U_blk_inv = U_blks_inv[0, ibl]
        d_rb = d_rb_all[:, ibl]
        # per-position weights of every sub-block's tiles (tile of matrix m, t = 16 r + c -> diag_w[m, s0 + c])
        wts_blk = diag_w[:, c0:c1].reshape(n_mat, 1, NUM_SUBBLOCKS, 1, SUBBLOCK_SIZE)
        wts_blk = wts_blk.expand(n_mat, tiles_per_mat, NUM_SUBBLOCKS, 16, SUBBLOCK_SIZE).permute(2, 0, 1, 3, 4)
        wts_blk = wts_blk.reshape(NUM_SUBBLOCKS, nt, 16 * SUBBLOCK_SIZE)
        G_pass, ldg = (G_buf, QK_K) if pk is None else (pk["G"][:, c0:], K)
        codes = (pk["idx"][:, c0:], pk["idx"].stride(0), pk["gi"][:, c0:], pk["gi"].stride(0)) if pk else None
        for ib in range(NUM_SUBBLOCKS):
            s1 = (ib + 1) * SUBBLOCK_SIZE
            if cfg.get("tb"):
                out = viterbi_ub_cuda(x_cur, lut, cfg["K"], cfg["nu"], cfg["m"], gains, sub=sub, wts=wts_blk[ib],
                                      n_cand=n_cand, tail_biting=True, tb_window=tb_window,
                                      m_extra=cfg.get("m_extra", ()), pair_parity=cfg.get("pp", False),
                                      return_code=pk is not None, _raw_code=True)
                rec, code = out if pk is not None else (out, None)
            elif cfg.get("carry"):  # the trellis state carries over to the next sub-block's tile of the same rows
                rec, carry = viterbi_ub_cuda(x_cur, lut, cfg["K"], cfg["nu"], cfg["m"], gains, sub=SUBBLOCK_SIZE,
                                             wts=wts_blk[ib], init_state=carry, return_end_state=True, n_cand=n_cand,
                                             **hi_kw)
                code = None
            else:
                rec = viterbi_ub_cuda(x_cur, lut, cfg["K"], cfg["nu"], cfg["m"], gains, sub=SUBBLOCK_SIZE,
                                      wts=wts_blk[ib], n_cand=n_cand, **hi_kw)
                code = None
            # G, the error feedback, the next sub-block's tiles and (PACK) the code / gain index scatter
            _check(lib.ltq_ldlq_sub(w_sub.data_ptr(), QK_K, rec.data_ptr(), d_rb.data_ptr(), nblocks,
                                    U_blk_inv.data_ptr(), QK_K, U_blk.data_ptr(), K, ib,
                                    G_pass.data_ptr(), ldg, x_nxt.data_ptr() if s1 < QK_K else None, M,
                                    code.data_ptr() if code is not None else None,
                                    codes[0].data_ptr() if codes else None, codes[1] if codes else 0,
                                    codes[2].data_ptr() if codes else None, codes[3] if codes else 0,
                                    fed[:, c0:].data_ptr() if fed is not None else None,
                                    fed.stride(0) if fed is not None else 0, stack, ubi_ms, u_ms, stream),
                   "ltq_ldlq_sub")
            x_cur, x_nxt = x_nxt, x_cur
        # the block's reconstruction and error (W_work[:, c0:c1] still holds the block's start)
        _check(lib.ltq_ldlq_err(W_work[:, c0:].data_ptr(), K, G_pass.data_ptr(), ldg, d_rb.data_ptr(), nblocks,
                                U_blk_inv.data_ptr(), QK_K, E_t.data_ptr(), M, W_hat_rot[:, c0:].data_ptr(), K, M,
                                stack, ubi_ms, stream), "ltq_ldlq_err")
        if c1 < K:
            _check(lib.ltq_ldlq_update(W_work[:, c1:].data_ptr(), K, E_t.data_ptr(), M, U[0, c0:c1, c1:].data_ptr(),
                                       K, M, K - c1, w_sub.data_ptr(), QK_K, x_cur.data_ptr(),
                                       d_rb_all[:, ibl + 1].data_ptr(), nblocks, stack, u_ms, stream),
                   "ltq_ldlq_update")
    if pk is not None:
        PACK["groups"].append({"spec": spec_name, "d_row": d_row, "e": e_rb, "idx": pk["idx"], "gi": pk["gi"],
                               "G": pk["G"]})
    return d_full, W_hat_rot


def _sq_sum(a: torch.Tensor) -> torch.Tensor:
    """Per column of a [256, M] (rows of the block's E-shaped products): the float64 sum of squares."""
    return a.double().square().sum(dim=0)


def _ldlq_rows_dcand(W_rot: torch.Tensor, U: torch.Tensor, U_blks_inv: torch.Tensor, diag_w: torch.Tensor, cfg: dict,
                     spec_name: str, n_pass: int = 2) -> Tuple[torch.Tensor, torch.Tensor]:
    """The branch without row scale (src/liqk_v2.py:982-1016). Per 256-column block: d_cand = fp16(rms of the
    block's start row * scale); n_pass passes of the sub-block loop with d = d_cand (tiles start free, or carry
    the state over), each followed by the least-squares refit d_refit = fp16(<A, B> / <B, B>) in the whitened
    space (A = w_start U_inv, B = G U_inv) and a per-row choice of the lower loss |A - d B|^2 between d_cand and
    d_refit (strictly lower replaces; the next pass starts from d_refit); the chosen d and its pass's G give the
    block's reconstruction and error feedback. The sub-block loop and every product with U_inv are the fixed-order
    kernels of the row-scale path; the block rms, the refit's inner products and the losses are float64 sums
    (the reference's are device fp32 reductions of no fixed order), so the oracle matches bit for bit."""
    device = W_rot.device
    lut, gains, hi_kw = _format_tables(cfg, device)
    M, K = W_rot.shape
    assert M % 16 == 0, "TCQ: number of rows must be divisible by 16"
    nt, nblocks = M // 16, K // QK_K
    n_cand = int(os.environ.get("TCQ_NCAND", cfg.get("n_cand", 0)))
    scale = torch.tensor(float(cfg.get("scale", 1.0)), dtype=torch.float32)
    lib, stream = _lib.lib(), _lib.stream_ptr()
    U, U_blks_inv = U.contiguous(), U_blks_inv.contiguous()
    W_work = W_rot.float().clone()
    W_hat_rot = torch.empty_like(W_work)
    d_full = torch.empty((M, nblocks), dtype=torch.float16, device=device)
    w_sub = torch.empty((M, QK_K), dtype=torch.float32, device=device)
    x_cur = torch.empty((nt, QK_K), dtype=torch.float32, device=device)
    x_nxt = torch.empty_like(x_cur)
    G_pass = torch.empty((M, QK_K), dtype=torch.float32, device=device)
    zero_g = torch.zeros((M, QK_K), dtype=torch.float32, device=device)
    zero_d = torch.zeros(M, dtype=torch.float32, device=device)
    minus_one = torch.full((M,), -1.0, dtype=torch.float32, device=device)
    A_t = torch.empty((QK_K, M), dtype=torch.float32, device=device)
    B_t = torch.empty_like(A_t)
    E_t = torch.empty_like(A_t)
    carry = None
    for ibl in range(nblocks):
        c0, c1 = ibl * QK_K, (ibl + 1) * QK_K
        w_start = W_work[:, c0:c1]
        U_blk, U_blk_inv = U[c0:c1, c0:c1], U_blks_inv[ibl]
        rms = w_start.double().square().mean(dim=1).sqrt().float()
        d_cand = (rms * scale.to(device)).to(torch.float16).float().clamp(min=1e-8)
        wts_blk = diag_w[c0:c1].reshape(NUM_SUBBLOCKS, 1, SUBBLOCK_SIZE).expand(NUM_SUBBLOCKS, 16, SUBBLOCK_SIZE)
        wts_blk = wts_blk.reshape(NUM_SUBBLOCKS, 16 * SUBBLOCK_SIZE)
        # A = w_start U_inv: the error kernel with d = 0 (w - 0 G)
        _check(lib.ltq_ldlq_err(w_start.data_ptr(), K, zero_g.data_ptr(), QK_K, zero_d.data_ptr(), 1,
                                U_blk_inv.data_ptr(), QK_K, A_t.data_ptr(), M, None, 0, M, 0, 0, stream), "ltq_ldlq_err")
        best_loss = torch.full((M,), float("inf"), dtype=torch.float64, device=device)
        best_d = d_cand.clone()
        G_best = torch.zeros((M, QK_K), dtype=torch.float32, device=device)
        for _ in range(n_pass):
            w_sub.copy_(w_start)
            _check(lib.ltq_ldlq_prep(w_sub.data_ptr(), QK_K, d_cand.data_ptr(), 1, x_cur.data_ptr(), M, stream),
                   "ltq_ldlq_prep")
            for ib in range(NUM_SUBBLOCKS):
                s1 = (ib + 1) * SUBBLOCK_SIZE
                if cfg.get("carry"):
                    rec, carry = viterbi_ub_cuda(x_cur, lut, cfg["K"], cfg["nu"], cfg["m"], gains, sub=SUBBLOCK_SIZE,
                                                 wts=wts_blk[ib], init_state=carry, return_end_state=True,
                                                 n_cand=n_cand, **hi_kw)
                else:
                    rec = viterbi_ub_cuda(x_cur, lut, cfg["K"], cfg["nu"], cfg["m"], gains, sub=SUBBLOCK_SIZE,
                                          wts=wts_blk[ib], n_cand=n_cand, **hi_kw)
                _check(lib.ltq_ldlq_sub(w_sub.data_ptr(), QK_K, rec.data_ptr(), d_cand.data_ptr(), 1,
                                        U_blk_inv.data_ptr(), QK_K, U_blk.data_ptr(), K, ib, G_pass.data_ptr(), QK_K,
                                        x_nxt.data_ptr() if s1 < QK_K else None, M, None, None, 0, None, 0, None, 0,
                                        0, 0, 0, stream), "ltq_ldlq_sub")
                x_cur, x_nxt = x_nxt, x_cur
            # B = G U_inv: the error kernel with w = 0, d = -1 (0 - (-1) G = G exactly)
            _check(lib.ltq_ldlq_err(zero_g.data_ptr(), QK_K, G_pass.data_ptr(), QK_K, minus_one.data_ptr(), 1,
                                    U_blk_inv.data_ptr(), QK_K, B_t.data_ptr(), M, None, 0, M, 0, 0, stream),
                   "ltq_ldlq_err")
            Ad, Bd = A_t.double(), B_t.double()
            num, den = (Ad * Bd).sum(dim=0), _sq_sum(B_t).clamp(min=1e-12)
            d_refit = torch.where(den > 0, num / den, d_cand.double()).float().to(torch.float16).float().clamp(min=1e-8)
            for d_try in (d_cand, d_refit):
                loss = (Ad - d_try.double().unsqueeze(0) * Bd).square().sum(dim=0)
                imp = loss < best_loss
                best_loss = torch.where(imp, loss, best_loss)
                best_d = torch.where(imp, d_try, best_d)
                G_best = torch.where(imp.unsqueeze(1), G_pass, G_best)
            d_cand = d_refit
        # the block's reconstruction fl(d G) and error (w_start - d G) U_inv with the chosen scale and pass
        _check(lib.ltq_ldlq_err(w_start.data_ptr(), K, G_best.data_ptr(), QK_K, best_d.data_ptr(), 1,
                                U_blk_inv.data_ptr(), QK_K, E_t.data_ptr(), M, W_hat_rot[:, c0:].data_ptr(), K, M, 0,
                                0, stream), "ltq_ldlq_err")
        d_full[:, ibl] = best_d.to(torch.float16)
        if c1 < K:
            _check(lib.ltq_ldlq_update(W_work[:, c1:].data_ptr(), K, E_t.data_ptr(), M, U[c0:c1, c1:].data_ptr(), K,
                                       M, K - c1, None, 0, None, None, 0, 0, 0, stream), "ltq_ldlq_update")
    return d_full, W_hat_rot


# ------------------------------------------------------------------------------------------------------------
# The matrix driver. A matrix job runs in stages: rotation (suh, FWHT) -> factors of the rotated Hessian ->
# every format's row group through the LDLQ + Viterbi loop -> the joint c_row / suh refit -> the .ltq fields.
# ------------------------------------------------------------------------------------------------------------

@dataclass
class RefitResult:
    """What the joint c_row / suh refit (src/liqk_v2.py:1139-1180) computed, kept for inspection.

    c_raw [M]: per-row least-squares gain <W_hat, W H> / <W_hat, W_hat H> of the pre-refit reconstruction;
    c_row [M]: c_raw where finite and strictly inside (0.5, 2), else 1; d_new [M, nblk] fp16(d c_row);
    c_eff [M]: mean over the row's blocks of d_new / d; A (lower triangle, ridge included; only with keep) and
    b [K]: the normal equations of the column scale; s_solved: the solve's fp32 output (None when the solve
    failed); suh_cand: fp16(s_solved) where inside (0.05, 10) in magnitude, else the old suh; the two weighted
    proxy losses and whether the candidate replaced the old scales (strictly lower loss)."""
    c_raw: torch.Tensor
    c_row: torch.Tensor
    d_new: torch.Tensor
    c_eff: torch.Tensor
    A: Optional[torch.Tensor]
    b: torch.Tensor
    s_solved: Optional[torch.Tensor]
    suh_cand: torch.Tensor
    loss_base: float
    loss_cand: float
    accepted: bool


def row_proxy(HW: torch.Tensor, HQ: torch.Tensor, W: torch.Tensor, W_hat: torch.Tensor) -> torch.Tensor:
    """[M]: sum_j ((W - W_hat) H)[m, j] (W - W_hat)[m, j], with (W - W_hat) H formed as HW - HQ (no extra
    M x K x K product)."""
    return ((HW - HQ) * (W - W_hat)).sum(dim=1)


@torch.no_grad()
def refit_scales(W: torch.Tensor, H: torch.Tensor, HW: torch.Tensor, U_base: torch.Tensor, suh: torch.Tensor,
                 d: torch.Tensor, rw: Optional[torch.Tensor],
                 keep: bool = False) -> Tuple[RefitResult, torch.Tensor, torch.Tensor]:
    """The refit for W [M, K] (fp32), H, HW = W H, U_base = FWHT of the rotated reconstruction (so that the
    reconstruction is U_base * suh), the per-(row, block) scales d [M, nblk] fp16 and the normalized row weights
    rw [M] (None: unweighted). Returns (the record, the reconstruction W_hat of the scales the record chose,
    W_hat H): (c_eff U_base) * suh_cand when accepted, else U_base * suh."""
    st = _refit_prepare(W, H, HW, U_base, suh, d, rw)
    return _refit_finish(st, linalg.cholesky_lower(st["A"]), keep)


def _refit_prepare(W, H, HW, U_base, suh, d, rw) -> dict:
    """The refit up to its SPD system: c_row, the new block scales, A (lower triangle, ridge included), b."""
    W_hat = U_base * suh.unsqueeze(0)
    HQ = W_hat @ H
    gain_num = (W_hat * HW).sum(dim=1)
    gain_den = (W_hat * HQ).sum(dim=1).clamp(min=1e-12)
    c_raw = gain_num / gain_den
    usable = torch.isfinite(c_raw) & (c_raw > 0.5) & (c_raw < 2.0)
    c_row = torch.where(usable, c_raw, torch.ones_like(c_raw))
    d32 = d.float()
    d_new = (d32 * c_row.unsqueeze(1)).to(torch.float16)
    c_eff = (d_new.float() / d32.clamp(min=1e-12)).mean(dim=1)
    # the column-scale normal equations (U_w^T U_s) o H s = sum over rows of U_w o HW, U_s = c_eff U_base,
    # U_w = rw U_s; the matrix is symmetric and only its lower triangle is formed (all the Cholesky reads)
    U_s = U_base * c_eff.unsqueeze(1)
    U_w = U_s if rw is None else U_s * rw.unsqueeze(1)
    A = linalg.gram_lower(U_w, U_s).mul_(H)
    b = (U_w * HW).sum(dim=0)
    A.diagonal().add_(1e-3 * A.diagonal().mean().clamp(min=1e-12))
    weight = torch.ones_like(c_row) if rw is None else rw
    loss_base = float((row_proxy(HW, HQ, W, W_hat) * weight).sum().item())
    return dict(W=W, H=H, HW=HW, suh=suh, W_hat=W_hat, HQ=HQ, c_raw=c_raw, c_row=c_row, d_new=d_new, c_eff=c_eff,
                U_s=U_s, A=A, b=b, weight=weight, loss_base=loss_base)


def _refit_finish(st: dict, factor, keep: bool = False) -> Tuple[RefitResult, torch.Tensor, torch.Tensor]:
    """The refit from A's Cholesky factor (L, info): solve, fp16 candidate scales, loss, acceptance."""
    W, H, HW, suh, A, b = st["W"], st["H"], st["HW"], st["suh"], st["A"], st["b"]
    s_solved, suh_cand, loss_cand, W_cand, HQ_cand = None, suh, float("inf"), None, None
    try:
        s_solved = linalg.spd_solve_factored(A, b, *factor)
    except RuntimeError:  # a singular system leaves the scales as they are (src/liqk_v2.py:1179-1180)
        pass
    if s_solved is not None:
        s16 = s_solved.to(torch.float16).to(torch.float32)
        good = torch.isfinite(s16) & (s16.abs() > 0.05) & (s16.abs() < 10.0)
        suh_cand = torch.where(good, s16, suh)
        W_cand = st["U_s"] * suh_cand.unsqueeze(0)
        HQ_cand = W_cand @ H
        loss_cand = float((row_proxy(HW, HQ_cand, W, W_cand) * st["weight"]).sum().item())
    accepted = loss_cand < st["loss_base"]
    rec = RefitResult(st["c_raw"], st["c_row"], st["d_new"], st["c_eff"], A if keep else None, b, s_solved, suh_cand,
                      st["loss_base"], loss_cand, accepted)
    return (rec, W_cand, HQ_cand) if accepted else (rec, st["W_hat"], st["HQ"])


def refit_jobs(jobs: Sequence["_MatrixJob"]) -> None:
    """job.refit() for each job, bit for bit, with the SPD systems of same-sized matrices of up to linalg.LEAF
    rows factored in one batched call."""
    As = [j.refit_prepare() for j in jobs]
    by_size: Dict[int, List[int]] = {}
    for i, A in enumerate(As):
        by_size.setdefault(A.shape[0], []).append(i)
    factors: List = [None] * len(jobs)
    for K, idx in by_size.items():
        if K > linalg.LEAF or not As[idx[0]].is_cuda:
            for i in idx:
                factors[i] = linalg.cholesky_lower(As[i])
            continue
        L, info = linalg.cholesky_many(torch.stack([As[i] for i in idx]))
        for j, i in enumerate(idx):
            factors[i] = (L[j], info[j])
    del As
    for j, f in zip(jobs, factors):
        j.refit_finish(f)


def _row_slices(spec_or_row_specs, M: int) -> List[Tuple[int, int, str]]:
    if isinstance(spec_or_row_specs, str):
        return [(0, M, spec_or_row_specs)]
    return [(int(r0), int(r1), sp) for r0, r1, sp in spec_or_row_specs]


def _rows_of(row_slices, device) -> Dict[str, torch.Tensor]:
    """format -> the (sorted by slice order) row indices it quantizes."""
    groups: Dict[str, List[torch.Tensor]] = {}
    for r0, r1, sp in row_slices:
        groups.setdefault(sp, []).append(torch.arange(r0, r1, device=device))
    return {sp: torch.cat(parts) for sp, parts in groups.items()}


class _MatrixJob:
    """One matrix through the quantizer (src/liqk_v2.py:1030-1198): the stages below share its state."""

    def __init__(self, W, H, row_slices, seed, damp, row_weights):
        self.W = W.float()
        self.H = H.float()
        self.M, self.K = self.W.shape
        self.nblk = self.K // QK_K
        self.row_slices = row_slices
        for _, _, sp in row_slices:
            if sp not in TCQ_CONFIG:
                raise NotImplementedError(f"{sp}: only TCQ formats are quantized on the GPU path")
        # TCQ formats take 10x the damping of the other families (src/liqk_v2.py:1061-1063)
        self.damp = damp * float(os.environ.get("TCQ_DAMP_MULT", "10"))
        self.seed = seed
        self.row_weights = row_weights

    def rotate_and_factor(self):
        H_rot = self.rotate()
        self.U, self.diag_w, self.U_blks_inv = factor_hessian(H_rot, self.damp)
        del H_rot
        _mark("factor")

    def rotate(self) -> torch.Tensor:
        """The rotation and suh; returns the rotated Hessian for the factorization."""
        self.W_rot, H_rot, self.suh = rotation.compute_optimal_suh(self.W, self.H, seed=self.seed,
                                                                   row_weights=self.row_weights)
        _mark("rotation")
        return H_rot

    def quantize_groups(self):
        """Each format's rows through the LDLQ loop; with PACK, the tile fields gathered into matrix order."""
        dev = self.W.device
        self.W_hat_rot = torch.empty_like(self.W_rot)
        self.d = torch.empty((self.M, self.nblk), dtype=torch.float16, device=dev)
        self.fields = None
        if PACK is not None:
            PACK["groups"] = []
            self.fields = {"idx": torch.empty((self.M, self.K), dtype=torch.int16, device=dev),
                           "gi": torch.empty((self.M, self.K), dtype=torch.uint8, device=dev),
                           "G": torch.empty((self.M, self.K), dtype=torch.float32, device=dev),
                           "d_row": torch.empty(self.M, device=dev),
                           "e": torch.empty((self.M, self.nblk), dtype=torch.int8, device=dev)}
        for sp, rows in _rows_of(self.row_slices, dev).items():
            d_g, W_hat_g = _quantize_rows_tcq_ldlq(self.W_rot[rows], self.U, self.U_blks_inv, self.diag_w, sp)
            self.W_hat_rot[rows] = W_hat_g
            self.d[rows] = d_g
            if self.fields is not None:
                got = PACK["groups"].pop()
                for name, dst in self.fields.items():
                    dst[rows] = got[name].to(dst.dtype)
        _mark("rows")

    def refit(self):
        self.refit_finish(linalg.cholesky_lower(self.refit_prepare()))

    def refit_prepare(self) -> torch.Tensor:
        """The refit up to its SPD system; returns the system's matrix (lower triangle) to factor."""
        self.HW = self.W @ self.H
        U_base = rotation.fwht_inplace(self.W_hat_rot, block_size=QK_K)
        rw = None
        if self.row_weights is not None:
            rw = rotation.normalized_row_weights(self.row_weights.to(self.W.device)).float()
        self._refit = _refit_prepare(self.W, self.H, self.HW, U_base, self.suh, self.d, rw)
        return self._refit["A"]

    def refit_finish(self, factor):
        rec, self.W_hat, self.HQ = _refit_finish(self._refit, factor)
        del self._refit
        global LAST_REFIT
        LAST_REFIT = rec
        self.c_pack = torch.ones(self.M, device=self.W.device)
        if rec.accepted:
            self.suh, self.d, self.c_pack = rec.suh_cand, rec.d_new, rec.c_eff

    def write_fields(self):
        """PACK["matrix"]: the .ltq fields, and the reconstruction the file decodes to (src/liqk_v2.py:1182-1190).
        The decoded matrix equals the refit's reconstruction with row m scaled by rho_m = fp16(d_row c) /
        (d_row c) (same tile values and fp16 suh), so W_hat H is the refit's HQ scaled by row; rows whose block
        scale met the 1e-8 clamp are multiplied out."""
        f = self.fields
        d_row_file = (f["d_row"] * self.c_pack).to(torch.float16)
        suh_file = self.suh.to(torch.float16)
        scale = block_scale(d_row_file, f["e"])
        W_rot_file = (scale.unsqueeze(2) * f["G"].view(self.M, self.nblk, QK_K)).view(self.M, self.K)
        self.W_hat = rotation.fwht_inplace(W_rot_file, block_size=QK_K) * suh_file.float().unsqueeze(0)
        rho = d_row_file.float() / (f["d_row"] * self.c_pack)
        self.HQ = self.HQ * rho.unsqueeze(1)
        clamped = (block_scale(f["d_row"], f["e"]) < 1e-8).any(dim=1)
        if bool(clamped.any()):
            self.HQ[clamped] = self.W_hat[clamped] @ self.H
        PACK["matrix"] = {"row_slices": self.row_slices, "idx": f["idx"], "gi": f["gi"], "G": f["G"],
                          "d_row": d_row_file, "e": f["e"], "suh": suh_file}

    def relative_loss(self) -> float:
        num = float(row_proxy(self.HW, self.HQ, self.W, self.W_hat).sum().item())
        den = float((self.HW * self.W).sum().clamp(min=1e-12).item())
        return num / den


@torch.no_grad()
def quantize_matrix_liqk_v2(W: torch.Tensor, H: torch.Tensor, spec_or_row_specs, seed: int = 1337, damp: float = 0.02,
                            row_weights: Optional[torch.Tensor] = None, cd_sweeps: int = 2,
                            out_rot: bool = False) -> Tuple[Dict[str, torch.Tensor], torch.Tensor, float]:
    """W [M, K] with input Hessian H [K, K] -> (qdata {d, suh, row_slices[, s_out]}, W_hat [M, K], relative proxy
    loss tr(dW H dW^T) / tr(W H W^T)) for one TCQ format or row slices [(r0, r1, format), ...]
    (src/liqk_v2.py:1030-1198; cd_sweeps is accepted and unused, as there). With out_rot the rows are first
    rotated by a block FWHT-256 with Rademacher signs s_out (seed + 7919); row weights are then averaged per
    256 rows, and the result is rotated back."""
    s_out = None
    if out_rot:
        s_out = rotation.make_rademacher_signs(W.shape[0], seed=seed + 7919, device=W.device)
        W = rotation.fwht_cols(W.float(), s_out, mode=2)
        if row_weights is not None:
            row_weights = row_weights.float().view(-1, QK_K).mean(dim=1).repeat_interleave(QK_K)
    _mark("start")
    job = _MatrixJob(W, H, _row_slices(spec_or_row_specs, W.shape[0]), seed, damp, row_weights)
    job.rotate_and_factor()
    job.quantize_groups()
    job.refit()
    if job.fields is not None:
        job.write_fields()
    rel = job.relative_loss()
    q = {"d": job.d, "suh": job.suh.to(torch.float16), "row_slices": job.row_slices}
    W_hat = job.W_hat
    if s_out is not None:
        q["s_out"] = s_out.to(torch.int8)
        W_hat = rotation.fwht_cols(W_hat) * s_out.unsqueeze(1)
    _mark("refit")
    return q, W_hat, rel
