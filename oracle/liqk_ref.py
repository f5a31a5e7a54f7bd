"""TEST INFRASTRUCTURE ONLY -- CPU restatement of the TCQ matrix quantizer around the Viterbi (the checker
for ltq_amd.liqk). Only tests/ import it.

Reference anchors (torch on the CPU, float32, the reference's order of operations):
  row_scale_ref          src/liqk_v2.py:938-946 (the quantizer's bit-exact definition; row_scale_torch_fp32 is
                         the reference's torch text, kept to count rounding-boundary flips against it)
  suh_ref                src/liqk_v2.py:409-441 (scale vector in float64; suh_torch_fp32 is the reference's
                         fp32 torch text, kept to count fp16 flips against it)
  factor_hessian_ref     src/liqk_v2.py:1066-1088
  quantize_rows_ref      src/liqk_v2.py:877-1021, row-scale branch with tail-biting formats (quant_sub at
                         :913-921 via the C oracle's two-pass tail-biting driver; the feedback sums through
                         oracle/ldlq_oracle.c in the kernels' fixed order)
  ldlq_identity_residual the loop's defining identity W_rot - W_hat = E U (float64), the pin of the loop
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import ref

QK_K = 256
SUB = 16


def _exp2_table(e_step: float, e_bits: int) -> np.ndarray:
    """2^(e_step (k - 2^(e_bits-1))) for k < 2^e_bits, float64 rounded once to float32: the block-exponent
    factors (src/liqk_v2.py:946 evaluates torch.exp2 on them; the values agree, checked in tests)."""
    half = 1 << (e_bits - 1)
    return np.array([2.0 ** (e_step * (k - half)) for k in range(2 * half)], np.float32)


def block_rms_ref(W_rot: np.ndarray, scale: float) -> np.ndarray:
    """[M, K/256] fp32: max(sqrt(s / 256), 1e-10) * scale with the block sum of squares s in a fixed order:
    the 4 squares of each of 64 groups of consecutive elements summed left to right, then a butterfly over
    group offsets 32, 16, 8, 4, 2, 1 (p_l + p_(l ^ o)). src/liqk_v2.py:941 (`square().mean(2).sqrt()`)."""
    M, K = W_rot.shape
    x = np.ascontiguousarray(W_rot, np.float32).reshape(M, K // 256, 64, 4)
    sq = x * x
    p = ((sq[..., 0] + sq[..., 1]) + sq[..., 2]) + sq[..., 3]          # [M, nb, 64] fp32
    lanes = np.arange(64)
    for o in (32, 16, 8, 4, 2, 1):
        p = p + p[..., lanes ^ o]
    s = p[..., 0]
    r = np.maximum(np.sqrt(s / np.float32(256)), np.float32(1e-10))
    return (r * np.float32(scale)).astype(np.float32)


def row_scale_ref(W_rot, cfg: dict):
    """(rms [M, nb] fp32, d_row [M] fp32 (fp16 values), e [M, nb] int8, d [M, nb] fp32) as defined to the bit
    for the quantizer (src/liqk_v2.py:938-946 with the float64 evaluation of log / mean / exp / log2):
      d_row = max(fp16(fp32(exp(sum_b log(rms_b) / nb))), 1e-8)   (float64 log / exp, sum in block order)
      e     = clamp(round_half_even(log2(fp32(rms / d_row)) / e_step), -2^(bits-1), 2^(bits-1) - 1)
      d     = max(d_row * tab[e], 1e-8)                            (tab: the shared float32 exponent table)"""
    W = W_rot.numpy() if hasattr(W_rot, "numpy") else np.asarray(W_rot)
    rms = block_rms_ref(W, cfg.get("scale", 1.0))
    M, nb = rms.shape
    e_step, e_bits = float(cfg.get("e_step", 0.25)), int(cfg.get("e_bits", 5))
    e_max = 1 << (e_bits - 1)
    tab = _exp2_table(e_step, e_bits)
    d_row = np.empty(M, np.float32)
    e = np.empty((M, nb), np.int8)
    for i in range(M):
        ls = 0.0
        for b in range(nb):
            ls += math.log(float(rms[i, b]))
        dr = np.float32(np.float16(np.float32(math.exp(ls / nb))))
        d_row[i] = max(dr, np.float32(1e-8))
        for b in range(nb):
            ratio = np.float32(rms[i, b]) / d_row[i]
            ev = round(math.log2(float(ratio)) / e_step)   # Python round: half to even
            e[i, b] = min(max(ev, -e_max), e_max - 1)
    d = np.maximum(d_row[:, None] * tab[e.astype(np.int64) + e_max], np.float32(1e-8)).astype(np.float32)
    return rms, d_row, e, d


def row_scale_torch_fp32(W_rot: torch.Tensor, cfg: dict):
    """The reference's own formulation, verbatim in torch fp32 on the CPU (src/liqk_v2.py:941-946): used only to
    count where the fp32 reductions and transcendental functions put d_row or e on the other side of a rounding
    boundary than the exact definition above."""
    M, K = W_rot.shape
    nblocks = K // QK_K
    rms_rb = W_rot.float().view(M, nblocks, QK_K).square().mean(dim=2).sqrt().clamp(min=1e-10) * cfg.get("scale", 1.0)
    d_row = torch.exp(torch.log(rms_rb).mean(dim=1)).to(torch.float16).to(torch.float32).clamp(min=1e-8)
    e_step, e_max = cfg.get("e_step", 0.25), 1 << (cfg.get("e_bits", 5) - 1)
    e_rb = torch.round(torch.log2(rms_rb / d_row.unsqueeze(1)) / e_step).clamp(-e_max, e_max - 1)
    d_rb_all = d_row.unsqueeze(1) * torch.exp2(e_step * e_rb)
    return rms_rb, d_row, e_rb, d_rb_all


def suh_ref(W, H, seed: int = 1337, row_weights=None) -> np.ndarray:
    """suh [K] float32 (fp16 values) of src/liqk_v2.py:409-441 evaluated in float64 (numpy): exact squares,
    column means, the normalizations, col_rms^0.5 h_std^-0.25 clamped to [0.25, 4], times the Rademacher signs
    (the reference's own torch CPU generator draw, src/iqk_format.py:173-179), rounded once to fp16."""
    W = (W.float().numpy() if hasattr(W, "numpy") else np.asarray(W, np.float32)).astype(np.float64)
    Hd = np.diag(H.double().numpy() if hasattr(H, "numpy") else np.asarray(H, np.float64)).astype(np.float64)
    M, K = W.shape
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    signs = (torch.randint(0, 2, (K,), generator=gen, dtype=torch.int64) * 2 - 1).numpy().astype(np.float64)
    sq = W * W
    if row_weights is not None:
        rw = np.asarray(row_weights, np.float64)
        rw = np.maximum(rw, rw.mean() * 0.1)
        rw = np.clip(rw / max(rw.mean(), 1e-12), 0.25, 4.0)
        sq = sq * rw[:, None]
    col_rms = np.maximum(np.sqrt(sq.sum(axis=0) / M), 1e-6)
    col_rms = col_rms / max(col_rms.mean(), 1e-6)
    h_std = np.sqrt(np.maximum(Hd, 1e-8))
    h_std = h_std / max(h_std.mean(), 1e-6)
    scale = np.clip(np.sqrt(col_rms) * np.power(h_std, -0.25), 0.25, 4.0)
    return (signs * scale).astype(np.float16).astype(np.float32)


def suh_torch_fp32(W: torch.Tensor, H: torch.Tensor, seed: int = 1337) -> torch.Tensor:
    """The reference's fp32 torch text of the same scale (src/liqk_v2.py:419-434, no row weights), to count the
    fp16 rounding-boundary flips of the fp32 evaluation against the float64 one."""
    K = W.shape[1]
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    signs = (torch.randint(0, 2, (K,), generator=gen, dtype=torch.int64) * 2 - 1).float()
    col_rms = W.float().square().mean(dim=0).sqrt().clamp(min=1e-6)
    col_rms = col_rms / col_rms.mean().clamp(min=1e-6)
    h_std = torch.diagonal(H.float()).clamp(min=1e-8).sqrt()
    h_std = h_std / h_std.mean().clamp(min=1e-6)
    return (signs * ((col_rms ** 0.5) * (h_std ** -0.25)).clamp(0.25, 4.0)).to(torch.float16).to(torch.float32)


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


def _ptr(a):
    return None if a is None else a.ctypes.data


def quantize_rows_ref(W_rot, U, U_blks_inv, diag_w, cfg: dict, gains: np.ndarray, tb_window: int = 32,
                      n_cand: int | None = None, d_rb_all=None, mistake: str = "", trace: dict | None = None,
                      lut=None, hi: dict | None = None):
    """The row quantizer's LDLQ loop (src/liqk_v2.py:948-980, row-scale branch) over the C oracle's Viterbi and
    its LDLQ restatements (oracle/ldlq_oracle.c: fma chains in ascending order, as the kernels define the sums).
    Tiles are tail-biting (cfg "tb"), or carry the trellis state from one sub-block to the next (cfg "carry",
    src/liqk_v2.py:926-929), or start free. lut overrides cfg["lut"]; hi = {"small_hi", "gains_hi"} gives a
    half-integer format's odd-row tables (src/liqk_v2.py:887-892: the caller premultiplies each table by its
    format's scale). Returns (d_full fp16 [M, nblk], W_hat_rot [M, K], codes {idx int16, gi uint8} (tail-biting
    formats, else None), fed [M, K]): fed holds every weight's value when its sub-block was quantized. d_rb_all may be given ([M, nblk]); by default the row scale
    comes from row_scale_ref. `mistake` plants one error for the tests that check the identities catch it:
    "sign" (the sub-block feedback added instead of subtracted), "slice" (the inter-block update from the
    factor's rows shifted by one) or "index" (the next sub-block fed from the wrong column). With a `trace`
    dict, trace["x"] [M, K] receives the Viterbi inputs in matrix layout."""
    if not cfg.get("row_scale"):
        d_full, W_hat = quantize_rows_dcand_ref(W_rot, U, U_blks_inv, diag_w, cfg, gains, n_cand=n_cand, lut=lut,
                                                hi=hi)
        return d_full, W_hat, None, None
    L = ref.lib()
    W = np.ascontiguousarray(W_rot.numpy() if hasattr(W_rot, "numpy") else W_rot, np.float32)
    Uf = np.ascontiguousarray(U.numpy() if hasattr(U, "numpy") else U, np.float32)
    Ubi = np.ascontiguousarray(U_blks_inv.numpy() if hasattr(U_blks_inv, "numpy") else U_blks_inv, np.float32)
    dw = np.ascontiguousarray(diag_w.numpy() if hasattr(diag_w, "numpy") else diag_w, np.float32)
    M, K = W.shape
    nt, nblocks = M // 16, K // QK_K
    n_cand = cfg.get("n_cand", 0) if n_cand is None else n_cand
    lut = np.asarray(cfg["lut"] if lut is None else lut, np.float32)
    hi_kw = {} if hi is None else dict(small_hi=np.asarray(hi["small_hi"], np.float32),
                                       gains_hi=np.asarray(hi["gains_hi"], np.float32), mix=SUB)
    carry = None
    m_extra = tuple(cfg.get("m_extra", ()))
    if d_rb_all is None:
        _, _, _, d_rb_all = row_scale_ref(W, cfg)
    d_all = np.ascontiguousarray(d_rb_all.numpy() if hasattr(d_rb_all, "numpy") else d_rb_all, np.float32)
    d_all = np.maximum(d_all, np.float32(1e-8))
    W_work = W.copy()
    W_hat = np.empty_like(W)
    fed = np.empty_like(W)
    xs_all = np.empty_like(W) if trace is not None else None
    idx = np.empty((M, K), np.int16)
    gim = np.empty((M, K), np.uint8)
    G = np.empty((M, QK_K), np.float32)
    E = np.empty((M, QK_K), np.float32)
    for ibl in range(nblocks):
        c0, c1 = ibl * QK_K, (ibl + 1) * QK_K
        w_sub = np.ascontiguousarray(W_work[:, c0:c1])
        U_blk = np.ascontiguousarray(Uf[c0:c1, c0:c1])
        if mistake == "sign":
            U_blk = -U_blk
        Ubi_b = Ubi[ibl]
        d = np.ascontiguousarray(d_all[:, ibl])
        inv = np.float32(1.0) / d
        x = np.ascontiguousarray((w_sub[:, :SUB] * inv[:, None]).reshape(nt, 256))
        fed_b = np.empty((M, QK_K), np.float32)
        for ib in range(QK_K // SUB):
            s0, s1 = ib * SUB, (ib + 1) * SUB
            wts = np.tile(dw[c0 + s0:c0 + s1], 16)
            if xs_all is not None:
                xs_all[:, c0 + s0:c0 + s1] = x.reshape(M, SUB)
            if cfg.get("tb"):
                rec, gi, ix = ref.viterbi_ub_cuda_ref(x, lut, cfg["K"], 10, cfg["m"], gains, sub=cfg.get("sub", 16),
                                                      wts=wts, n_cand=n_cand, tail_biting=True, tb_window=tb_window,
                                                      m_extra=m_extra, pair_parity=int(cfg.get("pp", 0)),
                                                      return_code=True)
                idx[:, c0 + s0:c0 + s1] = np.asarray(ix).reshape(M, SUB).astype(np.int16)
                gim[:, c0 + s0:c0 + s1] = np.asarray(gi).reshape(M, SUB).astype(np.uint8)
            elif cfg.get("carry"):  # the state carries over to the next sub-block (src/liqk_v2.py:926-929)
                rec, carry = ref.viterbi_ub_cuda_ref(x, lut, cfg["K"], 10, cfg["m"], gains, sub=SUB, wts=wts,
                                                     init_state=carry, return_end_state=True, n_cand=n_cand, **hi_kw)
                carry = np.ascontiguousarray(carry, np.int32)
            else:
                rec = ref.viterbi_ub_cuda_ref(x, lut, cfg["K"], 10, cfg["m"], gains, sub=SUB, wts=wts, n_cand=n_cand,
                                              **hi_kw)
            rec = np.ascontiguousarray(rec, np.float32)
            x_next = np.empty((nt, 256), np.float32)
            L.ltq_oracle_ldlq_sub(_ptr(w_sub), QK_K, _ptr(rec), _ptr(d), 1, _ptr(Ubi_b), QK_K, _ptr(U_blk), QK_K, ib,
                                  _ptr(G), QK_K, _ptr(x_next) if s1 < QK_K else None, M, _ptr(fed_b), QK_K)
            if mistake == "index" and s1 < QK_K:
                j = min(s1 + 1, QK_K - SUB)
                x_next = np.ascontiguousarray((w_sub[:, j:j + SUB] * inv[:, None]).reshape(nt, 256))
            x = x_next
        fed[:, c0:c1] = fed_b
        wh = np.empty((M, QK_K), np.float32)
        ws = np.ascontiguousarray(W_work[:, c0:c1])
        L.ltq_oracle_ldlq_err(_ptr(ws), QK_K, _ptr(G), QK_K, _ptr(d), 1, _ptr(Ubi_b), QK_K, _ptr(E), QK_K, _ptr(wh),
                              QK_K, M)
        W_hat[:, c0:c1] = wh
        if c1 < K:
            r0 = c0 + 1 if mistake == "slice" else c0   # c1 < K, so rows r0 .. r0 + 255 exist
            Up = np.ascontiguousarray(Uf[r0:r0 + QK_K, c1:])
            rest = np.ascontiguousarray(W_work[:, c1:])
            L.ltq_oracle_ldlq_update(_ptr(rest), K - c1, _ptr(E), QK_K, _ptr(Up), K - c1, M, K - c1)
            W_work[:, c1:] = rest
    d_full = d_all.astype(np.float16)
    if trace is not None:
        trace["x"] = xs_all
    return d_full, W_hat, ({"idx": idx, "gi": gim} if cfg.get("tb") else None), fed


def quantize_rows_dcand_ref(W_rot, U, U_blks_inv, diag_w, cfg: dict, gains: np.ndarray, n_pass: int = 2,
                            n_cand: int | None = None, lut=None, hi: dict | None = None, mistake: str = "",
                            trace: dict | None = None):
    """The branch without row scale (src/liqk_v2.py:982-1016): per 256-column block, d_cand = fp16(rms * scale)
    of the block's start rows, n_pass passes of the sub-block loop at d_cand (tiles start free, or carry the
    state over with cfg "carry"), each followed by the refit d_refit = fp16(<A, B> / <B, B>) with A = w_start
    U_inv and B = G U_inv, and the per-row choice of the strictly lower |A - d B|^2 between d_cand and d_refit;
    the next pass starts from d_refit. The products with U_inv and the feedback are the oracle's fma chains; the
    rms, the inner products and the losses are float64 sums. Returns (d_full fp16 [M, nblk], W_hat [M, K]).
    `mistake` "no_refit" keeps d_cand in every pass (for the test that the refit is pinned). With a `trace` dict,
    trace["blocks"][b] lists every pass's (d_cand, G, d_refit) and trace["start"][b] the block's start rows."""
    L = ref.lib()
    W = np.ascontiguousarray(W_rot.numpy() if hasattr(W_rot, "numpy") else W_rot, np.float32)
    Uf = np.ascontiguousarray(U.numpy() if hasattr(U, "numpy") else U, np.float32)
    Ubi = np.ascontiguousarray(U_blks_inv.numpy() if hasattr(U_blks_inv, "numpy") else U_blks_inv, np.float32)
    dw = np.ascontiguousarray(diag_w.numpy() if hasattr(diag_w, "numpy") else diag_w, np.float32)
    M, K = W.shape
    nt, nblocks = M // 16, K // QK_K
    n_cand = cfg.get("n_cand", 0) if n_cand is None else n_cand
    lut = np.asarray(cfg["lut"] if lut is None else lut, np.float32)
    hi_kw = {} if hi is None else dict(small_hi=np.asarray(hi["small_hi"], np.float32),
                                       gains_hi=np.asarray(hi["gains_hi"], np.float32), mix=SUB)
    scale = np.float32(cfg.get("scale", 1.0))
    W_work = W.copy()
    W_hat = np.empty_like(W)
    d_full = np.empty((M, nblocks), np.float16)
    zero_g = np.zeros((M, QK_K), np.float32)
    carry = None
    for ibl in range(nblocks):
        c0, c1 = ibl * QK_K, (ibl + 1) * QK_K
        w_start = np.ascontiguousarray(W_work[:, c0:c1])
        U_blk = np.ascontiguousarray(Uf[c0:c1, c0:c1])
        Ubi_b = Ubi[ibl]
        rms = np.sqrt(np.mean(np.square(w_start.astype(np.float64)), axis=1)).astype(np.float32)
        d_cand = np.maximum((rms * scale).astype(np.float16).astype(np.float32), np.float32(1e-8))
        A = np.empty((M, QK_K), np.float32)
        L.ltq_oracle_ldlq_err(_ptr(w_start), QK_K, _ptr(zero_g), QK_K, _ptr(np.zeros(M, np.float32)), 1,
                              _ptr(Ubi_b), QK_K, _ptr(A), QK_K, None, QK_K, M)
        best_loss = np.full(M, np.inf)
        best_d = d_cand.copy()
        G_best = np.zeros((M, QK_K), np.float32)
        passes = []
        if trace is not None:
            trace.setdefault("blocks", []).append(passes)
            trace.setdefault("start", []).append(w_start.copy())
        for _ in range(n_pass):
            w_sub = w_start.copy()
            G = np.empty((M, QK_K), np.float32)
            x = np.ascontiguousarray((w_sub[:, :SUB] * (np.float32(1) / d_cand)[:, None]).reshape(nt, 256))
            for ib in range(QK_K // SUB):
                s0, s1 = ib * SUB, (ib + 1) * SUB
                wts = np.tile(dw[c0 + s0:c0 + s1], 16)
                if cfg.get("carry"):
                    rec, carry = ref.viterbi_ub_cuda_ref(x, lut, cfg["K"], 10, cfg["m"], gains, sub=SUB, wts=wts,
                                                         init_state=carry, return_end_state=True, n_cand=n_cand,
                                                         **hi_kw)
                    carry = np.ascontiguousarray(carry, np.int32)
                else:
                    rec = ref.viterbi_ub_cuda_ref(x, lut, cfg["K"], 10, cfg["m"], gains, sub=SUB, wts=wts,
                                                  n_cand=n_cand, **hi_kw)
                rec = np.ascontiguousarray(rec, np.float32)
                x_next = np.empty((nt, 256), np.float32)
                L.ltq_oracle_ldlq_sub(_ptr(w_sub), QK_K, _ptr(rec), _ptr(d_cand), 1, _ptr(Ubi_b), QK_K, _ptr(U_blk),
                                      QK_K, ib, _ptr(G), QK_K, _ptr(x_next) if s1 < QK_K else None, M, None, QK_K)
                x = x_next
            B = np.empty((M, QK_K), np.float32)
            L.ltq_oracle_ldlq_err(_ptr(zero_g), QK_K, _ptr(G), QK_K, _ptr(np.full(M, -1.0, np.float32)), 1,
                                  _ptr(Ubi_b), QK_K, _ptr(B), QK_K, None, QK_K, M)
            Ad, Bd = A.astype(np.float64), B.astype(np.float64)
            num, den = np.sum(Ad * Bd, axis=1), np.maximum(np.sum(Bd * Bd, axis=1), 1e-12)
            ratio = np.where(den > 0, num / den, d_cand.astype(np.float64)).astype(np.float32)
            d_refit = np.maximum(ratio.astype(np.float16).astype(np.float32), np.float32(1e-8))
            if mistake == "no_refit":
                d_refit = d_cand
            passes.append((d_cand.copy(), G.copy(), d_refit.copy()))
            for d_try in (d_cand, d_refit):
                loss = np.sum(np.square(Ad - d_try.astype(np.float64)[:, None] * Bd), axis=1)
                imp = loss < best_loss
                best_loss = np.where(imp, loss, best_loss)
                best_d = np.where(imp, d_try, best_d)
                G_best = np.where(imp[:, None], G, G_best)
            d_cand = d_refit
        E = np.empty((M, QK_K), np.float32)
        wh = np.empty((M, QK_K), np.float32)
        G_best = np.ascontiguousarray(G_best, np.float32)
        best_d = np.ascontiguousarray(best_d, np.float32)
        L.ltq_oracle_ldlq_err(_ptr(w_start), QK_K, _ptr(G_best), QK_K, _ptr(best_d), 1, _ptr(Ubi_b), QK_K, _ptr(E),
                              QK_K, _ptr(wh), QK_K, M)
        W_hat[:, c0:c1] = wh
        d_full[:, ibl] = best_d.astype(np.float16)
        if c1 < K:
            Up = np.ascontiguousarray(Uf[c0:c1, c1:])
            rest = np.ascontiguousarray(W_work[:, c1:])
            L.ltq_oracle_ldlq_update(_ptr(rest), K - c1, _ptr(E), QK_K, _ptr(Up), K - c1, M, K - c1)
            W_work[:, c1:] = rest
    return d_full, W_hat


def ldlq_identity_residual(W_rot, W_hat, fed, U, U_blks_inv):
    """The defining identity of the LDLQ loop, in float64: with E_j = (fed_j - W_hat_j) U_jj^-1 for every 16-column
    sub-block j (U_jj^-1 the diagonal 16 x 16 block of the block inverse), W_rot - W_hat = E U exactly. Returns
    (R = (W_rot - W_hat) - E U, B = |W_rot| + |E| |U|): an fp32 implementation of the loop leaves |R| within a
    few hundred units of roundoff of B, while a wrong sign, slice or feedback index leaves residuals of the
    size of B itself."""
    Wr = np.asarray(W_rot, np.float64)
    Wh = np.asarray(W_hat, np.float64)
    F = np.asarray(fed, np.float64)
    Ud = np.asarray(U, np.float64)
    Ubi = np.asarray(U_blks_inv, np.float64)
    M, K = Wr.shape
    E = np.empty_like(Wr)
    for c0 in range(0, K, SUB):
        b, s0 = c0 // QK_K, c0 % QK_K
        Uinv_jj = Ubi[b, s0:s0 + SUB, s0:s0 + SUB]
        E[:, c0:c0 + SUB] = (F[:, c0:c0 + SUB] - Wh[:, c0:c0 + SUB]) @ Uinv_jj
    R = (Wr - Wh) - E @ Ud
    B = np.abs(Wr) + np.abs(E) @ np.abs(Ud)
    return R, B
