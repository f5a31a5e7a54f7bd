"""TEST INFRASTRUCTURE ONLY -- the reference's CPU path in torch, the CPU baseline bench.py times.

The reference's CPU Viterbi is the torch function viterbi_ub (src/tcq_proto.py:327-419): a step loop over
[N tiles, G gain slots, S states] tensors. It covers the integer, 4-subset, free-start, all-gains subset; the
semantics of the production formats (extended labels, D4 parity groups, gain candidates, tail-biting, middle
states) exist only in the CUDA kernel (src/cuda/tcq_viterbi.cu:97-683). This module restates both in the same
torch-on-tensors style, eager, with the same fp32 order of operations and tie rules as the kernel:
  branch metric  E = w * min over levels u (u = parity class mod 2 in D4) of fl(fl(x - fl(g tab))^2)
                 (src/tcq_proto.py:376-385)
  integer step   D'(s) = min(D(p0), D(p1)) + E(lb(s)), p_h = h S/2 + (s >> 1), p0 on ties (:327-332, cu:501-554)
  D4 group       phase A: I_b = min(D(p)) + E_t(b); C_c = min over b (b = 0 on ties) of min(I_b(q)) +
                 E_t+1(b ^ c); phase B: J_cb = min(C_c(p)) + E_t+2(b); D' = first minimum over (c, b) in order
                 00, 01, 10, 11 of min(J_cb(q)) + E_t+3(b ^ c) (cu:217-267, 322-443)
  gain merge     at t = j sub > 0, D(g, s) <- min over g' (lowest g') (tcq_proto.py:393-396, cu:184-201)
  candidates     per sub-block the G gains of lowest sequentially summed scalar error, ascending (cu:155-180)
  end / tail     argmin over g S + s (lowest), with tail only s = init (cu:561-578)
  output         u = first minimum over allowed u, rec = fl(g tab), code = gi << 16 | lb U + u (cu:662-682)
Only tests/ and bench.py's cpu_baseline import it. Pinned by tests/test_torch_viterbi.py against the reference's
own viterbi_ub outputs (tests/golden/viterbi_ub.npz) and against the C oracle bit for bit.
"""
from __future__ import annotations

import numpy as np
import torch

SENT = 3.4e38


def _parity(v: torch.Tensor) -> torch.Tensor:
    v = v ^ (v >> 16)
    v = v ^ (v >> 8)
    v = v ^ (v >> 4)
    v = v ^ (v >> 2)
    v = v ^ (v >> 1)
    return v & 1


def labels(S: int, masks) -> torch.Tensor:
    """lb(s) = (s & 1) | par((s >> 1) & m_i) << (i + 1) for the label masks m_0 (primary), m_1, ... [S]."""
    s = torch.arange(S, dtype=torch.int64)
    lb = s & 1
    for i, m in enumerate(masks):
        lb = lb | (_parity((s >> 1) & m) << (i + 1))
    return lb


@torch.no_grad()
def tcq_viterbi_torch(x, w, tab, gains, *, masks=(359,), K=3, pp=0, sub=16, n_cand=0, init_st=None, tail=False,
                      steps=0, rot=0, mid_t=0, S=1024):
    """One pass over tiles x, w [N, ld] (float32 torch tensors, the rotated window (t + rot) % ld of `steps`
    samples, default ld). Returns {rec, code, best, end, mid} with the reference C ABI's meaning."""
    if pp not in (0, 2):
        raise NotImplementedError("the torch restatement covers the integer and D4 modes")
    x = torch.as_tensor(x, dtype=torch.float32)
    w = torch.as_tensor(w, dtype=torch.float32)
    tab = torch.as_tensor(tab, dtype=torch.float32)
    gains = torch.as_tensor(gains, dtype=torch.float32)
    N, ld = x.shape
    T = steps or ld
    nl = 2 << len(masks)
    U = tab.numel() // nl
    Gf = gains.numel()
    G = n_cand if 0 < n_cand < Gf else Gf
    HALF = S // 2
    pos = (torch.arange(T) + rot) % ld
    xr, wr = x[:, pos], w[:, pos]                                   # [N, T]
    lb_of = labels(S, masks)
    lo = torch.arange(S) >> 1
    hi = lo + HALF
    nsub = T // sub
    # slot -> global gain index per (tile, sub-block)
    if G < Gf:
        err_all = (xr.unsqueeze(-1).unsqueeze(-1) - gains.view(1, 1, Gf, 1) * tab.view(1, 1, 1, -1)).square()
        emin = err_all.amin(dim=3) * wr.unsqueeze(-1)              # [N, T, Gf]
        ce = torch.zeros((N, nsub, Gf))
        for k in range(sub):                                       # summed in step order
            ce = ce + emin[:, k::sub][:, :nsub]
        order = torch.sort(ce, dim=2, stable=True).indices[:, :, :G]
        gidx = order                                               # [N, nsub, G]
    else:
        gidx = torch.arange(G).view(1, 1, G).expand(N, nsub, G)
    gstep = gidx.repeat_interleave(sub, dim=1)                     # [N, T, G]
    gval = gains[gstep]                                            # [N, T, G]
    vals = gval.unsqueeze(-1) * tab.view(1, 1, 1, -1)              # [N, T, G, nl U]
    sq = (xr.view(N, T, 1, 1) - vals).square().view(N, T, G, nl, U)
    NP = 2 if pp else 1
    if pp:
        em = torch.stack([sq[..., p::2].amin(dim=-1) for p in range(2)], dim=-1)   # [N, T, G, nl, 2]
    else:
        em = sq.amin(dim=-1, keepdim=True)
    E = em * wr.view(N, T, 1, 1, 1)
    Es = E[:, :, :, lb_of, :]                                      # [N, T, G, S, NP]: by state

    if init_st is not None:
        init = torch.as_tensor(np.asarray(init_st), dtype=torch.int64).view(N)
        allowed = ((torch.arange(S).view(1, S) >> 1) == (init.view(N, 1) & (HALF - 1))).view(N, 1, S)
    else:
        init = None
        allowed = torch.ones((N, 1, S), dtype=torch.bool)
    sent = torch.tensor(SENT, dtype=torch.float32)

    def pred_min(D):
        a0, a1 = D[..., lo], D[..., hi]
        d = a1 < a0
        return torch.where(d, a1, a0), d

    gsel = {}
    dec = {}
    D = None
    if pp == 0:
        for t in range(T):
            if t == 0:
                D = torch.where(allowed, Es[:, 0, :, :, 0], sent)
                continue
            if G > 1 and t % sub == 0:
                D, gsel[t // sub] = _merge(D)
            m, d = pred_min(D)
            dec[t] = d
            D = m + Es[:, t, :, :, 0]
    else:
        for t in range(0, T, 4):
            if t > 0 and G > 1 and t % sub == 0:
                D, gsel[t // sub] = _merge(D)
            # phase A
            if t == 0:
                I = [torch.where(allowed, Es[:, 0, :, :, b], sent) for b in range(2)]
                dA = None
            else:
                m, dA = pred_min(D)
                I = [m + Es[:, t, :, :, b] for b in range(2)]
            mq, dq = zip(*[pred_min(I[b]) for b in range(2)])
            C, bs = [], []
            for c in range(2):
                c0 = mq[0] + Es[:, t + 1, :, :, c]
                c1 = mq[1] + Es[:, t + 1, :, :, 1 ^ c]
                sel = c1 < c0
                C.append(torch.where(sel, c1, c0))
                bs.append(sel)
            # phase B
            J, dr = [], []
            for c in range(2):
                m, d = pred_min(C[c])
                dr.append(d)
                J.append([m + Es[:, t + 2, :, :, b] for b in range(2)])
            best, choice, ds = None, None, []
            for cb in range(4):
                c, b = cb >> 1, cb & 1
                m, d = pred_min(J[c][b])
                ds.append(d)
                cand = m + Es[:, t + 3, :, :, b ^ c]
                if cb == 0:
                    best, choice = cand, torch.zeros_like(cand, dtype=torch.int64)
                else:
                    sel = cand < best
                    best = torch.where(sel, cand, best)
                    choice = torch.where(sel, torch.full_like(choice, cb), choice)
            D = best
            dec[t] = (dA, dq, bs, dr, ds, choice)

    # end state: lowest g S + s among the minima (with tail, among s = init)
    if tail:
        cand = D[torch.arange(N), :, init]                         # [N, G]
        g_end = cand.argmin(dim=1)
        s_end = init.clone()
    else:
        flat = D.reshape(N, G * S).argmin(dim=1)
        g_end, s_end = flat // S, flat % S
    best_idx = g_end * S + s_end

    # traceback
    ar = torch.arange(N)
    states = torch.empty((N, T), dtype=torch.int64)
    par = torch.zeros((N, T), dtype=torch.int64)
    slot = torch.empty((N, T), dtype=torch.int64)
    st, gs = s_end.clone(), g_end.clone()

    def back(bit, s):
        return (bit.to(torch.int64) << (HALF.bit_length() - 1)) | (s >> 1)

    if pp == 0:
        for t in range(T - 1, -1, -1):
            states[:, t] = st
            slot[:, t] = gs
            if t > 0:
                st = back(dec[t][ar, gs, st], st)
                if G > 1 and t % sub == 0:
                    gs = gsel[t // sub][ar, st]
    else:
        for t in range(T - 4, -1, -4):
            dA, dq, bs, dr, ds, choice = dec[t]
            s4 = st
            cb = choice[ar, gs, s4]
            c, bb = cb >> 1, cb & 1
            dsx = torch.stack(ds)[cb, ar, gs, s4]
            s3 = back(dsx, s4)
            s2 = back(torch.stack(dr)[c, ar, gs, s3], s3)
            bstar = torch.stack(bs)[c, ar, gs, s2].to(torch.int64)
            s1 = back(torch.stack(dq)[bstar, ar, gs, s2], s2)
            states[:, t], states[:, t + 1], states[:, t + 2], states[:, t + 3] = s1, s2, s3, s4
            par[:, t], par[:, t + 1], par[:, t + 2], par[:, t + 3] = bstar, bstar ^ c, bb, bb ^ c
            slot[:, t:t + 4] = gs.view(N, 1)
            if t > 0:
                st = back(dA[ar, gs, s1], s1)
                if G > 1 and t % sub == 0:
                    gs = gsel[t // sub][ar, st]

    # reconstruction and codes
    lbt = lb_of[states]                                            # [N, T]
    gi = gidx.repeat_interleave(sub, dim=1)[ar.view(N, 1), torch.arange(T).view(1, T), slot]   # [N, T]
    gv = gains[gi]
    lv = tab.view(nl, U)[lbt]                                      # [N, T, U]
    vv = gv.unsqueeze(-1) * lv
    err = (xr.unsqueeze(-1) - vv).square()
    if pp:
        uu = torch.arange(U).view(1, 1, U)
        err = torch.where((uu & 1) == par.unsqueeze(-1), err, torch.full_like(err, float("inf")))
    u = err.argmin(dim=-1)
    rec_t = vv.gather(2, u.unsqueeze(-1)).squeeze(-1)
    code_t = (gi << 16) | (lbt * U + u)
    rec = torch.zeros((N, ld), dtype=torch.float32)
    code = torch.zeros((N, ld), dtype=torch.int32)
    rec[:, pos] = rec_t
    code[:, pos] = code_t.to(torch.int32)
    out = {"rec": rec.numpy(), "code": code.numpy(), "best": best_idx.to(torch.int32).numpy(),
           "end": s_end.to(torch.int32).numpy()}
    if mid_t:
        out["mid"] = states[:, mid_t - 1].to(torch.int32).numpy()
    return out


def _merge(D):
    """D(g, s) <- min over g' (lowest g' on ties) and the chosen slot per (tile, state)."""
    best, bg = D[:, 0], torch.zeros(D.shape[0], D.shape[2], dtype=torch.int64)
    for g in range(1, D.shape[1]):
        sel = D[:, g] < best
        best = torch.where(sel, D[:, g], best)
        bg = torch.where(sel, torch.full_like(bg, g), bg)
    return best.unsqueeze(1).expand_as(D).contiguous(), bg


@torch.no_grad()
def viterbi_ub_cuda_torch(x, small, K, nu, m, gains, sub=16, wts=None, n_cand=0, tail_biting=True, tb_window=0,
                          m_extra=(), pair_parity=0):
    """The two-pass tail-biting driver of src/tcq_proto.py:584-609 over tcq_viterbi_torch: pass 1 finds the
    middle state (over the window [h - w, h + w) when tb_window > 0), pass 2 closes the path there at rotation
    h. Returns (rec, gain index, level index) as numpy arrays."""
    x = torch.as_tensor(np.ascontiguousarray(x, np.float32))
    N, T = x.shape
    w = torch.ones_like(x) if wts is None else torch.as_tensor(
        np.ascontiguousarray(np.broadcast_to(np.asarray(wts, np.float32).reshape(-1, T), (N, T))))
    masks = (m,) + tuple(m_extra)
    kw = dict(masks=masks, K=K, pp=int(pair_parity), sub=sub, n_cand=n_cand, S=1 << nu)
    h = T // 2
    if not tail_biting:
        o = tcq_viterbi_torch(x, w, small, gains, **kw)
    else:
        if tb_window:
            p1 = tcq_viterbi_torch(x, w, small, gains, steps=2 * tb_window, rot=h - tb_window, mid_t=tb_window, **kw)
        else:
            p1 = tcq_viterbi_torch(x, w, small, gains, mid_t=h, **kw)
        o = tcq_viterbi_torch(x, w, small, gains, init_st=p1["mid"], tail=True, rot=h % T, **kw)
    code = o["code"].astype(np.int64)
    return o["rec"], code >> 16, code & 0xFFFF


@torch.no_grad()
def viterbi_ub_torch(x, small, K, nu, m, gains=None, sub=16, wts=None):
    """The reference's own viterbi_ub call convention (src/tcq_proto.py:363-419): integer mode, 4 subsets, free
    start, all gains. Returns (rec, labels, u, gidx) as numpy arrays."""
    x = np.ascontiguousarray(x, np.float32)
    N, T = x.shape
    w = np.ones_like(x) if wts is None else np.ascontiguousarray(np.broadcast_to(np.asarray(wts, np.float32).reshape(-1, T), (N, T)))
    g = np.asarray(gains, np.float32) if gains is not None else np.ones(1, np.float32)
    o = tcq_viterbi_torch(torch.from_numpy(x.copy()), torch.from_numpy(w.copy()), small, g, masks=(m,), K=K, pp=0, sub=sub,
                          S=1 << nu)
    code = o["code"].astype(np.int64)
    U = 1 << (K - 1)
    lev = code & 0xFFFF
    gidx = (code >> 16)[:, ::sub]
    return o["rec"], lev // U, lev % U, gidx
