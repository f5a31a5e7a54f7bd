"""TEST INFRASTRUCTURE ONLY -- ctypes wrapper of the C oracle (liboracle.so) plus numpy restatements.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module; the
product path (ltq-research_amd/) never does, and it must fail loudly when its HIP library is missing
rather than fall back to anything here.

Reference anchors:
  viterbi_ub_cuda_ref  -> src/tcq_proto.py:567-657 (driver, incl. two-pass tail-biting :584-609)
  viterbi_ub_ref       -> src/tcq_proto.py:363-419 (return convention of the torch reference)
  make_gains_ref       -> src/tcq_proto.py:247-249
  fwht256_ref          -> src/iqk_format.py:153-170
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB = None


def build(force: bool = False) -> Path:
    so = _DIR / "liboracle.so"
    if force or not so.exists():
        subprocess.run(["make", "-s", "-C", str(_DIR), "-B" if force else "liboracle.so"], check=True)
    return so


def lib():
    global _LIB
    if _LIB is None:
        so = _DIR / "liboracle.so"
        if not so.exists():
            build()
        L = ctypes.CDLL(str(so))
        vp, ci = ctypes.c_void_p, ctypes.c_int
        L.ltq_oracle_tcq_viterbi.restype = ci
        L.ltq_oracle_tcq_viterbi.argtypes = [vp] * 13 + [ci] * 19 + [vp, ci]
        L.ltq_oracle_fwht256.restype = None
        L.ltq_oracle_fwht256.argtypes = [vp, ctypes.c_long]
        L.ltq_oracle_lut_subs.restype = None
        L.ltq_oracle_lut_subs.argtypes = [vp] * 4 + [ctypes.c_long, ctypes.c_float, ctypes.c_float, ci]
        L.ltq_oracle_labels.restype = None
        L.ltq_oracle_labels.argtypes = [ci] * 6 + [vp]
        cl = ctypes.c_long
        L.ltq_oracle_ldlq_sub.restype = None
        L.ltq_oracle_ldlq_sub.argtypes = [vp, cl, vp, vp, cl, vp, cl, vp, cl, ci, vp, cl, vp, cl, vp, cl]
        L.ltq_oracle_ldlq_err.restype = None
        L.ltq_oracle_ldlq_err.argtypes = [vp, cl, vp, cl, vp, cl, vp, cl, vp, cl, vp, cl, cl]
        L.ltq_oracle_ldlq_update.restype = None
        L.ltq_oracle_ldlq_update.argtypes = [vp, cl, vp, cl, vp, cl, cl, cl]
        L.ltq_brute_force.restype = ctypes.c_double
        L.ltq_brute_force.argtypes = [vp] + [ci] * 12 + [vp, vp, vp]
        _LIB = L
    return _LIB


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def tcq_viterbi(x, w, tab, gains, *, init_st=None, tab_hi=None, gains_hi=None, n_cand=0, mid_t=0, tail=False,
                S=1024, U=None, m=359, sub=16, mix=0, m_extra=(), steps=0, rot=0, pp=0, want_code=True,
                want_end=False, want_gsel=False, nthreads=0):
    """One oracle call with the semantics of the reference C ABI tcq_viterbi (tcq_viterbi.cu:743-766).

    x, w: [N, ld] float32. Returns a dict with rec, code, best, end, mid, gcand (gsel optional)."""
    x, w = _f32(x), _f32(w)
    N, ld = x.shape
    T = steps or ld
    nl = 4 << len(m_extra)
    tab = _f32(tab)
    gains = _f32(gains)
    if U is None:
        U = tab.size // nl
    tab_hi_a = _f32(tab_hi) if tab_hi is not None else tab
    g_hi = _f32(gains_hi) if gains_hi is not None else gains
    U_hi = tab_hi_a.size // nl
    Gfull = gains.size
    G = n_cand if 0 < n_cand < Gfull else Gfull
    rec = np.zeros((N, ld), np.float32)
    code = np.zeros((N, ld), np.int32) if want_code else None
    best = np.zeros(N, np.int32)
    end = np.zeros(N, np.int32) if want_end else None
    mid = np.zeros(N, np.int32) if mid_t else None
    gcand = np.zeros((N, T // sub, G), np.uint8) if G < Gfull else None
    gsel = np.zeros((N, T // sub, S), np.uint8) if want_gsel else None
    init = np.ascontiguousarray(np.asarray(init_st, dtype=np.int32)) if init_st is not None else None
    me = (list(m_extra) + [0, 0, 0])[:3]
    rc = lib().ltq_oracle_tcq_viterbi(
        _p(x), _p(w), _p(tab), _p(gains), _p(rec), _p(init), _p(end), _p(tab_hi_a), _p(g_hi), _p(gcand), _p(best),
        _p(code), _p(mid), mid_t, int(tail), N, T, S, U, G, Gfull, m, sub, U_hi, mix if tab_hi is not None else 0,
        me[0], me[1], me[2], nl, ld, rot, int(pp), _p(gsel), nthreads)
    if rc != 0:
        raise RuntimeError(f"oracle tcq_viterbi: error code {rc}")
    return {"rec": rec, "code": code, "best": best, "end": end, "mid": mid, "gcand": gcand, "gsel": gsel}


def viterbi_ub_cuda_ref(x, small, K, nu, m, gains=None, sub=16, wts=None, init_state=None, return_end_state=False,
                        small_hi=None, gains_hi=None, mix=0, n_cand=0, return_code=False, tail_biting=False,
                        tb_passes=2, tb_cand1=0, tb_window=0, m_extra=(), pair_parity=False, _mid=0, _tail=False,
                        _steps=0, _rot=0, nthreads=0):
    """The reference driver viterbi_ub_cuda (tcq_proto.py:567-657) over the oracle, numpy in / out."""
    x = _f32(x)
    N, ld = x.shape
    if tail_biting:
        T = ld
        h = T // 2
        kw = dict(sub=sub, small_hi=small_hi, gains_hi=gains_hi, mix=mix, n_cand=n_cand, m_extra=m_extra,
                  pair_parity=pair_parity, nthreads=nthreads)
        w_full = None if wts is None else np.ascontiguousarray(
            np.broadcast_to(np.asarray(wts, np.float32).reshape(-1, T), (N, T)))
        kw1 = dict(kw, n_cand=tb_cand1) if tb_cand1 else kw
        if tb_window:
            _, mid = viterbi_ub_cuda_ref(x, small, K, nu, m, gains, wts=w_full, _mid=tb_window, _steps=2 * tb_window,
                                         _rot=h - tb_window, **kw1)
        else:
            _, mid = viterbi_ub_cuda_ref(x, small, K, nu, m, gains, wts=w_full, _mid=h, **kw1)
        shift = 0
        out = None
        for p in range(1, tb_passes):
            shift = (shift + h) % T
            if p + 1 < tb_passes:
                _, mid = viterbi_ub_cuda_ref(x, small, K, nu, m, gains, wts=w_full, init_state=mid, _tail=True, _mid=h,
                                             _rot=shift, **kw)
            else:
                out = viterbi_ub_cuda_ref(x, small, K, nu, m, gains, wts=w_full, init_state=mid,
                                          return_code=return_code, _tail=True, _rot=shift, **kw)
        return out
    S, U = 1 << nu, 1 << (K - 1)
    w = np.ones_like(x) if wts is None else np.ascontiguousarray(
        np.broadcast_to(np.asarray(wts, np.float32).reshape(-1, ld), (N, ld)))
    g = np.ones(1, np.float32) if gains is None else _f32(gains)
    r = tcq_viterbi(x, w, small, g, init_st=init_state, tab_hi=small_hi, gains_hi=gains_hi if small_hi is not None else None,
                    n_cand=n_cand, mid_t=_mid, tail=_tail, S=S, U=U, m=m, sub=sub,
                    mix=mix if small_hi is not None else 0, m_extra=m_extra, steps=_steps, rot=_rot,
                    pp=int(pair_parity), want_code=True, want_end=return_end_state, nthreads=nthreads)
    if _mid:
        return r["rec"], r["mid"]
    if return_code:
        return r["rec"], r["code"] >> 16, r["code"] & 0xFFFF
    return (r["rec"], r["end"]) if return_end_state else r["rec"]


def viterbi_ub_ref(x, small, K, nu, m, gains=None, sub=16, wts=None):
    """The torch reference viterbi_ub's outputs (rec, labels, u, gidx) (tcq_proto.py:363-419), via the oracle.
    viterbi_ub is the free-start, all-gains, 4-subset, integer special case of the kernel semantics."""
    x = _f32(x)
    N, T = x.shape
    U = 1 << (K - 1)
    g = np.ones(1, np.float32) if gains is None else _f32(gains)
    w = np.ones_like(x) if wts is None else np.ascontiguousarray(np.broadcast_to(_f32(wts).reshape(-1, T), (N, T)))
    r = tcq_viterbi(x, w, small, g, S=1 << nu, U=U, m=m, sub=sub if g.size > 1 else sub)
    code = r["code"]
    gi = code >> 16
    idx = code & 0xFFFF
    return r["rec"], idx // U, idx % U, gi[:, ::sub]


def make_gains_ref(h: int, step: float) -> np.ndarray:
    """CPU float32 gains 2^((g - (2^h - 1)/2) * step) (tcq_proto.py:247-249), computed by torch on the CPU."""
    import torch
    G = 1 << h
    return (2.0 ** ((torch.arange(G, dtype=torch.float32) - (G - 1) / 2) * step)).numpy()


def fwht256_ref(x) -> np.ndarray:
    """Normalized block FWHT-256 over the last dimension (iqk_format.py:153-170)."""
    a = _f32(x).copy()
    assert a.shape[-1] % 256 == 0
    lib().ltq_oracle_fwht256(_p(a), a.size // 256)
    return a


def lut_subs_ref(xs, dh, lut, inv_step: float, half_b: float) -> np.ndarray:
    """The reference's lut_subs_quant (tcq_viterbi.cu:768-811) over the oracle: xs, dh [S, 16], lut [nb, 64]."""
    x = np.ascontiguousarray(xs, np.float32).reshape(-1, 16)
    d = np.ascontiguousarray(dh, np.float32).reshape(x.shape)
    t = np.ascontiguousarray(lut, np.float32)
    assert t.shape[1] == 64
    out = np.empty_like(x)
    lib().ltq_oracle_lut_subs(_p(x), _p(d), _p(t), _p(out), x.shape[0], inv_step, half_b, t.shape[0])
    return out


def labels_ref(S=1024, m=359, m_extra=()) -> np.ndarray:
    nl = 4 << len(m_extra)
    me = (list(m_extra) + [0, 0, 0])[:3]
    out = np.zeros(S, np.int32)
    lib().ltq_oracle_labels(S, m, me[0], me[1], me[2], nl, _p(out))
    return out


def step_metrics(x, w, tab, gains, U, nl, pp):
    """[T, G, nl, 2] float32 branch metrics of one tile as the Viterbi uses them (no candidates, no mix)."""
    x, w, tab, gains = _f32(x), _f32(w), _f32(tab), _f32(gains)
    T, G = x.shape[0], gains.size
    E = np.zeros((T, G, nl, 2), np.float32)
    for g in range(G):
        vals = (gains[g] * tab.reshape(nl, U)).astype(np.float32)  # fl(g * tab)
        d = (x[:, None, None] - vals[None]).astype(np.float32)
        dd = (d * d).astype(np.float32)
        if pp:
            for p in range(2):
                E[:, g, :, p] = np.minimum(dd[:, :, p::2].min(axis=2), np.float32(3.4e38)) * w[:, None]
        else:
            E[:, g, :, 0] = np.minimum(dd.min(axis=2), np.float32(3.4e38)) * w[:, None]
    return E


def brute_force(x, w, tab, gains, *, S=1024, U=4, m=359, m_extra=(), sub=16, pp=0, init=-1, tail=False):
    """Exhaustive optimum of one tiny tile (oracle/ltq_brute.c). Returns (cost, states, g per sub-block, low bits)."""
    nl = 4 << len(m_extra)
    E = np.ascontiguousarray(step_metrics(x, w, tab, gains, U, nl, pp))
    T = E.shape[0]
    me = (list(m_extra) + [0, 0, 0])[:3]
    st = np.zeros(T, np.int32)
    gs = np.zeros(T // sub, np.int32)
    lo = np.zeros(T, np.int32)
    c = lib().ltq_brute_force(_p(E), T, S, gains.size, sub, m, me[0], me[1], me[2], nl, pp, init, int(tail), _p(st),
                              _p(gs), _p(lo))
    return c, st, gs, lo
