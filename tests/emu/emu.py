"""TEST INFRASTRUCTURE: ctypes driver of the CPU emulation of the gfx950 Viterbi kernel (tests/emu/tcq_emu.cpp).

Same argument convention as the reference ABI tcq_viterbi (src/cuda/tcq_viterbi.cu:743-746) with host
(numpy) buffers, and scratch sized exactly as the reference driver allocates it (src/tcq_proto.py:621-640)."""
from __future__ import annotations

import ctypes
import fcntl
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB = {}


def build(asan: bool = False) -> Path:
    """Compile the emulator library; written under a temporary name and renamed, so a concurrent loader never
    maps a half-written file."""
    so = _DIR / ("libtcq_emu_asan.so" if asan else "libtcq_emu.so")
    tmp = so.with_name(f"{so.name}.{os.getpid()}.tmp")
    cmd = ["g++", "-std=c++20", "-O1" if asan else "-O2", "-g", "-fPIC", "-shared", "-ffp-contract=off",
           "-fno-fast-math", "-pthread", "-o", str(tmp), str(_DIR / "tcq_emu.cpp")]
    if asan:
        cmd.insert(1, "-fsanitize=address")
    try:
        subprocess.run(cmd, check=True)
        os.replace(tmp, so)
    finally:
        tmp.unlink(missing_ok=True)
    return so


def lib(asan: bool = False):
    if asan not in _LIB:
        so = _DIR / ("libtcq_emu_asan.so" if asan else "libtcq_emu.so")
        srcs = (_DIR / "tcq_emu.cpp", _DIR.parent.parent / "ltq-research_amd" / "csrc" / "tcq_trellis.h")
        with open(_DIR / ".build.lock", "w") as lk:  # one rebuild among parallel test workers
            fcntl.flock(lk, fcntl.LOCK_EX)
            if not so.exists() or so.stat().st_mtime < max(f.stat().st_mtime for f in srcs):
                build(asan)  # missing, or older than the kernel body it emulates
        L = ctypes.CDLL(str(so))
        L.tcq_viterbi_emu.restype = ctypes.c_int
        L.tcq_viterbi_emu.argtypes = [ctypes.c_void_p] * 15 + [ctypes.c_int] * 18 + [ctypes.c_void_p, ctypes.c_int]
        L.tcq_needed_words_emu.restype = ctypes.c_long
        L.tcq_needed_words_emu.argtypes = [ctypes.c_int] * 4
        L.tcq_viterbi_compact_emu.restype = ctypes.c_int
        L.tcq_viterbi_compact_emu.argtypes = [ctypes.c_void_p] * 12 + [ctypes.c_int] * 16 + [ctypes.c_long]
        L.tcq_viterbi_tb_emu.restype = ctypes.c_int
        L.tcq_viterbi_tb_emu.argtypes = [ctypes.c_void_p] * 14 + [ctypes.c_int] * 17 + [ctypes.c_void_p] + [ctypes.c_int] * 4
        _LIB[asan] = L
    return _LIB[asan]


def _p(a):
    return None if a is None else a.ctypes.data


def tcq_viterbi(x, w, tab, gains, *, init_st=None, tab_hi=None, gains_hi=None, n_cand=0, mid_t=0, tail=False,
                S=1024, U=None, m=359, sub=16, mix=0, m_extra=(), steps=0, rot=0, pp=0, asan=False):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    N, ld = x.shape
    T = steps or ld
    nl = 4 << len(m_extra)
    tab = np.ascontiguousarray(tab, np.float32)
    gains = np.ascontiguousarray(gains, np.float32)
    U = tab.size // nl if U is None else U
    tab_hi_a = np.ascontiguousarray(tab_hi, np.float32) if tab_hi is not None else tab
    g_hi = np.ascontiguousarray(gains_hi, np.float32) if gains_hi is not None else gains
    Gfull = gains.size
    G = n_cand if 0 < n_cand < Gfull else Gfull
    rec = np.zeros((N, ld), np.float32)
    bp = np.zeros((N, T, G, S // 32), np.int32)
    gsel = np.zeros((N, max(T // sub, 1), S), np.uint8)
    best = np.zeros(N, np.int32)
    code = np.zeros((N, ld), np.int32)
    end = np.zeros(N, np.int32)
    mid = np.zeros(N, np.int32) if mid_t else None
    cand = np.zeros((N, T // sub, G), np.uint8) if G < Gfull else None
    if pp >= 2:
        pbits = np.zeros((N, T // 4, G, 9, S // 32), np.int32)
    elif pp == 1:
        pbits = np.zeros((N, T // 2, G, S // 32), np.int32)
    else:
        pbits = None
    init = np.ascontiguousarray(init_st, np.int32) if init_st is not None else None
    me = (list(m_extra) + [0, 0, 0])[:3]
    rc = lib(asan).tcq_viterbi_emu(
        _p(x), _p(w), _p(tab), _p(gains), _p(rec), _p(bp), _p(gsel), _p(init), _p(end), _p(tab_hi_a), _p(g_hi),
        _p(cand), _p(best), _p(code), _p(mid), mid_t, int(tail), N, T, S, U, G, Gfull, m, sub,
        tab_hi_a.size // nl, mix if tab_hi is not None else 0, me[0], me[1], me[2], nl, ld, rot, _p(pbits), int(pp))
    if rc != 0:
        raise RuntimeError(f"tcq_viterbi_emu: error code {rc}")
    return {"rec": rec, "code": code, "best": best, "end": end, "mid": mid, "gcand": cand}


def tcq_viterbi_tb(x, w, tab, gains, *, n_cand=0, S=1024, U=None, m=359, sub=16, m_extra=(), pp=0, window=0,
                   asan=False):
    """Both tail-biting passes in one emulated launch (the fused entry point): pass 1 over the window
    [h - window, h + window) (the whole tile when window is 0) for the middle state, then the closed pass from it
    at rotation h. Returns rec, code and the closing pass's best (g, s)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    N, T = x.shape
    h = T // 2
    nl = 4 << len(m_extra)
    tab = np.ascontiguousarray(tab, np.float32)
    gains = np.ascontiguousarray(gains, np.float32)
    U = tab.size // nl if U is None else U
    Gfull = gains.size
    G = n_cand if 0 < n_cand < Gfull else Gfull
    rec = np.zeros((N, T), np.float32)
    bp = np.zeros((N, T, G, S // 32), np.int32)
    gsel = np.zeros((N, max(T // sub, 1), S), np.uint8)
    best = np.zeros(N, np.int32)
    code = np.zeros((N, T), np.int32)
    mid = np.zeros(N, np.int32)
    cand = np.zeros((N, T // sub, G), np.uint8) if G < Gfull else None
    if pp >= 2:
        pbits = np.zeros((N, T // 4, G, 9, S // 32), np.int32)
    elif pp == 1:
        pbits = np.zeros((N, T // 2, G, S // 32), np.int32)
    else:
        pbits = None
    me = (list(m_extra) + [0, 0, 0])[:3]
    steps1, rot1, mid1 = (2 * window, h - window, window) if window else (T, 0, h)
    rc = lib(asan).tcq_viterbi_tb_emu(
        _p(x), _p(w), _p(tab), _p(gains), _p(rec), _p(bp), _p(gsel), _p(mid), None, _p(tab), _p(gains), _p(cand),
        _p(best), _p(code), 1, N, T, S, U, G, Gfull, m, sub, U, 0, me[0], me[1], me[2], nl, T, h % T, _p(pbits),
        int(pp), steps1, rot1, mid1)
    if rc != 0:
        raise RuntimeError(f"tcq_viterbi_tb_emu: error code {rc}")
    return {"rec": rec, "code": code, "best": best}


def tcq_viterbi_compact(x, w, tab, gains, *, init_st=None, n_cand=0, mid_t=0, tail=False, S=1024, m=359, sub=16,
                        m_extra=(), steps=0, rot=0, pp=0, guard=4096, asan=False):
    """The kernel body with the compact decision-scratch window of tcq_viterbi_static: tile_words = the words a
    tile needs rounded up to 64, the buffer exactly N * tile_words words plus `guard` sentinel words after it.
    Returns (the tcq_viterbi-style result dict, whether every guard word is untouched)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    N, ld = x.shape
    T = steps or ld
    nl = 4 << len(m_extra)
    tab = np.ascontiguousarray(tab, np.float32)
    gains = np.ascontiguousarray(gains, np.float32)
    U = tab.size // nl
    Gfull = gains.size
    G = n_cand if 0 < n_cand < Gfull else Gfull
    L = lib(asan)
    need = L.tcq_needed_words_emu(T, S, G, pp)
    assert need > 0
    tw = (need + 63) // 64 * 64
    bp = np.full(N * tw + guard, 0xDEADBEEF, np.uint32)
    rec = np.zeros((N, ld), np.float32)
    code = np.zeros((N, ld), np.int32)
    best = np.zeros(N, np.int32)
    end = np.zeros(N, np.int32)
    mid = np.zeros(N, np.int32) if mid_t else None
    gcand = np.zeros((N, T // sub, G), np.uint8) if G < Gfull else None
    init = np.ascontiguousarray(np.asarray(init_st, dtype=np.int32)) if init_st is not None else None
    me = (list(m_extra) + [0, 0])[:2]
    rc = L.tcq_viterbi_compact_emu(_p(x), _p(w), _p(tab), _p(gains), _p(rec), _p(bp), _p(init), _p(end), _p(gcand),
                                   _p(best), _p(code), _p(mid), mid_t, int(tail), N, T, S, U, G, Gfull, m, sub, nl,
                                   me[0], me[1], ld, rot, int(pp), tw)
    if rc != 0:
        raise RuntimeError(f"emulated compact tcq_viterbi: error code {rc}")
    guard_ok = bool(np.all(bp[N * tw:] == 0xDEADBEEF))
    return {"rec": rec, "code": code, "best": best, "end": end, "mid": mid}, guard_ok
