"""Drop-in Python surface of the reference's TCQ Viterbi drivers, running the gfx950 HIP kernels.

Mirrors (same names, argument meaning, return conventions and errors):
  make_gains           src/tcq_proto.py:247-249
  viterbi_ub_cuda      src/tcq_proto.py:567-657 (single pass and the two-pass tail-biting driver :584-609)
  lut_subs_quant_cuda  src/tcq_proto.py:537-548

Every call goes to libltq_hip.so (ltq_amd._lib); there is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib

# timing hook (off by default): a list receives one record per sampled call -- a tail-biting call (both passes)
# or a single pass -- for calls 0, LAUNCH_SAMPLE, 2 LAUNCH_SAMPLE, ... counted from the last reset of
# _launch_count. A record is a dict: "ev" a list of (start, end) event pairs, "tiles", "launches" ((steps, gain
# slots run) of each pass), "pp" (parity mode).
LAUNCH_EVENTS: list | None = None
LAUNCH_SAMPLE = 1
_launch_count = 0
# the hook's event type: None for torch.cuda.Event, one pair recorded on the stream around the whole call; or
# a callable returning an object with `handle` (its hipEvent_t) and elapsed_time(end) in ms, handed to the kernel
# launch itself (ltq_viterbi_timing), which stamps it with the dispatch's own start / end: each kernel launch of
# the call then gets its own pair, so the record holds the kernels' durations and not the dispatch gap between
# two dependent launches.
EVENT_FACTORY = None
_PER_LAUNCH: list | None = None  # pairs of the launches of the sampled call in progress


def _timed_call(fn, tiles, launches, pp, kernels=None):
    """fn() with timing events when the timing hook samples this call. kernels=1: fn issues one kernel launch
    (inside a sampled composite call it then takes its own event pair)."""
    global _launch_count, _PER_LAUNCH
    if _PER_LAUNCH is not None and kernels == 1:
        e0, e1 = EVENT_FACTORY(), EVENT_FACTORY()
        _lib.lib().ltq_viterbi_timing(e0.handle, e1.handle, 1)
        try:
            out = fn()
        finally:
            _lib.lib().ltq_viterbi_timing(None, None, 0)
        _PER_LAUNCH.append((e0, e1))
        return out
    take = LAUNCH_EVENTS is not None and _launch_count % LAUNCH_SAMPLE == 0
    if LAUNCH_EVENTS is not None:
        _launch_count += 1
    if not take:
        return fn()
    if EVENT_FACTORY is not None:
        _PER_LAUNCH = []
        try:
            out = _timed_call(fn, tiles, launches, pp, kernels) if kernels == 1 else fn()
            pairs = _PER_LAUNCH
        finally:
            _PER_LAUNCH = None
    else:
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        out = fn()
        e1.record(st)
        pairs = [(e0, e1)]
    LAUNCH_EVENTS.append({"ev": pairs, "tiles": tiles, "launches": launches, "pp": pp})
    return out


def make_gains(h: int, step: float, device="cuda") -> torch.Tensor:
    """2^((g - (2^h - 1)/2) * step) for g < 2^h, float32 (src/tcq_proto.py:247-249).

    The values are evaluated on the CPU by torch and then moved to `device`, so that the quantizer and the
    .ltq decoder see exactly the same gain table on any device."""
    G = 1 << h
    g = 2.0 ** ((torch.arange(G, dtype=torch.float32) - (G - 1) / 2) * step)
    return g.to(device)


@torch.no_grad()
def lut_subs_quant_cuda(x_subs: torch.Tensor, dh: torch.Tensor, lut_val: torch.Tensor, inv_step: float,
                        half_b: float) -> torch.Tensor:
    """x_subs, dh [S, 16] -> [S, 16]: per 16-weight sub-block, the best of 64 LUT candidates (src/tcq_proto.py:537-548)."""
    assert lut_val.shape[1] == 64
    _lib.require_device(x_subs)
    x = x_subs.float().contiguous()
    d = dh.float().reshape(x.shape).contiguous()
    t = lut_val.float().contiguous()
    out = torch.empty_like(x)
    rc = _lib.lib().lut_subs_quant(x.data_ptr(), d.data_ptr(), t.data_ptr(), out.data_ptr(), x.shape[0], inv_step,
                                   half_b, t.shape[0], _lib.stream_ptr())
    if rc != 0:
        raise RuntimeError(f"lut_subs_quant: HIP error code {rc}" if rc > 0 else "lut_subs_quant: rejected arguments")
    return out


def _rows(wts: torch.Tensor | None, N: int, T: int) -> torch.Tensor | None:
    if wts is None:
        return None
    return (wts.view(1, T).expand(N, T) if wts.dim() == 1 else wts).float().contiguous()


def _tail_biting(x, small, K, nu, m, gains, sub, wts, small_hi, gains_hi, mix, n_cand, return_code, tb_passes,
                 tb_cand1, tb_window, m_extra, pair_parity, _raw_code, _fuse):
    """The two-pass tail-biting driver (src/tcq_proto.py:584-609); the single passes run with the hook off."""
    global LAUNCH_EVENTS
    saved, LAUNCH_EVENTS = LAUNCH_EVENTS, None
    try:
        N, T = x.shape
        h = T // 2
        common = dict(sub=sub, small_hi=small_hi, gains_hi=gains_hi, mix=mix, m_extra=m_extra, pair_parity=pair_parity)
        w_full = _rows(wts, N, T)
        xf = x.float().contiguous()
        # pass 1 only locates the path state in the middle of the tile: over the window [h-w, h+w) when
        # tb_window > 0 (shift + step count, no copies), over the whole tile otherwise
        nc1 = tb_cand1 if tb_cand1 else n_cand
        if tb_passes == 2 and nc1 == n_cand and _fuse:  # both passes in one launch
            fused = (2 * tb_window, h - tb_window, tb_window) if tb_window else (T, 0, h)
            return viterbi_ub_cuda(xf, small, K, nu, m, gains, wts=w_full, n_cand=n_cand, return_code=return_code,
                                   _tail=True, _rot=h % T, _raw_code=_raw_code, _fused=fused, **common)
        if tb_window:
            _, mid = viterbi_ub_cuda(xf, small, K, nu, m, gains, wts=w_full, n_cand=nc1, _mid=tb_window,
                                     _steps=2 * tb_window, _rot=h - tb_window, **common)
        else:
            _, mid = viterbi_ub_cuda(xf, small, K, nu, m, gains, wts=w_full, n_cand=nc1, _mid=h, **common)
        shift, out = 0, None
        for p in range(1, tb_passes):
            shift = (shift + h) % T
            last = p + 1 == tb_passes
            if not last:  # another closed pass, only for its middle state
                _, mid = viterbi_ub_cuda(xf, small, K, nu, m, gains, wts=w_full, n_cand=n_cand, init_state=mid,
                                         _tail=True, _mid=h, _rot=shift, **common)
            else:  # closed pass writing rec / code back at the original positions
                out = viterbi_ub_cuda(xf, small, K, nu, m, gains, wts=w_full, n_cand=n_cand, init_state=mid,
                                      return_code=return_code, _tail=True, _rot=shift, _raw_code=_raw_code,
                                      **common)
        return out
    finally:
        LAUNCH_EVENTS = saved


@torch.no_grad()
def viterbi_ub_cuda(x: torch.Tensor, small: torch.Tensor, K: int, nu: int, m: int, gains: torch.Tensor | None = None,
                    sub: int = 16, wts: torch.Tensor | None = None, init_state: torch.Tensor | None = None,
                    return_end_state: bool = False, small_hi: torch.Tensor | None = None,
                    gains_hi: torch.Tensor | None = None, mix: int = 0, n_cand: int = 0, return_code: bool = False,
                    tail_biting: bool = False, tb_passes: int = 2, tb_cand1: int = 0, tb_window: int = 0,
                    m_extra: tuple = (), pair_parity=False, _mid: int = 0, _tail: bool = False, _steps: int = 0,
                    _rot: int = 0, _raw_code: bool = False, _fuse: bool = False, _fused: tuple | None = None):
    """Joint (gain, trellis) Viterbi over tiles x [N, T] on the GPU; see src/tcq_proto.py:567-583 for the meaning
    of every argument. Returns rec [N, T]; or (rec, gain index, level index) with return_code; or (rec, end
    state) with return_end_state; or (rec, mid state) for an internal first tail-biting pass. _raw_code with
    return_code gives (rec, code) with the kernel's packed int32 code (gain index << 16 | level index).
    _fuse=True runs both tail-biting passes (same gain slots) in one launch (tcq_viterbi_tb, identical results).
    It is off by default: on gfx950 the fused kernel measures ~30 us slower per 4096-tile sub-block than the two
    launches (the pass loop keeps both argument sets live, 140 SGPR spills)."""
    _lib.require_device(x)
    if tail_biting:
        N, T = x.shape
        G_run = n_cand if 0 < n_cand < (gains.numel() if gains is not None else 1) else (
            gains.numel() if gains is not None else 1)
        G1 = tb_cand1 if tb_cand1 else G_run
        launches = [(2 * tb_window if tb_window else T, G1)] + [(T, G_run)] * (tb_passes - 1)
        return _timed_call(lambda: _tail_biting(x, small, K, nu, m, gains, sub, wts, small_hi, gains_hi, mix, n_cand,
                                                return_code, tb_passes, tb_cand1, tb_window, m_extra, pair_parity,
                                                _raw_code, _fuse), N, launches, int(pair_parity))
    N, ld = x.shape
    T = _steps or ld
    S, U = 1 << nu, 1 << (K - 1)
    dev = x.device
    xf = x.float().contiguous()
    w = torch.ones_like(xf) if wts is None else _rows(wts, N, ld)
    g = (gains if gains is not None else torch.ones(1, device=dev)).float().contiguous()
    tab = small.float().contiguous()
    Gfull = g.numel()
    G_run = n_cand if 0 < n_cand < Gfull else Gfull
    rec = torch.empty_like(xf)
    # scratch with the reference's shapes: decision words of the HIP kernel live in bp (and pbits)
    bp = torch.empty((N, T, G_run, S // 32), dtype=torch.int32, device=dev)
    gsel = torch.empty((N, max(T // sub, 1), S), dtype=torch.uint8, device=dev)
    tab_hi = small_hi.float().contiguous() if small_hi is not None else tab
    g_hi = gains_hi.float().contiguous() if gains_hi is not None else g
    init = init_state.to(torch.int32).contiguous() if init_state is not None else None
    end = torch.empty(N, dtype=torch.int32, device=dev) if return_end_state else None
    best = torch.empty(N, dtype=torch.int32, device=dev)
    code = torch.empty((N, ld), dtype=torch.int32, device=dev) if return_code else None
    mid = torch.empty(N, dtype=torch.int32, device=dev) if _mid else None
    pp = int(pair_parity)
    if pp >= 2:
        pbits = torch.empty((N, T // 4, G_run, 9, S // 32), dtype=torch.int32, device=dev)
    elif pp == 1:
        pbits = torch.empty((N, T // 2, G_run, S // 32), dtype=torch.int32, device=dev)
    else:
        pbits = None
    nl = 4 << len(m_extra)
    cand = torch.empty((N, T // sub, G_run), dtype=torch.uint8, device=dev) if G_run < Gfull else None
    me = (list(m_extra) + [0, 0, 0])[:3]
    p = _lib.ptr
    mix_arg = mix if small_hi is not None else 0
    def launch():
        if _fused:  # both tail-biting passes: pass 1's middle states land in mid_buf, the closing pass starts there
            if init_state is not None:
                raise ValueError("the fused tail-biting launch computes its own start states")
            mid_buf = torch.empty(N, dtype=torch.int32, device=dev)
            return _lib.lib().tcq_viterbi_tb(p(xf), p(w), p(tab), p(g), p(rec), p(bp), p(gsel), p(mid_buf), p(end),
                                             p(tab_hi), p(g_hi), p(cand), p(best), p(code), int(_tail), N, T, S, U,
                                             G_run, Gfull, m, sub, tab_hi.numel() // nl, mix_arg, me[0], me[1], me[2],
                                             nl, ld, _rot, p(pbits), pp, _fused[0], _fused[1], _fused[2],
                                             _lib.stream_ptr())
        return _lib.lib().tcq_viterbi(p(xf), p(w), p(tab), p(g), p(rec), p(bp), p(gsel), p(init), p(end), p(tab_hi),
                                      p(g_hi), p(cand), p(best), p(code), p(mid), _mid, int(_tail), N, T, S, U, G_run,
                                      Gfull, m, sub, tab_hi.numel() // nl, mix_arg, me[0], me[1], me[2], nl, ld, _rot,
                                      p(pbits), pp, _lib.stream_ptr())

    rc = _timed_call(launch, N, [(_fused[0], G_run), (T, G_run)] if _fused else [(T, G_run)], pp, kernels=1)
    if rc != 0:
        raise RuntimeError(f"tcq_viterbi: HIP error code {rc}")
    if _mid:
        return rec, mid
    if return_code:
        return (rec, code) if _raw_code else (rec, code >> 16, code & 0xFFFF)
    return (rec, end) if return_end_state else rec
