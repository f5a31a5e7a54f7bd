"""tcq_viterbi_static, the entry point that allocates nothing, against tcq_viterbi on the same inputs.

Both run through the C ABI. For each case the static entry runs twice in a row, the second call on a smaller
input (fewer tiles, and for the tail-biting case fewer steps), and every output (reconstruction, codes, best
index, end / middle states) must equal tcq_viterbi's bit for bit. A call too large for the static array is
refused with -2 before any device work.
"""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

DEV = "cuda"


def _p(t):
    return None if t is None else t.data_ptr()


def _inputs(N, T, K, nl, G, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((N, T), generator=g)
    w = torch.rand((N, T), generator=g) + 0.5
    U = 1 << (K - 1)
    tab = torch.randn(nl * U, generator=g)
    gains = 2.0 ** ((torch.arange(G, dtype=torch.float32) - (G - 1) / 2) * 0.2)
    return x.to(DEV), w.to(DEV), tab.to(DEV), gains.to(DEV)


def _call(static, x, w, tab, gains, *, T, K, nl, G_run, pp, masks, sub=16, init=None, tail=0, mid_t=0, rot=0):
    from ltq_amd import _lib
    L = _lib.lib()
    N, ld = x.shape
    S, U = 1024, 1 << (K - 1)
    Gfull = gains.numel()
    rec = torch.full((N, ld), -1.0, device=DEV)
    code = torch.full((N, ld), -7, dtype=torch.int32, device=DEV)
    best = torch.full((N,), -7, dtype=torch.int32, device=DEV)
    end = torch.full((N,), -7, dtype=torch.int32, device=DEV)
    mid = torch.full((N,), -7, dtype=torch.int32, device=DEV) if mid_t else None
    me = (list(masks[1:]) + [0, 0, 0])[:3]
    args_tail = (mid_t, tail, N, T, S, U, G_run, Gfull, masks[0], sub, U, 0, me[0], me[1], me[2], nl, ld, rot)
    stream = torch.cuda.current_stream().cuda_stream
    if static:
        rc = L.tcq_viterbi_static(_p(x), _p(w), _p(tab), _p(gains), _p(rec), _p(init), _p(end), _p(tab), _p(gains),
                                  _p(best), _p(code), _p(mid), *args_tail, pp, stream)
    else:
        bp = torch.empty((N, T, G_run, S // 32), dtype=torch.int32, device=DEV)
        gsel = torch.empty((N, T // sub, S), dtype=torch.uint8, device=DEV)
        cand = torch.empty((N, T // sub, G_run), dtype=torch.uint8, device=DEV) if G_run < Gfull else None
        pb = None
        if pp >= 2:
            pb = torch.empty((N, T // 4, G_run, 9, S // 32), dtype=torch.int32, device=DEV)
        elif pp == 1:
            pb = torch.empty((N, T // 2, G_run, S // 32), dtype=torch.int32, device=DEV)
        rc = L.tcq_viterbi(_p(x), _p(w), _p(tab), _p(gains), _p(rec), _p(bp), _p(gsel), _p(init), _p(end), _p(tab),
                           _p(gains), _p(cand), _p(best), _p(code), _p(mid), *args_tail, _p(pb), pp, stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    out = {"rec": rec.cpu(), "code": code.cpu(), "best": best.cpu(), "end": end.cpu()}
    if mid is not None:
        out["mid"] = mid.cpu()
    return out


def _same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        av, bv = a[k].numpy(), b[k].numpy()
        if av.dtype == np.float32:
            av, bv = av.view(np.uint32), bv.view(np.uint32)
        assert np.array_equal(av, bv), k


# (name, K, masks, pp, G_run, Gfull): the headline D4 format, D2, integer with gain candidates (C2), 16 subsets
CASES = [("TCQ275X2", 3, (359, 241), 2, 4, 4), ("TCQ25X", 3, (359, 241), 1, 2, 2),
         ("TCQ3X3", 3, (359, 241), 0, 4, 8), ("C4-16sub", 3, (359, 40, 475), 2, 4, 8)]


@pytest.mark.gpu
@pytest.mark.parametrize("name,K,masks,pp,G_run,Gfull", CASES)
def test_gpu_static_entry_matches_tcq_viterbi(name, K, masks, pp, G_run, Gfull):
    nl = 2 << len(masks)
    for call, (N, seed) in enumerate(((256, 1), (40, 2))):
        print(f"no-alloc {name}: call {call + 1}, {N} tiles x 256 steps", flush=True)
        x, w, tab, gains = _inputs(N, 256, K, nl, Gfull, seed)
        kw = dict(T=256, K=K, nl=nl, G_run=G_run, pp=pp, masks=masks)
        _same(_call(True, x, w, tab, gains, **kw), _call(False, x, w, tab, gains, **kw))


@pytest.mark.gpu
def test_gpu_static_entry_two_pass_tail_biting():
    """The two tail-biting passes of src/tcq_proto.py:584-609 (window 32) through the static entry, then a
    smaller closing pass right after (fewer tiles, 128 steps), each against tcq_viterbi."""
    K, masks, pp, G = 3, (359, 241), 2, 4
    nl = 8
    for call, (N, T, seed) in enumerate(((256, 256, 3), (24, 128, 4))):
        print(f"no-alloc tail-biting: call {call + 1}, {N} tiles x {T} steps", flush=True)
        x, w, tab, gains = _inputs(N, T, K, nl, G, seed)
        h, win = T // 2, 32
        kw = dict(K=K, nl=nl, G_run=G, pp=pp, masks=masks)
        p1s = _call(True, x, w, tab, gains, T=2 * win, mid_t=win, rot=h - win, **kw)
        p1r = _call(False, x, w, tab, gains, T=2 * win, mid_t=win, rot=h - win, **kw)
        _same(p1s, p1r)
        init = p1s["mid"].to(DEV)
        p2s = _call(True, x, w, tab, gains, T=T, init=init, tail=1, rot=h, **kw)
        p2r = _call(False, x, w, tab, gains, T=T, init=init, tail=1, rot=h, **kw)
        _same(p2s, p2r)
