"""TEST INFRASTRUCTURE ONLY -- numpy restatement of the .ltq tile bit layout (the checker for the HIP packer).

Only tests/ and __graft_entry__.smoke() use this module; the product path never does.

Reference anchors:
  states_from_codes   src/ltq_format.py:77-86   (tail-biting state of every position from the code bits)
  labels_from_states  src/ltq_format.py:89-93
  pack_tile           src/ltq_format.py:104-124 (codes / planes / lsb / gains fields of one tile or ring)
  decode_tile         src/ltq_format.py:127-147
  slice layout        src/ltq_file.py:67-96     (tile order, four SoA regions on 64-byte boundaries)
  decode_slice        src/ltq_file.py:119-140
"""
from __future__ import annotations

import numpy as np

NU = 10
TILE = 256


def parity(x):
    x = np.asarray(x).astype(np.uint32)
    out = np.zeros_like(x)
    while np.any(x):
        out ^= x & 1
        x = x >> 1
    return out


def states_from_codes(c):
    """s_t = sum_j c[(t - j) mod L] << j for j < 10 (the start continues the end)."""
    c = np.asarray(c).astype(np.uint32)
    L = len(c)
    s = np.zeros(L, np.uint32)
    for j in range(NU):
        s |= np.roll(c, j) << j
    return s


def labels_from_states(s, masks):
    s = np.asarray(s).astype(np.uint32)
    lb = (s & 1) | (parity((s >> 1) & masks[0]) << 1)
    for i, m in enumerate(masks[1:]):
        lb |= parity((s >> 1) & m) << (2 + i)
    return lb


def lsb_words(frac, L=TILE):
    return ({0: L, 1: L // 2, 2: 3 * L // 4}[frac] + 15) // 16


def gain_words(h, sub, L=TILE):
    return (L // sub * h + 15) // 16


def _to_words(bits, n_words):
    """bit j of word w = element 16 w + j."""
    b = np.zeros(n_words * 16, np.uint32)
    b[: len(bits)] = bits
    return (b.reshape(n_words, 16) << np.arange(16, dtype=np.uint32)).sum(axis=1).astype(np.uint16)


def _from_words(words, n_bits):
    w = np.asarray(words).astype(np.uint32)
    return ((w[:, None] >> np.arange(16, dtype=np.uint32)) & 1).reshape(-1)[:n_bits]


def pack_tile(labels, u, gidx, K, frac, h, sub):
    L = len(labels)
    W = L // 16
    labels = np.asarray(labels).astype(np.uint32)
    u = np.asarray(u).astype(np.uint32)
    codes = _to_words(labels & 1, W)
    planes = (np.stack([_to_words((u >> p) & 1, W) for p in range(1, K - 1)]) if K > 2
              else np.zeros((0, W), np.uint16))
    lsb = u & 1
    if frac == 1:
        lsb = lsb[0::2]
    elif frac == 2:
        lsb = lsb.reshape(-1, 4)[:, :3].reshape(-1)
    lsbw = _to_words(lsb, lsb_words(frac, L))
    g = np.asarray(gidx).astype(np.uint32)[::sub]
    gb = ((g[:, None] >> np.arange(h, dtype=np.uint32)) & 1).reshape(-1) if h else np.zeros(0, np.uint32)
    gains = _to_words(gb, gain_words(h, sub, L)) if h else np.zeros(0, np.uint16)
    return {"L": L, "codes": codes, "planes": planes, "lsb": lsbw, "gains": gains}


def decode_tile(f, K, frac, h, sub, masks, lut, gain_tab):
    L = f["L"]
    U = 1 << (K - 1)
    c = _from_words(f["codes"], L)
    lb = labels_from_states(states_from_codes(c), masks)
    if frac == 0:
        lsb = _from_words(f["lsb"], L)
    elif frac == 1:
        lsb = np.repeat(_from_words(f["lsb"], L // 2), 2)
    else:
        b3 = _from_words(f["lsb"], 3 * L // 4).reshape(-1, 3)
        lsb = np.concatenate([b3, b3.sum(axis=1, keepdims=True) & 1], axis=1).reshape(-1)  # even quad sum
    u = lsb.astype(np.uint32)
    for p in range(1, K - 1):
        u |= _from_words(f["planes"][p - 1], L) << p
    if h:
        gb = _from_words(f["gains"], L // sub * h).reshape(-1, h)
        g = (gb << np.arange(h, dtype=np.uint32)).sum(axis=1)
        gain = np.asarray(gain_tab, np.float32)[np.repeat(g, sub)]
    else:
        gain = np.ones(L, np.float32)
    return (gain * np.asarray(lut, np.float32)[lb * U + u]).astype(np.float32)


def tiles(x):
    """[R, K] -> [T, 256]: tile (row group, column block), position t = 16 r + c."""
    R, K = x.shape
    return x.reshape(R // 16, 16, K // 16, 16).transpose(0, 2, 1, 3).reshape(-1, TILE)


def untiles(t, R, K):
    return t.reshape(R // 16, K // 16, 16, 16).transpose(0, 2, 1, 3).reshape(R, K)


def region_sizes(K, frac, h, sub):
    return [16, 16 * max(K - 2, 0), lsb_words(frac) if K > 1 else 0, gain_words(h, sub) if h else 0]


def pack_slice(idx, gi, K, frac, h, sub) -> bytes:
    """[R, K] (label * U + u, gain index) -> the four regions, each starting on a 64-byte boundary."""
    U = 1 << (K - 1)
    ix, g = tiles(np.asarray(idx).astype(np.int64)), tiles(np.asarray(gi).astype(np.int64))
    fields = [pack_tile(t // U, t % U, gg, K, frac, h, sub) for t, gg in zip(ix, g)]
    regs = [np.stack([f["codes"] for f in fields]),
            np.stack([f["planes"].reshape(-1) for f in fields]),
            np.stack([f["lsb"] for f in fields]),
            np.stack([f["gains"] for f in fields])]
    out = bytearray()
    for r in regs:
        out += bytes(((len(out) + 63) // 64) * 64 - len(out))
        out += r.astype(np.uint16).tobytes()
    return bytes(out)


def decode_slice(data, R, Kc, K, frac, h, sub, masks, lut, gain_tab):
    T = (R // 16) * (Kc // 16)
    sizes = region_sizes(K, frac, h, sub)
    regs, off = [], 0
    for n in sizes:
        off = ((off + 63) // 64) * 64
        regs.append(np.frombuffer(bytes(data[off: off + 2 * T * n]), dtype=np.uint16).reshape(T, n) if n else None)
        off += 2 * T * n
    out = np.zeros((T, TILE), np.float32)
    for i in range(T):
        f = {"L": TILE, "codes": regs[0][i], "planes": regs[1][i].reshape(max(K - 2, 0), 16) if regs[1] is not None
             else np.zeros((0, 16), np.uint16), "lsb": regs[2][i], "gains": regs[3][i] if regs[3] is not None else None}
        out[i] = decode_tile(f, K, frac, h, sub, masks, lut, gain_tab)
    return untiles(out, R, Kc)
