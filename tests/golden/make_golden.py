"""Writes the golden fixtures under tests/golden/ from the reference's own pure-torch / numpy functions.

Run in the build container only (the reference tree is not on the GPU box):

    TCQ_NO_COMPILE=1 python tests/golden/make_golden.py /root/reference

It imports only functions whose exact outputs no closed form, invariant or brute force pins:
  - src/tcq_proto.py:363 viterbi_ub      (exact codes incl. torch min/argmin first-index tie rules)
  - src/tcq_proto.py:247 make_gains      (CPU float32 values)
  - src/iqk_format.py:153 fwht_inplace   (bit pattern of the fp32 butterfly tree)
  - src/iqk_format.py:173 make_rademacher_signs (torch CPU generator stream)
  - src/ltq_format.py:104,126 pack_tile / decode_tile, src/ltq_file.py:79,119 pack_slice / decode_slice
    (exact word / byte layout, 64-byte region alignment)
Fixtures are data only (inputs and expected outputs), stored as .npz / .json.
"""
from __future__ import annotations

import json
import os
import sys
import zlib
from pathlib import Path

import numpy as np

os.environ["TCQ_NO_COMPILE"] = "1"
OUT = Path(__file__).resolve().parent


def main(ref_root: str):
    sys.path.insert(0, ref_root)
    import torch
    from src.tcq_proto import viterbi_ub, make_gains
    from src.iqk_format import fwht_inplace, make_rademacher_signs
    from src.ltq_format import LtqFormat, pack_tile, decode_tile, states_from_codes, labels_from_states
    from src.ltq_file import pack_slice, decode_slice

    tables = json.loads((Path(ref_root) / "results" / "tcq_x_tables.json").read_text())

    # ---- make_gains (CPU) for every (h, step) used by a format -----------------------------------
    gains = {}
    for name, t in tables.items():
        key = f"{t['h']}_{t['step']}"
        gains[key] = make_gains(t["h"], t["step"], "cpu").numpy().astype(np.float32).tolist()
    for h, step in ((1, 0.4), (2, 0.3), (3, 0.15), (2, 0.25), (2, 0.4), (0, 0.0)):
        gains[f"{h}_{step}"] = make_gains(h, step, "cpu").numpy().astype(np.float32).tolist()
    (OUT / "gains_cpu.json").write_text(json.dumps(gains, indent=0))

    # ---- Rademacher sign streams ----------------------------------------------------------------
    signs = {}
    for dim, seed in ((256, 4242), (256, 1337), (4096, 1337), (14336, 1337), (2048, 1337), (768, 1337), (512, 7)):
        s = make_rademacher_signs(dim, seed, "cpu").numpy()
        signs[f"{dim}_{seed}"] = np.packbits(s > 0)
    np.savez_compressed(OUT / "signs.npz", **signs)

    # ---- FWHT-256 ---------------------------------------------------------------------------------
    g = torch.Generator().manual_seed(11)
    xf = torch.randn((6, 768), generator=g) * torch.logspace(-3, 3, 768)
    yf = fwht_inplace(xf.clone(), block_size=256)
    np.savez_compressed(OUT / "fwht.npz", x=xf.numpy(), y=yf.numpy())

    # ---- viterbi_ub (integer, 4 subsets, free start, all gains) -----------------------------------
    cases = {}
    luts = {2: [-1.7691, 0.1581, -0.9582, 0.5299, -0.5294, 0.9609, -0.1571, 1.7674],
            3: [-2.1129, -0.5914, 0.0734, 0.7905, -1.4204, -0.4043, 0.2426, 1.0537, -1.0546, -0.2453, 0.4021, 1.4203,
                -0.7924, -0.0751, 0.5916, 2.1165]}
    lut4 = [-2.4689, -1.0897, -0.6307, -0.2814, 0.0376, 0.3596, 0.7259, 1.2576, -1.7803, -0.9513, -0.5342, -0.1954,
            0.1209, 0.448, 0.8359, 1.47, -1.4681, -0.8349, -0.4492, -0.12, 0.1953, 0.5335, 0.9513, 1.7807, -1.2568,
            -0.7259, -0.36, -0.0359, 0.281, 0.6301, 1.0894, 2.4651]
    luts[4] = lut4
    specs = [  # name, K, nu, h, step, sub, N, T, weights, ties
        ("k2_h2", 2, 10, 2, 0.3, 16, 6, 64, None, False),
        ("k3_h1_w", 3, 10, 1, 0.4, 16, 6, 64, "row", False),
        ("k3_h2_wfull", 3, 10, 2, 0.3, 16, 4, 96, "full", False),
        ("k4_h3", 4, 10, 3, 0.15, 16, 4, 64, None, False),
        ("k3_h0", 3, 10, 0, 0.0, 16, 4, 48, None, False),
        ("k3_nu8_h2", 3, 8, 2, 0.3, 16, 6, 64, None, False),
        ("k2_sub8_h1", 2, 10, 1, 0.4, 8, 4, 64, None, False),
        ("k3_ties_h1", 3, 10, 1, 0.4, 16, 6, 64, None, True),
        ("k2_ties_h0", 2, 10, 0, 0.0, 16, 6, 32, None, True),
        ("k4_ties_h2", 4, 8, 2, 0.3, 16, 4, 64, "row", True),
    ]
    for name, K, nu, h, step, sub, N, T, wmode, ties in specs:
        gg = torch.Generator().manual_seed(zlib.crc32(name.encode()))
        x = torch.randn((N, T), generator=gg)
        if ties:  # coarse grid and a symmetric table: many exactly equal metrics and path sums
            x = torch.round(x * 2) / 2
        small = torch.tensor(luts[K], dtype=torch.float32)
        if ties:
            small = torch.round(small * 4) / 4
        gains_t = make_gains(h, step, "cpu") if h > 0 else None
        wts = None
        if wmode == "row":
            wts = (torch.rand((T,), generator=gg) * 2 + 0.25).float()
            if ties:
                wts = torch.round(wts * 2) / 2
        elif wmode == "full":
            wts = (torch.rand((N, T), generator=gg) * 2 + 0.25).float()
        rec, labels, u, gidx = viterbi_ub(x, small, K, nu, 359, gains_t, sub=sub, wts=wts)
        cases[name] = dict(K=K, nu=nu, h=h, step=step, sub=sub, x=x.numpy(), small=small.numpy(),
                           gains=(gains_t.numpy() if gains_t is not None else np.ones(1, np.float32)),
                           wts=(wts.numpy() if wts is not None else np.zeros(0, np.float32)),
                           rec=rec.numpy(), labels=labels.numpy().astype(np.int32), u=u.numpy().astype(np.int32),
                           gidx=gidx.numpy().astype(np.int32))
    flat = {}
    for name, d in cases.items():
        for k, v in d.items():
            flat[f"{name}.{k}"] = np.asarray(v)
    np.savez_compressed(OUT / "viterbi_ub.npz", **flat)

    # ---- tile / ring packing and the container slice layout ---------------------------------------
    pk = {}
    fmts = ["TCQ275X2", "TCQ275X", "TCQ375X", "TCQ25X", "TCQ3X3", "TCQ4X", "TCQ2X0", "TCQ3W2", "TCQ5X", "TCQ3X16",
            "TCQ475X", "TCQ45X"]
    rng = np.random.default_rng(5)
    for name in fmts:
        t = tables[name]
        frac = int(t.get("pp", 0))
        masks = (359,) + tuple(t["m_extra"])
        gt = make_gains(t["h"], t["step"], "cpu").numpy().astype(np.float32)
        f = LtqFormat(name, t["K"], frac, masks, t["h"], float(t["step"]), t.get("sub", 16),
                      np.asarray(t["lut"], np.float32), gt)
        R, Kc = 32, 512
        ntile = (R // 16) * (Kc // 16)
        codes = rng.integers(0, 2, size=(ntile, 256))
        lab = np.stack([labels_from_states(states_from_codes(c), f) for c in codes]).astype(np.int64)
        u = rng.integers(0, f.U, size=(ntile, 256))
        if frac == 1:
            lo = rng.integers(0, 2, size=(ntile, 128))
            u = (u & ~1) | np.repeat(lo, 2, axis=1)
        elif frac == 2:
            lo = rng.integers(0, 2, size=(ntile, 64, 3))
            lo = np.concatenate([lo, lo.sum(axis=2, keepdims=True) & 1], axis=2).reshape(ntile, 256)
            u = (u & ~1) | lo
        gsub = rng.integers(0, 1 << t["h"], size=(ntile, 256 // f.sub)) if t["h"] else np.zeros((ntile, 256 // f.sub), int)
        gi = np.repeat(gsub, f.sub, axis=1)
        idx_t = lab * f.U + u
        # tiles -> [R, K] (position t = 16 r + c of tile (row group, kb)), the inverse of ltq_file._tiles
        idx = idx_t.reshape(R // 16, Kc // 16, 16, 16).transpose(0, 2, 1, 3).reshape(R, Kc)
        gim = gi.reshape(R // 16, Kc // 16, 16, 16).transpose(0, 2, 1, 3).reshape(R, Kc)
        raw = pack_slice(torch.tensor(idx, dtype=torch.int16), torch.tensor(gim, dtype=torch.uint8), f)
        dec = decode_slice(raw, R, Kc, f, "cpu").numpy()
        pk[f"{name}.idx"] = idx.astype(np.int16)
        pk[f"{name}.gi"] = gim.astype(np.uint8)
        pk[f"{name}.bytes"] = np.frombuffer(raw, dtype=np.uint8)
        pk[f"{name}.decoded"] = dec.astype(np.float32)
        # per-tile fields of the first tile, and a 160-long ring for sub = 16 formats
        tf = pack_tile(lab[0], u[0], gi[0], f)
        for k in ("codes", "planes", "lsb", "gains"):
            pk[f"{name}.tile0.{k}"] = np.asarray(tf[k]).astype(np.uint16)
        pk[f"{name}.tile0.decoded"] = decode_tile(tf, f)
        if f.sub == 16:
            L = 160
            c = rng.integers(0, 2, size=L)
            lb = labels_from_states(states_from_codes(c), f).astype(np.int64)
            uu = rng.integers(0, f.U, size=L)
            if frac == 1:
                uu = (uu & ~1) | np.repeat(rng.integers(0, 2, size=L // 2), 2)
            elif frac == 2:
                q = rng.integers(0, 2, size=(L // 4, 3))
                q = np.concatenate([q, q.sum(axis=1, keepdims=True) & 1], axis=1).reshape(L)
                uu = (uu & ~1) | q
            gr = np.repeat(rng.integers(0, 1 << t["h"], size=L // 16) if t["h"] else np.zeros(L // 16, int), 16)
            rf = pack_tile(lb, uu, gr, f)
            pk[f"{name}.ring.lab"] = lb.astype(np.int32)
            pk[f"{name}.ring.u"] = uu.astype(np.int32)
            pk[f"{name}.ring.gi"] = gr.astype(np.int32)
            for k in ("codes", "planes", "lsb", "gains"):
                pk[f"{name}.ring.{k}"] = np.asarray(rf[k]).astype(np.uint16)
            pk[f"{name}.ring.decoded"] = decode_tile(rf, f)
    np.savez_compressed(OUT / "packing.npz", **pk)
    print("golden fixtures written to", OUT)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
