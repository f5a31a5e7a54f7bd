"""Ring mode for row tables (src/ple_quant.py:28-67) and ring records (src/ltq_format.py:42-50, 104-147).

CPU: the oracle's ring fields and decode reproduce the reference's own 160-value rings for the 11 formats with a
gain per 16 values (tests/golden/packing.npz); the oracle ring quantizer keeps, per ring, the scale with the
lowest error and its packed fields decode to its values.
GPU: the HIP ring packer writes the reference's fields byte for byte; quantize_rings agrees with the oracle
(bit-exact codes and table wherever the fp16 ring scales agree) with and without the rotation; the packed ring
records decode exactly to the returned table.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

DEV = "cuda"
RING_FORMATS = ["TCQ275X2", "TCQ275X", "TCQ375X", "TCQ25X", "TCQ3X3", "TCQ4X", "TCQ2X0", "TCQ3X16", "TCQ5X",
                "TCQ475X", "TCQ45X"]


@pytest.fixture(scope="module")
def pk(golden_dir):
    return np.load(golden_dir / "packing.npz")


def _table(rows, cols, seed):
    """C5-like rows: N(0, 0.02^2) times a per-row log-normal(0, 0.5) norm."""
    g = torch.Generator().manual_seed(seed)
    W = torch.randn((rows, cols), generator=g) * 0.02
    W *= torch.exp(0.5 * torch.randn((rows, 1), generator=g))
    return W.to(torch.bfloat16)


def _fields_bytes(f):
    return np.concatenate([np.asarray(f[k], np.uint16).reshape(-1) for k in ("codes", "planes", "lsb", "gains")])


@pytest.mark.parametrize("name", RING_FORMATS)
def test_oracle_ring_fields_match_reference(pk, name):
    from oracle import pack
    from ltq_amd.formats import make_format
    f = make_format(name)
    lab, u, gi = pk[f"{name}.ring.lab"], pk[f"{name}.ring.u"], pk[f"{name}.ring.gi"]
    assert len(lab) == 160
    tf = pack.pack_tile(lab, u, gi, f.K, f.frac, f.h, f.sub)
    for k in ("codes", "planes", "lsb", "gains"):
        assert np.array_equal(np.asarray(tf[k]).astype(np.uint16), pk[f"{name}.ring.{k}"]), k
    dec = pack.decode_tile(tf, f.K, f.frac, f.h, f.sub, f.masks, f.lut, f.gain_tab)
    assert np.array_equal(dec.view(np.uint32), pk[f"{name}.ring.decoded"].view(np.uint32))
    assert 2 * len(_fields_bytes(tf)) == f.tile_bytes(160)


def test_oracle_rings_choose_lowest_error_and_decode():
    """Per ring the oracle keeps the first scale with the lowest error; its codes pack and decode to its values."""
    from oracle import pack, ple_ref
    from ltq_amd.formats import TCQ_CONFIG, make_format
    name = "TCQ375X"
    f, cfg = make_format(name), TCQ_CONFIG[name]
    W = _table(4, 512, seed=3)
    scales = (0.9, 1.0, 1.12)
    table, d, code, u = ple_ref.quantize_rings_ref(W, cfg, f, rot=False, scales=scales)
    x = W.reshape(-1, 256).float()
    rms = x.square().mean(dim=1, keepdim=True).sqrt().clamp(min=1e-8) * cfg["scale"]
    cand = torch.stack([(rms * s).half().float().squeeze(1) for s in scales], 1)
    assert all(float(d[i]) in cand[i].tolist() for i in range(len(d)))
    assert torch.equal(table, (u * d.float().unsqueeze(1)).to(torch.bfloat16).view_as(W))
    for i in range(code.shape[0]):
        c = code[i].numpy().astype(np.int64)
        ix, gi = c & 0xFFFF, c >> 16
        tf = pack.pack_tile(ix // f.U, ix % f.U, gi, f.K, f.frac, f.h, f.sub)
        dec = pack.decode_tile(tf, f.K, f.frac, f.h, f.sub, f.masks, f.lut, f.gain_tab)
        assert np.array_equal(dec.view(np.uint32), u[i].numpy().view(np.uint32))


# ---------------------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("name", RING_FORMATS)
def test_gpu_ring_pack_matches_reference_fields(pk, name):
    from ltq_amd.formats import make_format
    from ltq_amd.ltq_file import pack_rings_device, ring_bytes
    f = make_format(name)
    print(f"ring pack {name}", flush=True)
    lab, u, gi = (torch.from_numpy(pk[f"{name}.ring.{k}"].astype(np.int64)) for k in ("lab", "u", "gi"))
    idx = (lab * f.U + u).view(1, 160)
    rows = torch.cat([idx, idx.roll(16, 1), idx.flip(1)], 0)  # three different rings
    gis = torch.cat([gi.view(1, 160)] * 3, 0)
    out = pack_rings_device(rows.to(DEV), gis.to(DEV), f).cpu().numpy()
    torch.cuda.synchronize()
    assert out.shape == (3, ring_bytes(160, f)) == (3, f.tile_bytes(160))
    want = _fields_bytes({k: pk[f"{name}.ring.{k}"] for k in ("codes", "planes", "lsb", "gains")})
    assert np.array_equal(out[0].view(np.uint16), want)
    from oracle import pack
    for r in (1, 2):
        ix = rows[r].numpy()
        g = gis[r].numpy()
        tf = pack.pack_tile(ix // f.U, ix % f.U, g, f.K, f.frac, f.h, f.sub)
        assert np.array_equal(out[r].view(np.uint16), _fields_bytes(tf))


@pytest.mark.gpu
@pytest.mark.parametrize("name,rot", [("TCQ375X", True), ("TCQ375X", False), ("TCQ4X", True), ("TCQ275X2", True)])
def test_gpu_quantize_rings_vs_oracle(name, rot):
    from oracle import pack, ple_ref
    from ltq_amd import ple_quant
    from ltq_amd.formats import TCQ_CONFIG, make_format
    f, cfg = make_format(name), TCQ_CONFIG[name]
    W = _table(32, 1024, seed=7)  # 128 rings
    print(f"quantize_rings {name} rot={rot}", flush=True)
    table, bpv, packed, d = ple_quant.quantize_rings_packed(W, name, rot, chunk=48)
    table2, bpv2 = ple_quant.quantize_rings(W.to(DEV), name, rot)
    torch.cuda.synchronize()
    assert table.dtype == W.dtype and table.device == W.device and table2.is_cuda
    assert bpv == bpv2 == f.tile_bytes() * 8 / 256 + 16 / 256
    assert torch.equal(table, table2.cpu())
    t_ref, d_ref, code_ref, u_ref = ple_ref.quantize_rings_ref(W, cfg, f, rot)
    d, packed = d.cpu(), packed.cpu().numpy()
    same_d = d == d_ref
    assert same_d.float().mean().item() >= 0.98
    rows_same = same_d.nonzero().flatten().tolist()
    for i in rows_same:
        dec = pack.decode_tile({"L": 256, **_split_fields(packed[i], f)}, f.K, f.frac, f.h, f.sub, f.masks, f.lut,
                               f.gain_tab)
        assert np.array_equal(dec.view(np.uint32), u_ref[i].numpy().view(np.uint32)), i
    tr = table.reshape(-1, 256)
    trr = t_ref.reshape(-1, 256)
    if rot:  # the inverse rotation mixes a ring's values only within the ring
        assert torch.equal(tr[rows_same], trr[rows_same])
    else:
        assert torch.equal(tr[same_d], trr[same_d])


def _split_fields(rec, f, L=256):
    w = rec.view(np.uint16)
    n = [L // 16, L // 16 * max(f.K - 2, 0), f.lsb_words(L) if f.K > 1 else 0, f.gain_words(L) if f.h else 0]
    o = np.cumsum([0] + n)
    return {"codes": w[o[0]:o[1]], "planes": w[o[1]:o[2]].reshape(max(f.K - 2, 0), L // 16), "lsb": w[o[2]:o[3]],
            "gains": w[o[3]:o[4]]}


@pytest.mark.gpu
@pytest.mark.parametrize("rot", [False, True])
def test_gpu_ring_records_decode_to_table(rot):
    """The '0 decode mismatches' bar for rings: record i decoded, times fp16 scale i, (inverse-rotated) is the
    returned table's ring i, bit for bit."""
    from oracle import pack, ref
    from ltq_amd import ple_quant
    from ltq_amd.formats import make_format
    name = "TCQ375X"
    f = make_format(name)
    W = _table(64, 2560, seed=11)  # 640 rings, 10 per row as in a 2560-wide table
    print(f"ring records decode rot={rot}", flush=True)
    table, _, packed, d = ple_quant.quantize_rings_packed(W.to(DEV), name, rot)
    torch.cuda.synchronize()
    packed, d, table = packed.cpu().numpy(), d.cpu().float(), table.cpu().reshape(-1, 256)
    vals = np.stack([pack.decode_tile({"L": 256, **_split_fields(packed[i], f)}, f.K, f.frac, f.h, f.sub, f.masks,
                                      f.lut, f.gain_tab) for i in range(packed.shape[0])])
    rec = torch.from_numpy(vals) * d.unsqueeze(1)
    if rot:
        rec = torch.from_numpy(ref.fwht256_ref(rec.numpy())) * ple_quant.hadamard_signs()
    assert torch.equal(rec.to(torch.bfloat16), table)
