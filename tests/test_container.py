"""The .ltq container (src/ltq_file.py): writer, reader, spec decoder, assemble.

CPU: the file layout (magic, version, reserve, 4096-aligned data, 64-byte aligned tensors, space-padded JSON
header), every tensor dtype and the header's format description read back exactly.
GPU: the HIP slice decoder reproduces the reference's own decoded values for 12 formats (tests/golden/
packing.npz), and quantize -> LtqWriter.add_matrix (decode-verified) -> LtqFile.decode_matrix gives the
quantizer's reconstruction bit for bit, for a single-format matrix and for row slices of two formats, and at the
benchmark's full C3 size.
"""
import struct

import numpy as np
import pytest

torch = pytest.importorskip("torch")

FORMATS = ["TCQ275X2", "TCQ275X", "TCQ375X", "TCQ25X", "TCQ3X3", "TCQ4X", "TCQ2X0", "TCQ3W2", "TCQ5X", "TCQ3X16",
           "TCQ475X", "TCQ45X"]
RESERVE = 4096 - 16


def test_file_layout_and_tensors_round_trip(tmp_path):
    from ltq_amd.formats import make_format
    from ltq_amd.ltq_file import LtqFile, LtqWriter, format_json, MAGIC, VERSION
    fmts = [make_format("TCQ275X2"), make_format("TCQ4X")]
    p = tmp_path / "t.ltq"
    w = LtqWriter(p, fmts, reserve=RESERVE)
    g = torch.Generator().manual_seed(0)
    ts = {"a.f32": torch.randn((3, 5), generator=g), "b.f16": torch.randn(7, generator=g).half(),
          "c.bf16": torch.randn((2, 9), generator=g).bfloat16(), "d.i8": torch.randint(-100, 100, (11,), dtype=torch.int8),
          "e.u8": torch.randint(0, 255, (13,), dtype=torch.uint8), "f.i32": torch.randint(-9, 9, (4, 4), dtype=torch.int32)}
    for k, v in ts.items():
        w.add_tensor(k, v)
    w.finalize({"quantization": {"formats": [format_json(f) for f in fmts], "bits_per_weight": 2.9}})
    raw = p.read_bytes()
    assert raw[:4] == MAGIC and struct.unpack("<IQ", raw[4:16]) == (VERSION, RESERVE)
    assert raw[16:16 + RESERVE].rstrip(b" ").endswith(b"}")
    lf = LtqFile(p)
    assert lf.data_off == 4096
    for k, v in ts.items():
        assert lf.header["tensors"][k]["offset"] % 64 == 0
        got = lf.tensor(k)
        assert got.dtype == v.dtype and torch.equal(got.view(torch.int16) if v.dtype == torch.bfloat16 else got,
                                                   v.view(torch.int16) if v.dtype == torch.bfloat16 else v)
    for f, r in zip(fmts, lf.formats):
        assert (r.name, r.K, r.frac, r.masks, r.h, r.sub) == (f.name, f.K, f.frac, tuple(f.masks), f.h, f.sub)
        assert np.array_equal(r.lut.view(np.uint32), np.asarray(f.lut, np.float32).view(np.uint32))
        assert np.array_equal(r.gain_tab.view(np.uint32), np.asarray(f.gain_tab, np.float32).view(np.uint32))


def test_header_overflow_is_rejected(tmp_path):
    from ltq_amd.ltq_file import LtqWriter
    w = LtqWriter(tmp_path / "o.ltq", [], reserve=RESERVE)
    with pytest.raises(AssertionError):
        w.finalize({"quantization": {"formats": []}, "pad": "x" * 5000})


# ---------------------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("name", FORMATS)
def test_gpu_decode_slice_matches_reference(golden_dir, name):
    from ltq_amd.formats import make_format
    from ltq_amd.ltq_file import decode_slice
    pk = np.load(golden_dir / "packing.npz")
    f = make_format(name)
    print(f"decode {name}", flush=True)
    dec = decode_slice(pk[f"{name}.bytes"].tobytes(), 32, 512, f, "cuda").cpu().numpy()
    assert np.array_equal(dec.view(np.uint32), pk[f"{name}.decoded"].view(np.uint32))


def _synthetic(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((M, K), generator=g)
    chi2 = sum(torch.randn((M, K), generator=g).square() for _ in range(5))
    W = (z / (chi2 / 5).sqrt()) * 0.02
    X = torch.randn((300, K), generator=g)
    return W, X.T @ X / 300


@pytest.mark.gpu
@pytest.mark.parametrize("specs", ["TCQ275X2", [(0, 32, "TCQ275X2"), (32, 64, "TCQ375X")]])
def test_gpu_quantize_write_read_decode(tmp_path, specs):
    from ltq_amd import liqk
    from ltq_amd.formats import make_format
    from ltq_amd.ltq_file import LtqFile, LtqWriter, format_json
    W, H = _synthetic(64, 512, seed=3)
    print(f"quantize -> .ltq -> decode {specs}", flush=True)
    liqk.PACK = {}
    try:
        q, W_hat, rel = liqk.quantize_matrix_liqk_v2(W.cuda(), H.cuda(), specs, damp=0.02)
        pm = liqk.PACK["matrix"]
    finally:
        liqk.PACK = None
    names = sorted({sp for _, _, sp in pm["row_slices"]})
    fmts = [make_format(n) for n in names]
    p = tmp_path / "m.ltq"
    w = LtqWriter(p, fmts, reserve=RESERVE)
    nbytes = w.add_matrix("layer.w", pm, verify=True)
    w.finalize({"quantization": {"formats": [format_json(f) for f in fmts]}})
    assert nbytes > 0
    Wd = LtqFile(p).decode_matrix("layer.w", device="cuda")
    torch.cuda.synchronize()
    assert torch.equal(Wd.view(torch.int32), W_hat.float().contiguous().view(torch.int32))


@pytest.mark.gpu
def test_gpu_full_c3_write_read_decode(tmp_path):
    """The benchmark's C3 matrix (4096 x 14336 bf16 Student-t with outlier columns, H from 2048 activation rows,
    TCQ275X2) through quantize -> .ltq -> decode at full size (256 row groups x 56 column blocks): the file holds
    M K 2.75 / 8 bytes of codes plus the gain indices and decodes to the quantizer's reconstruction bit for bit."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import bench
    from ltq_amd import liqk
    from ltq_amd.formats import make_format
    from ltq_amd.ltq_file import LtqFile, LtqWriter, format_json
    print("full C3 quantize -> .ltq -> decode", flush=True)
    W, H, _ = bench.prepare(torch.device("cuda"))
    liqk.PACK = {}
    try:
        q, W_hat, rel = liqk.quantize_matrix_liqk_v2(W, H, "TCQ275X2", damp=0.02)
        pm = liqk.PACK["matrix"]
    finally:
        liqk.PACK = None
    del H
    f = make_format("TCQ275X2")
    p = tmp_path / "c3.ltq"
    w = LtqWriter(p, [f], reserve=RESERVE)
    nbytes = w.add_matrix("down_proj", pm, verify=True)
    w.finalize({"quantization": {"formats": [format_json(f)]}})
    M, K = W.shape
    print(f"full C3: {nbytes} bytes, relative proxy loss {rel:.6f}", flush=True)
    assert nbytes >= M * K * 11 // 32
    Wd = LtqFile(p).decode_matrix("down_proj", device="cuda")
    torch.cuda.synchronize()
    assert Wd.shape == (M, K)
    assert torch.equal(Wd.view(torch.int32), W_hat.float().contiguous().view(torch.int32))
