"""The C ABI: libltq_hip.so loads on a machine without a GPU and exports every function include/*.h declares,
with the argument counts the Python loader binds (no compute calls here)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declarations():
    out = {}
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(?:int|long)\s+(\w+)\s*\(([^;{]*)\)\s*;", text):
            args = [a for a in m.group(2).replace("\n", " ").split(",") if a.strip() and a.strip() != "void"]
            out[m.group(1)] = len(args)
    return out


def test_header_declares_entry_points():
    decl = _declarations()
    assert {"tcq_viterbi", "ltq_fwht256_rows", "ltq_fwht256_cols", "ltq_pack_slice", "ltq_slice_bytes"} <= set(decl)
    assert decl["tcq_viterbi"] == 36  # the reference's ctypes binding: 15 pointers, 18 ints, pbits, pp, stream


def test_library_exports_every_declared_symbol():
    from ltq_amd import _lib
    so = ROOT / "ltq-research_amd" / "ltq_amd" / "libltq_hip.so"
    if not so.exists():
        pytest.skip("libltq_hip.so not built (run __graft_entry__.build())")
    L = ctypes.CDLL(str(so))
    for name, nargs in _declarations().items():
        assert hasattr(L, name), f"{name} declared in include/ but not exported"
        assert name in _lib.SIGNATURES, f"{name} not bound by ltq_amd._lib"
        assert len(_lib.SIGNATURES[name][1]) == nargs, name


def test_product_path_fails_loudly_without_device():
    """No CPU fallback: on a machine without a HIP device every kernel entry raises."""
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a device is present")
    from ltq_amd import _lib
    from ltq_amd.rotation import fwht_rows
    from ltq_amd.tcq_proto import viterbi_ub_cuda
    with pytest.raises(_lib.LtqLibraryMissing):
        fwht_rows(torch.zeros((1, 256)))
    with pytest.raises(_lib.LtqLibraryMissing):
        viterbi_ub_cuda(torch.zeros((1, 32)), torch.zeros(16), 3, 10, 359)


def test_hessian_entry_points_reject_bad_arguments_without_a_device():
    """ltq_cov_accumulate / ltq_cov_finalize validate their arguments before any device call (-1)."""
    from ltq_amd import _lib
    so = ROOT / "ltq-research_amd" / "ltq_amd" / "libltq_hip.so"
    if not so.exists():
        pytest.skip("libltq_hip.so not built (run __graft_entry__.build())")
    L = ctypes.CDLL(str(so))
    for name, (res, args) in _lib.SIGNATURES.items():
        if name.startswith("ltq_cov"):
            getattr(L, name).restype, getattr(L, name).argtypes = res, args
    buf = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    acc, fin = L.ltq_cov_accumulate, L.ltq_cov_finalize
    assert acc(buf, -1, 8, 8, 0, buf, 8, None) == -1     # negative rows
    assert acc(buf, 4, 0, 8, 0, buf, 8, None) == -1      # K < 1
    assert acc(buf, 4, 8, 7, 0, buf, 8, None) == -1      # ldx < K
    assert acc(buf, 4, 8, 8, 2, buf, 8, None) == -1      # element type flag
    assert acc(buf, 4, 8, 8, 0, None, 8, None) == -1     # no H
    assert acc(None, 4, 8, 8, 0, buf, 8, None) == -1     # rows but no X
    assert acc(None, 0, 8, 8, 0, buf, 8, None) == 0      # n == 0: nothing to add
    assert fin(buf, 0, 8, 1.0, buf, 8, None) == -1
    assert fin(buf, 8, 7, 1.0, buf, 8, None) == -1
    assert fin(None, 8, 8, 1.0, buf, 8, None) == -1


def test_static_entry_refuses_oversized_calls_before_device_work():
    """tcq_viterbi_static checks its scratch need against the static array first: an oversized call returns -2
    without touching a device (this machine has none), and an invalid one -1."""
    from ltq_amd import _lib
    so = ROOT / "ltq-research_amd" / "ltq_amd" / "libltq_hip.so"
    if not so.exists():
        pytest.skip("libltq_hip.so not built (run __graft_entry__.build())")
    L = _lib.lib()
    cap = L.tcq_viterbi_static_bytes()
    assert cap == 96 << 20
    fake = 4096  # stand-in addresses: the call must return before using them
    # TCQ275X2's closing pass needs 320 KiB per tile: 1000 tiles do not fit
    args = [fake] * 5 + [None, None, fake, fake, fake, fake, None]
    ints = [0, 1, 1000, 256, 1024, 4, 4, 4, 359, 16, 4, 0, 241, 0, 0, 8, 256, 128]
    assert L.tcq_viterbi_static(*args, *ints, 2, None) == -2
    ints[2] = 300  # 300 tiles fit; but T not a multiple of sub is invalid -> -1 (still before any device call)
    ints[3] = 250
    ints[16] = 256
    assert L.tcq_viterbi_static(*args, *ints, 2, None) == -1


# tcq_viterbi's integer arguments, in order (the reference's ctypes binding, src/cuda/tcq_viterbi.cu:743-746)
_VIT_INTS = ("mid_t", "tail", "N", "T", "S", "U", "G", "Gfull", "m", "sub", "U_hi", "mix", "m2", "m3", "m4", "nl",
             "ld", "rot")
_MAX = 4 * 128  # nl * U and nl * U_hi limit: 4 * MAX_U (tcq_viterbi.cu:17, 750)

# (change to TCQ275X2's closing-pass arguments, whether the reference accepts it). Clauses of
# src/cuda/tcq_viterbi.cu:748-751 (argument checks), 721-728 (G in {1, 2, 3, 4, 8}) and 763 (S in {256, 1024}).
_VIT_RULES = [
    ({}, True),
    ({"G": 17}, False),                                   # G > MAX_G
    ({"Gfull": 17, "gcand": True}, False),                # Gfull > MAX_G
    ({"Gfull": 8}, False),                                # candidates (Gfull != G) without gcand
    ({"Gfull": 8, "gcand": True}, True),
    ({"U": 129}, False),                                  # U > MAX_U
    ({"U_hi": 129}, False),                               # U_hi > MAX_U
    ({"T": 248}, False),                                  # T % sub != 0
    ({"sub": 6, "T": 36, "ld": 36, "pp": 0}, True),
    ({"sub": 3, "T": 36, "ld": 36, "pp": 0}, False),      # odd sub
    ({"sub": 8, "T": 264, "ld": 264}, False),             # T / sub > MAX_SUBS
    ({"sub": 32, "T": 544, "ld": 544}, False),            # T > MAX_T
    ({"sub": 32, "T": 512, "ld": 512}, True),
    ({"sub": 34, "T": 68, "ld": 68, "pp": 0}, False),     # sub > 32
    ({"nl": 32, "U": 1, "U_hi": 1, "sub": 32, "T": 256}, False),  # sub * G * nl * 2 > 4096 with pair parity
    ({"nl": 32, "U": 1, "U_hi": 1, "sub": 32, "T": 256, "pp": 0, "G": 4}, True),  # 4096 without it
    ({"S": 256, "nl": 4, "U": 8, "U_hi": 8}, False),      # pair parity needs S = 1024
    ({"S": 256, "nl": 4, "U": 8, "U_hi": 8, "pp": 0}, True),
    ({"S": 256, "pp": 0}, False),                         # S != 1024 needs nl = 4
    ({"S": 512, "nl": 4, "U": 8, "U_hi": 8, "pp": 0}, False),  # S neither 1024 nor 256
    ({"mix": 1}, False),                                  # pair parity with a mixed table
    ({"sub": 18, "T": 36, "ld": 36}, False),              # D4 (pp >= 2) needs sub % 4 == 0
    ({"sub": 18, "T": 36, "ld": 36, "pp": 1}, True),
    ({"pp": 4}, False),                                   # pp > 3
    ({"nl": 12}, False),                                  # nl not in {4, 8, 16, 32}
    ({"ld": 255}, False),                                 # ld < T
    ({"U": 65}, False),                                   # nl * U > 4 * MAX_U
    ({"U": 64}, True),
    ({"U_hi": 65}, False),                                # nl * U_hi > 4 * MAX_U
    ({"G": 5, "Gfull": 5}, False),                        # no kernel for G = 5
    ({"G": 8, "Gfull": 8}, True),
]


@pytest.mark.parametrize("change,accepted", _VIT_RULES, ids=[str(c) for c, _ in _VIT_RULES])
def test_viterbi_argument_rules_match_the_reference_without_a_device(change, accepted):
    """tcq_viterbi accepts and rejects the argument sets the reference does, before any device call: with N = 0 an
    accepted set gets the zero-block launch's error (hipErrorInvalidConfiguration, 9, as CUDA's 9 for the
    reference's <<<0, ...>>> launch) and a rejected one -1."""
    from ltq_amd import _lib
    so = ROOT / "ltq-research_amd" / "ltq_amd" / "libltq_hip.so"
    if not so.exists():
        pytest.skip("libltq_hip.so not built (run __graft_entry__.build())")
    L = _lib.lib()
    v = dict(mid_t=0, tail=1, N=0, T=256, S=1024, U=4, G=4, Gfull=4, m=359, sub=16, U_hi=4, mix=0, m2=241, m3=0, m4=0,
             nl=8, ld=256, rot=128, pp=2, gcand=False)
    v.update(change)
    assert v["nl"] * v["U"] <= _MAX or not accepted
    fake = 4096  # stand-in addresses: every call here returns before using them
    ptrs = [fake] * 5 + [fake, None, None, None, None, None, fake if v["gcand"] else None, fake, None, None]
    rc = L.tcq_viterbi(*ptrs, *[v[k] for k in _VIT_INTS], fake, v["pp"], None)
    assert rc == (9 if accepted else -1)
    # with no tiles, empty torch buffers arrive as null pointers: still the zero-block launch's error, not -1
    if accepted:
        nulls = [fake, fake, fake, fake, None, None, None, None, None, None, None, fake if v["gcand"] else None, None,
                 None, None]
        assert L.tcq_viterbi(*nulls, *[v[k] for k in _VIT_INTS], None, v["pp"], None) == 9
    # a negative tile count is rejected outright
    if accepted:
        v["N"] = -1
        assert L.tcq_viterbi(*ptrs, *[v[k] for k in _VIT_INTS], fake, v["pp"], None) == -1


def test_lut_subs_argument_rules_without_a_device():
    """lut_subs_quant: no sub-blocks is the reference's zero-block launch, CUDA / HIP error 9, which its caller
    raises on (src/cuda/tcq_viterbi.cu:806-811, src/tcq_proto.py:544-547); a negative count or an empty table -1.
    All three return before any device call."""
    from ltq_amd import _lib
    so = ROOT / "ltq-research_amd" / "ltq_amd" / "libltq_hip.so"
    if not so.exists():
        pytest.skip("libltq_hip.so not built (run __graft_entry__.build())")
    L = _lib.lib()
    fake = 4096
    assert L.lut_subs_quant(fake, fake, fake, fake, 0, 1.0, 8.0, 16, None) == 9
    assert L.lut_subs_quant(fake, fake, fake, fake, -1, 1.0, 8.0, 16, None) == -1
    assert L.lut_subs_quant(fake, fake, fake, fake, 4, 1.0, 8.0, 0, None) == -1


@pytest.mark.parametrize("K,frac,h,sub", [(2, 1, 0, 32), (3, 2, 2, 16), (3, 1, 3, 32), (4, 0, 4, 64), (5, 2, 8, 16),
                                          (8, 1, 5, 256), (4, 1, 3, 4)])
def test_slice_bytes_equal_the_oracle_layout_without_a_device(K, frac, h, sub):
    """ltq_slice_bytes (what the packer and the decoder size their buffers by) equals the length of the oracle's
    packed slice (src/ltq_file.py:79-102: four regions, each on a 64-byte boundary) for ragged row-group and
    column-block counts; sizes off the 16 x 16 tile grid, negative sizes and unknown formats are -1."""
    from ltq_amd import _lib
    from oracle import pack
    so = ROOT / "ltq-research_amd" / "ltq_amd" / "libltq_hip.so"
    if not so.exists():
        pytest.skip("libltq_hip.so not built (run __graft_entry__.build())")
    L = _lib.lib()
    rng = np.random.default_rng(K * 100 + sub)
    for R, Kc in ((16, 16), (48, 16 * 37), (32, 256)):
        idx = rng.integers(0, 1 << 15, (R, Kc)).astype(np.int16)
        gi = rng.integers(0, 256, (R, Kc)).astype(np.uint8)
        assert L.ltq_slice_bytes(R, Kc, K, frac, h, sub) == len(pack.pack_slice(idx, gi, K, frac, h, sub))
    assert L.ltq_slice_bytes(0, 0, K, frac, h, sub) == 0
    assert L.ltq_slice_bytes(24, 16, K, frac, h, sub) == -1
    assert L.ltq_slice_bytes(16, 40, K, frac, h, sub) == -1
    assert L.ltq_slice_bytes(-16, 16, K, frac, h, sub) == -1
    assert L.ltq_slice_bytes(16, 16, K, frac, h, 3) == -1


def test_hbm_entry_points_argument_rules_without_a_device():
    """The rotation, row-scale and packing entry points return 0 for empty inputs and -1 for shapes, strides,
    modes or pointers they cannot serve, all before any device call."""
    from ltq_amd import _lib
    so = ROOT / "ltq-research_amd" / "ltq_amd" / "libltq_hip.so"
    if not so.exists():
        pytest.skip("libltq_hip.so not built (run __graft_entry__.build())")
    L = _lib.lib()
    a = 4096  # stand-in address, 16-byte aligned; every call here returns before using it
    # FWHT along rows: (x, dtype, y, rows, cols, ldx, ldy, s, smode)
    assert L.ltq_fwht256_rows(a, 0, a, 0, 512, 512, 512, None, 0, None) == 0
    assert L.ltq_fwht256_rows(a, 0, a, 4, 0, 0, 0, None, 0, None) == 0
    assert L.ltq_fwht256_rows(a, 0, a, 4, 300, 300, 300, None, 0, None) == -1    # cols not a multiple of 256
    assert L.ltq_fwht256_rows(a, 0, a, 4, 512, 256, 512, None, 0, None) == -1    # ldx < cols
    assert L.ltq_fwht256_rows(a, 0, a, 4, 512, 514, 512, None, 0, None) == -1    # ldx not a multiple of 4
    assert L.ltq_fwht256_rows(a, 3, a, 4, 512, 512, 512, None, 0, None) == -1    # element type
    assert L.ltq_fwht256_rows(a, 0, a, 4, 512, 512, 512, None, 1, None) == -1    # scale mode without a scale
    assert L.ltq_fwht256_rows(a + 4, 0, a, 4, 512, 512, 512, None, 0, None) == -1  # fp32 rows need 16-byte alignment
    # FWHT along columns: (x, y, rows, cols, ldx, ldy, s, smode)
    assert L.ltq_fwht256_cols(a, a, 0, 64, 64, 64, None, 0, None) == 0
    assert L.ltq_fwht256_cols(a, a, 300, 64, 64, 64, None, 0, None) == -1       # rows not a multiple of 256
    assert L.ltq_fwht256_cols(a, a, 256, 64, 32, 64, None, 0, None) == -1       # ldx < cols
    assert L.ltq_fwht256_cols(a, a, 256, 64, 64, 64, None, 3, None) == -1       # scale mode
    # row scale: (w, M, K, ldw, scale, e_step, e_bits, exp2_tab, d_row, e, lde, d, ldd)
    assert L.ltq_row_scale(a, 0, 512, 512, 1.1, 0.25, 5, a, a, a, 2, a, 2, None) == 0
    assert L.ltq_row_scale(a, 16, 300, 300, 1.1, 0.25, 5, a, a, a, 2, a, 2, None) == -1  # K not a multiple of 256
    assert L.ltq_row_scale(a, 16, 512, 512, 1.1, 0.25, 9, a, a, a, 2, a, 2, None) == -1  # e_bits
    assert L.ltq_row_scale(a, 16, 512, 512, 0.0, 0.25, 5, a, a, a, 2, a, 2, None) == -1  # scale
    assert L.ltq_row_scale(a, 16, 512, 512, 1.1, 0.25, 5, a, a, a, 1, a, 2, None) == -1  # lde < blocks
    # packing and decoding: an output smaller than the slice, or strides below K
    need = L.ltq_slice_bytes(16, 256, 3, 2, 2, 16)
    assert need > 0
    assert L.ltq_pack_slice(a, 256, a, 256, 0, 0, 3, 2, 2, 16, a, 0, None) == 0
    assert L.ltq_pack_slice(a, 256, a, 256, 16, 256, 3, 2, 2, 16, a, need - 1, None) == -1
    assert L.ltq_pack_slice(a, 255, a, 256, 16, 256, 3, 2, 2, 16, a, need, None) == -1
    assert L.ltq_unpack_slice(a, need - 1, 16, 256, 3, 2, 2, 16, 359, 241, 0, 0, 2, a, a, a, 256, None) == -1
    assert L.ltq_unpack_slice(a, need, 16, 256, 3, 2, 2, 16, 359, 241, 0, 0, 5, a, a, a, 256, None) == -1  # masks
    assert L.ltq_unpack_slice(a, need, 16, 256, 3, 2, 2, 16, 359, 241, 0, 0, 2, a, a, a, 255, None) == -1  # ld_out
