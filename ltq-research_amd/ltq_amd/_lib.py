"""Loader of the gfx950 HIP library (libltq_hip.so, built in-tree by ltq-research_amd/build.py).

There is no fallback: if the library or the device is missing, every entry point raises. The C ABI is
declared in include/ltq_hip.h; argument conventions follow the reference's ctypes glue
(src/tcq_proto.py:515-534)."""
from __future__ import annotations

import ctypes
from pathlib import Path

_SO = Path(__file__).resolve().parent / "libltq_hip.so"
_LIB = None

vp, ci, cf, cl, cd = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_long, ctypes.c_double

# name -> (restype, argtypes)
SIGNATURES = {
    # src/cuda/tcq_viterbi.cu:743-746; ctypes argtypes as src/tcq_proto.py:529
    "tcq_viterbi": (ci, [vp] * 15 + [ci] * 18 + [vp, ci, vp]),
    # both tail-biting passes in one launch (no reference counterpart; the two calls of src/tcq_proto.py:584-609)
    "tcq_viterbi_tb": (ci, [vp] * 14 + [ci] * 17 + [vp, ci, ci, ci, ci, vp]),
    # tcq_viterbi without caller workspace (no reference counterpart): 12 pointers, 19 ints, stream
    "tcq_viterbi_static": (ci, [vp] * 12 + [ci] * 19 + [vp]),
    "tcq_viterbi_static_bytes": (cl, []),
    # timing hook for benchmarks (no reference counterpart): start / stop HIP events carried by the next launches
    "ltq_viterbi_timing": (ci, [vp, vp, ci]),
    "ltq_kernel_timing": (ci, [vp, vp, ci]),
    # src/cuda/tcq_viterbi.cu:806-807; src/tcq_proto.py:531-532
    "lut_subs_quant": (ci, [vp] * 4 + [ci, cf, cf, ci, vp]),
    # FWHT-256 (src/iqk_format.py:153-170), rows with a fused scale / columns
    "ltq_fwht256_rows": (ci, [vp, ci, vp, cl, cl, cl, cl, vp, ci, vp]),
    "ltq_fwht256_cols": (ci, [vp, vp, cl, cl, cl, cl, vp, ci, vp]),
    # .ltq slice packing (src/ltq_file.py:79-96)
    "ltq_slice_bytes": (cl, [ci] * 6),
    "ltq_pack_slice": (ci, [vp, cl, vp, cl, ci, ci, ci, ci, ci, ci, vp, cl, vp]),
    "ltq_unpack_slice": (ci, [vp, cl] + [ci] * 11 + [vp, vp, vp, cl, vp]),
    "ltq_ring_bytes": (cl, [ci, ci, ci, ci, ci]),
    "ltq_pack_rings": (ci, [vp, cl, vp, cl, cl, ci, ci, ci, ci, ci, vp, cl, vp]),
    # row scale and LDLQ sub-block feedback (src/liqk_v2.py:938-967)
    # src/liqk_v2.py:207-231 (_CovAccumulator.add / get)
    "ltq_cov_accumulate": (ci, [vp, cl, ci, cl, ci, vp, cl, vp]),
    "ltq_cov_finalize": (ci, [vp, ci, cl, cd, vp, cl, vp]),
    "ltq_row_scale": (ci, [vp, cl, cl, cl, cf, cf, ci, vp, vp, vp, cl, vp, cl, vp]),
    "ltq_ldlq_prep": (ci, [vp, cl, vp, cl, vp, cl, vp]),
    "ltq_ldlq_sub": (ci, [vp, cl, vp, vp, cl, vp, cl, vp, cl, ci, vp, cl, vp, cl, vp, vp, cl, vp, cl, vp, cl, cl, cl, cl,
                          vp]),
    # LDLQ block error and inter-block update on the matrix cores (src/liqk_v2.py:972-979)
    "ltq_ldlq_err": (ci, [vp, cl, vp, cl, vp, cl, vp, cl, vp, cl, vp, cl, cl, cl, cl, vp]),
    "ltq_ldlq_update": (ci, [vp, cl, vp, cl, vp, cl, cl, cl, vp, cl, vp, vp, cl, cl, cl, vp]),
}


class LtqLibraryMissing(RuntimeError):
    pass


def lib():
    global _LIB
    if _LIB is None:
        if not _SO.exists():
            raise LtqLibraryMissing(f"{_SO} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(str(_SO))
        for name, (res, args) in SIGNATURES.items():
            if hasattr(L, name):
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
        _LIB = L
    return _LIB


def require_device(t) -> None:
    import torch
    if not torch.cuda.is_available():
        raise LtqLibraryMissing("no HIP device: the LTQ kernels run only on an MI355X (gfx950)")
    if not t.is_cuda:
        raise ValueError("LTQ kernels take device tensors")


def stream_ptr():
    import torch
    return torch.cuda.current_stream().cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()
