"""The .ltq slice packing of the quantizer's PACK output, on the GPU.

Mirrors src/ltq_file.py:79-96 (`pack_slice`): a row slice [R, K] of codes (label * U + u) and gain indices
becomes four structure-of-arrays regions (codes, uncoded bit planes, lowest uncoded bit, gain indices), each
starting on a 64-byte boundary, tiles ordered by row group then 16-column block (position t = 16 r + c).
The bytes are produced by the HIP kernel ltq_pack_slice.
"""
from __future__ import annotations

import torch

from . import _lib
from .formats import LtqFormat


def slice_bytes(R: int, K: int, f: LtqFormat) -> int:
    n = _lib.lib().ltq_slice_bytes(R, K, f.K, f.frac, f.h, f.sub)
    if n < 0:
        raise ValueError(f"slice [{R}, {K}] cannot hold format {f.name} tiles (R and K must be multiples of 16)")
    return n


@torch.no_grad()
def pack_slice_device(idx: torch.Tensor, gi: torch.Tensor, f: LtqFormat) -> torch.Tensor:
    """Packed slice as a uint8 device tensor."""
    _lib.require_device(idx)
    R, K = idx.shape
    ix = idx.to(torch.int16)
    g = gi.to(torch.uint8)
    if ix.stride(1) != 1:
        ix = ix.contiguous()
    if g.stride(1) != 1:
        g = g.contiguous()
    n = slice_bytes(R, K, f)
    out = torch.empty(n, dtype=torch.uint8, device=idx.device)
    rc = _lib.lib().ltq_pack_slice(ix.data_ptr(), ix.stride(0), g.data_ptr(), g.stride(0), R, K, f.K, f.frac, f.h,
                                   f.sub, out.data_ptr(), n, _lib.stream_ptr())
    if rc != 0:
        raise RuntimeError(f"ltq_pack_slice: HIP error code {rc}" if rc > 0 else "ltq_pack_slice: rejected arguments")
    return out


def pack_slice(idx: torch.Tensor, gi: torch.Tensor, f: LtqFormat) -> bytes:
    """Row slice data [R, K] (label * U + u and gain index per position) -> bytes, as the reference returns."""
    return bytes(pack_slice_device(idx, gi, f).cpu().numpy().tobytes())


def ring_bytes(L: int, f: LtqFormat) -> int:
    """Bytes of one packed ring of L positions (src/ltq_format.py:48-50, `tile_bytes(L)`; scale excluded)."""
    n = _lib.lib().ltq_ring_bytes(L, f.K, f.frac, f.h, f.sub)
    if n < 0:
        raise ValueError(f"rings of {L} values cannot hold format {f.name} (L % 16 == 0, L % sub == 0, L <= 512)")
    return n


@torch.no_grad()
def pack_rings_device(idx: torch.Tensor, gi: torch.Tensor, f: LtqFormat) -> torch.Tensor:
    """Rings [n, L] of codes (label * U + u) and gain indices -> uint8 device tensor [n, ring_bytes(L)], each row
    the fields codes / planes / lsb / gains of src/ltq_format.py:104-124 back to back."""
    _lib.require_device(idx)
    n, L = idx.shape
    ix = idx.to(torch.int16)
    g = gi.to(torch.uint8)
    if ix.stride(1) != 1:
        ix = ix.contiguous()
    if g.stride(1) != 1:
        g = g.contiguous()
    rb = ring_bytes(L, f)
    out = torch.empty((n, rb), dtype=torch.uint8, device=idx.device)
    rc = _lib.lib().ltq_pack_rings(ix.data_ptr(), ix.stride(0), g.data_ptr(), g.stride(0), n, L, f.K, f.frac, f.h,
                                   f.sub, out.data_ptr(), out.numel(), _lib.stream_ptr())
    if rc != 0:
        raise RuntimeError(f"ltq_pack_rings: HIP error code {rc}" if rc > 0 else "ltq_pack_rings: rejected arguments")
    return out
