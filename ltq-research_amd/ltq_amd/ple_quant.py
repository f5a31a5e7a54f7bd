"""Row tables quantized as LTQ rings on the GPU (embeddings, n-gram and per-layer-embedding tables).

Mirrors src/ple_quant.py:28-67 (same names, arguments and results):
  RING             256 values per ring
  hadamard_signs   the ring rotation's random signs (torch CPU generator, seed 4242)
  quantize_rings   W [rows, n * 256] -> (reconstructed table, bits per value): per ring an optional signed
                   FWHT-256, rms x format scale, and for each of `scales` an fp16 ring scale d and a tail-biting
                   Viterbi (no Hessian, unit weights) of x / d; the ring keeps the scale with the lowest squared
                   error (the first on ties), then the rotation is undone.
and, for the `.ltq` ring records of src/ltq_format.py:42-50, 104-147:
  quantize_rings_packed   the same, plus the packed ring records and the fp16 ring scales.

The Viterbi is the HIP kernel (two passes per ring, tb_window 0), the rotation the HIP FWHT, the packing the
HIP ring packer; the per-ring rms / error / selection are element-wise torch on the device.
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib, ltq_file, rotation
from .formats import TCQ_CONFIG, load_formats
from .tcq_proto import viterbi_ub_cuda

RING = 256


def hadamard_signs(seed: int = 4242) -> torch.Tensor:
    """+-1 float32 [256] (CPU): the rotation's signs are data, drawn as the reference draws them."""
    bits = torch.randint(0, 2, (RING,), generator=torch.Generator().manual_seed(seed))
    return (bits * 2 - 1).float()


def _device(W: torch.Tensor) -> torch.device:
    return W.device if W.is_cuda else torch.device("cuda")


@torch.no_grad()
def _rings(W: torch.Tensor, spec: str, rot: bool, chunk: int, scales, want_fields: bool):
    fmt = load_formats([spec])[spec]
    cfg = TCQ_CONFIG[spec]
    dev = _device(W)
    if not torch.cuda.is_available():
        raise _lib.LtqLibraryMissing("quantize_rings needs a HIP device")
    lut = torch.tensor(fmt.lut, device=dev)
    gains = torch.tensor(fmt.gain_tab, device=dev)
    signs = hadamard_signs().to(dev)
    rings = W.view(-1, RING)
    n = rings.shape[0]
    out = torch.empty_like(rings)
    if want_fields:
        rb = ltq_file.ring_bytes(RING, fmt)
        packed = torch.empty((n, rb), dtype=torch.uint8, device=dev)
        d_out = torch.empty(n, dtype=torch.float16, device=dev)
    for i in range(0, n, chunk):
        x = rings[i:i + chunk].to(dev).float()
        if rot:
            x = rotation.fwht_inplace((x * signs).contiguous(), block_size=RING)
        rms = x.square().mean(dim=1, keepdim=True).sqrt().clamp(min=1e-8) * cfg.get("scale", 1.0)
        best = best_err = best_code = best_d = None
        for sc in scales:
            d = (rms * sc).half().float()
            res = viterbi_ub_cuda(x / d, lut, fmt.K, 10, fmt.masks[0], gains, sub=fmt.sub, tail_biting=True,
                                  m_extra=fmt.masks[1:], pair_parity=fmt.frac, n_cand=cfg.get("n_cand", 0),
                                  return_code=want_fields, _raw_code=True)
            rec, code = res if want_fields else (res, None)
            rec = rec * d
            err = (rec - x).square().sum(dim=1)
            if best is None:
                best, best_err, best_code, best_d = rec, err, code, d
            else:
                better = err < best_err
                best = torch.where(better.unsqueeze(1), rec, best)
                best_err = torch.where(better, err, best_err)
                if want_fields:
                    best_code = torch.where(better.unsqueeze(1), code, best_code)
                    best_d = torch.where(better.unsqueeze(1), d, best_d)
        if want_fields:
            packed[i:i + chunk] = ltq_file.pack_rings_device(best_code & 0xFFFF, best_code >> 16, fmt)
            d_out[i:i + chunk] = best_d.squeeze(1).half()
        if rot:
            best = rotation.fwht_inplace(best.contiguous(), block_size=RING) * signs
        out[i:i + chunk] = best.to(out.dtype).to(out.device)
    bpv = fmt.tile_bytes() * 8 / RING + 16 / RING
    fields = (packed, d_out) if want_fields else None
    return out.view_as(W), bpv, fields


@torch.no_grad()
def quantize_rings(W: torch.Tensor, spec: str, rot: bool, chunk: int = 1 << 17,
                   scales=(0.9, 1.0, 1.12)) -> Tuple[torch.Tensor, float]:
    """W [rows, n * 256] (any device, any float dtype) -> reconstructed table (W's device and dtype) and bits per
    value. The ring scale is fp16, the MSE-best of `scales` x rms x format multiplier."""
    table, bpv, _ = _rings(W, spec, rot, chunk, scales, False)
    return table, bpv


@torch.no_grad()
def quantize_rings_packed(W: torch.Tensor, spec: str, rot: bool, chunk: int = 1 << 17, scales=(0.9, 1.0, 1.12)):
    """quantize_rings plus the ring records: (table, bits per value, packed uint8 [n_rings, ring_bytes] and fp16
    scales [n_rings], both on the device). Ring i decodes (src/ltq_format.py:127-147) to the unscaled values whose
    product with scale i is the table's ring i before the inverse rotation."""
    table, bpv, (packed, d) = _rings(W, spec, rot, chunk, scales, True)
    return table, bpv, packed, d
