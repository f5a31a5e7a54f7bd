"""Incoherence rotation of the quantizer: Rademacher signs, suh pre-scaling and the block FWHT-256.

Mirrors (same names, argument meaning and results):
  fwht_inplace           src/iqk_format.py:153-170   (HIP kernel ltq_fwht256_rows; bit-identical stage order)
  make_rademacher_signs  src/iqk_format.py:173-179   (the reference's own CPU torch generator draw)
  compute_optimal_suh    src/liqk_v2.py:409-441      (scale from column rms and diag(H); W and H rotated by
                                                      the HIP kernels with the scale fused into their loads)
  fwht_cols              src/liqk_v2.py:1023-1026 (_fwht_rows: the transform along dim 0)

Differences a caller cannot observe: the reference's fwht_inplace also leaves the unnormalized transform in
its (contiguous) input; every caller passes a temporary, so this one leaves the input untouched.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

QK_K = 256
_DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def make_rademacher_signs(dim: int, seed: int, device) -> torch.Tensor:
    """Deterministic +-1 float32 vector: bits from torch.randint on a CPU generator seeded with `seed`."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    bits = torch.randint(0, 2, (dim,), generator=gen, dtype=torch.int64)
    return (bits * 2 - 1).to(dtype=torch.float32, device=device)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: HIP error code {rc}" if rc > 0 else f"{what}: rejected arguments")


def fwht_rows(x: torch.Tensor, s: Optional[torch.Tensor] = None, mode: int = 0,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Normalized FWHT-256 over the last dimension of a 2-D fp32/bf16/fp16 device tensor, fp32 out.
    mode 1 transforms x / s[col], mode 2 x * s[col] (s: fp32 [cols]), each rounded once as torch does."""
    _lib.require_device(x)
    if x.dim() != 2 or x.dtype not in _DT or x.shape[1] % QK_K:
        raise ValueError("fwht_rows: 2-D fp32/bf16/fp16 tensor with a multiple of 256 columns")
    if x.stride(1) != 1 or x.stride(0) % 4 or x.data_ptr() % 16:
        x = x.contiguous()
    rows, cols = x.shape
    if out is None:
        out = torch.empty((rows, cols), dtype=torch.float32, device=x.device)
    sp = None
    if mode:
        s = s.to(device=x.device, dtype=torch.float32).contiguous()
        if s.numel() != cols:
            raise ValueError("fwht_rows: scale vector must have one entry per column")
        sp = s.data_ptr()
    _check(_lib.lib().ltq_fwht256_rows(x.data_ptr(), _DT[x.dtype], out.data_ptr(), rows, cols, x.stride(0),
                                       out.stride(0), sp, mode, _lib.stream_ptr()), "ltq_fwht256_rows")
    return out


def fwht_cols(x: torch.Tensor, s: Optional[torch.Tensor] = None, mode: int = 0,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Normalized FWHT-256 along dim 0 (256-row blocks) of a 2-D fp32 device tensor; mode 1 / 2 scale by
    s[row] first. Equals fwht_inplace(x.T * s).T of the reference, bit for bit."""
    _lib.require_device(x)
    if x.dim() != 2 or x.dtype != torch.float32 or x.shape[0] % QK_K:
        raise ValueError("fwht_cols: 2-D fp32 tensor with a multiple of 256 rows")
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, cols = x.shape
    if out is None:
        out = torch.empty((rows, cols), dtype=torch.float32, device=x.device)
    sp = None
    if mode:
        s = s.to(device=x.device, dtype=torch.float32).contiguous()
        if s.numel() != rows:
            raise ValueError("fwht_cols: scale vector must have one entry per row")
        sp = s.data_ptr()
    _check(_lib.lib().ltq_fwht256_cols(x.data_ptr(), out.data_ptr(), rows, cols, x.stride(0), out.stride(0), sp, mode,
                                       _lib.stream_ptr()), "ltq_fwht256_cols")
    return out


def fwht_inplace(x: torch.Tensor, block_size: int = 256) -> torch.Tensor:
    """Normalized block FWHT over the last dimension (orthogonal, self-inverse); fp32 in, fp32 out."""
    if block_size != QK_K:
        raise ValueError("fwht_inplace: the LTQ formats use block_size 256 only")
    if x.dtype != torch.float32:
        raise TypeError("fwht_inplace: fp32 input (the reference's callers always pass .float())")
    shape = x.shape
    if shape[-1] % block_size:
        raise AssertionError(f"Dimension {shape[-1]} is not a multiple of {block_size}")
    y = fwht_rows(x.reshape(-1, shape[-1]))
    return y.view(shape)


def _fwht_rows(X: torch.Tensor) -> torch.Tensor:
    """The transform along dim 0 (src/liqk_v2.py:1023-1026), contiguous fp32 result."""
    return fwht_cols(X.float())


def normalized_row_weights(row_weights: torch.Tensor) -> torch.Tensor:
    """The row-weight normalization of src/liqk_v2.py:423-425 / :1150-1152 (floor at a tenth of the mean,
    unit mean, clamp to [0.25, 4]), evaluated in float64."""
    rw = row_weights.double()
    rw = rw.clamp(min=float(rw.mean().item()) * 0.1)
    return (rw / rw.mean().clamp(min=1e-12)).clamp(0.25, 4.0)


@torch.no_grad()
def column_sumsq(W: torch.Tensor, rw: Optional[torch.Tensor] = None, chunk: int = 1024) -> torch.Tensor:
    """float64 [K]: sum over rows of W^2 (times the row weight), every square exact in float64; row chunks keep
    the float64 temporary small."""
    M, K = W.shape
    acc = torch.zeros(K, dtype=torch.float64, device=W.device)
    for r0 in range(0, M, chunk):
        blk = W[r0:r0 + chunk].double().square_()
        if rw is not None:
            blk.mul_(rw[r0:r0 + chunk].unsqueeze(1))
        acc += blk.sum(dim=0)
    return acc


@torch.no_grad()
def compute_optimal_suh(W: torch.Tensor, H: torch.Tensor, seed: int = 1337,
                        row_weights: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(W_rot, H_rot, suh): suh = fp16(signs * clamp(col_rms^0.5 * h_std^-0.25, 0.25, 4)),
    W_rot = FWHT_rows(W / suh), H_rot = FWHT_cols(FWHT_rows(H * suh) * suh).

    The scale vector is evaluated in float64 from exact squares (the reference's fp32 column reduction and
    powers, src/liqk_v2.py:419-434, depend on the device's summation order): suh is the fp16 rounding of the
    scale's exact value except within ~1e-13 of an fp16 rounding boundary, so a CPU restatement gets the same
    bits."""
    device = W.device
    M, K = W.shape
    signs = make_rademacher_signs(K, seed=seed, device=device)
    rw = normalized_row_weights(row_weights.to(device)) if row_weights is not None else None
    col_rms = (column_sumsq(W, rw) / M).sqrt().clamp(min=1e-6)
    col_rms = col_rms / col_rms.mean().clamp(min=1e-6)
    h_std = torch.diagonal(H).double().clamp(min=1e-8).sqrt()
    h_std = h_std / h_std.mean().clamp(min=1e-6)
    scale = (col_rms.sqrt() * h_std.pow(-0.25)).clamp(0.25, 4.0)
    suh = (signs.double() * scale).to(torch.float16).to(torch.float32)
    W_rot = fwht_rows(W if W.dtype in _DT else W.float(), suh, mode=1)
    H_tmp = fwht_rows(H.float(), suh, mode=2)
    H_rot = fwht_cols(H_tmp, suh, mode=2, out=H_tmp)
    return W_rot, H_rot, suh
