"""Input-covariance (Hessian) accumulation of the matrix quantizer: the _CovAccumulator of src/liqk_v2.py:207-231.

CovAccumulator keeps the running sum of X^T X in fp64 on the batch's device and the row count; get() returns
H = sum / count in fp32. bf16 / fp16 batches go through ltq_cov_accumulate (one gfx950 kernel: the batch's
X^T X on the matrix cores with fp32 accumulation, added straight into the fp64 sum, lower-triangle tiles
only); fp32 batches take the reference's own fp32 GEMM (src/liqk_v2.py:223-224). get() is ltq_cov_finalize,
which reads the lower triangle, so the result is exactly symmetric.

Differences from the reference that stay within fp32 rounding: the order of the fp32 sums over a batch's rows
(any two GEMMs differ there), and exact symmetry (a full GEMM's (i, j) and (j, i) entries may differ in the
last bit).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (code {rc})")


class CovAccumulator:
    """H = (1/N) sum X^T X over the batches passed to add(), without storing X (src/liqk_v2.py:207-231).

    `H` is the fp64 running sum; after bf16 / fp16 batches only its tiles on and below the diagonal hold the
    sum (get() reads the lower triangle). `n` is the number of rows added."""

    def __init__(self):
        self.H: Optional[torch.Tensor] = None
        self.n = 0

    def add(self, x: torch.Tensor):
        x_2d = x.detach().reshape(-1, x.shape[-1])
        if self.H is None:
            self.H = torch.zeros((x_2d.shape[1],) * 2, dtype=torch.float64, device=x_2d.device)
        if x_2d.dtype in (torch.bfloat16, torch.float16):
            _lib.require_device(x_2d)
            if x_2d.stride(1) != 1 or x_2d.stride(0) < x_2d.shape[1]:
                x_2d = x_2d.contiguous()
            n, K = x_2d.shape
            lib = _lib.lib()
            _check(lib.ltq_cov_accumulate(x_2d.data_ptr(), n, K, max(x_2d.stride(0), K),
                                          1 if x_2d.dtype == torch.float16 else 0, self.H.data_ptr(),
                                          self.H.stride(0), _lib.stream_ptr()), "ltq_cov_accumulate")
        else:
            x_2d = x_2d.float()
            gram = x_2d.T @ x_2d
            self.H.add_(gram.to(torch.float64))
        self.n += x_2d.shape[0]

    def get(self) -> torch.Tensor:
        if self.H is None:
            raise TypeError("CovAccumulator.get: no batch was added")
        _lib.require_device(self.H)
        K = self.H.shape[0]
        out = torch.empty((K, K), dtype=torch.float32, device=self.H.device)
        _check(_lib.lib().ltq_cov_finalize(self.H.data_ptr(), K, self.H.stride(0), 1.0 / max(self.n, 1),
                                           out.data_ptr(), out.stride(0), _lib.stream_ptr()), "ltq_cov_finalize")
        return out
