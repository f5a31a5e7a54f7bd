"""TEST INFRASTRUCTURE ONLY -- CPU restatement of the input-covariance accumulator (the checker for
ltq_amd.hessian). Only tests/ import it.

Reference anchor: src/liqk_v2.py:207-231 (_CovAccumulator): add() sums X^T X of every batch (rows flattened
over the leading dimensions) into an fp64 running sum and counts rows; get() = (sum / max(count, 1)) in fp32.

Here the sum is exact: bf16 / fp16 values are exact in fp64, their products too, and numpy's fp64 matmul adds
at most ~1e-16 relative error, far below the fp32 accumulation the reference (and the GPU path) does within a
batch. get() scales as torch's device kernel does: a multiplication by the fp64 reciprocal of the count.

Pinned by (tests/test_hessian.py): a pure-Python triple loop on tiny inputs, closed forms (one-hot rows give
a diagonal of row counts, constant rows give a constant matrix, two orthogonal directions give a known rank-2
matrix) and batching invariance.
"""
from __future__ import annotations

import numpy as np


class CovAccumulatorRef:
    def __init__(self):
        self.H = None
        self.n = 0

    def add(self, x: np.ndarray):
        x2 = np.asarray(x, dtype=np.float64).reshape(-1, np.shape(x)[-1])
        if self.H is None:
            self.H = np.zeros((x2.shape[1],) * 2, dtype=np.float64)
        self.H += x2.T @ x2
        self.n += x2.shape[0]

    def abs_sum(self, batches):
        """sum over batches of |X|^T |X| (the scale of the fp32 rounding error bound of each entry)."""
        out = None
        for x in batches:
            a = np.abs(np.asarray(x, dtype=np.float64).reshape(-1, np.shape(x)[-1]))
            out = a.T @ a if out is None else out + a.T @ a
        return out

    def get(self) -> np.ndarray:
        inv = 1.0 / max(self.n, 1)
        return (self.H * inv).astype(np.float32)


def cov_loop(x) -> list:
    """X^T X by explicit loops (tiny inputs only): the independent check of the matmul form."""
    rows = [[float(v) for v in r] for r in x]
    K = len(rows[0]) if rows else 0
    H = [[0.0] * K for _ in range(K)]
    for r in rows:
        for i in range(K):
            for j in range(K):
                H[i][j] += r[i] * r[j]
    return H
