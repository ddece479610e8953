"""Varlen softmax along the ragged dimension (test oracle; see oracle/__init__.py).

Restates ``src/scree/kernels/reference/varlen_softmax.py:53-61`` (the numpy
branch): per sequence, max-subtracted ``exp`` along axis 0, divided by the
sum along axis 0.  The gradient is the softmax Jacobian-vector product
``dx = y * (dy - sum_rows(y * dy))`` per sequence and column.
"""

from __future__ import annotations

import numpy as np


def varlen_softmax(values, offsets, dtype=np.float64):
    x = np.asarray(values, dtype=dtype)
    off = np.asarray(offsets, dtype=np.int64)
    out = np.empty_like(x)
    for i in range(len(off) - 1):
        s, e = int(off[i]), int(off[i + 1])
        if e <= s:
            continue
        row = x[s:e]
        ex = np.exp(row - row.max(axis=0, keepdims=True))
        out[s:e] = ex / ex.sum(axis=0, keepdims=True)
    return out


def varlen_softmax_bwd(y, dy, offsets, dtype=np.float64):
    y = np.asarray(y, dtype=dtype)
    dy = np.asarray(dy, dtype=dtype)
    off = np.asarray(offsets, dtype=np.int64)
    dx = np.empty_like(y)
    for i in range(len(off) - 1):
        s, e = int(off[i]), int(off[i + 1])
        if e <= s:
            continue
        dx[s:e] = y[s:e] * (dy[s:e] - (y[s:e] * dy[s:e]).sum(axis=0, keepdims=True))
    return dx
