"""Packed <-> padded conversions (test oracle; see oracle/__init__.py).

Restates the numpy branch of the reference's ``to_padded``
(``src/scree/_core.py:245-266``) and ``from_padded`` (``:292-298``).
"""

from __future__ import annotations

import numpy as np


def to_padded(values, offsets, side="right", fill_value=0.0):
    values = np.asarray(values)
    off = np.asarray(offsets, dtype=np.int64)
    lengths = [int(off[i + 1] - off[i]) for i in range(len(off) - 1)]
    max_len = max(lengths) if lengths else 0
    batch = len(lengths)
    padded = np.full((batch, max_len, *values.shape[1:]), fill_value, dtype=values.dtype)
    mask = np.zeros((batch, max_len), dtype=np.bool_)
    for i, n in enumerate(lengths):
        row = values[off[i]:off[i] + n]
        if side == "right":
            padded[i, :n] = row
            mask[i, :n] = True
        else:
            padded[i, max_len - n:] = row
            mask[i, max_len - n:] = True
    return padded, mask


def from_padded(padded, mask):
    padded = np.asarray(padded)
    lengths = [int(np.asarray(mask)[i].sum()) for i in range(padded.shape[0])]
    values = np.concatenate([padded[i, :lengths[i]] for i in range(padded.shape[0])], axis=0)
    offsets = np.zeros(len(lengths) + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(lengths)
    return values, offsets
