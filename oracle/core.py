"""Offsets arithmetic (oracle; test infrastructure only).

Follows ``src/scree/_core.py:137-138`` of the reference: offsets are the int32
vector ``[0, cumsum(lengths)]``.
"""

from __future__ import annotations

import numpy as np


def offsets_from_lengths(lengths) -> np.ndarray:
    lengths = [int(x) for x in lengths]
    out = np.zeros(len(lengths) + 1, dtype=np.int32)
    acc = 0
    for i, n in enumerate(lengths):
        acc += n
        out[i + 1] = acc
    return out


def lengths_from_offsets(offsets) -> np.ndarray:
    offsets = np.asarray(offsets, dtype=np.int64)
    return (offsets[1:] - offsets[:-1]).astype(np.int32)
