"""Tile schedule enumeration (oracle; test infrastructure only).

The reference has no scheduler: it launches a padded ``(B, cdiv(max_seq, 64),
H)`` grid and lets programs past a sequence's end return
(``src/scree/kernels/triton/varlen_attention.py:63-76,236``).  The HIP library
instead builds a dense work list on the device.  This module states that list
in plain Python so the device output can be compared bit for bit.

For block size ``BM`` a sequence of length ``L`` has ``nblk = ceil(L / BM)``
row blocks.  Sequences are ranked by ``(-nblk, seq)``.  The list holds one
``(seq, blk)`` pair per row block of every sequence, ordered longest-work
first:

* causal: the work of row block ``blk`` grows with ``blk + 1`` (the number of
  key blocks it reads), so items are grouped by ``c = blk + 1`` from the
  largest ``c`` down to 1, and inside a group by sequence rank;
* non-causal: every row block of a sequence reads all ``nblk`` key blocks, so
  sequences appear in rank order, each with its blocks ``0..nblk-1``.

The key-block-major list used by the dK/dV pass is the same list with
``blk -> nblk - 1 - blk``, whose work ``nblk - blk`` then matches ``c``.

A second list holds the same items sequence by sequence (``build_schedule_by_sequence``):
sequences in rank order, each with its blocks from the last down.  Launches
that give each XCD one head at a time read it, so that the resident
workgroups of an XCD share one sequence's K/V.
"""

from __future__ import annotations

import numpy as np


def block_counts(offsets, block: int) -> np.ndarray:
    off = np.asarray(offsets, dtype=np.int64)
    lengths = off[1:] - off[:-1]
    return ((lengths + block - 1) // block).astype(np.int64)


def seq_order(nblk) -> list:
    return sorted(range(len(nblk)), key=lambda s: (-int(nblk[s]), s))


def build_schedule(offsets, block: int, causal: bool, max_class: int = 4096,
                   max_batch: int = 2048) -> np.ndarray:
    """Return an ``(T, 2)`` int32 array of ``(seq, blk)`` items.

    ``max_class`` is the device scheduler's limit on row blocks per sequence
    for the causal ordering, ``max_batch`` its limit on sequences for any
    ordering; past either the list falls back to natural order (sequence by
    sequence, blocks ascending).
    """
    nblk = block_counts(offsets, block)
    order = seq_order(nblk)
    items = []
    if len(nblk) > max_batch or (causal and len(nblk) and int(nblk.max()) > max_class):
        for s in range(len(nblk)):
            for b in range(int(nblk[s])):
                items.append((s, b))
    elif causal:
        cmax = int(nblk.max()) if len(nblk) else 0
        for c in range(cmax, 0, -1):
            for s in order:
                if nblk[s] >= c:
                    items.append((s, c - 1))
    else:
        for s in order:
            for b in range(int(nblk[s])):
                items.append((s, b))
    return np.asarray(items, dtype=np.int32).reshape(-1, 2)


def item_cost(item, nblk, causal: bool) -> int:
    s, b = int(item[0]), int(item[1])
    return b + 1 if causal else int(nblk[s])


def build_schedule_by_sequence(offsets, block: int, max_batch: int = 2048) -> np.ndarray:
    """The sequence-major list: ``(seq, blk)`` for sequences in ``(-nblk, seq)``
    rank order (index order past ``max_batch`` sequences), each sequence's
    blocks ``nblk - 1`` down to ``0``."""
    nblk = block_counts(offsets, block)
    seqs = range(len(nblk)) if len(nblk) > max_batch else seq_order(nblk)
    items = [(s, b) for s in seqs for b in range(int(nblk[s]) - 1, -1, -1)]
    return np.asarray(items, dtype=np.int32).reshape(-1, 2)

