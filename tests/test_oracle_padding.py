"""Pins the padding oracle and the host path (CPU): the reference's own tests, restated."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import scree_amd
from oracle.padding import from_padded, to_padded
from scree_amd.bridges import from_hf_padded, to_hf_padded


def _seqs(lengths, feat=4, seed=0):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((n, feat)).astype(np.float32) for n in lengths]


def test_reference_roundtrip_shapes():
    # tests/test_core.py:58-68 of the reference
    arr = scree_amd.pack(_seqs([3, 5, 2, 7]))
    padded, mask = to_padded(arr.values, arr.offsets)
    assert padded.shape == (4, 7, 4) and mask.shape == (4, 7) and mask.sum() == 17
    values, offsets = from_padded(padded, mask)
    np.testing.assert_array_equal(values, arr.values)
    np.testing.assert_array_equal(offsets, arr.offsets)


def test_reference_left_side_mask():
    # tests/test_core.py:71-78 of the reference
    arr = scree_amd.pack(_seqs([3, 5]))
    _, mask = to_padded(arr.values, arr.offsets, side="left")
    assert mask[0].tolist() == [False, False, True, True, True]
    assert mask[1].tolist() == [True, True, True, True, True]


@pytest.mark.parametrize("side", ["right", "left"])
def test_index_identity(side):
    lengths = [0, 1, 6, 3, 0, 9]
    arr = scree_amd.pack(_seqs(lengths, feat=3, seed=1))
    padded, mask = to_padded(arr.values, arr.offsets, side=side, fill_value=-7.0)
    off = arr.offsets
    T = max(lengths)
    for b, n in enumerate(lengths):
        lo = 0 if side == "right" else T - n
        for t in range(T):
            if lo <= t < lo + n:
                assert mask[b, t]
                np.testing.assert_array_equal(padded[b, t], arr.values[off[b] + t - lo])
            else:
                assert not mask[b, t] and np.all(padded[b, t] == -7.0)


def test_host_path_matches_oracle():
    arr = scree_amd.pack(_seqs([4, 0, 2, 8], seed=2))
    for side in ("right", "left"):
        p1, m1 = scree_amd.to_padded(arr, side=side, fill_value=1.5)
        p2, m2 = to_padded(arr.values, arr.offsets, side=side, fill_value=1.5)
        np.testing.assert_array_equal(p1, p2)
        np.testing.assert_array_equal(m1, m2)
    tarr = scree_amd.pack([torch.from_numpy(s) for s in _seqs([4, 0, 2, 8], seed=2)])
    p, m = scree_amd.to_padded(tarr)
    back = scree_amd.from_padded(p, m)
    assert torch.equal(back.values, tarr.values) and torch.equal(back.offsets, tarr.offsets)


def test_reference_hf_bridge():
    # tests/test_bridges.py:17-37 of the reference
    arr = scree_amd.pack(_seqs([3, 5, 2]))
    hidden, mask = to_hf_padded(arr)
    assert mask.dtype == np.int64 and mask.sum() == arr.total_length
    arr2 = from_hf_padded(hidden, mask)
    np.testing.assert_array_equal(arr.values, arr2.values)
    np.testing.assert_array_equal(arr.offsets, arr2.offsets)
    _, mask = to_hf_padded(scree_amd.pack(_seqs([2, 5])))
    assert mask[0].tolist() == [1, 1, 0, 0, 0] and mask[1].tolist() == [1, 1, 1, 1, 1]


def test_from_padded_takes_first_rows():
    """The reference takes the first mask.sum() rows, wherever the mask's Trues are."""
    padded = np.arange(2 * 4 * 1, dtype=np.float32).reshape(2, 4, 1)
    mask = np.array([[False, True, False, True], [True, True, True, False]])
    values, offsets = from_padded(padded, mask)
    np.testing.assert_array_equal(values[:, 0], [0, 1, 4, 5, 6])
    np.testing.assert_array_equal(offsets, [0, 2, 5])
