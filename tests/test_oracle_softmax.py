"""Pins the softmax oracle (CPU): reference known answers, torch, finite differences."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.core import offsets_from_lengths
from oracle.softmax import varlen_softmax, varlen_softmax_bwd


def _pack(seqs):
    return np.concatenate(seqs, axis=0), offsets_from_lengths([len(s) for s in seqs])


def test_reference_sums_to_one():
    # tests/test_varlen_kernels.py:119-126 of the reference, restated
    rng = np.random.default_rng(0)
    seqs = [rng.standard_normal((n,)).astype(np.float32) for n in [3, 5, 2]]
    x, off = _pack(seqs)
    y = varlen_softmax(x, off)
    for i in range(3):
        np.testing.assert_allclose(y[off[i]:off[i + 1]].sum(), 1.0, atol=1e-5)


def test_reference_per_sequence_baseline():
    # tests/test_varlen_kernels.py:129-139 of the reference, restated
    rng = np.random.default_rng(0)
    seqs = [rng.standard_normal((n, 3)).astype(np.float32) for n in [3, 5, 2]]
    x, off = _pack(seqs)
    y = varlen_softmax(x, off, dtype=np.float32)
    for i, seq in enumerate(seqs):
        e = np.exp(seq - seq.max(axis=0, keepdims=True))
        np.testing.assert_allclose(y[off[i]:off[i + 1]], e / e.sum(axis=0, keepdims=True), atol=1e-5)


@pytest.mark.parametrize("shape", [(), (3,), (2, 5)])
def test_matches_torch_per_sequence(shape):
    rng = np.random.default_rng(1)
    lengths = [1, 4, 0, 9, 2]
    x = rng.standard_normal((sum(lengths),) + shape) * 3
    off = offsets_from_lengths(lengths)
    y = varlen_softmax(x, off)
    for i in range(len(lengths)):
        s, e = off[i], off[i + 1]
        if e > s:
            want = torch.softmax(torch.from_numpy(x[s:e]), dim=0).numpy()
            np.testing.assert_allclose(y[s:e], want, rtol=1e-12, atol=1e-14)


def test_bwd_matches_autograd_and_finite_differences():
    rng = np.random.default_rng(2)
    lengths = [3, 1, 6]
    x = rng.standard_normal((10, 4))
    dy = rng.standard_normal((10, 4))
    off = offsets_from_lengths(lengths)
    y = varlen_softmax(x, off)
    dx = varlen_softmax_bwd(y, dy, off)
    tx = torch.from_numpy(x).requires_grad_(True)
    ty = torch.cat([torch.softmax(tx[off[i]:off[i + 1]], dim=0) for i in range(3)], 0)
    ty.backward(torch.from_numpy(dy))
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-12, atol=1e-14)
    # finite differences of <dy, softmax(x)>
    h = 1e-6
    for idx in [(0, 0), (3, 2), (7, 1), (9, 3)]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        fd = ((varlen_softmax(xp, off) - varlen_softmax(xm, off)) * dy).sum() / (2 * h)
        assert abs(fd - dx[idx]) < 1e-7
    for i in range(3):  # invariant: gradients of a normalised row sum to zero
        np.testing.assert_allclose(dx[off[i]:off[i + 1]].sum(axis=0), 0.0, atol=1e-12)


def test_planted_mistake_is_caught():
    """Softmax over the whole buffer (ignoring offsets) must fail the per-sequence check."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 2))
    off = offsets_from_lengths([2, 4])
    wrong = varlen_softmax(x, offsets_from_lengths([6]))
    assert not np.allclose(wrong, varlen_softmax(x, off))


def test_non_finite_columns_match_torch():
    """NaN, one or two +inf, all -inf, and -inf beside one finite value: the
    oracle's NaN pattern and finite values are torch.softmax's."""
    inf, nan = np.inf, np.nan
    cols = [[0.5, nan, 2.0, -1.0], [1.0, inf, 0.0, 3.0], [inf, 1.0, inf, 0.0],
            [-inf, -inf, -inf, -inf], [-inf, 4.0, -inf, -inf], [-inf, nan, -inf, -inf]]
    x = np.array(cols, dtype=np.float64).T  # 4 rows, 6 columns: one sequence
    off = offsets_from_lengths([4])
    got = varlen_softmax(x, off)
    want = torch.softmax(torch.from_numpy(x), dim=0).numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_allclose(got[~np.isnan(want)], want[~np.isnan(want)], rtol=1e-15)
    assert np.isnan(got[:, [0, 1, 2, 3, 5]]).all() and got[1, 4] == 1.0
