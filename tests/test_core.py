"""The scree.Array contract: invariants, error messages and bit-exact offsets.

Mirrors the reference's ``tests/test_core.py`` (invariants ``:20-55``,
round trips ``:59-170``) and adds bit-exact offset checks against the oracle's
closed form (``src/scree/_core.py:137-138``).
"""

import numpy as np
import pytest
import torch

import scree_amd as scree
from oracle.core import offsets_from_lengths


def test_array_basic_invariants_numpy():
    values = np.arange(20, dtype=np.float32).reshape(10, 2)
    offsets = np.array([0, 3, 7, 10], dtype=np.int32)
    arr = scree.Array(values=values, offsets=offsets, ragged_dim=0)
    assert arr.batch_size == 3
    assert arr.total_length == 10
    assert arr.dtype == np.float32
    assert arr.feature_shape == (2,)
    assert len(arr) == 3


def test_array_rejects_bad_offsets():
    values = np.zeros((10, 2), dtype=np.float32)
    with pytest.raises(ValueError, match=r"offsets\[0\]"):
        scree.Array(values=values, offsets=np.array([1, 5, 10], dtype=np.int32))
    with pytest.raises(ValueError, match=r"offsets\[-1\]"):
        scree.Array(values=values, offsets=np.array([0, 5, 8], dtype=np.int32))


def test_array_rejects_bad_offsets_ndim():
    values = np.zeros((10, 2), dtype=np.float32)
    with pytest.raises(ValueError, match=r"offsets must be 1-D"):
        scree.Array(values=values, offsets=np.array([[0, 5, 10]], dtype=np.int32))


def test_array_rejects_short_offsets_and_scalar_values():
    with pytest.raises(ValueError, match=r"length >= 2"):
        scree.Array(values=np.zeros((0, 2)), offsets=np.array([0], dtype=np.int32))
    with pytest.raises(ValueError, match=r"at least 1-D"):
        scree.Array(values=np.float32(1.0), offsets=np.array([0, 1], dtype=np.int32))


def test_array_rejects_bad_ragged_dim():
    values = np.zeros((10, 2), dtype=np.float32)
    offsets = np.array([0, 5, 10], dtype=np.int32)
    with pytest.raises(ValueError, match=r"ragged_dim"):
        scree.Array(values=values, offsets=offsets, ragged_dim=5)


def test_pack_unpack_roundtrip_numpy():
    rng = np.random.default_rng(0)
    seqs = [rng.standard_normal((n, 4)).astype(np.float32) for n in [3, 5, 2, 7]]
    arr = scree.pack(seqs)
    assert arr.batch_size == 4
    assert arr.total_length == 17
    out = scree.unpack(arr)
    assert len(out) == 4
    for a, b in zip(seqs, out):
        np.testing.assert_array_equal(a, b)


def test_pack_empty_list_raises():
    with pytest.raises(ValueError, match=r"empty"):
        scree.pack([])


def test_to_from_padded_roundtrip_numpy():
    rng = np.random.default_rng(0)
    seqs = [rng.standard_normal((n, 4)).astype(np.float32) for n in [3, 5, 2, 7]]
    arr = scree.pack(seqs)
    padded, mask = scree.to_padded(arr)
    assert padded.shape == (4, 7, 4)
    assert mask.shape == (4, 7)
    assert mask.sum() == 17
    arr2 = scree.from_padded(padded, mask)
    np.testing.assert_array_equal(arr.values, arr2.values)
    np.testing.assert_array_equal(arr.offsets, arr2.offsets)


def test_to_padded_left_side():
    rng = np.random.default_rng(0)
    seqs = [rng.standard_normal((n, 4)).astype(np.float32) for n in [3, 5]]
    arr = scree.pack(seqs)
    padded, mask = scree.to_padded(arr, side="left")
    assert mask[0].tolist() == [False, False, True, True, True]
    assert mask[1].tolist() == [True, True, True, True, True]
    np.testing.assert_array_equal(padded[0, 2:], seqs[0])


def test_to_padded_rejects_bad_side():
    arr = scree.pack([np.zeros((2, 1), dtype=np.float32)])
    with pytest.raises(ValueError, match=r"side"):
        scree.to_padded(arr, side="middle")


def test_from_cu_seqlens_numpy():
    values = np.zeros((10, 2), dtype=np.float32)
    cu_seqlens = np.array([0, 3, 7, 10], dtype=np.int32)
    arr = scree.from_cu_seqlens(values, cu_seqlens)
    assert arr.batch_size == 3
    assert arr.total_length == 10
    assert arr.values is values
    assert arr.offsets is cu_seqlens


def test_lengths_property():
    values = np.zeros((10, 2), dtype=np.float32)
    offsets = np.array([0, 3, 7, 10], dtype=np.int32)
    arr = scree.Array(values=values, offsets=offsets)
    np.testing.assert_array_equal(arr.lengths, np.array([3, 4, 3], dtype=np.int32))


def test_repr_does_not_crash():
    values = np.zeros((10, 2), dtype=np.float32)
    offsets = np.array([0, 3, 7, 10], dtype=np.int32)
    s = repr(scree.Array(values=values, offsets=offsets))
    assert "scree.Array" in s and "batch_size=3" in s


def test_pack_unpack_roundtrip_torch():
    gen = torch.Generator().manual_seed(0)
    seqs = [torch.randn(n, 4, generator=gen) for n in [3, 5, 2, 7]]
    arr = scree.pack(seqs)
    assert arr.batch_size == 4 and arr.total_length == 17
    assert arr.offsets.dtype == torch.int32
    for a, b in zip(seqs, scree.unpack(arr)):
        torch.testing.assert_close(a, b)


def test_to_from_padded_roundtrip_torch():
    gen = torch.Generator().manual_seed(0)
    seqs = [torch.randn(n, 4, generator=gen) for n in [3, 5, 2, 7]]
    arr = scree.pack(seqs)
    padded, mask = scree.to_padded(arr)
    assert padded.shape == (4, 7, 4) and mask.shape == (4, 7)
    arr2 = scree.from_padded(padded, mask)
    torch.testing.assert_close(arr.values, arr2.values)
    torch.testing.assert_close(arr.offsets, arr2.offsets)


@pytest.mark.parametrize("seed", range(5))
def test_offsets_bit_exact_against_closed_form(seed):
    rng = np.random.default_rng(seed)
    lengths = [int(x) for x in rng.integers(0, 3000, size=int(rng.integers(1, 200)))]
    seqs_np = [np.zeros((n, 1), dtype=np.float32) for n in lengths]
    want = offsets_from_lengths(lengths)
    got_np = scree.pack(seqs_np).offsets
    got_t = scree.pack([torch.from_numpy(s) for s in seqs_np]).offsets
    assert got_np.dtype == np.int32 and got_t.dtype == torch.int32
    np.testing.assert_array_equal(got_np, want)
    np.testing.assert_array_equal(got_t.numpy(), want)
    np.testing.assert_array_equal(want[1:], np.cumsum(lengths).astype(np.int32))


def test_pack_offsets_match_reference_test_expectations():
    # reference tests/test_core.py:20-55 build these offsets by hand
    arr = scree.pack([np.zeros((n, 2), dtype=np.float32) for n in [3, 4, 3]])
    np.testing.assert_array_equal(arr.offsets, np.array([0, 3, 7, 10], dtype=np.int32))


def test_grad_flows_through_pack_unpack():
    seqs = [torch.randn(n, 4, requires_grad=True) for n in [3, 5, 2]]
    out = scree.unpack(scree.pack(seqs))
    sum(t.sum() for t in out).backward()
    for s in seqs:
        assert s.grad is not None and s.grad.shape == s.shape
        assert torch.isfinite(s.grad).all()
