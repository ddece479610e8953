"""The packed Array contract on the host: validation, offsets, packing, padding.

The error-message patterns are part of the interface (callers match on the
reference's wording, ``src/scree/_core.py:44-62``).  Offsets are checked
bit-exactly against the closed form ``[0, cumsum(L)]`` int32
(``_core.py:137-138``), restated independently in ``oracle/core.py``.
Round trips are checked as properties over random length lists, including
empty sequences, several feature axes and a non-zero ragged axis.
"""

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

import scree_amd as scree
from oracle.core import lengths_from_offsets, offsets_from_lengths

lengths_lists = st.lists(st.integers(min_value=0, max_value=40), min_size=1, max_size=12)


def _seqs_np(lengths, feat=(3,), seed=0, dtype=np.float32):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((n, *feat)).astype(dtype) for n in lengths]


# ----------------------------------------------------------------- validation
# (values shape, offsets, ragged_dim, message pattern)
BAD_CONSTRUCTIONS = [
    ((6, 2), [2, 4, 6], 0, r"offsets\[0\]"),
    ((6, 2), [0, 4, 5], 0, r"offsets\[-1\]"),
    ((6, 2), [[0, 6]], 0, r"offsets must be 1-D"),
    ((6, 2), [0], 0, r"length >= 2"),
    ((6, 2), [0, 6], 2, r"ragged_dim"),
    ((6, 2), [0, 6], -1, r"ragged_dim"),
    ((2, 6), [0, 3, 6], 0, r"offsets\[-1\]"),  # offsets describe axis 1, not axis 0
]


@pytest.mark.parametrize("shape,offsets,ragged_dim,pattern", BAD_CONSTRUCTIONS)
def test_invalid_arrays_are_rejected_with_reference_messages(shape, offsets, ragged_dim, pattern):
    with pytest.raises(ValueError, match=pattern):
        scree.Array(values=np.ones(shape, np.float16), offsets=np.array(offsets, np.int32),
                    ragged_dim=ragged_dim)


def test_zero_dimensional_values_are_rejected():
    with pytest.raises(ValueError, match=r"at least 1-D"):
        scree.Array(values=np.float64(3.0), offsets=np.array([0, 1], np.int32))


def test_torch_offsets_are_validated_like_numpy_offsets():
    vals = torch.zeros(9, 4)
    with pytest.raises(ValueError, match=r"offsets\[-1\]"):
        scree.Array(values=vals, offsets=torch.tensor([0, 4, 8], dtype=torch.int32))
    arr = scree.Array(values=vals, offsets=torch.tensor([0, 4, 9], dtype=torch.int32))
    assert arr.total_length == 9 and arr.batch_size == 2


def test_properties_on_a_non_leading_ragged_axis():
    # 5 sequences packed along axis 1 of a (2, 12, 3) tensor
    offsets = np.array([0, 1, 1, 6, 10, 12], np.int32)
    arr = scree.Array(values=np.zeros((2, 12, 3), np.float32), offsets=offsets, ragged_dim=1)
    assert len(arr) == arr.batch_size == 5
    assert arr.total_length == 12
    assert arr.feature_shape == (2, 3)
    assert arr.dtype == np.float32
    np.testing.assert_array_equal(arr.lengths, [1, 0, 5, 4, 2])
    text = repr(arr)
    assert text.startswith("scree.Array(") and "batch_size=5" in text and "total_length=12" in text


# --------------------------------------------------------------------- offsets
@settings(max_examples=60, deadline=None)
@given(lengths=lengths_lists)
def test_pack_offsets_are_the_int32_prefix_sum(lengths):
    want = offsets_from_lengths(lengths)
    got_np = scree.pack(_seqs_np(lengths, feat=(1,))).offsets
    got_t = scree.pack([torch.zeros(n, 1) for n in lengths]).offsets
    assert got_np.dtype == np.int32 and got_t.dtype == torch.int32
    np.testing.assert_array_equal(got_np, want)
    np.testing.assert_array_equal(got_t.numpy(), want)
    np.testing.assert_array_equal(lengths_from_offsets(got_np), lengths)


def test_offsets_stay_exact_near_the_int32_limit():
    # lengths whose running sum approaches 2^31 - 1: no float rounding may enter
    lengths = [2 ** 30 - 3, 2 ** 29 + 7, 2 ** 28 + 1]
    want = offsets_from_lengths(lengths)
    assert int(want[-1]) == sum(lengths) < 2 ** 31
    got = scree._core._offsets_from_lengths_np(lengths)
    np.testing.assert_array_equal(got, want)


def test_from_cu_seqlens_wraps_without_copying():
    vals = torch.arange(14.0).reshape(7, 2)
    cu = torch.tensor([0, 2, 2, 7], dtype=torch.int32)
    arr = scree.from_cu_seqlens(vals, cu)
    assert arr.values is vals and arr.offsets is cu and arr.ragged_dim == 0
    assert arr.lengths.tolist() == [2, 0, 5]


# --------------------------------------------------------------- pack / unpack
def test_pack_of_nothing_is_an_error():
    with pytest.raises(ValueError, match=r"empty"):
        scree.pack([])


@settings(max_examples=40, deadline=None)
@given(lengths=lengths_lists, seed=st.integers(0, 1000))
def test_unpack_inverts_pack_numpy(lengths, seed):
    seqs = _seqs_np(lengths, feat=(2, 3), seed=seed)
    arr = scree.pack(seqs)
    assert arr.values.shape == (sum(lengths), 2, 3)
    back = scree.unpack(arr)
    assert [b.shape[0] for b in back] == lengths
    for a, b in zip(seqs, back):
        np.testing.assert_array_equal(a, b)


def test_unpack_inverts_pack_along_axis_one():
    seqs = [np.full((3, n), float(n), np.float32) for n in (4, 0, 2)]
    arr = scree.pack(seqs, ragged_dim=1)
    assert arr.values.shape == (3, 6)
    np.testing.assert_array_equal(arr.offsets, [0, 4, 4, 6])
    for a, b in zip(seqs, scree.unpack(arr)):
        np.testing.assert_array_equal(a, b)


def test_unpack_returns_views_of_the_packed_tensor():
    arr = scree.pack([torch.zeros(3, 2), torch.zeros(4, 2)])
    parts = scree.unpack(arr)
    parts[1][0, 0] = 5.0
    assert float(arr.values[3, 0]) == 5.0


def test_torch_pack_keeps_dtype_and_is_differentiable():
    g = torch.Generator().manual_seed(3)
    seqs = [torch.randn(n, 5, generator=g, dtype=torch.float64, requires_grad=True)
            for n in (2, 7, 1)]
    arr = scree.pack(seqs)
    assert arr.values.dtype == torch.float64
    weights = torch.arange(arr.total_length, dtype=torch.float64)[:, None]
    (arr.values * weights).sum().backward()
    start = 0
    for s in seqs:
        n = s.shape[0]
        expect = torch.arange(start, start + n, dtype=torch.float64)[:, None].expand(n, 5)
        torch.testing.assert_close(s.grad, expect)
        start += n


# ------------------------------------------------------------------- padding
@settings(max_examples=40, deadline=None)
@given(lengths=lengths_lists.filter(lambda ls: sum(ls) > 0), fill=st.sampled_from([0.0, -1.5]))
def test_padding_layout_and_round_trip_numpy(lengths, fill):
    seqs = _seqs_np(lengths, feat=(2,), seed=len(lengths))
    arr = scree.pack(seqs)
    width = max(lengths)
    for side in ("right", "left"):
        padded, mask = scree.to_padded(arr, side=side, fill_value=fill)
        assert padded.shape == (len(lengths), width, 2) and mask.shape == (len(lengths), width)
        assert mask.dtype == np.bool_ and int(mask.sum()) == sum(lengths)
        for i, (n, s) in enumerate(zip(lengths, seqs)):
            cols = slice(0, n) if side == "right" else slice(width - n, width)
            np.testing.assert_array_equal(padded[i, cols], s)
            assert mask[i, cols].all() and int(mask[i].sum()) == n
            assert np.all(padded[i][~mask[i]] == fill)
    padded, mask = scree.to_padded(arr)
    again = scree.from_padded(padded, mask)
    np.testing.assert_array_equal(again.values, arr.values)
    np.testing.assert_array_equal(again.offsets, arr.offsets)


def test_padding_round_trip_torch_host():
    g = torch.Generator().manual_seed(1)
    arr = scree.pack([torch.randn(n, 3, generator=g) for n in (6, 1, 0, 4)])
    padded, mask = scree.to_padded(arr, fill_value=7.0)
    assert padded.shape == (4, 6, 3) and mask.dtype == torch.bool
    assert bool((padded[~mask] == 7.0).all())
    again = scree.from_padded(padded, mask)
    assert torch.equal(again.values, arr.values)
    assert torch.equal(again.offsets, arr.offsets)


def test_padding_side_must_be_left_or_right():
    arr = scree.pack([np.zeros((2, 1), np.float32)])
    with pytest.raises(ValueError, match=r"side"):
        scree.to_padded(arr, side="center")
