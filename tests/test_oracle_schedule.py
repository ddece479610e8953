"""Pins the schedule oracle by brute force: coverage, order and tie-breaking."""

import numpy as np
import pytest

from oracle.core import offsets_from_lengths
from oracle.schedule import block_counts, build_schedule, item_cost, seq_order
from scree_amd import workloads


def _cases():
    yield [1]
    yield [0, 5, 0]
    yield [128, 129, 127, 1, 256]
    yield workloads.config3().lengths
    yield workloads.config3(fixed=True).lengths
    yield workloads.config5().lengths
    rng = np.random.default_rng(0)
    for _ in range(5):
        yield [int(x) for x in rng.integers(0, 2000, size=int(rng.integers(1, 60)))]


@pytest.mark.parametrize("causal", [False, True])
def test_schedule_covers_each_block_once_in_cost_order(causal):
    for lengths in _cases():
        off = offsets_from_lengths(lengths)
        nblk = block_counts(off, 128)
        items = build_schedule(off, 128, causal)
        want = {(s, b) for s in range(len(lengths)) for b in range(int(nblk[s]))}
        got = [tuple(map(int, it)) for it in items]
        assert len(got) == len(want) and set(got) == want
        costs = [item_cost(it, nblk, causal) for it in items]
        assert all(a >= b for a, b in zip(costs, costs[1:]))
        # inside one cost the order follows the (-nblk, seq) rank
        rank = {s: r for r, s in enumerate(seq_order(nblk))}
        for (a, ca), (b, cb) in zip(zip(got, costs), zip(got[1:], costs[1:])):
            if ca == cb and a[0] != b[0]:
                assert rank[a[0]] < rank[b[0]]


def test_schedule_small_causal_example_by_hand():
    # lengths 300, 100, 200 -> nblk 3, 1, 2; rank: seq0, seq2, seq1
    items = build_schedule(offsets_from_lengths([300, 100, 200]), 128, True)
    assert items.tolist() == [[0, 2], [0, 1], [2, 1], [0, 0], [2, 0], [1, 0]]
    items = build_schedule(offsets_from_lengths([300, 100, 200]), 128, False)
    assert items.tolist() == [[0, 0], [0, 1], [0, 2], [2, 0], [2, 1], [1, 0]]


def test_sequence_major_list_by_hand_and_coverage():
    from oracle.schedule import build_schedule_by_sequence

    # lengths 300, 100, 200 -> nblk 3, 1, 2; rank: seq0, seq2, seq1
    items = build_schedule_by_sequence(offsets_from_lengths([300, 100, 200]), 128)
    assert items.tolist() == [[0, 2], [0, 1], [0, 0], [2, 1], [2, 0], [1, 0]]
    for lengths in _cases():
        off = offsets_from_lengths(lengths)
        a = build_schedule_by_sequence(off, 128)
        b = build_schedule(off, 128, True)
        assert sorted(map(tuple, a.tolist())) == sorted(map(tuple, b.tolist()))
        # each sequence's blocks are contiguous and descending
        seqs = a[:, 0].tolist()
        for s in set(seqs):
            idx = [i for i, x in enumerate(seqs) if x == s]
            assert idx == list(range(idx[0], idx[0] + len(idx)))
        for i in range(1, len(a)):
            if a[i, 0] == a[i - 1, 0]:
                assert a[i, 1] == a[i - 1, 1] - 1



def test_large_batch_lists_fall_back_to_natural_order():
    """Past max_batch sequences both lists keep index order: the first by
    sequence then block ascending, the second by sequence then block
    descending, covering the same items as the sorted lists would."""
    from oracle.schedule import build_schedule_by_sequence

    lengths = [300, 0, 100, 200, 129]
    off = offsets_from_lengths(lengths)
    for causal in (False, True):
        items = build_schedule(off, 128, causal, max_batch=4)
        assert items.tolist() == [[0, 0], [0, 1], [0, 2], [2, 0], [3, 0], [3, 1], [4, 0], [4, 1]]
        assert build_schedule(off, 128, causal, max_batch=5).tolist() != items.tolist()
    seq = build_schedule_by_sequence(off, 128, max_batch=4)
    assert seq.tolist() == [[0, 2], [0, 1], [0, 0], [2, 0], [3, 1], [3, 0], [4, 1], [4, 0]]
