"""GPU parity of the varlen softmax (forward and backward) against the oracle.

Bounds: fp32 1e-5, half 1e-3 max-abs (the norms' half-precision bound),
plus for fp16/bf16 results the output-rounding term u*|reference|.  The
oracle runs in fp64 on the same rounded inputs.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle.softmax import varlen_softmax, varlen_softmax_bwd
from parity import UNIT, check_close, cu_of, np64, randn, say

pytestmark = pytest.mark.gpu

ATOL = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 1e-3}
LENGTHS = [1, 0, 5, 64, 65, 300, 2, 2001, 17]


def _run(lengths, features, dtype, seed, scale=3.0):
    from scree_amd.kernels.hip import varlen_softmax_hip, varlen_softmax_hip_backward

    n = int(sum(lengths))
    say(f"case: B={len(lengths)} N={n} features={features} {dtype}")
    off, cu = cu_of(lengths)
    x = randn((n,) + features, dtype, seed, scale=scale)
    dy = randn((n,) + features, dtype, seed + 1)
    y = varlen_softmax_hip(x, cu)
    assert y.dtype == dtype and y.shape == x.shape
    ry = varlen_softmax(np64(x), off)
    u = 0.0 if dtype == torch.float32 else UNIT[dtype]  # output rounding of a half result
    check_close("y", np64(y), ry, ATOL[dtype], extra=np.abs(ry), unit=u)
    dx = varlen_softmax_hip_backward(y, dy, cu)
    # the backward consumes the rounded y the forward produced
    rdx = varlen_softmax_bwd(np64(y), np64(dy), off)
    check_close("dx", np64(dx), rdx, ATOL[dtype], extra=np.abs(rdx), unit=u)
    return y


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("features", [(), (3,), (8,), (4, 16), (1000,)])
def test_softmax_shapes(dtype, features):
    _run(LENGTHS, features, dtype, seed=len(features) + 3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_register_capacity_boundary(dtype):
    """64 features: the forward narrows to 8 column lanes (full 128-byte
    lines) of 512 threads, whose 64 row lanes hold 8 rows each in registers
    (512 rows; from 513 on, the rows past 512 are streamed first and
    re-read).  The backward stops at 8 column lanes too, whose 64 row lanes
    hold 10 rows of y and dy (640 rows; 641 are re-read)."""
    _run([512, 513, 640, 641, 1024, 1025, 3], (64,), dtype, seed=11)


def test_rows_sum_to_one_and_masked_entries():
    from scree_amd.kernels.hip import varlen_softmax_hip

    lengths = [3, 7, 1, 40]
    off, cu = cu_of(lengths)
    x = randn((51, 24), torch.float32, 11)
    x[0:2, 5] = float("-inf")       # masked entries inside a sequence
    x[5, :] = float("-inf")         # a fully masked row of sequence 1 (rows 3..9)
    y = varlen_softmax_hip(x, cu)
    yn = y.cpu().numpy()
    assert np.all(yn[0:2, 5] == 0.0) and np.all(yn[5] == 0.0)
    for i in range(len(lengths)):
        np.testing.assert_allclose(yn[off[i]:off[i + 1]].sum(axis=0), 1.0, atol=1e-5)
    ry = varlen_softmax(np64(x), off)
    check_close("y", yn.astype(np.float64), ry, 1e-5)
    # a sequence whose column is -inf throughout has no softmax: NaN, as torch.softmax
    x[10, :] = float("-inf")        # sequence 2 is the single row 10
    y = varlen_softmax_hip(x, cu).cpu()
    assert torch.isnan(y[10]).all()
    assert torch.isnan(torch.softmax(x[10:11].cpu(), dim=0)).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("length", [300, 5000])
def test_non_finite_inputs_match_two_pass_semantics(length, dtype):
    """NaN, +inf and all -inf columns give what the max-subtracted two-pass
    formula (the oracle, pinned to torch.softmax) gives: NaN throughout the
    affected column.  5000 rows of 8 fp32 columns exceed what the forward keeps
    in registers (8 rows per row lane: 2,048 rows in fp32, whose 8 columns
    are two 16-byte vectors, 256 row lanes; 4,096 in bf16, one vector, 512
    row lanes), so the online update of the rows past those, its merge with
    the held rows' result and the row-lane merge all see non-finite values
    (column 3 has a +inf on each side: rows 5 and length - 3); 300 rows stay
    held."""
    from scree_amd.kernels.hip import varlen_softmax_hip

    say(f"case: non-finite softmax length {length} {dtype}")
    lengths = [length, 7]
    off, cu = cu_of(lengths)
    x = randn((sum(lengths), 8), dtype, 31)
    x[length // 3, 1] = float("nan")
    x[length - 2, 2] = float("inf")
    x[5, 3] = float("inf")
    x[length - 3, 3] = float("inf")                   # two +inf in one column
    x[:length, 4] = float("-inf")                      # a column with no finite value
    x[7, 5] = float("nan")
    x[:length, 5][x[:length, 5] == x[:length, 5]] = float("-inf")  # only -inf and one NaN
    x[:length, 6] = float("-inf")
    x[length - 1, 6] = 1.0                             # one finite value among -inf
    y = varlen_softmax_hip(x, cu)
    torch.cuda.synchronize()
    want = varlen_softmax(np64(x), off)
    got = np64(y)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    u = 0.0 if dtype == torch.float32 else UNIT[dtype]
    check_close("y (finite entries)", got[fin], want[fin], ATOL[dtype], extra=np.abs(want[fin]), unit=u)
    assert np.isnan(got[:length, 1:6]).all()
    assert got[length - 1, 6] == 1.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_nan_held_alone_in_its_row_lane(dtype):
    """A NaN among finite values of a short sequence: every row lane holds at
    most one row, so the lane holding the NaN has no other value.  Its max
    (v_max3 skips NaN) is -inf, and its sum must still carry the NaN so that
    the column is NaN throughout, as in the two-pass formula."""
    from scree_amd.kernels.hip import varlen_softmax_hip

    say(f"case: NaN alone in its row lane {dtype}")
    lengths = [10, 3, 40]
    off, cu = cu_of(lengths)
    x = randn((sum(lengths), 8), dtype, 41)
    x[4, 1] = float("nan")           # sequence 0
    x[13 + 20, 6] = float("nan")     # sequence 2
    y = varlen_softmax_hip(x, cu)
    torch.cuda.synchronize()
    want = varlen_softmax(np64(x), off)
    got = np64(y)
    assert np.isnan(want[0:10, 1]).all() and np.isnan(want[13:53, 6]).all()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    u = 0.0 if dtype == torch.float32 else UNIT[dtype]
    check_close("y (finite entries)", got[fin], want[fin], ATOL[dtype], extra=np.abs(want[fin]), unit=u)


def test_non_contiguous_view():
    from scree_amd.kernels.hip import varlen_softmax_hip

    lengths = [9, 33]
    off, cu = cu_of(lengths)
    base = randn((42, 17), torch.float16, 12)
    x = base[:, 1:]  # a strided view: the launcher reads a contiguous copy
    y = varlen_softmax_hip(x, cu)
    check_close("y", np64(y), varlen_softmax(np64(x), off), 1e-3)


def test_config2_shape_full_size():
    """Config-2 lengths and width (19,758 x 4096, bf16): sums to one everywhere, parity on samples."""
    from scree_amd import workloads
    from scree_amd.kernels.hip import varlen_softmax_hip

    cfg = workloads.config2()
    off, cu = cu_of(cfg.lengths)
    x = randn((cfg.total, cfg.hidden), torch.bfloat16, 13, scale=2.0)
    y = varlen_softmax_hip(x, cu)
    seg = torch.repeat_interleave(torch.arange(len(cfg.lengths), device="cuda"),
                                  torch.tensor(cfg.lengths, device="cuda"))
    sums = torch.zeros(len(cfg.lengths), cfg.hidden, device="cuda").index_add_(0, seg, y.float())
    # each column of each sequence sums to 1 up to bf16 output rounding (u per term)
    worst = float((sums - 1).abs().max())
    say(f"  column sums: max |sum - 1| = {worst:.3e}")
    assert worst < 2e-2
    for i in (0, 7, int(np.argmax(cfg.lengths)), len(cfg.lengths) - 1):
        s, e = int(off[i]), int(off[i + 1])
        ry = varlen_softmax(np64(x[s:e]), np.array([0, e - s]))
        check_close(f"seq {i}", np64(y[s:e]), ry, 1e-3, extra=np.abs(ry), unit=UNIT[torch.bfloat16])


def test_autograd_and_array_api():
    import scree_amd
    from scree_amd.kernels import varlen_softmax as array_softmax

    lengths = [4, 0, 19]
    off, cu = cu_of(lengths)
    x = randn((23, 6), torch.float32, 14).requires_grad_(True)
    dy = randn((23, 6), torch.float32, 15)
    arr = scree_amd.Array(values=x, offsets=cu, ragged_dim=0)
    out = array_softmax(arr)
    assert out.offsets is arr.offsets
    out.values.backward(dy)
    yo = varlen_softmax(np64(x), off)
    check_close("y", np64(out.values), yo, 1e-5)
    check_close("dx", np64(x.grad), varlen_softmax_bwd(yo, np64(dy), off), 1e-5)


def test_softmax_deterministic():
    from scree_amd.kernels.hip import varlen_softmax_hip

    off, cu = cu_of(LENGTHS)
    x = randn((sum(LENGTHS), 64), torch.bfloat16, 16)
    a = varlen_softmax_hip(x, cu)
    b = varlen_softmax_hip(x, cu)
    assert torch.equal(a, b)


def test_matches_golden():
    from scree_amd.kernels.hip import varlen_softmax_hip, varlen_softmax_hip_backward

    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "softmax_4x16.npz"))
    x = torch.from_numpy(g["x"]).cuda()
    cu = torch.from_numpy(g["offsets"]).cuda()
    y = varlen_softmax_hip(x, cu)
    check_close("y", np64(y), g["y"].astype(np.float64), 1e-3)
    dx = varlen_softmax_hip_backward(y, torch.from_numpy(g["dy"]).cuda(), cu)
    want = g["dx"].astype(np.float64)
    check_close("dx", np64(dx), want, 1e-3, extra=np.abs(want), unit=UNIT[torch.float16])
