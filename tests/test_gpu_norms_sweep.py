"""Seeded random sweep of norm and varlen-softmax shapes against the oracle.

The hand-picked shapes of the other norm tests cover the vector path, odd
widths and tiny rows; these draw row counts (log-uniform, 1 to ~4,000) and
widths (powers of two up to 8,192 on the vector path, arbitrary widths up to
6,000 on the generic one, and widths past the vector path's register
capacity) with every dtype and parameter combination, through the same
checks.  The draw is fixed by its seed; each case prints its parameters
before it touches the GPU.
"""

import numpy as np
import pytest
import torch

from test_gpu_add_rmsnorm import test_add_rmsnorm_fwd_bwd as _add_case
from test_gpu_norms import test_layernorm_fwd_bwd as _ln_case
from test_gpu_norms import test_rmsnorm_fwd_bwd as _rms_case

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _draw(rng):
    rows = int(np.exp(rng.uniform(0, np.log(4000))))
    kind = rng.integers(3)
    if kind == 0:
        dim = int(2 ** rng.integers(3, 14))       # 8 .. 8192
    elif kind == 1:
        dim = int(rng.integers(1, 6000))          # any width: generic path unless aligned
    else:
        dim = int(rng.choice([4104, 8200, 12288]))  # past one row per wave's registers for some dtypes
    return rows, dim, DTYPES[int(rng.integers(3))]


def _cases(seed, n):
    rng = np.random.default_rng(seed)
    return [(i, *_draw(rng), int(rng.integers(4))) for i in range(n)]


RMS = _cases(11, 16)
LN = _cases(12, 16)
ADD = _cases(13, 10)


@pytest.mark.parametrize("case", RMS, ids=[f"rms{c[0]}" for c in RMS])
def test_random_rmsnorm(case):
    _, rows, dim, dtype, flags = case
    _rms_case(dtype, (rows, dim), with_w=bool(flags & 1))


@pytest.mark.parametrize("case", LN, ids=[f"ln{c[0]}" for c in LN])
def test_random_layernorm(case):
    _, rows, dim, dtype, flags = case
    _ln_case(dtype, (rows, dim), params=["wb", "w", "none", "b"][flags])


@pytest.mark.parametrize("case", ADD, ids=[f"add{c[0]}" for c in ADD])
def test_random_add_rmsnorm(case):
    _, rows, dim, dtype, flags = case
    with_w, with_dh = [(True, True), (True, False), (False, True), (True, True)][flags]
    _add_case(dtype, (rows, dim), with_w, with_dh)


def _softmax_cases(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        batch = int(rng.integers(1, 40))
        lengths = [int(x) for x in rng.choice([0, 1, 2, 63, 64, 65, 511, 512, 513, 640, 641, 1024, 1025,
                                                int(rng.integers(1, 3000))], batch)]
        feats = [(), (int(rng.integers(1, 9)),), (int(rng.integers(1, 200)),), (2, int(rng.integers(1, 40)))]
        features = feats[int(rng.integers(4))]
        while sum(lengths) * max(1, int(np.prod(features))) > 3_000_000:
            lengths[int(np.argmax(lengths))] //= 2
        out.append((i, lengths, features, DTYPES[int(rng.integers(3))]))
    return out


SOFTMAX = _softmax_cases(14, 12)


@pytest.mark.parametrize("case", SOFTMAX, ids=[f"softmax{c[0]}" for c in SOFTMAX])
def test_random_varlen_softmax(case):
    from test_gpu_softmax import _run

    i, lengths, features, dtype = case
    if sum(lengths) == 0:
        lengths = lengths + [1]
    _run(lengths, features, dtype, seed=900 + i)
