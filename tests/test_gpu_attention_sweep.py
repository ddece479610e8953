"""Seeded random sweep of attention shapes against the oracle.

The other GPU tests pick their shapes by hand (edge lengths, the configs,
head ratios).  These draw them: batch sizes, lengths (log-normal, uniform,
and the 64/128-row tile edges mixed in), head counts with every grouped-query
ratio that divides them, head_dim 16-256, fp16 / bf16 / fp32, causal or not.
The draw is fixed by its seed, so every run checks the same cases; each case
prints its parameters before it touches the GPU.  Sizes stay small enough
for the fp64 oracle (at most ~2,400 tokens).
"""

import numpy as np
import pytest
import torch

from test_gpu_attention import _run_case
from test_gpu_attention_fp32 import run_fp32_case

pytestmark = pytest.mark.gpu

TILE_EDGES = [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 191, 255, 256, 257]


def _draw(rng, max_tokens):
    kind = rng.integers(3)
    batch = int(rng.integers(1, 24))
    if kind == 0:  # log-normal around a random mean
        mean = float(rng.uniform(16, 300))
        lengths = np.maximum(1, rng.lognormal(np.log(mean), 0.8, batch)).astype(int)
    elif kind == 1:  # uniform
        lengths = rng.integers(1, 400, batch)
    else:  # tile edges, with empty sequences among them
        lengths = rng.choice(TILE_EDGES + [0], batch)
    lengths = [int(x) for x in lengths]
    while sum(lengths) > max_tokens:
        lengths[int(np.argmax(lengths))] //= 2
    if sum(lengths) == 0:
        lengths[0] = 1
    heads = int(rng.choice([1, 2, 3, 4, 6, 8]))
    ratios = [r for r in (1, 2, 3, 4, 6, 8) if heads % r == 0]
    kv_heads = heads // int(rng.choice(ratios))
    return lengths, heads, kv_heads


def _cases(seed, n, max_tokens):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        lengths, heads, kv_heads = _draw(rng, max_tokens)
        dim = int(rng.choice([16, 32, 64, 128, 256]))
        causal = bool(rng.integers(2))
        out.append((i, lengths, heads, kv_heads, dim, causal))
    return out


HALF = _cases(2024, 24, 2400)
FP32 = _cases(7, 8, 900)


@pytest.mark.parametrize("case", HALF, ids=[f"half{c[0]}" for c in HALF])
def test_random_shapes_half(case):
    i, lengths, heads, kv_heads, dim, causal = case
    dtype = torch.float16 if i % 2 == 0 else torch.bfloat16
    _run_case(lengths, heads, dim, dtype, causal, seed=100 + i, kv_heads=kv_heads)


@pytest.mark.parametrize("case", FP32, ids=[f"fp32_{c[0]}" for c in FP32])
def test_random_shapes_fp32(case):
    i, lengths, heads, kv_heads, dim, causal = case
    run_fp32_case(lengths, heads, dim, causal, seed=300 + i, kv_heads=kv_heads)
