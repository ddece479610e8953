"""Synthetic varlen workloads and their algorithmic work.

Sequence lengths follow the reference's benchmark sampler
(``benchmarks/bench_throughput.py:31-34``): ``rng.lognormal(mean=ln(mean_len),
sigma, size=B)`` with ``np.random.default_rng(seed)``, truncated by ``int()``
and clipped.  The attention configs that name a total token count rescale the
draw to that total: scale, floor, clamp to the minimum, then hand the
remaining tokens to the largest fractional remainders.

The FLOP and byte counts are the algorithmic work the throughput numbers are
quoted on:

* attention forward ``F = 4 * H * D * pairs``, ``pairs = sum L(L+1)/2`` when
  causal and ``sum L^2`` otherwise; forward+backward ``= 3.5 * F`` (two GEMMs
  forward, five backward); recomputation and masked tile work are not counted;
* norms: compulsory HBM bytes, ``2*s*N*Hd + s*Hd*(1 RMS | 2 LN)`` forward and
  ``3*s*N*Hd + s*Hd + s*Hd*(1 RMS | 2 LN)`` backward, ``s`` bytes per element.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

# Fixed 16-sequence list of the reference's H100 benchmark
# (benchmarks/modal_bench.py:81); sums to 12160 tokens.
MODAL_BENCH_LENGTHS = [512, 1024, 768, 256, 2048, 384, 896, 640, 1536, 320, 1152, 480, 704, 192, 832, 416]


def lognormal_lengths(num_seqs: int, mean_len: float, sigma: float, seed: int = 0,
                      lo: int = 1, hi: Optional[int] = None) -> List[int]:
    rng = np.random.default_rng(seed)
    draw = rng.lognormal(mean=np.log(mean_len), sigma=sigma, size=num_seqs)
    out = []
    for x in draw:
        n = max(lo, int(x))
        if hi is not None:
            n = min(hi, n)
        out.append(n)
    return out


def rescaled_lengths(num_seqs: int, total: int, sigma: float, seed: int = 0, lo: int = 1) -> List[int]:
    rng = np.random.default_rng(seed)
    draw = rng.lognormal(mean=np.log(total / num_seqs), sigma=sigma, size=num_seqs)
    exact = draw * (total / draw.sum())
    base = [max(lo, int(math.floor(x))) for x in exact]
    rem = total - sum(base)
    frac = sorted(range(num_seqs), key=lambda i: (-(exact[i] - math.floor(exact[i])), i))
    i = 0
    while rem > 0:
        base[frac[i % num_seqs]] += 1
        rem -= 1
        i += 1
    while rem < 0:  # only when clamping to lo overshot; take from the longest
        j = max(range(num_seqs), key=lambda t: (base[t], -t))
        base[j] -= 1
        rem += 1
    return base


def causal_pairs(lengths) -> int:
    return int(sum(int(n) * (int(n) + 1) // 2 for n in lengths))


def full_pairs(lengths) -> int:
    return int(sum(int(n) * int(n) for n in lengths))


def attn_fwd_flops(lengths, heads: int, head_dim: int, causal: bool) -> float:
    pairs = causal_pairs(lengths) if causal else full_pairs(lengths)
    return 4.0 * heads * head_dim * pairs


def attn_fwd_bwd_flops(lengths, heads: int, head_dim: int, causal: bool) -> float:
    return 3.5 * attn_fwd_flops(lengths, heads, head_dim, causal)


def norm_fwd_bytes(rows: int, dim: int, elem_bytes: int, layer: bool) -> float:
    return 2.0 * elem_bytes * rows * dim + elem_bytes * dim * (2 if layer else 1)


def norm_bwd_bytes(rows: int, dim: int, elem_bytes: int, layer: bool) -> float:
    return 3.0 * elem_bytes * rows * dim + elem_bytes * dim + elem_bytes * dim * (2 if layer else 1)


@dataclass
class AttnConfig:
    name: str
    lengths: List[int]
    heads: int
    head_dim: int
    dtype: str
    causal: bool = True
    backward: bool = False

    @property
    def total(self) -> int:
        return int(sum(self.lengths))

    def fwd_flops(self) -> float:
        return attn_fwd_flops(self.lengths, self.heads, self.head_dim, self.causal)

    def step_flops(self) -> float:
        f = self.fwd_flops()
        return 3.5 * f if self.backward else f


@dataclass
class NormConfig:
    name: str
    lengths: List[int]
    hidden: int
    dtype: str
    eps: float = 1e-6
    extra: dict = field(default_factory=dict)

    @property
    def total(self) -> int:
        return int(sum(self.lengths))


def config1_lengths() -> List[int]:
    return lognormal_lengths(16, 128, 0.6, seed=0, lo=1, hi=512)


def config2() -> NormConfig:
    return NormConfig("cfg2_norms_bf16_64x4096", lognormal_lengths(64, 256, 0.6, seed=0, lo=1, hi=2048),
                      4096, "bf16", eps=1e-6)


def config3(fixed: bool = False) -> AttnConfig:
    lengths = list(MODAL_BENCH_LENGTHS) if fixed else rescaled_lengths(16, 12160, 0.6, seed=0, lo=1)
    tag = "fixed" if fixed else "rescaled"
    return AttnConfig(f"cfg3_attn_fwd_fp16_12160tok_16x64_{tag}", lengths, 16, 64, "fp16", True, False)


def config4(fixed: bool = False) -> AttnConfig:
    c = config3(fixed)
    c.name = c.name.replace("cfg3_attn_fwd", "cfg4_attn_fwdbwd")
    c.backward = True
    return c


def config5() -> AttnConfig:
    lengths = lognormal_lengths(32, 2048, 1.2, seed=0, lo=16, hi=16384)
    return AttnConfig("cfg5_attn_fwdbwd_bf16_32x128", lengths, 32, 128, "bf16", True, True)
