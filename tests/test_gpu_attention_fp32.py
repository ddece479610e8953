"""GPU parity of the fp32 attention kernels (the Array-level call on fp32
values) against the fp64 oracle.

The reference's Array-level ``varlen_attention`` computes fp32 arrays as
given (its torch branch, ``reference/varlen_attention.py:90-113``); here they
run on the FP32-FMA kernels through the same C entry points, with autograd.
Every operand stays fp32.  Bound: the reference's own fp32 one
(``tests/test_varlen_kernels.py`` of the reference: 1e-5), plus the rounding
of the stored result (``2^-24 |ref|``) and ``E_ref``, the amount by which the
reference's fp32 arithmetic itself departs from the fp64 oracle beyond that
rounding on the same inputs (``parity.reference_excess``): a key early in a
long causal sequence, summed over a head group, collects dV from ~1,000
queries, and fp32 sums of that many terms carry ~1e-5 of absolute error at
|dV| ~ 30 in either arithmetic.  The logsumexp is held to 1e-5.
"""

import numpy as np
import pytest
import torch

from oracle.attention import attention_bwd, attention_fwd
from parity import check_attn, check_close, cu_of, np64, randn, reference_excess, say

pytestmark = pytest.mark.gpu

EDGE_LENGTHS = [1, 63, 64, 65, 127, 128, 129, 255, 300, 2]
TOL = 1e-5


def run_fp32_case(lengths, heads, dim, causal, seed, kv_heads=None, sigma=1.0):
    import scree_amd
    from scree_amd.kernels import varlen_attention
    from scree_amd.kernels.hip import attention as A

    kv_heads = heads if kv_heads is None else kv_heads
    say(f"case: fp32 lengths[:6]={lengths[:6]} B={len(lengths)} N={sum(lengths)} H={heads} "
        f"Hkv={kv_heads} D={dim} causal={causal} sigma={sigma}")
    n = sum(lengths)
    off, cu = cu_of(lengths)
    q = randn((n, heads, dim), torch.float32, seed, scale=sigma)
    k = randn((n, kv_heads, dim), torch.float32, seed + 1, scale=sigma)
    v = randn((n, kv_heads, dim), torch.float32, seed + 2)
    do = randn((n, heads, dim), torch.float32, seed + 3)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    arr = lambda t: scree_amd.Array(values=t, offsets=cu)  # noqa: E731
    out = varlen_attention(arr(qa), arr(ka), arr(va), causal=causal)
    assert out.values.dtype == torch.float32 and out.offsets is cu
    out.values.backward(do)
    # the LSE through the launcher-level entry (same kernels, fp32 buffers)
    lse = torch.empty((n, heads), dtype=torch.float32, device="cuda")
    o2 = torch.empty_like(q)
    ws = A.prepare_workspace(cu, n, dim, causal, heads)
    A._attn_fwd(q, k, v, cu, causal, o2, lse, ws)
    torch.cuda.synchronize()
    assert torch.equal(o2, out.values.detach())
    q64, k64, v64, do64 = np64(q), np64(k), np64(v), np64(do)
    lse64 = lse.cpu().numpy().astype(np.float64)
    ref_o, ref_lse = attention_fwd(q64, k64, v64, off, causal=causal)
    e_ref = reference_excess(q64, k64, v64, do64, off, causal, torch.float32,
                             o=np64(out.values), lse=lse64)
    check_attn("O", np64(out.values), ref_o, TOL, torch.float32, e_ref["O"])
    check_close("LSE", lse64, ref_lse, TOL)
    rdq, rdk, rdv, _ = attention_bwd(do64, q64, k64, v64, np64(out.values), ref_lse, off,
                                     causal=causal)
    check_attn("dQ", np64(qa.grad), rdq, TOL, torch.float32, e_ref["dQ"])
    check_attn("dK", np64(ka.grad), rdk, TOL, torch.float32, e_ref["dK"])
    check_attn("dV", np64(va.grad), rdv, TOL, torch.float32, e_ref["dV"])


@pytest.mark.parametrize("dim", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_edge_lengths(dim, causal):
    run_fp32_case(EDGE_LENGTHS, 2, dim, causal, seed=300 + dim)


@pytest.mark.parametrize("dim", [32, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_grouped_query(dim, causal):
    """8 query heads on 2 K/V heads: dK / dV sum over each group of 4."""
    run_fp32_case(EDGE_LENGTHS, 8, dim, causal, seed=400 + dim, kv_heads=2)


def test_fp32_large_logits():
    """q, k ~ N(0, 2^2): scaled scores with standard deviation 4, where a
    softmax without the running maximum would overflow nothing in fp32 but
    loses every weight but the largest to rounding."""
    run_fp32_case([700, 33, 1], 2, 64, True, seed=500, sigma=2.0)


def test_fp32_past_64_sequences():
    """80 sequences: the work list comes from the scheduler launch, not the
    forward's own derivation."""
    from scree_amd.kernels.hip import attention as A

    rng = np.random.default_rng(7)
    lengths = [int(x) for x in rng.integers(1, 200, size=80)]
    assert A.needs_schedule(len(lengths), sum(lengths), 2, 64)
    run_fp32_case(lengths, 2, 64, True, seed=600)


def f32_form(lengths, heads, dim):
    """The column layout an fp32 launch takes: "narrow" (16 columns per lane)
    unless that form would give the 1,024 SIMDs less than a wave each and
    head_dim is below 256 ("wide": max(4, dim / 16) columns per lane).
    Restates the launchers' choice so each test knows which form it checks."""
    tmax = -(-sum(lengths) // 128) + len(lengths)
    tpr = dim // 16
    rows = 64 if 64 * tpr <= 512 else 512 // tpr
    waves = -(-(rows * tpr) // 64)
    if max(4, dim // 16) == 16:
        return "narrow"
    return "wide" if tmax * heads * 2 * waves < 1024 else "narrow"


@pytest.mark.parametrize("dim,heads", [(16, 72), (32, 40), (64, 20), (128, 10)])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_narrow_form(dim, heads, causal):
    """Launches large enough for the narrow form (the other tests here are
    small enough for the wide one)."""
    lengths = [200, 129, 64, 300, 17, 1, 90, 255, 128, 40, 77, 150, 33, 96, 5, 250]
    assert f32_form(lengths, heads, dim) == "narrow"
    run_fp32_case(lengths, heads, dim, causal, seed=800 + dim, kv_heads=heads // 2)


def test_fp32_forms_of_the_other_tests():
    """Both forms are covered at every head_dim below 256."""
    for dim in (16, 32, 64, 128):
        assert f32_form(EDGE_LENGTHS, 2, dim) == "wide"
    assert f32_form(EDGE_LENGTHS, 8, 128) == "narrow"  # the grouped-query case
    assert f32_form(EDGE_LENGTHS, 2, 256) == "narrow"


def test_fp32_run_to_run_identical():
    import scree_amd
    from scree_amd.kernels import varlen_attention

    lengths = [129, 1, 300]
    say(f"case: fp32 determinism lengths={lengths} H=4 D=64 causal")
    off, cu = cu_of(lengths)
    n = sum(lengths)
    q, k, v = (randn((n, 4, 64), torch.float32, 700 + s) for s in range(3))
    outs = [varlen_attention(*(scree_amd.Array(values=t, offsets=cu) for t in (q, k, v)),
                             causal=True).values for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("heads", [4, 40])  # the wide form, then the narrow one
def test_fp32_strided_views_match_contiguous(heads):
    """q, k, v as views into one packed (tokens, 3, heads, 64) fp32 buffer, read
    in place with its strides: the same values as contiguous copies, and the
    same gradients."""
    import scree_amd
    from scree_amd.kernels import varlen_attention

    lengths = [70, 33, 190, 1]
    say(f"case: fp32 strided qkv views H={heads}")
    n = sum(lengths)
    _, cu = cu_of(lengths)
    qkv = randn((n, 3, heads, 64), torch.float32, 17)
    do = randn((n, heads, 64), torch.float32, 18)

    def run(q, k, v):
        qa, ka, va = (t.detach().requires_grad_(True) for t in (q, k, v))
        out = varlen_attention(*(scree_amd.Array(values=t, offsets=cu) for t in (qa, ka, va)),
                               causal=True)
        out.values.backward(do)
        return out.values.detach(), qa.grad, ka.grad, va.grad

    strided = run(qkv[:, 0], qkv[:, 1], qkv[:, 2])
    contig = run(qkv[:, 0].contiguous(), qkv[:, 1].contiguous(), qkv[:, 2].contiguous())
    torch.cuda.synchronize()
    assert not qkv[:, 0].is_contiguous()
    for a, b in zip(strided, contig):
        assert torch.equal(a, b)
