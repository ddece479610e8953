"""GPU parity of the HIP attention kernels against the oracle.

Every case prints its name before touching the GPU.  Inputs are seeded,
rounded to the kernel dtype, and the oracle runs in fp64 on those rounded
values.  Tolerances: see ``tests/parity.py``.
"""

import numpy as np
import pytest
import torch

from oracle.attention import attention_bwd, attention_fwd
from oracle.schedule import build_schedule, build_schedule_by_sequence
from parity import UNIT, check_attn, check_close, cu_of, np64, randn, reference_excess, say
from scree_amd import workloads

pytestmark = pytest.mark.gpu

EDGE_LENGTHS = [1, 63, 64, 65, 127, 128, 129, 255, 300, 2]


def _run_case(lengths, heads, dim, dtype, causal, seed=0, backward=True, kv_heads=None):
    kv_heads = heads if kv_heads is None else kv_heads
    say(f"case: lengths[:6]={lengths[:6]} B={len(lengths)} N={sum(lengths)} H={heads} "
        f"Hkv={kv_heads} D={dim} {dtype} causal={causal}")
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    n = sum(lengths)
    off, cu = cu_of(lengths)
    q = randn((n, heads, dim), dtype, seed)
    k = randn((n, kv_heads, dim), dtype, seed + 1)
    v = randn((n, kv_heads, dim), dtype, seed + 2)
    out, lse = varlen_attention_hip(q, k, v, cu, causal=causal, return_lse=True)
    torch.cuda.synchronize()
    q64, k64, v64 = np64(q), np64(k), np64(v)
    ref_o, ref_lse = attention_fwd(q64, k64, v64, off, causal=causal)
    bf16 = dtype == torch.bfloat16
    do = randn((n, heads, dim), dtype, seed + 3) if backward else None
    do64 = np64(do) if backward else None

    def check(name, got, want, atol):
        if bf16:  # atol + u|ref| + the reference arithmetic's own excess (tests/parity.py)
            return check_attn(name, got, want, atol, dtype, e_ref[name])
        return check_close(name, got, want, atol)

    e_ref = (reference_excess(q64, k64, v64, do64, off, causal, dtype, o=np64(out),
                              lse=lse.cpu().numpy().astype(np.float64)) if bf16 else None)
    check("O", np64(out), ref_o, 2e-3)
    check_close("LSE", lse.cpu().numpy().astype(np.float64), ref_lse, 1e-4 + 1e-5 * np.abs(ref_lse).max())
    if not backward:
        return
    dq, dk, dv = varlen_attention_hip_backward(do, q, k, v, out, lse, cu, causal=causal)
    torch.cuda.synchronize()
    rdq, rdk, rdv, _ = attention_bwd(do64, q64, k64, v64, np64(out), ref_lse, off, causal=causal)
    check("dQ", np64(dq), rdq, 5e-3)
    check("dK", np64(dk), rdk, 5e-3)
    check("dV", np64(dv), rdv, 5e-3)


@pytest.mark.parametrize("dim", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
def test_edge_lengths(dim, dtype, causal):
    _run_case(EDGE_LENGTHS, 2, dim, dtype, causal, seed=dim)


@pytest.mark.parametrize("dim", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
def test_grouped_query_edge_lengths(dim, dtype, causal):
    """Grouped-query attention: 8 query heads on 2 K/V heads (groups of 4)."""
    _run_case(EDGE_LENGTHS, 8, dim, dtype, causal, seed=100 + dim, kv_heads=2)


@pytest.mark.parametrize("heads,kv_heads", [(4, 1), (6, 3), (16, 8), (32, 4)])
def test_grouped_query_head_ratios(heads, kv_heads):
    """Group sizes 4, 2, 2, 8 (the last two with heads a multiple of 8, where the
    grid keeps each group on one XCD)."""
    _run_case([300, 17, 129, 640], heads, 64, torch.float16, True, seed=heads + kv_heads,
              kv_heads=kv_heads)


def test_grouped_query_autograd_matches_launchers():
    """The autograd path gives the launchers' dq / dk / dv bit for bit (GQA)."""
    from scree_amd.kernels.hip import (varlen_attention_hip, varlen_attention_hip_autograd,
                                       varlen_attention_hip_backward)

    lengths = [200, 1, 77, 512]
    say(f"case: gqa autograd lengths={lengths} H=8 Hkv=2 D=64 fp16")
    off, cu = cu_of(lengths)
    n = sum(lengths)
    q = randn((n, 8, 64), torch.float16, 7)
    k = randn((n, 2, 64), torch.float16, 8)
    v = randn((n, 2, 64), torch.float16, 9)
    do = randn((n, 8, 64), torch.float16, 10)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = varlen_attention_hip_autograd(qa, ka, va, cu, causal=True)
    out.backward(do)
    o2, lse = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    dq, dk, dv = varlen_attention_hip_backward(do, q, k, v, o2, lse, cu, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), o2)
    assert torch.equal(qa.grad, dq) and torch.equal(ka.grad, dk) and torch.equal(va.grad, dv)
    assert ka.grad.shape == (n, 2, 64)
    # the forward keeps only the schedule between the passes; this shape takes
    # the split dK/dV path, whose larger workspace lives only during backward
    from scree_amd.kernels.hip import attention as A
    out2 = varlen_attention_hip_autograd(qa, ka, va, cu, causal=True)
    saved_ws = out2.grad_fn.saved_tensors[-1]
    assert saved_ws.numel() == A.workspace_bytes(len(lengths), n, 64)
    assert A.bwd_workspace_bytes(len(lengths), n, 8, 2, 64) > saved_ws.numel()


@pytest.mark.parametrize("heads,kv_heads,dim", [(8, 4, 128), (8, 2, 64), (16, 1, 32)])
def test_grouped_query_split_dkv_matches_single_pass(heads, kv_heads, dim):
    """Grouped-query dK/dV with each head group split over several workgroups
    (workspace sized by bwd_workspace_bytes: here 2, 4 and 16 parts) against
    the one-workgroup-per-group pass (schedule-only workspace): the same up to
    fp32 summation order before the final rounding, dQ untouched, and the
    split result bit-identical run to run."""
    from scree_amd.kernels.hip import attention as A
    from scree_amd.kernels.hip import varlen_attention_hip

    lengths = EDGE_LENGTHS
    n = sum(lengths)
    say(f"case: split dK/dV H={heads} Hkv={kv_heads} D={dim} N={n} fp16 causal")
    off, cu = cu_of(lengths)
    q = randn((n, heads, dim), torch.float16, 21)
    k = randn((n, kv_heads, dim), torch.float16, 22)
    v = randn((n, kv_heads, dim), torch.float16, 23)
    do = randn((n, heads, dim), torch.float16, 24)
    out, lse = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    small = A.attention_schedule(cu, n, dim, True)
    big = A.attention_schedule(cu, n, dim, True, A._bwd_workspace(cu, n, heads, kv_heads, dim))
    assert big.numel() > small.numel()

    def run(ws):
        dq, dk, dv = (torch.empty_like(t) for t in (q, k, v))
        delta = torch.empty(n, heads, device=q.device, dtype=torch.float32)
        A._attn_bwd(do, q, k, v, out, lse, cu, True, dq, dk, dv, delta, ws)
        torch.cuda.synchronize()
        return dq, dk, dv

    one, split, again = run(small), run(big), run(big)
    assert torch.equal(one[0], split[0])
    for name, a, b, c in zip(("dK", "dV"), one[1:], split[1:], again[1:]):
        assert torch.equal(b, c), f"{name}: split pass not deterministic"
        diff = (a.float() - b.float()).abs()
        # one fp16 ulp (2u relative): two fp32 sums on either side of a rounding boundary
        bound = 2 * UNIT[torch.float16] * torch.maximum(a.float().abs(), b.float().abs()) + 1e-5
        worst = float((diff - bound).max())
        say(f"  {name}: max |single - split| = {float(diff.max()):.3e}")
        assert worst <= 0, f"{name}: split and single pass differ by more than one rounding"


def test_single_token_sequences():
    _run_case([1, 1, 1, 1], 3, 64, torch.float16, True)


def test_empty_sequences_in_batch():
    _run_case([0, 70, 0, 0, 130, 0], 2, 64, torch.float16, True)


@pytest.mark.parametrize("batch", [64, 65, 130])
@pytest.mark.parametrize("causal", [True, False])
def test_batches_past_one_wavefront(batch, causal):
    """Batches past one wavefront of sequences (the scheduler's sort and
    scans then span several waves), with empty and multi-block sequences."""
    rng = np.random.default_rng(batch)
    lengths = [int(x) for x in rng.integers(0, 300, size=batch)]
    lengths[3] = 0
    lengths[-1] = 400
    _run_case(lengths, 2, 64, torch.float16, causal, seed=batch)


@pytest.mark.parametrize("dim,dtype", [(16, torch.float16), (256, torch.bfloat16)])
def test_scheduled_batches_at_the_extreme_head_dims(dim, dtype):
    """head_dim 16 (the 32-column kernels on zero-padded rows) and 256 (one
    wave per SIMD) past 64 sequences, where the forward reads the scheduler's
    list instead of deriving its items, with grouped K/V heads."""
    rng = np.random.default_rng(dim)
    lengths = [int(x) for x in rng.integers(0, 260, size=90)]
    lengths[7] = 0
    lengths[-1] = 513
    _run_case(lengths, 4, dim, dtype, True, seed=dim + 3, kv_heads=2)


@pytest.mark.parametrize("causal", [True, False])
def test_batch_past_the_sorting_scheduler(causal):
    """2,500 sequences (beyond the 2,048 the sorting scheduler holds in LDS):
    the lists come in natural order, with empty and multi-block sequences."""
    rng = np.random.default_rng(2500)
    lengths = [int(x) for x in rng.integers(0, 12, size=2500)]
    lengths[10] = 300
    _run_case(lengths, 2, 64, torch.float16, causal, seed=25)


@pytest.mark.parametrize("causal", [True, False])
def test_forward_publishes_the_schedule(causal):
    """A forward that needs no schedule derives its items and leaves in a
    workspace of stale bytes the header and the work-order list, bit for bit
    as the scheduler writes them (which the oracle pins): grouped-query head
    order, head_dim 128, empty sequences, one sequence, a full wave of 64,
    the largest launch that derives.  (The sequence-major list serves only
    head-major passes, which no problem small enough to derive has.)"""
    from scree_amd.kernels.hip import attention as A
    from scree_amd.kernels.hip import attention_schedule, needs_schedule, schedule_items

    rng = np.random.default_rng(31)
    c4 = workloads.config4().lengths
    cases = [  # (lengths, heads, kv_heads, head_dim)
        ([300, 17, 129, 640, 1, 0, 77], 4, 4, 64),
        ([300, 17, 129, 640, 1, 0, 77], 8, 8, 128),
        ([5], 2, 2, 32),
        (c4, 16, 16, 64),
        (c4, 18, 18, 64),                      # 1,998 workgroups: the largest that derive
        (c4, 16, 4, 64),                       # grouped-query head permutation
        ([int(x) for x in rng.integers(0, 400, size=64)], 2, 2, 32),
    ]
    for lengths, heads, kvh, d in cases:
        n, b = int(sum(lengths)), len(lengths)
        say(f"case: published schedule B={b} N={n} H={heads}/{kvh} D={d} causal={causal}")
        assert not needs_schedule(b, n, heads, d)
        off, cu = cu_of(lengths)
        q = randn((n, heads, d), torch.float16, 70)
        k, v = (randn((n, kvh, d), torch.float16, 71 + i) for i in range(2))
        stale = torch.full((A.workspace_bytes(b, n, d),), 255, dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q)
        lse = torch.empty((n, heads), dtype=torch.float32, device="cuda")
        A._attn_fwd(q, k, v, cu, causal, out, lse, stale)
        want = attention_schedule(cu, n, d, causal)
        torch.cuda.synchronize()
        assert stale[:16].view(torch.int32).tolist() == want[:16].view(torch.int32).tolist()
        cw, iw = schedule_items(want, with_ranges=True)
        cg, ig = schedule_items(stale, with_ranges=True)
        assert cg == cw
        np.testing.assert_array_equal(ig.numpy(), iw.numpy())


@pytest.mark.parametrize("causal", [True, False])
def test_backward_reads_the_forwards_lists(causal):
    """Forward then backward on one workspace of stale bytes, no schedule
    call: the same outputs and gradients, bit for bit, as the standalone
    backward, which schedules its own workspace."""
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward
    from scree_amd.kernels.hip import attention as A

    for lengths, heads in (([300, 17, 129, 640, 1, 0, 77], 4), (workloads.config4().lengths, 16)):
        n = sum(lengths)
        say(f"case: forward-built lists B={len(lengths)} N={n} H={heads} causal={causal}")
        off, cu = cu_of(lengths)
        q, k, v, do = (randn((n, heads, 64), torch.float16, 50 + i) for i in range(4))
        ref = varlen_attention_hip(q, k, v, cu, causal=causal, return_lse=True)
        ref_g = varlen_attention_hip_backward(do, q, k, v, ref[0], ref[1], cu, causal=causal)
        stale = torch.full((A.workspace_bytes(len(lengths), n, 64),), 255, dtype=torch.uint8,
                           device="cuda")
        got = varlen_attention_hip(q, k, v, cu, causal=causal, return_lse=True, workspace=stale)
        got_g = varlen_attention_hip_backward(do, q, k, v, got[0], got[1], cu, causal=causal,
                                              workspace=stale)
        torch.cuda.synchronize()
        assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])
        for a, b in zip(ref_g, got_g):
            assert torch.equal(a, b)


def test_backward_skips_items_no_schedule_wrote():
    """A backward handed a workspace whose list no schedule or forward wrote
    (crafted here: every item out of range in one of the ways the kernels
    check, the count past the grid) skips those items -- no access outside
    the tensors, the outputs left exactly as they were."""
    from scree_amd.kernels.hip import attention as A

    lengths = [300, 17, 129]
    n = sum(lengths)
    say(f"case: unscheduled workspace B={len(lengths)} N={n}")
    off, cu = cu_of(lengths)
    q, k, v, do = (randn((n, 2, 64), torch.float16, 80 + i) for i in range(4))
    o, lse = (torch.zeros((n, 2, 64), dtype=torch.float16, device="cuda"),
              torch.zeros((n, 2), dtype=torch.float32, device="cuda"))
    ws = A.attention_schedule(cu, n, 64, True)
    tmax = (n + 127) // 128 + len(lengths)
    bad = [(0, 0, -5, 10), (0, 0, 0, 0), (0, 0, n - 6, 10), (0, 3, 0, 300), (0, -1, 0, 300),
           (0, 0, 2 ** 30, 2 ** 30), (0, 0, 0, 2 ** 31 - 1)]
    items = torch.tensor([bad[p % len(bad)] for p in range(2 * tmax)], dtype=torch.int32)
    header = torch.tensor([tmax + 100, len(lengths), 128, 1], dtype=torch.int32)
    ws[:16].copy_(header.view(torch.uint8).cuda())
    ws[16:16 + 32 * tmax].copy_(items.view(torch.uint8).reshape(-1).cuda())
    outs = [torch.full_like(q, 7.0) for _ in range(3)]
    delta = torch.full((n, 2), 7.0, dtype=torch.float32, device="cuda")
    A._attn_bwd(do, q, k, v, o, lse, cu, True, *outs, delta, ws)
    torch.cuda.synchronize()
    for t in outs + [delta]:
        assert bool((t == 7.0).all())


def test_config3_fixed_list_fp16_causal():
    c = workloads.config3(fixed=True)
    _run_case(c.lengths, c.heads, c.head_dim, torch.float16, True, seed=3)


def test_config4_rescaled_lengths_fp16_causal_fwd_bwd():
    """The bench's own workload: config 3/4's rescaled length list, forward and backward."""
    c = workloads.config4()
    _run_case(c.lengths, c.heads, c.head_dim, torch.float16, True, seed=4, backward=True)


def test_config5_sampled_heads_bf16():
    """Config 5 shape on the GPU; the oracle checks two heads of four sequences
    (including the longest, 10555 tokens) -- heads are independent."""
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    c = workloads.config5()
    say(f"case: config5 N={c.total} H={c.heads} D={c.head_dim} bf16 causal")
    n, h, d = c.total, c.heads, c.head_dim
    off, cu = cu_of(c.lengths)
    q = randn((n, h, d), torch.bfloat16, 50)
    k = randn((n, h, d), torch.bfloat16, 51)
    v = randn((n, h, d), torch.bfloat16, 52)
    do = randn((n, h, d), torch.bfloat16, 53)
    out, lse = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    dq, dk, dv = varlen_attention_hip_backward(do, q, k, v, out, lse, cu, causal=True)
    torch.cuda.synchronize()
    longest = int(np.argmax(c.lengths))
    picks = sorted({longest, int(np.argmin(c.lengths)), 0, 5})
    heads = [0, 17]
    for s in picks:
        a, b = int(off[s]), int(off[s + 1])
        say(f"  seq {s} len {b - a} heads {heads}")
        sub = lambda t: np64(t[a:b][:, heads])  # noqa: E731
        q64, k64, v64, do64 = sub(q), sub(k), sub(v), sub(do)
        loff = np.array([0, b - a], dtype=np.int32)
        ro, rl = attention_fwd(q64, k64, v64, loff, causal=True, dtype=np.float64)
        e_ref = reference_excess(q64, k64, v64, do64, loff, True, torch.bfloat16, o=sub(out),
                                 lse=lse[a:b][:, heads].cpu().numpy().astype(np.float64))
        check_attn("O", sub(out), ro, 2e-3, torch.bfloat16, e_ref["O"])
        check_close("LSE", lse[a:b][:, heads].cpu().numpy().astype(np.float64), rl, 1e-4 + 1e-5 * np.abs(rl).max())
        rdq, rdk, rdv, _ = attention_bwd(do64, q64, k64, v64, sub(out), rl, loff, causal=True)
        check_attn("dQ", sub(dq), rdq, 5e-3, torch.bfloat16, e_ref["dQ"])
        check_attn("dK", sub(dk), rdk, 5e-3, torch.bfloat16, e_ref["dK"])
        check_attn("dV", sub(dv), rdv, 5e-3, torch.bfloat16, e_ref["dV"])


@pytest.mark.parametrize("heads,kv_heads", [(8, 8), (16, 4)])
def test_head_major_launch_fp16_d64_both_masks(heads, kv_heads):
    """A grid of many rounds per XCD (config 5's lengths: 689 items x 8 or 16
    heads) takes the head-major launch, the sequence-major item list and the
    downward query sweep of dK/dV -- with 4 query heads per K/V head also the
    dK/dV workgroup's loop over its group.  Checked on one K/V head's query
    heads for three sequences, causal and not."""
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    c = workloads.config5()
    n, d = c.total, 64
    group = heads // kv_heads
    off, cu = cu_of(c.lengths)
    q, do = (randn((n, heads, d), torch.float16, 80 + s) for s in (0, 3))
    k, v = (randn((n, kv_heads, d), torch.float16, 80 + s) for s in (1, 2))
    order = np.argsort(c.lengths)
    picks = sorted({int(order[0]), int(order[len(order) // 2]), int(order[-6])})
    kvh = 1  # its query heads are group .. 2 * group - 1 (and 1, 6 of the same-heads case)
    qh = list(range(kvh * group, (kvh + 1) * group)) if group > 1 else [1, 6]
    kh = [kvh] if group > 1 else qh
    u = UNIT[torch.float16]
    for causal in (True, False):
        say(f"case: head-major N={n} H={heads} Hkv={kv_heads} D={d} fp16 causal={causal}")
        out, lse = varlen_attention_hip(q, k, v, cu, causal=causal, return_lse=True)
        dq, dk, dv = varlen_attention_hip_backward(do, q, k, v, out, lse, cu, causal=causal)
        torch.cuda.synchronize()
        for s in picks:
            a, b = int(off[s]), int(off[s + 1])
            say(f"  seq {s} len {b - a} query heads {qh}")
            subq = lambda t: np64(t[a:b][:, qh])  # noqa: E731
            subk = lambda t: np64(t[a:b][:, kh])  # noqa: E731
            q64, k64, v64, do64 = subq(q), subk(k), subk(v), subq(do)
            loff = np.array([0, b - a], dtype=np.int32)
            ro, rl = attention_fwd(q64, k64, v64, loff, causal=causal, dtype=np.float64)
            check_close("O", subq(out), ro, 2e-3)
            check_close("LSE", lse[a:b][:, qh].cpu().numpy().astype(np.float64), rl,
                        1e-4 + 1e-5 * np.abs(rl).max())
            rdq, rdk, rdv, _ = attention_bwd(do64, q64, k64, v64, subq(out), rl, loff, causal=causal)
            check_close("dQ", subq(dq), rdq, 5e-3)
            check_close("dK", subk(dk), rdk, 5e-3)
            check_close("dV", subk(dv), rdv, 5e-3)


@pytest.mark.parametrize("causal", [True, False])
def test_schedule_bit_exact(causal):
    from scree_amd.kernels.hip import attention as A
    from scree_amd.kernels.hip import attention_schedule, schedule_items

    cases = [EDGE_LENGTHS, [5], [0, 0, 3], workloads.config3().lengths,
             workloads.config5().lengths, list(range(1, 2049)), [600000, 5, 200],
             # one wave of sequences, most sharing a block count (ties by index)
             [int(x) for x in np.random.default_rng(9).integers(0, 4, size=60) * 100],
             [int(x) for x in np.random.default_rng(7).integers(0, 300, size=3000)]]
    for lengths in cases:
        say(f"case: schedule B={len(lengths)} N={sum(lengths)} causal={causal}")
        off, cu = cu_of(lengths)
        n = int(sum(lengths))
        ws = torch.full((A.workspace_bytes(len(lengths), n, 64),), 255, dtype=torch.uint8,
                        device="cuda")  # stale bytes: the scheduler must rewrite what it uses
        attention_schedule(cu, n, 64, causal, ws)
        count, items = schedule_items(ws)
        want = build_schedule(off, 128, causal)
        assert count == len(want)
        np.testing.assert_array_equal(items.numpy(), want)
        header = ws[:16].view(torch.int32).cpu().tolist()
        assert header == [len(want), len(lengths), 128, int(causal)]
        tmax = (n + 127) // 128 + len(lengths)
        count2, items2 = schedule_items(ws, by_sequence=True, tmax=tmax)
        assert count2 == count
        np.testing.assert_array_equal(items2.numpy(), build_schedule_by_sequence(off, 128))


def test_strided_qkv_views_match_contiguous():
    from scree_amd.kernels.hip import varlen_attention_hip

    say("case: strided qkv views")
    lengths = [70, 33, 190]
    n = sum(lengths)
    _, cu = cu_of(lengths)
    qkv = randn((n, 3, 4, 64), torch.float16, 7)
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    assert not q.is_contiguous()
    a, la = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    b, lb = varlen_attention_hip(q.contiguous(), k.contiguous(), v.contiguous(), cu, causal=True,
                                 return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(la, lb)


def test_deterministic_forward_and_backward():
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    say("case: determinism")
    lengths = [300, 17, 129]
    n = sum(lengths)
    _, cu = cu_of(lengths)
    q, k, v, do = (randn((n, 4, 64), torch.bfloat16, s) for s in range(4))
    o1, l1 = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    o2, l2 = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    g1 = varlen_attention_hip_backward(do, q, k, v, o1, l1, cu, causal=True)
    g2 = varlen_attention_hip_backward(do, q, k, v, o2, l2, cu, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_config4_autograd_step_is_deterministic():
    """Config 4 through the autograd path (the forward derives its items and
    publishes the work list the backward reads): five steps give the same
    output and gradients bit for bit."""
    from scree_amd.kernels.hip import varlen_attention_hip_autograd

    c = workloads.config4()
    n = c.total
    say(f"case: config 4 autograd determinism N={n}")
    _, cu = cu_of(c.lengths)
    q, k, v, do = (randn((n, c.heads, c.head_dim), torch.float16, 90 + s) for s in range(4))
    first = None
    for _ in range(5):
        qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
        out = varlen_attention_hip_autograd(qa, ka, va, cu, causal=True)
        out.backward(do)
        got = (out.detach(), qa.grad, ka.grad, va.grad)
        if first is None:
            first = got
        else:
            for a, b in zip(first, got):
                assert torch.equal(a, b)
    torch.cuda.synchronize()


def test_autograd_wrapper_matches_explicit_backward():
    from scree_amd.kernels.hip import (varlen_attention_hip, varlen_attention_hip_autograd,
                                       varlen_attention_hip_backward)

    say("case: autograd wrapper")
    lengths = [64, 200, 3]
    n = sum(lengths)
    _, cu = cu_of(lengths)
    q, k, v, do = (randn((n, 2, 128), torch.float16, 10 + s) for s in range(4))
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = varlen_attention_hip_autograd(qa, ka, va, cu, causal=True)
    out.backward(do)
    o, lse = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    dq, dk, dv = varlen_attention_hip_backward(do, q, k, v, o, lse, cu, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), o)
    assert torch.equal(qa.grad, dq) and torch.equal(ka.grad, dk) and torch.equal(va.grad, dv)


def test_preallocated_out_and_lse_buffers():
    from scree_amd.kernels.hip import varlen_attention_hip

    say("case: out= / lse_buffer=")
    lengths = [40, 90]
    n = sum(lengths)
    _, cu = cu_of(lengths)
    q, k, v = (randn((n, 2, 32), torch.float16, 20 + s) for s in range(3))
    out = torch.empty_like(q)
    lse = torch.empty((n, 2), dtype=torch.float32, device="cuda")
    r = varlen_attention_hip(q, k, v, cu, causal=False, return_lse=True, out=out, lse_buffer=lse)
    torch.cuda.synchronize()
    assert r[0] is out and r[1] is lse
    o2 = varlen_attention_hip(q, k, v, cu, causal=False)
    assert torch.equal(o2, out)


def test_array_level_api_on_device():
    import scree_amd as scree
    from scree_amd.kernels import varlen_attention

    say("case: Array-level varlen_attention")
    seqs = [randn((n, 2, 64), torch.float16, n) for n in (5, 77, 130)]
    q = scree.pack(seqs)
    out = varlen_attention(q, q, q, causal=True)
    torch.cuda.synchronize()
    assert out.offsets is q.offsets
    off = q.offsets.cpu().numpy()
    ref, _ = attention_fwd(np64(q.values), np64(q.values), np64(q.values), off, causal=True)
    check_close("O", np64(out.values), ref, 2e-3)
    other = scree.pack([randn((n, 2, 64), torch.float16, 1) for n in (6, 76, 130)])
    with pytest.raises(ValueError, match="identical offsets"):
        varlen_attention(q, other, other)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_batch_without_tokens(dtype):
    """Every sequence empty: empty outputs and gradients, as the reference's
    torch branch returns (``reference/varlen_attention.py:96-113``), through
    the launchers, autograd and the Array-level call."""
    import scree_amd
    from scree_amd.kernels import varlen_attention
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    say(f"case: three empty sequences, H=4 D=64 {dtype}")
    off, cu = cu_of([0, 0, 0])
    q, k, v = (torch.empty((0, 4, 64), dtype=dtype, device="cuda") for _ in range(3))
    if dtype != torch.float32:
        out, lse = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
        assert out.shape == (0, 4, 64) and lse.shape == (0, 4)
        grads = varlen_attention_hip_backward(torch.empty_like(q), q, k, v, out, lse, cu, causal=True)
        assert all(g.shape == (0, 4, 64) for g in grads)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    res = varlen_attention(*(scree_amd.Array(values=t, offsets=cu) for t in (qa, ka, va)), causal=True)
    assert res.values.shape == (0, 4, 64) and res.values.dtype == dtype
    res.values.sum().backward()
    torch.cuda.synchronize()
    assert qa.grad.shape == (0, 4, 64) and ka.grad.shape == (0, 4, 64)
