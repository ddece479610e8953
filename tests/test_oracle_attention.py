"""Pins the attention oracle (forward, LSE, backward) before it is trusted.

* the reference's own known-answer tests (``tests/test_varlen_kernels.py:19-75``
  and ``tests/test_autograd.py:67-78``), restated;
* brute force with explicit Python loops in fp64 on tiny inputs;
* ``torch.nn.functional.scaled_dot_product_attention`` per sequence, and torch
  autograd through it for the backward;
* fp64 central finite differences of the backward;
* invariants: rows of exp(S - LSE) sum to 1, sum_k dS = 0, identical keys
  average the values.
A dropped term, wrong sign, transposed operand or misplaced mask fails at
least one of these.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import attention_bwd, attention_fwd, attention_lse
from oracle.core import offsets_from_lengths


def _inputs(lengths, heads, dim, seed=0):
    rng = np.random.default_rng(seed)
    n = sum(lengths)
    q = rng.standard_normal((n, heads, dim))
    k = rng.standard_normal((n, heads, dim))
    v = rng.standard_normal((n, heads, dim))
    return q, k, v, offsets_from_lengths(lengths)


def _brute(q, k, v, off, causal):
    n, h, d = q.shape
    out = np.zeros_like(q)
    lse = np.zeros((n, h))
    for b in range(len(off) - 1):
        s, e = off[b], off[b + 1]
        for hh in range(h):
            for i in range(s, e):
                keys = range(s, i + 1) if causal else range(s, e)
                sc = [sum(q[i, hh, t] * k[j, hh, t] for t in range(d)) / math.sqrt(d) for j in keys]
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                z = sum(w)
                lse[i, hh] = m + math.log(z)
                for t in range(d):
                    out[i, hh, t] = sum(wj * v[j, hh, t] for wj, j in zip(w, keys)) / z
    return out, lse


@pytest.mark.parametrize("causal", [False, True])
def test_forward_matches_brute_force(causal):
    q, k, v, off = _inputs([3, 1, 5, 2], 2, 4)
    want_o, want_l = _brute(q, k, v, off, causal)
    for impl in ("einsum", "matmul"):
        o, lse = attention_fwd(q, k, v, off, causal=causal, impl=impl)
        np.testing.assert_allclose(o, want_o, atol=1e-12)
        np.testing.assert_allclose(lse, want_l, atol=1e-12)


def test_reference_known_answer_per_sequence_baseline():
    # reference tests/test_varlen_kernels.py:19-43
    rng = np.random.default_rng(0)
    n_heads, head_dim, lengths = 2, 4, [3, 5, 2]
    sq = [rng.standard_normal((n, n_heads, head_dim)).astype(np.float32) for n in lengths]
    sk = [rng.standard_normal((n, n_heads, head_dim)).astype(np.float32) for n in lengths]
    sv = [rng.standard_normal((n, n_heads, head_dim)).astype(np.float32) for n in lengths]
    off = offsets_from_lengths(lengths)
    o, _ = attention_fwd(np.concatenate(sq), np.concatenate(sk), np.concatenate(sv), off,
                         causal=False, dtype=np.float32, impl="einsum")
    for i in range(len(lengths)):
        scores = np.einsum("ihd,jhd->hij", sq[i], sk[i]) / np.sqrt(head_dim)
        attn = np.exp(scores - scores.max(-1, keepdims=True))
        attn /= attn.sum(-1, keepdims=True)
        base = np.einsum("hij,jhd->ihd", attn, sv[i])
        np.testing.assert_allclose(o[off[i]:off[i + 1]], base, atol=1e-5)


def test_reference_known_answer_causal_first_token_is_v0():
    # reference tests/test_varlen_kernels.py:46-63
    q, k, v, off = _inputs([4, 6], 1, 4)
    o, _ = attention_fwd(q, k, v, off, causal=True)
    for i in range(2):
        np.testing.assert_allclose(o[off[i]], v[off[i]], atol=1e-12)


def test_rejects_mismatched_offsets():
    # reference tests/test_varlen_kernels.py:66-75
    q, k, v, off = _inputs([3, 5], 1, 4)
    with pytest.raises(ValueError, match=r"identical offsets"):
        attention_fwd(q, k, v, off, k_offsets=offsets_from_lengths([4, 4]))


def test_length_one_sequences():
    # reference tests/test_autograd.py:67-78: length-1 rows attend to themselves only
    q, k, v, off = _inputs([1, 1, 1], 2, 8)
    for causal in (False, True):
        o, lse = attention_fwd(q, k, v, off, causal=causal)
        np.testing.assert_allclose(o, v, atol=1e-12)
        np.testing.assert_allclose(lse, (q * k).sum(-1) / math.sqrt(8), atol=1e-12)


def test_identical_keys_average_values():
    lengths = [7]
    q, k, v, off = _inputs(lengths, 1, 4)
    k[:] = k[0]
    o, _ = attention_fwd(q, k, v, off, causal=False)
    np.testing.assert_allclose(o, np.broadcast_to(v.mean(0), o.shape), atol=1e-12)
    oc, _ = attention_fwd(q, k, v, off, causal=True)
    for i in range(7):
        np.testing.assert_allclose(oc[i], v[: i + 1].mean(0), atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_forward_matches_torch_sdpa(causal):
    lengths = [17, 1, 64, 33, 90]
    q, k, v, off = _inputs(lengths, 3, 16, seed=1)
    o, lse = attention_fwd(q, k, v, off, causal=causal)
    for b in range(len(lengths)):
        s, e = off[b], off[b + 1]
        tq, tk, tv = (torch.from_numpy(x[s:e]).permute(1, 0, 2) for x in (q, k, v))
        ref = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal).permute(1, 0, 2)
        np.testing.assert_allclose(o[s:e], ref.numpy(), atol=1e-10)
        sc = torch.einsum("hid,hjd->hij", tq, tk) / math.sqrt(16)
        if causal:
            sc = sc.masked_fill(torch.triu(torch.ones(e - s, e - s, dtype=torch.bool), 1), -math.inf)
        np.testing.assert_allclose(lse[s:e], torch.logsumexp(sc, -1).T.numpy(), atol=1e-10)


@pytest.mark.parametrize("causal", [False, True])
def test_lse_independent_and_normalises(causal):
    lengths = [9, 20, 3]
    q, k, v, off = _inputs(lengths, 2, 8, seed=2)
    _, lse = attention_fwd(q, k, v, off, causal=causal)
    np.testing.assert_allclose(lse, attention_lse(q, k, off, causal=causal), atol=1e-12)
    for b in range(len(lengths)):
        s, e = off[b], off[b + 1]
        sc = np.einsum("ihd,jhd->hij", q[s:e], k[s:e]) / math.sqrt(8)
        if causal:
            sc = np.where(np.triu(np.ones((e - s, e - s), bool), 1), -np.inf, sc)
        rows = np.exp(sc - lse[s:e].T[:, :, None]).sum(-1)
        np.testing.assert_allclose(rows, 1.0, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_torch_autograd(causal):
    lengths = [5, 12, 1, 30]
    q, k, v, off = _inputs(lengths, 2, 8, seed=3)
    do = np.random.default_rng(9).standard_normal(q.shape)
    o, lse = attention_fwd(q, k, v, off, causal=causal)
    dq, dk, dv, delta = attention_bwd(do, q, k, v, o, lse, off, causal=causal)
    np.testing.assert_allclose(delta, (o * do).sum(-1), atol=1e-12)
    for b in range(len(lengths)):
        s, e = off[b], off[b + 1]
        tq, tk, tv = (torch.from_numpy(x[s:e]).permute(1, 0, 2).clone().requires_grad_(True)
                      for x in (q, k, v))
        out = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal)
        out.backward(torch.from_numpy(do[s:e]).permute(1, 0, 2))
        np.testing.assert_allclose(dq[s:e], tq.grad.permute(1, 0, 2).numpy(), atol=1e-10)
        np.testing.assert_allclose(dk[s:e], tk.grad.permute(1, 0, 2).numpy(), atol=1e-10)
        np.testing.assert_allclose(dv[s:e], tv.grad.permute(1, 0, 2).numpy(), atol=1e-10)
    # einsum path agrees with matmul path
    dq2, dk2, dv2, _ = attention_bwd(do, q, k, v, o, lse, off, causal=causal, impl="einsum")
    np.testing.assert_allclose(dq2, dq, atol=1e-12)
    np.testing.assert_allclose(dk2, dk, atol=1e-12)
    np.testing.assert_allclose(dv2, dv, atol=1e-12)


def test_backward_finite_differences():
    lengths = [4, 3]
    q, k, v, off = _inputs(lengths, 1, 3, seed=4)
    do = np.random.default_rng(5).standard_normal(q.shape)

    def loss(q_, k_, v_):
        o_, _ = attention_fwd(q_, k_, v_, off, causal=True)
        return float((o_ * do).sum())

    o, lse = attention_fwd(q, k, v, off, causal=True)
    grads = attention_bwd(do, q, k, v, o, lse, off, causal=True)[:3]
    eps = 1e-6
    for which, g in enumerate(grads):
        base = [q, k, v]
        for idx in [(0, 0, 0), (2, 0, 1), (3, 0, 2), (5, 0, 0), (6, 0, 1)]:
            plus = [x.copy() for x in base]
            minus = [x.copy() for x in base]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fd = (loss(*plus) - loss(*minus)) / (2 * eps)
            assert abs(fd - g[idx]) < 1e-7, (which, idx, fd, g[idx])


def test_softmax_gradient_rows_sum_to_zero():
    lengths = [11]
    q, k, v, off = _inputs(lengths, 1, 4, seed=6)
    do = np.random.default_rng(7).standard_normal(q.shape)
    o, lse = attention_fwd(q, k, v, off, causal=True)
    _, _, _, delta = attention_bwd(do, q, k, v, o, lse, off, causal=True)
    sc = np.einsum("ihd,jhd->hij", q, k) / 2.0
    sc = np.where(np.triu(np.ones((11, 11), bool), 1), -np.inf, sc)
    p = np.exp(sc - lse.T[:, :, None])
    dp = np.einsum("ihd,jhd->hij", do, v)
    ds = p * (dp - delta.T[:, :, None])
    np.testing.assert_allclose(ds.sum(-1), 0.0, atol=1e-12)


def test_empty_sequence_is_skipped():
    q, k, v, off = _inputs([3, 0, 2], 1, 4)
    o, lse = attention_fwd(q, k, v, off, causal=True)
    o2, lse2 = attention_fwd(q, k, v, offsets_from_lengths([3, 2]), causal=True)
    np.testing.assert_array_equal(o, o2)
    np.testing.assert_array_equal(lse, lse2)


# ----------------------------------------------------------- grouped-query
def _sdpa_gqa(q, k, v, off, causal, want_grad=False, do=None):
    """torch SDPA with enable_gqa per sequence (fp64 CPU), and its autograd."""
    qt, kt, vt = (torch.tensor(a, requires_grad=want_grad) for a in (q, k, v))
    outs = []
    for b in range(len(off) - 1):
        s, e = int(off[b]), int(off[b + 1])
        if e <= s:
            continue
        o = F.scaled_dot_product_attention(qt[s:e].transpose(0, 1)[None], kt[s:e].transpose(0, 1)[None],
                                           vt[s:e].transpose(0, 1)[None], is_causal=causal,
                                           enable_gqa=True)
        outs.append(o[0].transpose(0, 1))
    out = torch.cat(outs)
    if not want_grad:
        return out.detach().numpy()
    out.backward(torch.tensor(do))
    return out.detach().numpy(), qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


@pytest.mark.parametrize("kv_heads", [1, 2, 3])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_forward_and_backward_match_sdpa(kv_heads, causal):
    lengths = [5, 1, 9, 3]
    rng = np.random.default_rng(kv_heads)
    n, h, d = sum(lengths), 6, 8
    off = offsets_from_lengths(lengths)
    q = rng.standard_normal((n, h, d))
    k = rng.standard_normal((n, kv_heads, d))
    v = rng.standard_normal((n, kv_heads, d))
    do = rng.standard_normal((n, h, d))
    o, lse = attention_fwd(q, k, v, off, causal=causal)
    want_o, wdq, wdk, wdv = _sdpa_gqa(q, k, v, off, causal, want_grad=True, do=do)
    np.testing.assert_allclose(o, want_o, atol=1e-12)
    np.testing.assert_allclose(lse, attention_lse(q, k, off, causal=causal), atol=1e-12)
    dq, dk, dv, _ = attention_bwd(do, q, k, v, o, lse, off, causal=causal)
    assert dk.shape == k.shape and dv.shape == v.shape
    np.testing.assert_allclose(dq, wdq, atol=1e-10)
    np.testing.assert_allclose(dk, wdk, atol=1e-10)
    np.testing.assert_allclose(dv, wdv, atol=1e-10)


def test_gqa_single_kv_head_gives_identical_query_heads():
    """With one K/V head, query heads holding the same queries see the same keys."""
    rng = np.random.default_rng(11)
    lengths = [7, 4]
    n, d = sum(lengths), 4
    off = offsets_from_lengths(lengths)
    q1 = rng.standard_normal((n, 1, d))
    q = np.repeat(q1, 3, axis=1)
    k = rng.standard_normal((n, 1, d))
    v = rng.standard_normal((n, 1, d))
    o, lse = attention_fwd(q, k, v, off, causal=True)
    o1, lse1 = attention_fwd(q1, k, v, off, causal=True)
    for hh in range(3):
        np.testing.assert_allclose(o[:, hh], o1[:, 0], atol=1e-13)
        np.testing.assert_allclose(lse[:, hh], lse1[:, 0], atol=1e-13)
    do = rng.standard_normal((n, 3, d))
    dq, dk, dv, _ = attention_bwd(do, q, k, v, o, lse, off, causal=True)
    # dK / dV of the shared head = sum of the three single-head gradients
    acc_k, acc_v = np.zeros_like(k), np.zeros_like(v)
    for hh in range(3):
        _, dk1, dv1, _ = attention_bwd(do[:, hh:hh + 1], q1, k, v, o1, lse1, off, causal=True)
        acc_k += dk1
        acc_v += dv1
    np.testing.assert_allclose(dk, acc_k, atol=1e-12)
    np.testing.assert_allclose(dv, acc_v, atol=1e-12)


def test_gqa_rejects_non_dividing_heads():
    q = np.zeros((3, 4, 8))
    k = np.zeros((3, 3, 8))
    with pytest.raises(ValueError):
        attention_fwd(q, k, k, np.array([0, 3]))


# ---- the reference-rounding variants (explain the bf16 error budget) ----

def _torch_rounded(q, k, v, do, off, causal, dt, block=64):
    """The same arithmetic in torch: P, dS cast with torch's own fp32 ->
    fp16/bf16 conversion (an implementation of the rounding independent of
    ``round_bf16``), sums in fp64."""
    rnd = lambda x: x.float().to(dt).double()  # noqa: E731
    tq, tk, tv, tdo = (torch.from_numpy(np.ascontiguousarray(a.transpose(1, 0, 2)))
                       for a in (q, k, v, do))
    d = q.shape[-1]
    o, lse = np.zeros_like(q), np.zeros(q.shape[:2])
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    for b in range(len(off) - 1):
        s, e = int(off[b]), int(off[b + 1])
        if e <= s:
            continue
        qs, ks, vs, dos = tq[:, s:e], tk[:, s:e], tv[:, s:e], tdo[:, s:e]
        sc = qs @ ks.transpose(1, 2) / math.sqrt(d)
        if causal:
            sc = sc.masked_fill(torch.ones(e - s, e - s, dtype=torch.bool).triu(1), -math.inf)
        m = torch.full((sc.shape[0], e - s, 1), -math.inf, dtype=torch.float64)
        l = torch.zeros_like(m)
        acc = torch.zeros_like(qs)
        for j in range(0, e - s, block):
            blk = sc[:, :, j:j + block]
            mn = torch.maximum(m, blk.amax(-1, keepdim=True))
            p = torch.exp(blk - mn)
            a = torch.exp(m - mn)
            l = a * l + p.sum(-1, keepdim=True)
            acc = a * acc + rnd(p) @ vs[:, j:j + block]
            m = mn
        ob = rnd(acc / l)
        lb = (m + torch.log(l))[..., 0]
        o[s:e], lse[s:e] = ob.transpose(0, 1).numpy(), lb.T.numpy()
        p = torch.exp(sc - lb[..., None])
        delta = (ob * dos).sum(-1, keepdim=True)
        ds = rnd(p * (dos @ vs.transpose(1, 2) - delta))
        dv[s:e] = (rnd(p).transpose(1, 2) @ dos).transpose(0, 1).numpy()
        dq[s:e] = (ds @ ks / math.sqrt(d)).transpose(0, 1).numpy()
        dk[s:e] = (ds.transpose(1, 2) @ qs / math.sqrt(d)).transpose(0, 1).numpy()
    return o, lse, tuple(rnd(torch.from_numpy(g)).numpy() for g in (dq, dk, dv))


@pytest.mark.parametrize("causal", [False, True])
def test_rounded_variant_without_rounding_is_the_oracle(causal):
    from oracle.attention import attention_bwd_rounded, attention_fwd_rounded

    q, k, v, off = _inputs([70, 1, 130, 64], 2, 16, seed=5)
    do = np.random.default_rng(6).standard_normal(q.shape)
    o, lse = attention_fwd(q, k, v, off, causal=causal)
    o2, lse2 = attention_fwd_rounded(q, k, v, off, causal=causal, operand="float64")
    np.testing.assert_allclose(o2, o, atol=1e-12)
    np.testing.assert_allclose(lse2, lse, atol=1e-12)
    for a, b in zip(attention_bwd(do, q, k, v, o, lse, off, causal=causal),
                    attention_bwd_rounded(do, q, k, v, o, lse, off, causal=causal, operand="float64")):
        np.testing.assert_allclose(b, a, atol=1e-12)
    # grouped K/V heads: the variant expands and folds them like the oracle
    kg, vg = k[:, :1], v[:, :1]
    o, lse = attention_fwd(q, kg, vg, off, causal=causal)
    o2, _ = attention_fwd_rounded(q, kg, vg, off, causal=causal, operand="float64")
    np.testing.assert_allclose(o2, o, atol=1e-12)
    for a, b in zip(attention_bwd(do, q, kg, vg, o, lse, off, causal=causal),
                    attention_bwd_rounded(do, q, kg, vg, o, lse, off, causal=causal, operand="float64")):
        np.testing.assert_allclose(b, a, atol=1e-12)


@pytest.mark.parametrize("operand,dt", [("bfloat16", torch.bfloat16), ("float16", torch.float16)])
@pytest.mark.parametrize("causal", [False, True])
def test_rounded_variant_matches_torch_casts(operand, dt, causal):
    """Rounding placement (P per 64-key block against the running maximum,
    dS, the stored results) against torch's own casts, and the rounding
    really applied: the result departs from the exact oracle, by no more
    than the operand roundings allow."""
    from oracle.attention import attention_bwd_rounded, attention_fwd_rounded

    q, k, v, off = _inputs([150, 1, 64, 65], 2, 32, seed=9)
    q, k = 1.5 * q, 1.5 * k  # peaked rows: the running maximum moves between blocks
    do = np.random.default_rng(10).standard_normal(q.shape)
    o, lse = attention_fwd_rounded(q, k, v, off, causal=causal, operand=operand)
    grads = attention_bwd_rounded(do, q, k, v, o, lse, off, causal=causal, operand=operand)
    to, tl, tg = _torch_rounded(q, k, v, do, off, causal, dt)
    np.testing.assert_allclose(o, to, atol=1e-12)
    np.testing.assert_allclose(lse, tl, atol=1e-12)
    for a, b in zip(grads[:3], tg):
        np.testing.assert_allclose(a, b, atol=1e-12)
    exact_o, exact_lse = attention_fwd(q, k, v, off, causal=causal)
    u = 2.0 ** -8 if operand == "bfloat16" else 2.0 ** -11
    err = np.abs(o - exact_o)
    assert err.max() > 0.1 * u
    assert (err <= u * (np.abs(v).max() + np.abs(exact_o)) + 1e-12).all()
    np.testing.assert_allclose(lse, exact_lse, atol=1e-12)  # the row sum is unrounded


def test_reference_excess_emulates_the_backward_on_the_given_forward_outputs():
    """``reference_excess`` runs the reference backward's arithmetic on the O and
    LSE it is given (the HIP forward's, in the GPU tests): given the emulated
    reference forward's own outputs it reproduces the default, and given
    another O its backward figures change while the forward's do not."""
    from oracle.attention import attention_fwd_rounded
    from parity import reference_excess

    q, k, v, off = _inputs([150, 1, 64, 65], 2, 32, seed=11)
    q, k = 2.0 * q, 2.0 * k
    do = np.random.default_rng(12).standard_normal(q.shape)
    eo, el = attention_fwd_rounded(q, k, v, off, causal=True, operand="bfloat16")
    base = reference_excess(q, k, v, do, off, True, torch.bfloat16)
    same = reference_excess(q, k, v, do, off, True, torch.bfloat16, o=eo, lse=el)
    assert base == same
    other_o = torch.from_numpy(eo + 2.0 ** -7 * np.abs(eo)).bfloat16().double().numpy()
    other = reference_excess(q, k, v, do, off, True, torch.bfloat16, o=other_o, lse=el)
    assert other["O"] == base["O"]
    assert any(other[g] != base[g] for g in ("dQ", "dK", "dV"))
