"""Varlen self-attention forward, logsumexp and backward (oracle; test infrastructure only).

Forward follows the numpy branch of the reference,
``src/scree/kernels/reference/varlen_attention.py:115-138``: per sequence,
``S = einsum("ihd,jhd->hij") * scale`` with ``scale = 1/sqrt(D)`` (``:31-32``),
causal positions above the diagonal set to ``-inf`` (``:129-132``),
max-subtracted softmax (``:133-135``) and ``O = einsum("hij,jhd->ihd")``
(``:136``).  The identical-offsets check raises the same ``ValueError``
(``:118-119``).

The log-sum-exp is the quantity the reference's GPU forward stores for the
backward (``src/scree/kernels/triton/varlen_attention.py:158-162``): natural
log, of the *scaled* scores, shape ``(total, heads)``.

The backward is the closed-form softmax-attention gradient the reference's
GPU backward evaluates (``src/scree/kernels/triton/_backward.py:53-69`` for
``Delta = rowsum(O * dO)``, ``:161-181`` for dK/dV, ``:270-282`` for dQ)::

    P  = exp(S - LSE)           dV = P^T dO
    dP = dO V^T                 dS = P * (dP - Delta)
    dQ = scale * dS K           dK = scale * dS^T Q

Grouped-query attention (``k`` / ``v`` with ``kv_heads`` dividing the
query heads; no counterpart in the reference, whose docs list it as missing,
``docs/kernels.md:177``) is defined by its identity with ordinary attention:
each K/V head is repeated for the ``g = heads // kv_heads`` consecutive query
heads of its group (query head ``h`` uses K/V head ``h // g``), and ``dK`` /
``dV`` are the repeated-head gradients summed over each group.

``impl="einsum"`` reproduces the reference's call pattern (``np.einsum``
without ``optimize``: single-threaded loops, the CPU baseline);
``impl="matmul"`` evaluates the same sums through ``np.matmul`` and is what
the tests use for speed.  ``dtype`` is the arithmetic type (numpy has no
bf16; half-precision inputs are upcast exactly).
"""

from __future__ import annotations

import math

import numpy as np


def _check_offsets(q_off, k_off, v_off) -> np.ndarray:
    q_off = np.asarray(q_off)
    if not np.array_equal(q_off, np.asarray(k_off)) or not np.array_equal(q_off, np.asarray(v_off)):
        raise ValueError("q, k, v must have identical offsets")
    return q_off.astype(np.int64)


def _scores(qi, ki, scale, impl):
    # qi, ki: (L, H, D) -> (H, L, L)
    if impl == "einsum":
        return np.einsum("ihd,jhd->hij", qi, ki) * scale
    return np.matmul(qi.transpose(1, 0, 2), ki.transpose(1, 2, 0)) * scale


def _pv(attn, vi, impl):
    # attn: (H, L, L), vi: (L, H, D) -> (L, H, D)
    if impl == "einsum":
        return np.einsum("hij,jhd->ihd", attn, vi)
    return np.matmul(attn, vi.transpose(1, 0, 2)).transpose(1, 0, 2)


def _expand_kv(t, heads):
    """Repeat each K/V head for the consecutive query heads of its group."""
    hkv = t.shape[1]
    if hkv == heads:
        return t
    if hkv < 1 or heads % hkv:
        raise ValueError("k/v heads must divide q heads")
    return np.repeat(t, heads // hkv, axis=1)


def _fold_kv(t, kv_heads):
    """Sum repeated-head gradients back onto their K/V head."""
    n, h, d = t.shape
    if h == kv_heads:
        return t
    return t.reshape(n, kv_heads, h // kv_heads, d).sum(axis=2)


def attention_fwd(q, k, v, offsets, causal=False, dtype=np.float64, impl="matmul",
                  k_offsets=None, v_offsets=None):
    """Return ``(O, LSE)`` for packed ``q, k, v`` of shape ``(N, H, D)``."""
    off = _check_offsets(offsets, offsets if k_offsets is None else k_offsets,
                         offsets if v_offsets is None else v_offsets)
    q = np.asarray(q, dtype=dtype)
    k = _expand_kv(np.asarray(k, dtype=dtype), q.shape[1])
    v = _expand_kv(np.asarray(v, dtype=dtype), q.shape[1])
    n, h, d = q.shape
    scale = 1.0 / math.sqrt(d)
    out = np.zeros_like(q)
    lse = np.zeros((n, h), dtype=dtype)
    for i in range(len(off) - 1):
        s, e = int(off[i]), int(off[i + 1])
        if e <= s:
            continue
        scores = _scores(q[s:e], k[s:e], scale, impl)
        if causal:
            length = e - s
            mask = np.triu(np.ones((length, length), dtype=bool), k=1)
            scores = np.where(mask, -np.inf, scores)
        smax = scores.max(axis=-1, keepdims=True)
        ex = np.exp(scores - smax)
        den = ex.sum(axis=-1, keepdims=True)
        out[s:e] = _pv(ex / den, v[s:e], impl)
        lse[s:e] = (smax + np.log(den))[..., 0].T
    return out, lse


def attention_lse(q, k, offsets, causal=False, dtype=np.float64):
    """LSE alone, computed independently of the forward's running max."""
    q = np.asarray(q, dtype=dtype)
    k = _expand_kv(np.asarray(k, dtype=dtype), q.shape[1])
    off = np.asarray(offsets, dtype=np.int64)
    n, h, d = q.shape
    scale = 1.0 / math.sqrt(d)
    lse = np.zeros((n, h), dtype=dtype)
    for i in range(len(off) - 1):
        s, e = int(off[i]), int(off[i + 1])
        for t in range(s, e):
            hi = t + 1 if causal else e
            sc = np.einsum("hd,jhd->hj", q[t], k[s:hi]) * scale
            m = sc.max(axis=-1)
            lse[t] = m + np.log(np.exp(sc - m[:, None]).sum(axis=-1))
    return lse


def attention_bwd(do, q, k, v, o, lse, offsets, causal=False, dtype=np.float64, impl="matmul"):
    """Return ``(dQ, dK, dV, Delta)`` given the forward's ``O`` and ``LSE``."""
    off = np.asarray(offsets, dtype=np.int64)
    do = np.asarray(do, dtype=dtype)
    q = np.asarray(q, dtype=dtype)
    kv_heads = np.shape(k)[1]
    k = _expand_kv(np.asarray(k, dtype=dtype), q.shape[1])
    v = _expand_kv(np.asarray(v, dtype=dtype), q.shape[1])
    o = np.asarray(o, dtype=dtype)
    lse = np.asarray(lse, dtype=dtype)
    n, h, d = q.shape
    scale = 1.0 / math.sqrt(d)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    delta = (o * do).sum(axis=-1)  # (N, H)
    for i in range(len(off) - 1):
        s, e = int(off[i]), int(off[i + 1])
        if e <= s:
            continue
        qi, ki, vi, doi = q[s:e], k[s:e], v[s:e], do[s:e]
        scores = _scores(qi, ki, scale, impl)
        if causal:
            length = e - s
            mask = np.triu(np.ones((length, length), dtype=bool), k=1)
            scores = np.where(mask, -np.inf, scores)
        p = np.exp(scores - lse[s:e].T[:, :, None])  # (H, Lq, Lk)
        if impl == "einsum":
            dv[s:e] = np.einsum("hij,ihd->jhd", p, doi)
            dp = np.einsum("ihd,jhd->hij", doi, vi)
        else:
            dv[s:e] = np.matmul(p.transpose(0, 2, 1), doi.transpose(1, 0, 2)).transpose(1, 0, 2)
            dp = np.matmul(doi.transpose(1, 0, 2), vi.transpose(1, 2, 0))
        ds = p * (dp - delta[s:e].T[:, :, None])
        if impl == "einsum":
            dq[s:e] = scale * np.einsum("hij,jhd->ihd", ds, ki)
            dk[s:e] = scale * np.einsum("hij,ihd->jhd", ds, qi)
        else:
            dq[s:e] = scale * np.matmul(ds, ki.transpose(1, 0, 2)).transpose(1, 0, 2)
            dk[s:e] = scale * np.matmul(ds.transpose(0, 2, 1), qi.transpose(1, 0, 2)).transpose(1, 0, 2)
    return dq, _fold_kv(dk, kv_heads), _fold_kv(dv, kv_heads), delta


def _rounder(operand):
    """Rounding of an fp32 value to the kernel operand type, returned as fp64."""
    if operand in (None, "float64"):
        return lambda x: x
    if operand == "float32":
        return lambda x: np.asarray(x, dtype=np.float32).astype(np.float64)
    if operand == "float16":
        return lambda x: np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float64)
    if operand == "bfloat16":
        from .norms import round_bf16
        return round_bf16
    raise ValueError(f"unknown operand type {operand}")


def attention_fwd_rounded(q, k, v, offsets, causal=False, operand="float16", block=64):
    """``(O, LSE)`` with the reference GPU forward's own roundings.

    Restates the loop of ``src/scree/kernels/triton/varlen_attention.py:105-162``:
    per 64-key block, the running maximum ``m_new = max(m, rowmax(S_blk))``,
    ``alpha = exp(m - m_new)``, ``p = exp(S_blk - m_new)``, ``l = alpha*l +
    rowsum(p)`` (unrounded ``p``), ``acc = alpha*acc + round(p) @ V_blk``
    (``p.to(v.dtype)``, ``:142``), then ``O = round(acc / l)`` and ``LSE = m +
    log(l)``.  ``round`` is the cast to ``operand``; everything else is fp64
    (the reference keeps it in fp32).  With ``operand="float64"`` this is
    :func:`attention_fwd` up to summation order.
    """
    rnd = _rounder(operand)
    off = np.asarray(offsets, dtype=np.int64)
    q = np.asarray(q, dtype=np.float64)
    k = _expand_kv(np.asarray(k, dtype=np.float64), q.shape[1])
    v = _expand_kv(np.asarray(v, dtype=np.float64), q.shape[1])
    n, h, d = q.shape
    scale = 1.0 / math.sqrt(d)
    out = np.zeros_like(q)
    lse = np.zeros((n, h))
    for i in range(len(off) - 1):
        s, e = int(off[i]), int(off[i + 1])
        length = e - s
        if length <= 0:
            continue
        scores = _scores(q[s:e], k[s:e], scale, "matmul")  # (H, L, L)
        if causal:
            scores = np.where(np.triu(np.ones((length, length), dtype=bool), k=1), -np.inf, scores)
        vt = v[s:e].transpose(1, 0, 2)
        m = np.full((h, length, 1), -np.inf)
        l = np.zeros((h, length, 1))
        acc = np.zeros((h, length, d))
        with np.errstate(invalid="ignore"):
            for j in range(0, length, block):
                sb = scores[:, :, j:j + block]
                m_new = np.maximum(m, sb.max(axis=-1, keepdims=True))
                alpha = np.exp(m - m_new)  # 0 on the first block (m = -inf)
                p = np.exp(sb - m_new)
                l = alpha * l + p.sum(axis=-1, keepdims=True)
                acc = alpha * acc + np.matmul(rnd(p), vt[:, j:j + block])
                m = m_new
        out[s:e] = rnd(acc / l).transpose(1, 0, 2)
        lse[s:e] = (m + np.log(l))[..., 0].T
    return out, lse


def attention_bwd_rounded(do, q, k, v, o, lse, offsets, causal=False, operand="float16"):
    """``(dQ, dK, dV, Delta)`` with the reference GPU backward's own roundings.

    Restates ``src/scree/kernels/triton/_backward.py``: ``Delta = rowsum(O*dO)``
    from the stored O (``:53-69``); ``P = exp(S - LSE)``; ``dV += round(P)^T dO``
    (``p.to(do.dtype)``, ``:174``); ``dS = P*(dP - Delta)``; ``dK += scale *
    round(dS)^T Q`` (``:181``) and ``dQ += scale * round(dS) K`` (``:282``);
    the three results rounded to ``operand`` when stored.  Grouped-query
    gradients are summed over each group before that rounding, as the HIP
    dK/dV pass does.  Sums run in fp64 (the reference: fp32).
    """
    rnd = _rounder(operand)
    off = np.asarray(offsets, dtype=np.int64)
    do = np.asarray(do, dtype=np.float64)
    q = np.asarray(q, dtype=np.float64)
    kv_heads = np.shape(k)[1]
    k = _expand_kv(np.asarray(k, dtype=np.float64), q.shape[1])
    v = _expand_kv(np.asarray(v, dtype=np.float64), q.shape[1])
    o = np.asarray(o, dtype=np.float64)
    lse = np.asarray(lse, dtype=np.float64)
    n, h, d = q.shape
    scale = 1.0 / math.sqrt(d)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    delta = (o * do).sum(axis=-1)
    for i in range(len(off) - 1):
        s, e = int(off[i]), int(off[i + 1])
        length = e - s
        if length <= 0:
            continue
        qi, ki, vi, doi = (t[s:e].transpose(1, 0, 2) for t in (q, k, v, do))
        scores = np.matmul(qi, ki.transpose(0, 2, 1)) * scale
        if causal:
            scores = np.where(np.triu(np.ones((length, length), dtype=bool), k=1), -np.inf, scores)
        p = np.exp(scores - lse[s:e].T[:, :, None])
        dv[s:e] = np.matmul(rnd(p).transpose(0, 2, 1), doi).transpose(1, 0, 2)
        dp = np.matmul(doi, vi.transpose(0, 2, 1))
        ds = rnd(p * (dp - delta[s:e].T[:, :, None]))
        dq[s:e] = scale * np.matmul(ds, ki).transpose(1, 0, 2)
        dk[s:e] = scale * np.matmul(ds.transpose(0, 2, 1), qi).transpose(1, 0, 2)
    return rnd(dq), rnd(_fold_kv(dk, kv_heads)), rnd(_fold_kv(dv, kv_heads)), delta
