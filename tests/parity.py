"""Helpers shared by the GPU parity tests: seeded inputs and tolerance rules.

Tolerances (north star): attention outputs within 2e-3 and dq/dk/dv within
5e-3 max-abs of an fp32-or-better reference, norms within 1e-3 (half) and 1e-5
(fp32).  The reference is the oracle evaluated in fp64 on the *same rounded
inputs* the GPU sees.  bf16 keeps 8 significant bits, so rounding an operand
(P or dS before an MFMA, the output itself) can exceed those flat bounds on
its own; for bf16 the bound adds that rounding term, computed elementwise
from the oracle: ``u * (|P| |V| + |O|)`` for O, and the analogous products
for the gradients, with ``u = 2^-8``.  fp16 uses the flat bounds unchanged.
"""

from __future__ import annotations

import math

import numpy as np
import torch

UNIT = {torch.float32: 2.0 ** -24, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def say(msg: str) -> None:
    print(msg, flush=True)


def randn(shape, dtype, seed, device="cuda", scale=1.0, mean=0.0):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g, dtype=torch.float32) * scale + mean
    return t.to(dtype).to(device)


def np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def cu_of(lengths, device="cuda"):
    off = np.zeros(len(lengths) + 1, dtype=np.int32)
    off[1:] = np.cumsum(lengths)
    return off, torch.from_numpy(off).to(device)


def attn_abs_terms(q, k, v, do, lse, off, causal):
    """Elementwise magnitudes that bound operand rounding (fp64, numpy).

    Returns (P|V|, P^T|dO|, scale*|dS||K|, scale*|dS|^T|Q|) given the oracle's
    lse; dS uses Delta computed from the same inputs.
    """
    n, h, d = q.shape
    scale = 1.0 / math.sqrt(d)
    pv = np.zeros_like(q)
    pdo = np.zeros_like(q)
    dsk = np.zeros_like(q)
    dsq = np.zeros_like(q)
    for b in range(len(off) - 1):
        s, e = int(off[b]), int(off[b + 1])
        if e <= s:
            continue
        qi, ki, vi = q[s:e].transpose(1, 0, 2), k[s:e].transpose(1, 0, 2), v[s:e].transpose(1, 0, 2)
        sc = qi @ ki.transpose(0, 2, 1) * scale
        if causal:
            sc = np.where(np.triu(np.ones((e - s, e - s), bool), 1), -np.inf, sc)
        p = np.exp(sc - lse[s:e].T[:, :, None])
        pv[s:e] = (p @ np.abs(vi)).transpose(1, 0, 2)
        if do is not None:
            doi = do[s:e].transpose(1, 0, 2)
            o = (p @ vi)
            delta = (o * doi).sum(-1)
            dp = doi @ vi.transpose(0, 2, 1)
            ds = np.abs(p * (dp - delta[:, :, None]))
            pdo[s:e] = (p.transpose(0, 2, 1) @ np.abs(doi)).transpose(1, 0, 2)
            dsk[s:e] = (scale * ds @ np.abs(ki)).transpose(1, 0, 2)
            dsq[s:e] = (scale * ds.transpose(0, 2, 1) @ np.abs(qi)).transpose(1, 0, 2)
    return pv, pdo, dsk, dsq


def check_close(name, got, want, atol, extra=None, unit=0.0):
    """Assert |got - want| <= atol + unit * extra (elementwise); print the figures.

    The printed line also says whether the flat bound ``atol`` alone holds
    (``flat=met``), which for bf16 is reported beside the widened bound.
    """
    err = np.abs(got - want)
    bound = atol + (unit * extra if extra is not None else 0.0)
    worst = float((err - bound).max()) if err.size else 0.0
    max_abs = float(err.max()) if err.size else 0.0
    say(f"  {name}: max_abs={max_abs:.3e} "
        f"(atol {atol:g}{' + u*terms' if extra is not None else ''}) margin={-worst:.3e} "
        f"flat={'met' if max_abs <= atol else 'exceeded'}")
    assert worst <= 0.0, f"{name}: exceeds tolerance by {worst:.3e}"
    return max_abs
