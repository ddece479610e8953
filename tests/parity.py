"""Helpers shared by the GPU parity tests: seeded inputs and tolerance rules.

Tolerances (north star): attention outputs within 2e-3 and dq/dk/dv within
5e-3 max-abs of an fp32-or-better reference, norms within 1e-3 (half) and 1e-5
(fp32).  The reference is the oracle evaluated in fp64 on the *same rounded
inputs* the GPU sees.  fp16 attention at ordinary logits uses the flat bounds
unchanged.  fp32 attention (the Array-level path) is held to 1e-5, the
reference's own fp32 bound, plus the same two terms with ``u = 2^-24`` and
``E_ref`` from the reference's fp32 arithmetic.

bf16 keeps 8 significant bits: rounding the stored result alone can exceed
the flat bounds, and so can rounding P and dS before their dots, which the
reference's GPU kernels do too (``triton/varlen_attention.py:142``,
``_backward.py:174,181,282``).  Attention in bf16, and at large logits in
either dtype, is therefore held to ``atol + u*|ref| + E_ref``: the flat bound,
the rounding of the stored result itself (``u = 2^-8`` for bf16, ``2^-11``
for fp16), and ``E_ref``, the largest amount by which the reference kernels'
own arithmetic (emulated by ``oracle.attention.attention_*_rounded``) departs
from the fp64 oracle beyond that same output rounding, on the same inputs
(:func:`reference_excess`).  Norms in half precision add the output-rounding
term ``u*|ref|`` to their flat bound.
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


def reference_excess(q, k, v, do, off, causal, dtype, o=None, lse=None):
    """``E_ref`` per output (O, dQ, dK, dV): max(|emulated - exact| - u|exact|, 0)
    for the reference kernels' arithmetic in ``dtype`` on these fp64 inputs.

    The backward's inputs include the forward's O and LSE.  Given ``o`` and
    ``lse`` (the ones the HIP backward consumed), the reference backward is
    emulated on exactly those, and the exact backward is evaluated at that O
    (the gradients depend on O through Delta), as the tests evaluate it.
    Without them both use the emulated reference forward's O and LSE.  The
    distinction matters at large logits in bf16: a different O moves every
    Delta, which re-draws the rounding of dS, and the largest excess of dK
    then moves by up to 40% (12.7e-3 -> 17.8e-3 on one D = 16 case, for the
    reference's own arithmetic) -- more than the flat bound that separates the
    two sides of the comparison.
    """
    from oracle.attention import (attention_bwd, attention_bwd_rounded, attention_fwd,
                                  attention_fwd_rounded)

    u = UNIT[dtype]
    ro, rl = attention_fwd(q, k, v, off, causal=causal)
    if dtype == torch.float32:
        # the reference's Array-level fp32 path: the same sums as GEMMs in
        # fp32 arithmetic (reference/varlen_attention.py:90-113)
        eo, el = attention_fwd(q, k, v, off, causal=causal, dtype=np.float32)

        def emulate(bo, bl):
            return attention_bwd(do, q, k, v, bo, bl, off, causal=causal, dtype=np.float32)[:3]
    else:
        operand = {torch.float16: "float16", torch.bfloat16: "bfloat16"}[dtype]
        eo, el = attention_fwd_rounded(q, k, v, off, causal=causal, operand=operand)

        def emulate(bo, bl):
            return attention_bwd_rounded(do, q, k, v, bo, bl, off, causal=causal, operand=operand)
    ex = lambda got, ref: max(0.0, float((np.abs(got - ref) - u * np.abs(ref)).max()))  # noqa: E731
    out = {"O": ex(eo, ro)}
    if do is not None:
        bo = eo if o is None else o
        bl = el if lse is None else lse
        emul = emulate(bo, bl)
        exact = attention_bwd(do, q, k, v, bo, rl, off, causal=causal)
        for name, a, b in zip(("dQ", "dK", "dV"), emul, exact):
            out[name] = ex(a, b)
    return out


def check_attn(name, got, want, atol, dtype, e_ref):
    """``|got - want| <= atol + E_ref + u*|want|`` (see the module docstring)."""
    u = UNIT[dtype]
    beyond = float((np.abs(got - want) - u * np.abs(want)).max()) if got.size else 0.0
    say(f"  {name}: beyond output rounding: hip {beyond:.3e}, reference arithmetic E_ref={e_ref:.3e}")
    return check_close(name, got, want, atol + e_ref, extra=np.abs(want), unit=UNIT[dtype])
