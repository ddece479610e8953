"""Varlen RMSNorm / LayerNorm forward and backward (oracle; test infrastructure only).

Forward formulas follow the numpy branches of the reference:

* RMSNorm, ``src/scree/kernels/reference/varlen_rmsnorm.py:58-65``:
  ``y = x / sqrt(mean(x*x, -1) + eps)``, times ``weight`` when given.
* LayerNorm, ``src/scree/kernels/reference/varlen_layernorm.py:64-74``:
  ``y = (x - mean) / sqrt(var + eps)`` with the population variance
  (``np.var`` default, torch ``unbiased=False`` at ``:58``), times ``weight``,
  plus ``bias``.

The reference's GPU launchers round ``weight`` / ``bias`` to the activation
dtype before the multiply (``triton/varlen_rmsnorm.py:79``,
``triton/varlen_layernorm.py:84,89``); callers of this oracle pass parameters
already rounded that way when they compare against the GPU path.

The reference has no norm backward.  These are the textbook closed forms,
with ``r = 1/sqrt(ms + eps)`` (RMS) or ``r = 1/sqrt(var + eps)`` (LN):

* RMS: ``g = dy*w``; ``dx = r*g - (r^3/D) * x * sum(x*g)``;
  ``dw = sum_rows(dy * x * r)``.
* LN: ``xhat = (x - mean)*r``; ``g = dy*w``;
  ``dx = r*(g - mean(g) - xhat*mean(g*xhat))``; ``dw = sum_rows(dy*xhat)``;
  ``db = sum_rows(dy)``.

All functions work on arrays whose last axis is the feature axis; every other
axis is a row axis.
"""

from __future__ import annotations

import numpy as np


def rmsnorm_fwd(x, weight=None, eps=1e-6, dtype=np.float64):
    """Return ``(y, rstd)``; ``rstd`` has the shape of ``x`` without its last axis."""
    x = np.asarray(x, dtype=dtype)
    rms = np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    y = x / rms
    if weight is not None:
        y = y * np.asarray(weight, dtype=dtype)
    return y, (1.0 / rms)[..., 0]


def rmsnorm_bwd(dy, x, weight=None, eps=1e-6, dtype=np.float64):
    """Return ``(dx, dweight)``; ``dweight`` is None when ``weight`` is None."""
    x = np.asarray(x, dtype=dtype)
    dy = np.asarray(dy, dtype=dtype)
    d = x.shape[-1]
    r = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    g = dy * np.asarray(weight, dtype=dtype) if weight is not None else dy
    dot = (x * g).sum(axis=-1, keepdims=True)
    dx = r * g - (r ** 3 / d) * x * dot
    dw = None
    if weight is not None:
        dw = (dy * x * r).reshape(-1, d).sum(axis=0)
    return dx, dw


def layernorm_fwd(x, weight=None, bias=None, eps=1e-5, dtype=np.float64):
    """Return ``(y, mean, rstd)``; stats have the shape of ``x`` without its last axis."""
    x = np.asarray(x, dtype=dtype)
    mean = x.mean(axis=-1, keepdims=True)
    var = x.var(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if weight is not None:
        y = y * np.asarray(weight, dtype=dtype)
    if bias is not None:
        y = y + np.asarray(bias, dtype=dtype)
    return y, mean[..., 0], (1.0 / np.sqrt(var + eps))[..., 0]


def layernorm_bwd(dy, x, weight=None, eps=1e-5, has_bias=False, dtype=np.float64):
    """Return ``(dx, dweight, dbias)``; absent parameters give None."""
    x = np.asarray(x, dtype=dtype)
    dy = np.asarray(dy, dtype=dtype)
    d = x.shape[-1]
    mean = x.mean(axis=-1, keepdims=True)
    r = 1.0 / np.sqrt(x.var(axis=-1, keepdims=True) + eps)
    xhat = (x - mean) * r
    g = dy * np.asarray(weight, dtype=dtype) if weight is not None else dy
    dx = r * (g - g.mean(axis=-1, keepdims=True) - xhat * (g * xhat).mean(axis=-1, keepdims=True))
    dw = (dy * xhat).reshape(-1, d).sum(axis=0) if weight is not None else None
    db = dy.reshape(-1, d).sum(axis=0) if has_bias else None
    return dx, dw, db


# ----------------------------------------------------- fused add + RMSNorm
# No counterpart in the reference: its transformer block adds the attention
# output to the residual stream and then normalises
# (``examples/03_train_step.py:46-48``).  The fused form returns both the sum
# ``h`` and ``y = rmsnorm(h)``; ``h`` is rounded to the storage dtype the way
# the separate half-precision addition rounds it (operands widened to fp32,
# summed in fp32, the fp32 sum rounded to nearest-even), and ``y`` is RMSNorm
# of that rounded ``h``.

def round_bf16(x):
    """Round to bfloat16 (nearest, ties to even) and return float64.

    Standard bit-level method on the fp32 pattern: add ``0x7fff`` plus the
    lowest kept bit, then clear the low 16 bits.  Inputs are first rounded to
    fp32 (numpy has no bfloat16); NaN is not expected here.
    """
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def add_rounded(x, residual, storage="float64"):
    """``x + residual`` as a ``storage``-dtype tensor addition produces it."""
    if storage == "float64":
        return np.asarray(x, dtype=np.float64) + np.asarray(residual, dtype=np.float64)
    s32 = np.asarray(x, dtype=np.float32) + np.asarray(residual, dtype=np.float32)
    if storage == "float32":
        return s32.astype(np.float64)
    if storage == "float16":
        return s32.astype(np.float16).astype(np.float64)
    if storage == "bfloat16":
        return round_bf16(s32)
    raise ValueError(f"unknown storage dtype {storage}")


def add_rmsnorm_fwd(x, residual, weight=None, eps=1e-6, storage="float64", dtype=np.float64):
    """Return ``(h, y, rstd)``: ``h = x + residual`` (rounded as ``storage``), ``y = rmsnorm(h)``."""
    h = add_rounded(x, residual, storage)
    y, rstd = rmsnorm_fwd(h, weight, eps, dtype)
    return h, y, rstd


def add_rmsnorm_bwd(dy, dh, h, weight=None, eps=1e-6, dtype=np.float64):
    """Return ``(dx, dweight)``: ``dx = dh + dRMSNorm(dy)`` at ``h`` is the
    gradient of both ``x`` and ``residual``; ``dh`` may be None."""
    dx, dw = rmsnorm_bwd(dy, h, weight, eps, dtype)
    if dh is not None:
        dx = dx + np.asarray(dh, dtype=dtype)
    return dx, dw
