"""Varlen RMSNorm / LayerNorm on the HIP kernels: tensor-level launchers.

* :func:`varlen_rmsnorm_hip` <- ``varlen_rmsnorm_triton``
  (``src/scree/kernels/triton/varlen_rmsnorm.py:49-99``)
* :func:`varlen_layernorm_hip` <- ``varlen_layernorm_triton``
  (``src/scree/kernels/triton/varlen_layernorm.py:52-109``)
* :func:`varlen_add_rmsnorm_hip` -- fused residual add + RMSNorm (no
  counterpart in the reference; its block adds then normalises,
  ``examples/03_train_step.py:46-48``)

As in the reference, ``x`` of any rank is normalised over its last axis,
``weight`` / ``bias`` are rounded to ``x``'s dtype before the multiply
(``varlen_rmsnorm.py:79``, ``varlen_layernorm.py:84,89``) and the statistics
are computed in fp32.  Unlike the reference, these launchers are
autograd-aware: when ``x``, ``weight`` or ``bias`` requires grad the call
records a ``torch.autograd.Function`` whose backward runs the HIP backward
kernels (the reference has no norm backward).  The explicit backward
launchers are :func:`varlen_rmsnorm_hip_backward` and
:func:`varlen_layernorm_hip_backward`.
"""

from __future__ import annotations

import torch

from . import _ffi


def _flat(x):
    assert x.is_cuda, "varlen norms on HIP require ROCm device tensors"
    d = x.shape[-1]
    return x.reshape(-1, d).contiguous(), d


def _param(p, d, device, dtype, name):
    if p is None:
        return None
    assert p.shape == (d,), f"{name} must have shape ({d},)"
    assert p.device == device, f"{name} must be on {device}"
    return p.to(dtype).contiguous()


def _dparam_code(p):
    return _ffi.dtype_code(p.dtype) if p.dtype in (torch.float32, torch.float16, torch.bfloat16) else _ffi.DTYPE_F32


def rmsnorm_fwd(x2, w, eps, want_stats):
    rows, d = x2.shape
    y = torch.empty_like(x2)
    rstd = torch.empty(rows, dtype=torch.float32, device=x2.device) if want_stats else None
    with _ffi.device_guard(x2.device):
        _ffi.check(_ffi.lib().scree_rmsnorm_fwd(
            _ffi.ptr(x2), _ffi.ptr(w), _ffi.ptr(y), _ffi.ptr(rstd), rows, d, float(eps),
            _ffi.dtype_code(x2.dtype), _ffi.stream_of(x2)))
    return y, rstd


def layernorm_fwd(x2, w, b, eps, want_stats):
    rows, d = x2.shape
    y = torch.empty_like(x2)
    mean = rstd = None
    if want_stats:
        mean = torch.empty(rows, dtype=torch.float32, device=x2.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x2.device)
    with _ffi.device_guard(x2.device):
        _ffi.check(_ffi.lib().scree_layernorm_fwd(
            _ffi.ptr(x2), _ffi.ptr(w), _ffi.ptr(b), _ffi.ptr(y), _ffi.ptr(mean), _ffi.ptr(rstd),
            rows, d, float(eps), _ffi.dtype_code(x2.dtype), _ffi.stream_of(x2)))
    return y, mean, rstd


def _workspace(rows, d, device):
    n = int(_ffi.lib().scree_norm_bwd_workspace_bytes(rows, d))
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def rmsnorm_bwd(dy2, x2, w, rstd, want_dw, dw_like=None):
    rows, d = x2.shape
    dx = torch.empty_like(x2)
    dw = None
    code = _ffi.DTYPE_F32
    if want_dw:
        code = _dparam_code(dw_like) if dw_like is not None else _ffi.DTYPE_F32
        dw = torch.empty(d, dtype=_code_dtype(code), device=x2.device)
    ws = _workspace(rows, d, x2.device)
    with _ffi.device_guard(x2.device):
        _ffi.check(_ffi.lib().scree_rmsnorm_bwd(
            _ffi.ptr(dy2), _ffi.ptr(x2), _ffi.ptr(w), _ffi.ptr(rstd), _ffi.ptr(dx), _ffi.ptr(dw),
            code, rows, d, _ffi.dtype_code(x2.dtype), _ffi.ptr(ws), ws.numel(),
            _ffi.stream_of(x2)))
    return dx, dw


def layernorm_bwd(dy2, x2, w, mean, rstd, want_dw, want_db, p_like=None):
    rows, d = x2.shape
    dx = torch.empty_like(x2)
    code = _dparam_code(p_like) if p_like is not None else _ffi.DTYPE_F32
    dw = torch.empty(d, dtype=_code_dtype(code), device=x2.device) if want_dw else None
    db = torch.empty(d, dtype=_code_dtype(code), device=x2.device) if want_db else None
    ws = _workspace(rows, d, x2.device)
    with _ffi.device_guard(x2.device):
        _ffi.check(_ffi.lib().scree_layernorm_bwd(
            _ffi.ptr(dy2), _ffi.ptr(x2), _ffi.ptr(w), _ffi.ptr(mean), _ffi.ptr(rstd),
            _ffi.ptr(dx), _ffi.ptr(dw), _ffi.ptr(db), code, rows, d, _ffi.dtype_code(x2.dtype),
            _ffi.ptr(ws), ws.numel(), _ffi.stream_of(x2)))
    return dx, dw, db


def add_rmsnorm_fwd(x2, r2, w, eps, want_stats):
    rows, d = x2.shape
    h = torch.empty_like(x2)
    y = torch.empty_like(x2)
    rstd = torch.empty(rows, dtype=torch.float32, device=x2.device) if want_stats else None
    with _ffi.device_guard(x2.device):
        _ffi.check(_ffi.lib().scree_add_rmsnorm_fwd(
            _ffi.ptr(x2), _ffi.ptr(r2), _ffi.ptr(w), _ffi.ptr(h), _ffi.ptr(y), _ffi.ptr(rstd),
            rows, d, float(eps), _ffi.dtype_code(x2.dtype), _ffi.stream_of(x2)))
    return h, y, rstd


def add_rmsnorm_bwd(dy2, dh2, h2, w, rstd, want_dw, dw_like=None):
    rows, d = h2.shape
    dx = torch.empty_like(h2)
    dw = None
    code = _ffi.DTYPE_F32
    if want_dw:
        code = _dparam_code(dw_like) if dw_like is not None else _ffi.DTYPE_F32
        dw = torch.empty(d, dtype=_code_dtype(code), device=h2.device)
    ws = _workspace(rows, d, h2.device)
    with _ffi.device_guard(h2.device):
        _ffi.check(_ffi.lib().scree_add_rmsnorm_bwd(
            _ffi.ptr(dy2), _ffi.ptr(dh2), _ffi.ptr(h2), _ffi.ptr(w), _ffi.ptr(rstd), _ffi.ptr(dx),
            _ffi.ptr(dw), code, rows, d, _ffi.dtype_code(h2.dtype), _ffi.ptr(ws), ws.numel(),
            _ffi.stream_of(h2)))
    return dx, dw


def _code_dtype(code):
    return {_ffi.DTYPE_F32: torch.float32, _ffi.DTYPE_F16: torch.float16,
            _ffi.DTYPE_BF16: torch.bfloat16}[code]


class _RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        x2, d = _flat(x)
        w = _param(weight, d, x.device, x.dtype, "weight")
        y, rstd = rmsnorm_fwd(x2, w, eps, want_stats=True)
        ctx.save_for_backward(x2, w, rstd, weight)
        ctx.shape = x.shape
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, w, rstd, weight = ctx.saved_tensors
        dy2 = dy.reshape(x2.shape).contiguous()
        want_dw = weight is not None and ctx.needs_input_grad[1]
        dx, dw = rmsnorm_bwd(dy2, x2, w, rstd, want_dw, dw_like=weight)
        if dw is not None and dw.dtype != weight.dtype:
            dw = dw.to(weight.dtype)
        return dx.reshape(ctx.shape), dw, None


class _LayerNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        x2, d = _flat(x)
        w = _param(weight, d, x.device, x.dtype, "weight")
        b = _param(bias, d, x.device, x.dtype, "bias")
        y, mean, rstd = layernorm_fwd(x2, w, b, eps, want_stats=True)
        ctx.save_for_backward(x2, w, mean, rstd, weight, bias)
        ctx.shape = x.shape
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, w, mean, rstd, weight, bias = ctx.saved_tensors
        dy2 = dy.reshape(x2.shape).contiguous()
        want_dw = weight is not None and ctx.needs_input_grad[1]
        want_db = bias is not None and ctx.needs_input_grad[2]
        like = weight if weight is not None else bias
        dx, dw, db = layernorm_bwd(dy2, x2, w, mean, rstd, want_dw, want_db, p_like=like)
        if dw is not None and dw.dtype != weight.dtype:
            dw = dw.to(weight.dtype)
        if db is not None and db.dtype != bias.dtype:
            db = db.to(bias.dtype)
        return dx.reshape(ctx.shape), dw, db, None


class _AddRMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, residual, weight, eps):
        x2, d = _flat(x)
        r2, _ = _flat(residual)
        w = _param(weight, d, x.device, x.dtype, "weight")
        h, y, rstd = add_rmsnorm_fwd(x2, r2, w, eps, want_stats=True)
        ctx.save_for_backward(h, w, rstd, weight)
        ctx.shape = x.shape
        return h.reshape(x.shape), y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dh, dy):
        h2, w, rstd, weight = ctx.saved_tensors
        want_dw = weight is not None and ctx.needs_input_grad[2]
        dy2 = (torch.zeros_like(h2) if dy is None else dy.reshape(h2.shape).contiguous())
        dh2 = None if dh is None else dh.reshape(h2.shape).contiguous()
        dx, dw = add_rmsnorm_bwd(dy2, dh2, h2, w, rstd, want_dw, dw_like=weight)
        if dw is not None and dw.dtype != weight.dtype:
            dw = dw.to(weight.dtype)
        dx = dx.reshape(ctx.shape)
        # x and residual receive the same gradient (as torch's own add backward does)
        return dx, dx, dw, None


def _needs_grad(*ts):
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def varlen_rmsnorm_hip(x, weight=None, eps: float = 1e-6):
    """RMSNorm over the last axis; same shape and dtype as ``x``."""
    if _needs_grad(x, weight):
        return _RMSNormFn.apply(x, weight, eps)
    x2, d = _flat(x)
    w = _param(weight, d, x.device, x.dtype, "weight")
    y, _ = rmsnorm_fwd(x2, w, eps, want_stats=False)
    return y.reshape(x.shape)


def varlen_layernorm_hip(x, weight=None, bias=None, eps: float = 1e-5):
    """LayerNorm (population variance) over the last axis; same shape and dtype as ``x``."""
    if _needs_grad(x, weight, bias):
        return _LayerNormFn.apply(x, weight, bias, eps)
    x2, d = _flat(x)
    w = _param(weight, d, x.device, x.dtype, "weight")
    b = _param(bias, d, x.device, x.dtype, "bias")
    y, _, _ = layernorm_fwd(x2, w, b, eps, want_stats=False)
    return y.reshape(x.shape)


def varlen_add_rmsnorm_hip(x, residual, weight=None, eps: float = 1e-6):
    """Fused residual add + RMSNorm: returns ``(h, y)`` with ``h = x + residual``
    (rounded to ``x``'s dtype exactly as ``x + residual`` is) and
    ``y = varlen_rmsnorm_hip(h, weight, eps)``, in one pass over HBM.

    The pre-norm transformer step of the reference's block
    (``examples/03_train_step.py:46-48``); autograd-aware like the other
    launchers (``x`` and ``residual`` receive the same gradient).
    """
    assert residual.shape == x.shape, "residual must have x's shape"
    assert residual.dtype == x.dtype and residual.device == x.device, (
        "residual must share x's dtype and device")
    if _needs_grad(x, residual, weight):
        return _AddRMSNormFn.apply(x, residual, weight, eps)
    x2, d = _flat(x)
    r2, _ = _flat(residual)
    w = _param(weight, d, x.device, x.dtype, "weight")
    h, y, _ = add_rmsnorm_fwd(x2, r2, w, eps, want_stats=False)
    return h.reshape(x.shape), y.reshape(x.shape)


def varlen_add_rmsnorm_hip_backward(dy, dh, h, weight=None, eps: float = 1e-6, rstd=None):
    """``(dx, dweight)`` of the fused add + RMSNorm: ``dx = dh + dRMSNorm(h)``
    (``dh`` may be None); ``rstd`` from the forward is recomputed when absent."""
    h2, d = _flat(h)
    w = _param(weight, d, h.device, h.dtype, "weight")
    if rstd is None:
        _, rstd = rmsnorm_fwd(h2, w, eps, want_stats=True)
    dh2 = None if dh is None else dh.reshape(h2.shape).contiguous()
    dx, dw = add_rmsnorm_bwd(dy.reshape(h2.shape).contiguous(), dh2, h2, w,
                             rstd.reshape(-1).contiguous(), weight is not None, dw_like=weight)
    return dx.reshape(h.shape), dw


def varlen_rmsnorm_hip_autograd(x, weight=None, eps: float = 1e-6):
    """Always records the autograd node (for callers that set requires_grad later)."""
    return _RMSNormFn.apply(x, weight, eps)


def varlen_layernorm_hip_autograd(x, weight=None, bias=None, eps: float = 1e-5):
    return _LayerNormFn.apply(x, weight, bias, eps)


def varlen_rmsnorm_hip_backward(dy, x, weight=None, eps: float = 1e-6, rstd=None):
    """``(dx, dweight)`` of RMSNorm; ``rstd`` from the forward is recomputed when absent."""
    x2, d = _flat(x)
    w = _param(weight, d, x.device, x.dtype, "weight")
    if rstd is None:
        _, rstd = rmsnorm_fwd(x2, w, eps, want_stats=True)
    dx, dw = rmsnorm_bwd(dy.reshape(x2.shape).contiguous(), x2, w, rstd.reshape(-1).contiguous(),
                         weight is not None, dw_like=weight)
    return dx.reshape(x.shape), dw


def varlen_layernorm_hip_backward(dy, x, weight=None, bias=None, eps: float = 1e-5, mean=None,
                                  rstd=None):
    """``(dx, dweight, dbias)`` of LayerNorm; statistics recomputed when absent."""
    x2, d = _flat(x)
    w = _param(weight, d, x.device, x.dtype, "weight")
    if mean is None or rstd is None:
        _, mean, rstd = layernorm_fwd(x2, w, None, eps, want_stats=True)
    like = weight if weight is not None else bias
    dx, dw, db = layernorm_bwd(dy.reshape(x2.shape).contiguous(), x2, w,
                               mean.reshape(-1).contiguous(), rstd.reshape(-1).contiguous(),
                               weight is not None, bias is not None, p_like=like)
    return dx.reshape(x.shape), dw, db
