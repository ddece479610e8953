"""Varlen softmax along the ragged dimension on the HIP kernels.

Counterpart of ``scree.kernels.reference.varlen_softmax``
(``src/scree/kernels/reference/varlen_softmax.py:13-63``), which has no GPU
kernel in the reference: its torch branch slices each sequence and calls
``torch.softmax(.., dim=0)`` in a host loop (``:44-51``).  Here one launch
normalises every sequence: for each sequence's rows and each trailing feature
column, ``y = exp(x - max) / sum(exp(x - max))``, statistics in fp32, ``y`` in
``x``'s dtype.  The call is autograd-aware (the reference's torch branch is
differentiable through ``torch.softmax``); the backward runs
``scree_varlen_softmax_bwd``.
"""

from __future__ import annotations

import torch

from . import _ffi


def _check(x, cu_seqlens):
    assert x.is_cuda, "varlen_softmax on HIP requires ROCm device tensors"
    assert x.dim() >= 1, "x must have a ragged leading axis"
    assert cu_seqlens.dtype == torch.int32, "cu_seqlens must be int32"
    assert cu_seqlens.device == x.device, "cu_seqlens must be on the same device as x"
    assert cu_seqlens.dim() == 1 and cu_seqlens.numel() >= 2, "cu_seqlens must have batch + 1 entries"
    assert x.dtype in (torch.float32, torch.float16, torch.bfloat16), f"unsupported dtype {x.dtype}"


def _features(x):
    f = 1
    for s in x.shape[1:]:
        f *= int(s)
    return f


def softmax_fwd(x, cu_seqlens, out=None):
    xc = x.contiguous()
    y = torch.empty_like(xc) if out is None else out
    assert y.shape == xc.shape and y.dtype == xc.dtype and y.is_contiguous()
    f = _features(xc)
    if xc.numel() == 0:
        return y
    with _ffi.device_guard(xc.device):
        _ffi.check(_ffi.lib().scree_varlen_softmax(
            _ffi.ptr(xc), _ffi.ptr(y), _ffi.ptr(cu_seqlens), cu_seqlens.numel() - 1,
            xc.shape[0], f, _ffi.dtype_code(xc.dtype), _ffi.stream_of(xc)))
    return y


def softmax_bwd(y, dy, cu_seqlens):
    yc, dyc = y.contiguous(), dy.contiguous().to(y.dtype)
    dx = torch.empty_like(yc)
    if yc.numel() == 0:
        return dx
    with _ffi.device_guard(yc.device):
        _ffi.check(_ffi.lib().scree_varlen_softmax_bwd(
            _ffi.ptr(yc), _ffi.ptr(dyc), _ffi.ptr(dx), _ffi.ptr(cu_seqlens), cu_seqlens.numel() - 1,
            yc.shape[0], _features(yc), _ffi.dtype_code(yc.dtype), _ffi.stream_of(yc)))
    return dx


class _VarlenSoftmaxFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cu_seqlens):
        y = softmax_fwd(x, cu_seqlens)
        ctx.save_for_backward(y, cu_seqlens)
        return y

    @staticmethod
    def backward(ctx, dy):
        y, cu = ctx.saved_tensors
        return softmax_bwd(y, dy, cu), None


def varlen_softmax_hip(x, cu_seqlens, out=None):
    """Softmax of packed ``x`` over its leading (ragged) axis within each sequence.

    ``x`` is ``(total_tokens, *features)``; ``cu_seqlens`` int32 ``(B+1)`` on
    the same device.  Returns a tensor like ``x`` (contiguous).  Rows of an
    empty sequence do not exist, so nothing is written for it.
    """
    _check(x, cu_seqlens)
    if torch.is_grad_enabled() and x.requires_grad:
        assert out is None, "out= is not supported when x requires grad"
        return _VarlenSoftmaxFn.apply(x, cu_seqlens)
    return softmax_fwd(x, cu_seqlens, out)


def varlen_softmax_hip_backward(y, dy, cu_seqlens):
    """Gradient wrt x of :func:`varlen_softmax_hip` given its output ``y`` and ``dy``."""
    _check(y, cu_seqlens)
    return softmax_bwd(y, dy, cu_seqlens)
