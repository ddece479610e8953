"""``torch.autograd.Function`` around the HIP attention forward and backward.

Mirrors ``varlen_attention_triton_autograd``
(``src/scree/kernels/triton/_autograd.py:17-72``): forward saves
``(q, k, v, out, lse, cu_seqlens)`` and backward returns ``(dq, dk, dv, None,
None)``.  Two differences: the Function class is defined once at import
(the reference rebuilds it on every call, ``_autograd.py:71``), and the
forward also keeps its workspace, which holds the device work lists
(schedule-sized: 16 bytes per 128-token block plus 16 per sequence; built by
the scheduler past 64 sequences, else by the forward kernel itself as it
derives its items from the offsets), so the backward launches no scheduler
and never synchronises the host.  When the grouped-query dK/dV
split pays, the backward allocates the larger workspace it needs for the
duration of the pass and copies the work list into it on the device.
"""

from __future__ import annotations

import torch

from . import _ffi
from . import attention as _attn


class VarlenAttentionHip(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens, causal):
        _attn._check_inputs(q, k, v, allow_fp32=True)
        total, n_heads, head_dim = q.shape
        cu = _attn._cu(cu_seqlens, q.device)
        qk, kk, vk = _attn._kernel_view(q), _attn._kernel_view(k), _attn._kernel_view(v)
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        lse = torch.empty((total, n_heads), dtype=torch.float32, device=q.device)
        with _ffi.device_guard(q.device):
            ws = _attn.prepare_workspace(cu, total, head_dim, causal, n_heads)
            _attn._attn_fwd(qk, kk, vk, cu, causal, out, lse, ws)
        ctx.save_for_backward(qk, kk, vk, out, lse, cu, ws)
        ctx.causal = causal
        return out

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, out, lse, cu, ws = ctx.saved_tensors
        do = _attn._kernel_view(grad_output)
        dq = torch.empty_like(q, memory_format=torch.contiguous_format)
        dk = torch.empty_like(k, memory_format=torch.contiguous_format)
        dv = torch.empty_like(v, memory_format=torch.contiguous_format)
        total, n_heads, _ = q.shape
        delta = torch.empty((total, n_heads), dtype=torch.float32, device=q.device)
        with _ffi.device_guard(q.device):
            need = _attn.bwd_workspace_bytes(cu.numel() - 1, total, n_heads, k.shape[1], q.shape[2])
            if need > ws.numel():  # grouped-query split: work list + fp32 partials
                big = torch.empty(need, dtype=torch.uint8, device=q.device)
                big[:ws.numel()].copy_(ws)
                ws = big
            _attn._attn_bwd(do, q, k, v, out, lse, cu, ctx.causal, dq, dk, dv, delta, ws)
        return dq, dk, dv, None, None


def varlen_attention_hip_autograd(q, k, v, cu_seqlens, causal: bool = False):
    """Autograd-aware varlen attention; ``out.backward()`` runs the HIP backward.

    fp16 / bf16, as the reference's Triton autograd (its launcher asserts
    them); the Array-level ``scree_amd.kernels.varlen_attention`` applies
    :class:`VarlenAttentionHip` to fp32 values as well."""
    _attn._check_inputs(q, k, v)
    return VarlenAttentionHip.apply(q, k, v, cu_seqlens, causal)
