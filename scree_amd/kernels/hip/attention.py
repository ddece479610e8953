"""Varlen self-attention on the HIP kernels: tensor-level launchers.

Signatures and behaviour mirror the reference's Triton launchers so callers
can switch by changing the import:

* :func:`varlen_attention_hip` <- ``varlen_attention_triton``
  (``src/scree/kernels/triton/varlen_attention.py:165-268``)
* :func:`varlen_attention_hip_backward` <- ``varlen_attention_triton_backward``
  (``src/scree/kernels/triton/_backward.py:288-396``)

Differences a caller can observe:

* ``block_m`` / ``block_n`` are accepted and ignored: tile shapes are fixed
  per head_dim inside the library.
* No host synchronisation: the reference reads ``max(seq_lens)`` with
  ``.item()`` (``varlen_attention.py:220-221``); here a device scheduler turns
  ``cu_seqlens`` into a work list (:func:`attention_schedule`).
* head_dim must be 16, 32, 64, 128 or 256 (the reference takes any power of
  two, ``varlen_attention.py:217``); q/k/v may be strided views whose last
  axis is contiguous (other layouts are copied to contiguous first).
* Grouped-query attention: ``k`` / ``v`` may have fewer heads than ``q`` (a
  divisor of its head count); query head ``h`` attends with K/V head
  ``h // (q_heads // kv_heads)`` and ``dk`` / ``dv`` sum over each group.
  The reference requires equal shapes (its docs list GQA as missing,
  ``docs/kernels.md:177``); equal shapes behave exactly as there.
"""

from __future__ import annotations

import functools
import math

import torch

from . import _ffi


def _check_inputs(q, k, v, allow_fp32: bool = False):
    """The launchers' checks (``triton/varlen_attention.py:213-215``): fp16 or
    bf16, as the reference's GPU launchers; ``allow_fp32`` for the
    Array-level path, which also takes fp32 (computed by the fp32 kernels)."""
    assert k.shape == v.shape, "k and v must have identical shape"
    assert q.dim() == 3 and k.dim() == 3, "q, k, v must be (total_tokens, n_heads, head_dim)"
    assert q.shape[0] == k.shape[0] and q.shape[2] == k.shape[2], (
        "q, k, v must share total_tokens and head_dim")
    assert k.shape[1] >= 1 and q.shape[1] % k.shape[1] == 0, (
        "k/v heads must divide q heads (grouped-query attention)")
    assert q.is_cuda, "varlen_attention_hip requires ROCm device tensors"
    dtypes = (torch.float16, torch.bfloat16, torch.float32) if allow_fp32 else (torch.float16,
                                                                               torch.bfloat16)
    assert q.dtype in dtypes, "fp16 or bf16 only" if not allow_fp32 else "fp16, bf16 or fp32 only"
    assert q.dtype == k.dtype == v.dtype, "q, k, v must share a dtype"
    assert q.dim() == 3, "q, k, v must be (total_tokens, n_heads, head_dim)"


# Row and head strides the kernels index with 32-bit element offsets.
_MAX_STRIDE = 1 << 24


def _kernel_view(t: torch.Tensor) -> torch.Tensor:
    """``t`` itself when the library can read it in place, else a contiguous copy.

    In place means: head_dim contiguous, row and head strides non-negative
    multiples of 8 elements below 2^24, a 16-byte aligned base, and rows that
    do not overlap -- exactly what ``check_tensor`` in the library accepts.
    """
    s0, s1, s2 = t.stride()
    ok = (
        s2 == 1
        and s0 % 8 == 0
        and s1 % 8 == 0
        and 0 <= s0 < _MAX_STRIDE
        and 0 <= s1 < _MAX_STRIDE
        and t.data_ptr() % 16 == 0
        and (t.shape[0] <= 1 or s0 >= t.shape[2])
    )
    return t if ok else t.contiguous()


def _cu(cu_seqlens: torch.Tensor, device) -> torch.Tensor:
    cu = cu_seqlens
    if cu.device != device:
        cu = cu.to(device)
    if cu.dtype != torch.int32:
        cu = cu.to(torch.int32)
    return cu.contiguous()


# The size and mode queries are pure functions of a few integers; a training
# loop asks them with the same arguments every step.
@functools.lru_cache(maxsize=256)
def workspace_bytes(batch: int, total: int, head_dim: int) -> int:
    return int(_ffi.lib().scree_attn_workspace_bytes(batch, total, head_dim))


@functools.lru_cache(maxsize=256)
def needs_schedule(batch: int, total: int, heads: int, head_dim: int) -> bool:
    """Whether the forward reads a work list that :func:`attention_schedule`
    must build first.  At most 64 sequences in a launch of a few rounds of
    workgroups need none: the forward derives its items from ``cu_seqlens``
    and leaves the lists in its workspace for the backward calls that follow
    on the same workspace."""
    return bool(_ffi.lib().scree_attn_needs_schedule(batch, total, heads, head_dim))


def prepare_workspace(cu_seqlens: torch.Tensor, total_tokens: int, head_dim: int, causal: bool,
                      heads: int, workspace: torch.Tensor = None,
                      for_backward: bool = False) -> torch.Tensor:
    """A workspace for the attention calls on these offsets: the work lists
    built into it when the forward reads them, or when ``for_backward`` (a
    backward that no forward on this workspace precedes), else the room alone
    (allocated when ``workspace`` is None), which the forward fills."""
    batch = cu_seqlens.numel() - 1
    if for_backward or needs_schedule(batch, total_tokens, heads, head_dim):
        return attention_schedule(cu_seqlens, total_tokens, head_dim, causal, workspace)
    if workspace is None:
        workspace = torch.empty(workspace_bytes(batch, total_tokens, head_dim), dtype=torch.uint8,
                                device=cu_seqlens.device)
    return workspace


@functools.lru_cache(maxsize=256)
def bwd_workspace_bytes(batch: int, total: int, heads: int, kv_heads: int, head_dim: int) -> int:
    """Workspace bytes for a forward + backward with ``kv_heads`` K/V heads:
    the schedule, plus room for the grouped-query dK/dV split when it pays."""
    return int(_ffi.lib().scree_attn_bwd_workspace_bytes_gqa(batch, total, heads, kv_heads,
                                                             head_dim))


def _bwd_workspace(cu_seqlens, total, heads, kv_heads, head_dim):
    nbytes = bwd_workspace_bytes(cu_seqlens.numel() - 1, total, heads, kv_heads, head_dim)
    return torch.empty(nbytes, dtype=torch.uint8, device=cu_seqlens.device)


def attention_schedule(cu_seqlens: torch.Tensor, total_tokens: int, head_dim: int, causal: bool,
                       workspace: torch.Tensor = None) -> torch.Tensor:
    """Build the device work list for ``cu_seqlens`` and return its workspace.

    The returned uint8 tensor can be passed as ``workspace=`` to the forward
    and backward launchers for the same ``cu_seqlens``/``head_dim``/``causal``.
    """
    lib = _ffi.lib()
    batch = cu_seqlens.numel() - 1
    nbytes = workspace_bytes(batch, total_tokens, head_dim)
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=cu_seqlens.device)
    with _ffi.device_guard(cu_seqlens.device):
        _ffi.check(lib.scree_attn_schedule(
            _ffi.ptr(cu_seqlens), batch, total_tokens, head_dim, int(bool(causal)),
            _ffi.ptr(workspace), workspace.numel(), _ffi.stream_of(cu_seqlens)))
    return workspace


def schedule_items(workspace: torch.Tensor, with_ranges: bool = False, by_sequence: bool = False,
                   tmax: int = 0):
    """Decode a schedule workspace into ``(count, items)`` on the host (tests).

    ``items`` is ``(count, 2)`` of ``(seq, blk)``, or ``(count, 4)`` with the
    sequence's clamped ``(start, len)`` when ``with_ranges``.  The workspace
    holds two lists of ``tmax = ceil(total / 128) + batch`` slots: longest work
    first, then (``by_sequence``) the same items sequence by sequence.
    """
    header = workspace[:16].view(torch.int32).cpu()
    count = int(header[0])
    base = 16 + (16 * tmax if by_sequence else 0)
    items = workspace[base:base + 16 * count].view(torch.int32).reshape(-1, 4).cpu()
    return count, (items if with_ranges else items[:, :2].contiguous())


def _attn_fwd(q, k, v, cu, causal, out, lse, workspace):
    lib = _ffi.lib()
    total, heads, head_dim = q.shape
    strides = _ffi.int64_array(q.stride()[:2] + k.stride()[:2] + v.stride()[:2] + out.stride()[:2])
    _ffi.check(lib.scree_attn_fwd_gqa(
        _ffi.ptr(q), _ffi.ptr(k), _ffi.ptr(v), _ffi.ptr(out), _ffi.ptr(lse), _ffi.ptr(cu),
        cu.numel() - 1, total, heads, k.shape[1], head_dim, strides, 1.0 / math.sqrt(head_dim),
        int(bool(causal)), _ffi.dtype_code(q.dtype), _ffi.ptr(workspace), workspace.numel(),
        _ffi.stream_of(q)))


def _attn_bwd(do, q, k, v, o, lse, cu, causal, dq, dk, dv, delta, workspace):
    lib = _ffi.lib()
    total, heads, head_dim = q.shape
    ts = (do, q, k, v, o, dq, dk, dv)
    strides = _ffi.int64_array(sum((t.stride()[:2] for t in ts), ()))
    _ffi.check(lib.scree_attn_bwd_gqa(
        _ffi.ptr(do), _ffi.ptr(q), _ffi.ptr(k), _ffi.ptr(v), _ffi.ptr(o), _ffi.ptr(lse),
        _ffi.ptr(dq), _ffi.ptr(dk), _ffi.ptr(dv), _ffi.ptr(delta), _ffi.ptr(cu),
        cu.numel() - 1, total, heads, k.shape[1], head_dim, strides, 1.0 / math.sqrt(head_dim),
        int(bool(causal)), _ffi.dtype_code(q.dtype), _ffi.ptr(workspace), workspace.numel(),
        _ffi.stream_of(q)))


def _attn_bwd_dq(do, q, k, v, o, lse, cu, causal, dq, delta, workspace):
    lib = _ffi.lib()
    total, heads, head_dim = q.shape
    strides = _ffi.int64_array(sum((t.stride()[:2] for t in (do, q, k, v, o, dq)), ()))
    _ffi.check(lib.scree_attn_bwd_dq_gqa(
        _ffi.ptr(do), _ffi.ptr(q), _ffi.ptr(k), _ffi.ptr(v), _ffi.ptr(o), _ffi.ptr(lse),
        _ffi.ptr(dq), _ffi.ptr(delta), _ffi.ptr(cu), cu.numel() - 1, total, heads, k.shape[1],
        head_dim, strides, 1.0 / math.sqrt(head_dim), int(bool(causal)),
        _ffi.dtype_code(q.dtype), _ffi.ptr(workspace), workspace.numel(), _ffi.stream_of(q)))


def _attn_bwd_dkv(do, q, k, v, lse, delta, cu, causal, dk, dv, workspace):
    lib = _ffi.lib()
    total, heads, head_dim = q.shape
    strides = _ffi.int64_array(sum((t.stride()[:2] for t in (do, q, k, v, dk, dv)), ()))
    _ffi.check(lib.scree_attn_bwd_dkv_gqa(
        _ffi.ptr(do), _ffi.ptr(q), _ffi.ptr(k), _ffi.ptr(v), _ffi.ptr(lse), _ffi.ptr(delta),
        _ffi.ptr(dk), _ffi.ptr(dv), _ffi.ptr(cu), cu.numel() - 1, total, heads, k.shape[1],
        head_dim, strides, 1.0 / math.sqrt(head_dim), int(bool(causal)),
        _ffi.dtype_code(q.dtype), _ffi.ptr(workspace), workspace.numel(), _ffi.stream_of(q)))


def varlen_attention_hip(q, k, v, cu_seqlens, causal: bool = False, block_m: int = 64,
                         block_n: int = 64, return_lse: bool = False, out=None, lse_buffer=None,
                         workspace=None):
    """Variable-length self-attention forward on the HIP kernels.

    Parameters follow ``varlen_attention_triton``: ``q, k, v`` are
    ``(total_tokens, n_heads, head_dim)`` fp16/bf16 device tensors,
    ``cu_seqlens`` the int32 ``(batch + 1,)`` offsets.  ``out`` /
    ``lse_buffer`` are optional preallocated outputs.  ``workspace`` is an
    optional workspace from :func:`prepare_workspace` (or a schedule from
    :func:`attention_schedule`) for these offsets.

    Returns ``out`` or ``(out, lse)`` with ``lse`` the natural-log
    logsumexp of the scaled scores, ``(total_tokens, n_heads)`` fp32.
    """
    del block_m, block_n  # tile shapes are fixed inside the library
    _check_inputs(q, k, v)
    total, n_heads, head_dim = q.shape
    if out is None:
        out = torch.empty_like(q)
    else:
        assert out.shape == q.shape and out.dtype == q.dtype and out.device == q.device
    if lse_buffer is None:
        lse = torch.empty((total, n_heads), dtype=torch.float32, device=q.device)
    else:
        assert lse_buffer.shape == (total, n_heads)
        assert lse_buffer.dtype == torch.float32 and lse_buffer.device == q.device
        assert lse_buffer.is_contiguous(), "lse_buffer must be contiguous"
        lse = lse_buffer
    cu = _cu(cu_seqlens, q.device)
    qk, kk, vk = _kernel_view(q), _kernel_view(k), _kernel_view(v)
    ok = _kernel_view(out)
    with _ffi.device_guard(q.device):
        if workspace is None:
            workspace = prepare_workspace(cu, total, head_dim, causal, n_heads)
        _attn_fwd(qk, kk, vk, cu, causal, ok, lse, workspace)
    if ok is not out:
        out.copy_(ok)
    if return_lse:
        return out, lse
    return out


def varlen_attention_hip_backward(do, q, k, v, o, lse, cu_seqlens, causal: bool = False,
                                  block_m: int = 64, block_n: int = 64, workspace=None,
                                  delta_buffer=None):
    """``(dq, dk, dv)`` for varlen self-attention; mirrors ``varlen_attention_triton_backward``.

    ``lse`` is the forward's logsumexp.  ``delta_buffer`` (optional,
    ``(total, heads)`` fp32) receives ``rowsum(o * do)``.
    """
    del block_m, block_n
    _check_inputs(q, k, v)
    assert do.shape == q.shape and o.shape == q.shape, "do and o must match q"
    total, n_heads, head_dim = q.shape
    assert lse.shape == (total, n_heads) and lse.dtype == torch.float32
    cu = _cu(cu_seqlens, q.device)
    # fresh, contiguous gradients (empty_like would copy a view's strides)
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    if delta_buffer is None:
        delta = torch.empty((total, n_heads), dtype=torch.float32, device=q.device)
    else:
        # the dQ kernel writes fp32 Delta at contiguous (token, head) offsets
        assert delta_buffer.shape == (total, n_heads), "delta_buffer must be (total_tokens, n_heads)"
        assert delta_buffer.dtype == torch.float32, "delta_buffer must be float32"
        assert delta_buffer.device == q.device, "delta_buffer must be on q's device"
        assert delta_buffer.is_contiguous(), "delta_buffer must be contiguous"
        delta = delta_buffer
    ins = [_kernel_view(t) for t in (do, q, k, v, o)]
    with _ffi.device_guard(q.device):
        if workspace is None:
            workspace = prepare_workspace(cu, total, head_dim, causal, n_heads,
                                          _bwd_workspace(cu, total, n_heads, k.shape[1], head_dim),
                                          for_backward=True)
        _attn_bwd(*ins, lse.contiguous(), cu, causal, dq, dk, dv, delta, workspace)
    return dq, dk, dv
