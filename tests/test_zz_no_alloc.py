"""The allocation-free attention forward (scree_attn_fwd_noalloc) against the
workspace forward it is a variant of (scheduler + scree_attn_fwd_gqa on a
caller-owned workspace): bit-identical outputs and LSE, on calls in a row of
decreasing size, plus the host-side size limit.  The sequence of calls
alternates the two ways the entry point gets its items: a forward that
derives them from the offsets (scree_attn_needs_schedule == 0) never reads
the static array, so the calls that schedule (100 sequences, past the
derivation's 64) sit between deriving calls of other sizes, where a stale or
misaddressed schedule in the static array would change the output."""

import ctypes
import math

import numpy as np
import pytest
import torch

from parity import cu_of, randn, say
from scree_amd import workloads
from scree_amd.kernels.hip import _ffi
from scree_amd.kernels.hip import attention as A

LIMIT = 1 << 21  # SCREE_ATTN_NOALLOC_SCHEDULE_BYTES


def _strides(*ts):
    return _ffi.int64_array([s for t in ts for s in (t.stride(0), t.stride(1))])


def _inputs(lengths, heads, kv_heads, dim, dtype, seed):
    n = sum(lengths)
    off, cu = cu_of(lengths)
    q = randn((n, heads, dim), dtype, seed)
    k = randn((n, kv_heads, dim), dtype, seed + 1)
    v = randn((n, kv_heads, dim), dtype, seed + 2)
    return cu, q, k, v


def _noalloc(cu, q, k, v, causal):
    lib = _ffi.lib()
    n, h, d = q.shape
    out = torch.empty_like(q)
    lse = torch.empty((n, h), dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _ffi.check(lib.scree_attn_fwd_noalloc(
            _ffi.ptr(q), _ffi.ptr(k), _ffi.ptr(v), _ffi.ptr(out), _ffi.ptr(lse), _ffi.ptr(cu),
            cu.numel() - 1, n, h, k.shape[1], d, _strides(q, k, v, out), 1.0 / math.sqrt(d),
            int(causal), _ffi.dtype_code(q.dtype), _ffi.stream_of(q)))
    return out, lse


def _with_workspace(cu, q, k, v, causal):
    lib = _ffi.lib()
    n, h, d = q.shape
    out = torch.empty_like(q)
    lse = torch.empty((n, h), dtype=torch.float32, device=q.device)
    ws = A.attention_schedule(cu, n, d, causal)
    with torch.cuda.device(q.device):
        _ffi.check(lib.scree_attn_fwd_gqa(
            _ffi.ptr(q), _ffi.ptr(k), _ffi.ptr(v), _ffi.ptr(out), _ffi.ptr(lse), _ffi.ptr(cu),
            cu.numel() - 1, n, h, k.shape[1], d, _strides(q, k, v, out), 1.0 / math.sqrt(d),
            int(causal), _ffi.dtype_code(q.dtype), _ffi.ptr(ws), ws.numel(), _ffi.stream_of(q)))
    return out, lse


def test_limit_is_rejected_before_any_launch():
    lib = _ffi.lib()
    null = ctypes.c_void_p(0)
    # 2^27 tokens need 2 * (2^20 + 1) * 16 + 16 bytes of schedule: over the limit
    rc = lib.scree_attn_fwd_noalloc(null, null, null, null, null, null, 1, 1 << 27, 1, 1, 64,
                                    null, 0.125, 1, _ffi.DTYPE_F16, null)
    assert rc == _ffi.SCREE_ERR_UNSUPPORTED
    assert "static scratch" in lib.scree_last_error().decode()
    assert lib.scree_attn_workspace_bytes(1, 1 << 27, 64) > LIMIT
    # the largest accepted problem fits exactly: two lists of tmax slots
    tmax = (LIMIT - 16) // 32
    assert lib.scree_attn_workspace_bytes(1, (tmax - 1) * 128, 64) <= LIMIT
    assert lib.scree_attn_workspace_bytes(1, tmax * 128, 64) > LIMIT


@pytest.mark.gpu
def test_two_calls_match_the_workspace_forward():
    big = workloads.config3().lengths        # 12160 tokens, 16 x 64, fp16, causal
    small = [300, 17, 129, 640, 1]           # smaller: a stale schedule would cover more work
    rng = np.random.default_rng(5)
    many = [int(x) for x in rng.integers(1, 200, size=100)]   # > 64 sequences: scheduled
    fewer = [int(x) for x in rng.integers(1, 120, size=70)]   # scheduled, smaller than `many`
    cases = [(big, 16, 16, 64, torch.float16, True),          # derives
             (many, 4, 4, 64, torch.float16, True),           # schedules into the static array
             (small, 8, 2, 128, torch.bfloat16, False),       # derives
             (fewer, 4, 2, 64, torch.bfloat16, False)]        # schedules again, smaller
    lib = _ffi.lib()
    first = None
    for i, (lengths, h, hk, d, dt, causal) in enumerate(cases):
        scheduled = bool(lib.scree_attn_needs_schedule(len(lengths), sum(lengths), h, d))
        assert scheduled == (len(lengths) > 64)
        say(f"case: noalloc call {i}: B={len(lengths)} N={sum(lengths)} H={h} Hkv={hk} D={d} "
            f"{dt} causal={causal} scheduled={scheduled}")
        cu, q, k, v = _inputs(lengths, h, hk, d, dt, 80 + i)
        got_o, got_l = _noalloc(cu, q, k, v, causal)
        torch.cuda.synchronize()
        want_o, want_l = _with_workspace(cu, q, k, v, causal)
        torch.cuda.synchronize()
        assert torch.equal(got_o, want_o), f"call {i}: output differs from the workspace forward"
        assert torch.equal(got_l, want_l), f"call {i}: LSE differs from the workspace forward"
        assert torch.isfinite(got_o).all() and torch.isfinite(got_l).all()
        if first is None:
            first = (cu, q, k, v, causal, got_o)
    # the first problem again after the smaller one: the array is rebuilt each call
    cu, q, k, v, causal, want = first
    again, _ = _noalloc(cu, q, k, v, causal)
    torch.cuda.synchronize()
    assert torch.equal(again, want)
