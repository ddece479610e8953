"""The C-ABI library: it loads, exports every function ``include/scree_hip.h``
declares, and rejects bad arguments on the host (no GPU needed: every call here
fails validation before anything is launched)."""

import ctypes
import re
from pathlib import Path

import pytest

from scree_amd.kernels.hip import _ffi

HEADER = Path(__file__).resolve().parents[1] / "include" / "scree_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(scree_[a-z0-9_]+)\s*\(", text)))


def test_library_loads():
    assert _ffi.HIP_AVAILABLE, f"library failed to load from {_ffi.library_path()}"
    assert _ffi.lib().scree_abi_version() == 1


def test_exports_every_declared_symbol():
    declared = _declared()
    assert declared, "no declarations parsed from the header"
    raw = ctypes.CDLL(str(_ffi.library_path()))
    for name in declared:
        assert hasattr(raw, name), f"{name} declared in scree_hip.h but not exported"
    assert sorted(_ffi.EXPORTED) == declared


def _err():
    return _ffi.lib().scree_last_error().decode()


def test_attention_validation_errors():
    lib = _ffi.lib()
    ws = ctypes.create_string_buffer(1 << 16)
    p = ctypes.c_void_p(ctypes.addressof(ws))
    strides = _ffi.int64_array([16 * 64, 64] * 8)
    null = ctypes.c_void_p(0)
    # null cu_seqlens
    rc = lib.scree_attn_fwd(p, p, p, p, p, null, 2, 10, 16, 64, strides, 0.125, 1, 1, p, 1 << 16, null)
    assert rc == _ffi.SCREE_ERR_INVALID and "cu_seqlens" in _err()
    # unsupported head_dim: powers of two from 16 to 256 only
    for bad_dim in (8, 48, 512):
        rc = lib.scree_attn_fwd(p, p, p, p, p, p, 2, 10, 16, bad_dim, strides, 0.125, 1, 1, p,
                                1 << 16, null)
        assert rc == _ffi.SCREE_ERR_UNSUPPORTED and "head_dim" in _err()
    # dtype codes other than fp32 / fp16 / bf16
    rc = lib.scree_attn_fwd(p, p, p, p, p, p, 2, 10, 16, 64, strides, 0.125, 1, 7, p, 1 << 16, null)
    assert rc == _ffi.SCREE_ERR_UNSUPPORTED and "dtype" in _err()
    # workspace too small
    rc = lib.scree_attn_fwd(p, p, p, p, p, p, 2, 10, 16, 64, strides, 0.125, 1, 1, p, 8, null)
    assert rc == _ffi.SCREE_ERR_WORKSPACE
    # stride not a multiple of 8 elements
    bad = _ffi.int64_array([16 * 64 + 4, 64] * 8)
    rc = lib.scree_attn_fwd(p, p, p, p, p, p, 2, 10, 16, 64, bad, 0.125, 1, 1, p, 1 << 16, null)
    assert rc == _ffi.SCREE_ERR_INVALID and "strides" in _err()
    # batch out of range
    rc = lib.scree_attn_schedule(p, 0, 10, 64, 1, p, 1 << 16, null)
    assert rc == _ffi.SCREE_ERR_UNSUPPORTED
    rc = lib.scree_attn_bwd(p, p, p, p, p, p, p, p, p, null, p, 2, 10, 16, 64, strides, 0.125, 1, 1,
                            p, 1 << 16, null)
    assert rc == _ffi.SCREE_ERR_INVALID and "delta" in _err()


def test_attention_without_tokens_needs_no_tensors():
    """No tokens (every sequence empty): empty tensors may have no storage,
    so null tensor pointers are accepted and nothing is launched."""
    lib = _ffi.lib()
    ws = ctypes.create_string_buffer(1 << 16)
    p = ctypes.c_void_p(ctypes.addressof(ws))
    null = ctypes.c_void_p(0)
    strides = _ffi.int64_array([16 * 64, 64] * 8)
    rc = lib.scree_attn_fwd(null, null, null, null, null, p, 3, 0, 16, 64, strides, 0.125, 1, 1, p,
                            1 << 16, null)
    assert rc == _ffi.SCREE_OK, _err()
    rc = lib.scree_attn_bwd(null, null, null, null, null, null, null, null, null, null, p, 3, 0, 16,
                            64, strides, 0.125, 1, 1, p, 1 << 16, null)
    assert rc == _ffi.SCREE_OK, _err()
    # with tokens the same nulls are rejected
    rc = lib.scree_attn_fwd(null, null, null, null, null, p, 3, 5, 16, 64, strides, 0.125, 1, 1, p,
                            1 << 16, null)
    assert rc == _ffi.SCREE_ERR_INVALID


def test_workspace_sizes():
    lib = _ffi.lib()
    # header + two lists of (ceil(N/128) + B) int4 items
    assert lib.scree_attn_workspace_bytes(16, 12160, 64) == 16 + 2 * 16 * (95 + 16)
    assert lib.scree_attn_workspace_bytes(0, 10, 64) == 0
    # a forward over at most 64 sequences (one wavefront) in a launch of at
    # most 2048 workgroups (1024 at head_dim 128), (ceil(N/128) + B) * heads,
    # derives its items and writes the lists itself: no schedule needed
    assert lib.scree_attn_needs_schedule(16, 1980, 4, 32) == 0      # config 1: 32 x 4
    assert lib.scree_attn_needs_schedule(16, 12160, 16, 64) == 0    # config 4: 111 x 16
    assert lib.scree_attn_needs_schedule(32, 83977, 32, 128) == 1   # config 5: 689 x 32
    assert lib.scree_attn_needs_schedule(16, 12160, 18, 64) == 0    # 111 x 18 = 1998
    assert lib.scree_attn_needs_schedule(16, 12160, 19, 64) == 1    # 2109
    assert lib.scree_attn_needs_schedule(16, 12160, 9, 128) == 0    # 999
    assert lib.scree_attn_needs_schedule(16, 12160, 10, 128) == 1   # 1110
    assert lib.scree_attn_needs_schedule(16, 12160, 4, 256) == 0    # 444: 512 at head_dim 256
    assert lib.scree_attn_needs_schedule(16, 12160, 5, 256) == 1    # 555
    assert lib.scree_attn_needs_schedule(16, 12160, 18, 16) == 0    # head_dim 16 runs as 32
    assert lib.scree_attn_needs_schedule(64, 1024, 1, 64) == 0
    assert lib.scree_attn_needs_schedule(65, 1024, 1, 64) == 1      # past one wavefront of sequences
    assert lib.scree_attn_needs_schedule(0, 10, 4, 64) == 1         # invalid: the call will say why
    # past 2048 sequences the (natural-order) scheduler keeps batch + 1
    # prefix sums after the lists, rounded up to 16 bytes
    lists = 16 + 2 * 16 * (24 + 3000)
    assert lib.scree_attn_workspace_bytes(3000, 3000, 64) == lists + 12004 + 12
    assert lib.scree_norm_bwd_workspace_bytes(19758, 4096) == 512 * 2 * 4096 * 4
    assert lib.scree_norm_bwd_workspace_bytes(10, 100) == 2 * 2 * 100 * 4


def test_grouped_query_backward_workspace_sizes():
    lib = _ffi.lib()
    base = lib.scree_attn_workspace_bytes(16, 12160, 64)
    # equal heads: nothing beyond the schedule
    assert lib.scree_attn_bwd_workspace_bytes_gqa(16, 12160, 16, 16, 64) == base
    # 111 items x 4 K/V heads = 444 workgroups < 1536: ceil(1536 / 444) = 4 parts,
    # a divisor of the group of 4; after the (256-aligned) schedule, fp32 dK and
    # dV of 128 keys per part
    tmax, kv, parts = 95 + 16, 4, 4
    align = lambda n: (n + 255) // 256 * 256  # noqa: E731
    part = 2 * 128 * 64 * 4
    want = align(base) + tmax * kv * parts * part
    assert lib.scree_attn_bwd_workspace_bytes_gqa(16, 12160, 16, 4, 64) == want
    # 2 K/V heads: ceil(1536 / 222) = 7 -> 8, the next divisor of the group of 8
    assert lib.scree_attn_bwd_workspace_bytes_gqa(16, 12160, 16, 2, 64) == align(base) + tmax * 2 * 8 * part
    # 4 K/V heads of 32 query heads: ceil(1536 / 444) = 4, a divisor of 8
    assert lib.scree_attn_bwd_workspace_bytes_gqa(16, 12160, 32, 4, 64) == align(base) + tmax * 4 * 4 * part
    # 3 K/V heads of 18: ceil(1536 / 333) = 5 -> 6, the next divisor of the group of 6
    assert lib.scree_attn_bwd_workspace_bytes_gqa(16, 12160, 18, 3, 64) == align(base) + tmax * 3 * 6 * part
    # a grid that already fills the GPU: no split
    big = lib.scree_attn_workspace_bytes(32, 83977, 128)
    assert lib.scree_attn_bwd_workspace_bytes_gqa(32, 83977, 32, 8, 128) == big
    # heads that do not group fall back to the schedule's size
    assert lib.scree_attn_bwd_workspace_bytes_gqa(16, 12160, 16, 3, 64) == base


def test_norm_validation_errors():
    lib = _ffi.lib()
    null = ctypes.c_void_p(0)
    buf = ctypes.create_string_buffer(256)
    p = ctypes.c_void_p(ctypes.addressof(buf))
    assert lib.scree_rmsnorm_fwd(null, null, null, null, 4, 8, 1e-6, 1, null) == _ffi.SCREE_ERR_INVALID
    assert lib.scree_rmsnorm_fwd(p, null, p, null, 4, 0, 1e-6, 1, null) == _ffi.SCREE_ERR_INVALID
    assert "dim" in _err()
    assert lib.scree_layernorm_fwd(p, null, null, p, null, null, 4, 8, 1e-6, 7, null) == _ffi.SCREE_ERR_UNSUPPORTED
    # nothing to do for zero rows
    assert lib.scree_rmsnorm_fwd(null, null, null, null, 0, 8, 1e-6, 1, null) == _ffi.SCREE_OK
    # dweight without weight
    rc = lib.scree_rmsnorm_bwd(p, p, null, p, p, p, 0, 4, 8, 1, p, 256, null)
    assert rc == _ffi.SCREE_ERR_INVALID and "dweight" in _err()
    # workspace too small for the parameter gradient
    rc = lib.scree_layernorm_bwd(p, p, p, p, p, p, p, null, 0, 4, 8, 1, p, 4, null)
    assert rc == _ffi.SCREE_ERR_WORKSPACE


def test_python_errors_map_codes():
    with pytest.raises(ValueError):
        _ffi.check(_ffi.lib().scree_rmsnorm_fwd(None, None, None, None, 4, 8, 1e-6, 1, None))
    with pytest.raises(NotImplementedError):
        _ffi.check(_ffi.lib().scree_rmsnorm_fwd(None, None, None, None, 4, 8, 1e-6, 9, None))


def test_cpu_tensors_are_rejected_by_the_hip_path():
    import numpy as np
    import torch

    import scree_amd as scree
    from scree_amd.kernels import varlen_attention, varlen_rmsnorm
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_rmsnorm_hip

    x = torch.zeros(4, 2, 32, dtype=torch.float16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(AssertionError, match="ROCm"):
        varlen_attention_hip(x, x, x, cu)
    with pytest.raises(AssertionError, match="ROCm"):
        varlen_rmsnorm_hip(torch.zeros(4, 8))
    arr = scree.pack([np.zeros((3, 8), dtype=np.float32)])
    with pytest.raises(TypeError, match="ROCm"):
        varlen_rmsnorm(arr)
    with pytest.raises(TypeError, match="ROCm"):
        varlen_attention(arr, arr, arr)


def test_host_call_helpers():
    """The argument helpers hand the C ABI plain integers and cached array types."""
    import torch

    assert _ffi.ptr(None) == 0
    t = torch.zeros(4)
    assert _ffi.ptr(t) == t.data_ptr()
    a = _ffi.int64_array((3, -1, 2 ** 40))
    b = _ffi.int64_array((7, 8, 9))
    assert type(a) is type(b) and list(a) == [3, -1, 2 ** 40]
    assert list(_ffi.int64_array(t.stride()[:1] + (5,))) == [1, 5]
    # no device switch is entered for a tensor without a device index
    with _ffi.device_guard(torch.device("cpu")):
        pass


def test_size_queries_are_cached():
    from scree_amd.kernels.hip import attention as A

    A.workspace_bytes.cache_clear()
    assert A.workspace_bytes(16, 12160, 64) == A.workspace_bytes(16, 12160, 64)
    assert A.workspace_bytes.cache_info().hits >= 1
    assert A.needs_schedule(16, 12160, 16, 64) is False
    assert A.needs_schedule(65, 1024, 1, 64) is True
