"""The drop-in surface on the host: the reference's names and argument lists,
and the in-place view rule of the attention launchers (no GPU needed)."""

import inspect

import pytest
import torch

from scree_amd.kernels import hip as H
from scree_amd.kernels.hip import attention as A

# Parameter names, in order, of the reference's launchers:
# src/scree/kernels/triton/varlen_attention.py:165-176, _backward.py:288-299,
# _autograd.py:51, varlen_rmsnorm.py:49, varlen_layernorm.py:52.
REFERENCE_PARAMS = {
    "varlen_attention_triton": ["q", "k", "v", "cu_seqlens", "causal", "block_m", "block_n",
                                "return_lse", "out", "lse_buffer"],
    "varlen_attention_triton_backward": ["do", "q", "k", "v", "o", "lse", "cu_seqlens", "causal",
                                         "block_m", "block_n"],
    "varlen_attention_triton_autograd": ["q", "k", "v", "cu_seqlens", "causal"],
    "varlen_rmsnorm_triton": ["x", "weight", "eps"],
    "varlen_layernorm_triton": ["x", "weight", "bias", "eps"],
}
REFERENCE_DEFAULTS = {
    "varlen_attention_triton": {"causal": False, "block_m": 64, "block_n": 64,
                                "return_lse": False, "out": None, "lse_buffer": None},
    "varlen_attention_triton_backward": {"causal": False, "block_m": 64, "block_n": 64},
    "varlen_attention_triton_autograd": {"causal": False},
    "varlen_rmsnorm_triton": {"weight": None, "eps": 1e-6},
    "varlen_layernorm_triton": {"weight": None, "bias": None, "eps": 1e-5},
}


@pytest.mark.parametrize("name", sorted(REFERENCE_PARAMS))
def test_reference_names_keep_the_reference_arguments(name):
    fn = getattr(H, name)
    params = list(inspect.signature(fn).parameters.values())
    want = REFERENCE_PARAMS[name]
    # the reference's parameters come first, in order; extra keyword-only
    # extensions (workspace=, delta_buffer=) may follow with defaults
    assert [p.name for p in params[:len(want)]] == want
    for p in params[len(want):]:
        assert p.default is not inspect.Parameter.empty, f"{name}: extra parameter {p.name} needs a default"
    defaults = {p.name: p.default for p in params if p.default is not inspect.Parameter.empty}
    for arg, value in REFERENCE_DEFAULTS[name].items():
        assert defaults[arg] == value, f"{name}({arg}=) default {defaults[arg]!r} != {value!r}"


def test_reference_names_are_the_hip_launchers():
    assert H.varlen_attention_triton is H.varlen_attention_hip
    assert H.varlen_attention_triton_backward is H.varlen_attention_hip_backward
    assert H.varlen_attention_triton_autograd is H.varlen_attention_hip_autograd
    assert H.varlen_rmsnorm_triton is H.varlen_rmsnorm_hip
    assert H.varlen_layernorm_triton is H.varlen_layernorm_hip
    assert H.TRITON_AVAILABLE is H.HIP_AVAILABLE
    for name in REFERENCE_PARAMS:
        assert name in H.__all__


@pytest.mark.parametrize("shape,strides,in_place", [
    ((4, 2, 64), (128, 64, 1), True),             # contiguous
    ((4, 2, 64), (3 * 128, 64, 1), True),         # qkv[:, i] view of a packed qkv
    ((4, 2, 64), (1 << 24, 64, 1), False),        # row stride at the 2^24 limit
    ((4, 2, 64), (128, 1 << 24, 1), False),       # head stride at the limit
    ((4, 2, 64), (132, 64, 1), False),            # row stride not a multiple of 8
    ((4, 2, 64), (64, 256, 1), True),             # head-major layout (rows do not overlap)
    ((4, 2, 64), (32, 64, 1), False),             # rows overlap
    ((4, 2, 64), (2, 1, 8), False),               # head_dim not contiguous
])
def test_kernel_view_copies_exactly_what_the_library_rejects(shape, strides, in_place):
    t = torch.empty_strided(shape, strides, dtype=torch.float16, device="meta")
    v = A._kernel_view(t)
    assert (v is t) == in_place
    if not in_place:
        assert v.is_contiguous() and v.shape == t.shape
