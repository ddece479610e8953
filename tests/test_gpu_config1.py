"""Config 1 on the HIP path, the reference's own CPU-runnable case, under parity.

Config 1 (``benchmarks/bench_throughput.py:113,122`` of the reference): 16
sequences with log-normal lengths (mean 128, sigma 0.6, clipped to [1, 512],
seed 0; 1,980 tokens), 4 heads of head_dim 32, causal and non-causal
attention; RMSNorm with gamma = 1 on the same packed tensor viewed as
(1980, 4, 32) and on a (1980, 128) tensor.  The reference runs attention in
fp32 on the CPU; its GPU launchers (and these) take fp16 / bf16, so attention
runs in both half types against the fp64 oracle on the same rounded inputs,
and in fp32 through the Array-level call (the fp32 kernels) with the 1e-5
bound.  RMSNorm runs in fp32 with the 1e-5 bound.

Also here: the reference's launcher names bound to the HIP launchers, a
schedule that fails on overlapping offsets (outputs NaN, never stale
memory), and the backward's ``delta_buffer`` checks.
"""

import numpy as np
import pytest
import torch

from oracle.norms import rmsnorm_bwd, rmsnorm_fwd
from parity import check_close, cu_of, np64, randn, say
from scree_amd import workloads
from test_gpu_attention import _run_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
def test_config1_attention_fwd_bwd(dtype, causal):
    lengths = workloads.config1_lengths()
    assert sum(lengths) == 1980 and len(lengths) == 16
    _run_case(lengths, 4, 32, dtype, causal, seed=1, backward=True)


@pytest.mark.parametrize("causal", [True, False])
def test_config1_fp32_attention_fwd_bwd(causal):
    """Config 1 as stated: fp32, through the Array-level call (the fp32
    kernels) with autograd, within the reference's fp32 bound of 1e-5."""
    from test_gpu_attention_fp32 import run_fp32_case

    lengths = workloads.config1_lengths()
    run_fp32_case(lengths, 4, 32, causal, seed=3)


def test_attention_rejects_other_dtypes():
    """fp64 (or mixed dtypes) raise TypeError at the Array level; the
    reference-named launchers keep their fp16 / bf16 assertion."""
    import scree_amd
    from scree_amd.kernels import varlen_attention
    from scree_amd.kernels.hip import varlen_attention_triton, varlen_attention_triton_autograd

    say("case: fp64 / mixed-dtype Array-level attention -> TypeError")
    lengths = [5, 9]
    _, cu = cu_of(lengths)
    x64 = scree_amd.Array(values=randn((14, 2, 32), torch.float64, 2), offsets=cu)
    with pytest.raises(TypeError, match="float32"):
        varlen_attention(x64, x64, x64, causal=True)
    x32 = scree_amd.Array(values=randn((14, 2, 32), torch.float32, 3), offsets=cu)
    x16 = scree_amd.Array(values=randn((14, 2, 32), torch.float16, 4), offsets=cu)
    with pytest.raises(TypeError, match="share a dtype"):
        varlen_attention(x32, x16, x16, causal=True)
    with pytest.raises(AssertionError, match="fp16 or bf16"):
        varlen_attention_triton(x32.values, x32.values, x32.values, cu)
    with pytest.raises(AssertionError, match="fp16 or bf16"):
        varlen_attention_triton_autograd(x32.values, x32.values, x32.values, cu)


@pytest.mark.parametrize("shape", [(1980, 4, 32), (1980, 128)])
def test_config1_rmsnorm_fp32_unit_gamma(shape):
    from scree_amd.kernels.hip import varlen_rmsnorm_hip

    say(f"case: config1 RMSNorm fp32 shape={shape} gamma=1")
    x = randn(shape, torch.float32, 5)
    gamma = torch.ones(shape[-1], device="cuda")
    dy = randn(shape, torch.float32, 6)
    xa = x.clone().requires_grad_(True)
    y = varlen_rmsnorm_hip(xa, gamma, eps=1e-6)
    y.backward(dy)
    torch.cuda.synchronize()
    flat = lambda t: np64(t).reshape(-1, shape[-1])  # noqa: E731
    ry, _ = rmsnorm_fwd(flat(x), np.ones(shape[-1]), eps=1e-6)
    rdx, _ = rmsnorm_bwd(flat(dy), flat(x), np.ones(shape[-1]), eps=1e-6)
    check_close("y", flat(y), ry, 1e-5)
    check_close("dx", flat(xa.grad), rdx, 1e-5)
    # without a weight the kernel normalises the same way
    y0 = varlen_rmsnorm_hip(x, None, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(y0, y.detach())


def test_reference_launcher_names_run_the_hip_kernels():
    """Every name of ``scree.kernels.triton`` (plus ``_backward``'s launcher)
    runs, with the reference's arguments, and returns what the HIP launcher
    of the same role returns, bit for bit."""
    from scree_amd.kernels import hip as H

    say("case: reference launcher names")
    lengths = [33, 1, 140]
    off, cu = cu_of(lengths)
    n = sum(lengths)
    q, k, v, do = (randn((n, 2, 64), torch.float16, 40 + s) for s in range(4))
    assert H.TRITON_AVAILABLE is True
    o_ref, lse_ref = H.varlen_attention_triton(q, k, v, cu, causal=True, block_m=64,
                                               block_n=64, return_lse=True)
    o_hip, lse_hip = H.varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    grads_ref = H.varlen_attention_triton_backward(do, q, k, v, o_ref, lse_ref, cu, causal=True,
                                                   block_m=64, block_n=64)
    grads_hip = H.varlen_attention_hip_backward(do, q, k, v, o_hip, lse_hip, cu, causal=True)
    qa = q.clone().requires_grad_(True)
    out = H.varlen_attention_triton_autograd(qa, k, v, cu, causal=True)
    out.backward(do)
    x = randn((n, 96), torch.bfloat16, 44)
    w = randn((96,), torch.bfloat16, 45, scale=0.02, mean=1.0)
    b = randn((96,), torch.bfloat16, 46, scale=0.02)
    y_rms = (H.varlen_rmsnorm_triton(x, w, eps=1e-6), H.varlen_rmsnorm_hip(x, w, eps=1e-6))
    y_ln = (H.varlen_layernorm_triton(x, w, b, eps=1e-5), H.varlen_layernorm_hip(x, w, b, eps=1e-5))
    torch.cuda.synchronize()
    assert torch.equal(o_ref, o_hip) and torch.equal(lse_ref, lse_hip)
    for a, c in zip(grads_ref, grads_hip):
        assert torch.equal(a, c)
    assert torch.equal(out.detach(), o_hip) and torch.equal(qa.grad, grads_hip[0])
    assert torch.equal(*y_rms) and torch.equal(*y_ln)


def test_failed_schedule_writes_nan_outputs():
    """Offsets that decrease ([0, 1000, 1, 1000]: sequences 0 and 2 overlap)
    describe 16 row blocks where the host bound allows 11.  The scheduler
    then publishes no work, and every attention kernel fills its outputs with
    NaN instead of leaving the (poisoned-on-purpose) buffers as they were."""
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    say("case: failed schedule -> NaN outputs")
    n = 1000
    cu = torch.tensor([0, 1000, 1, 1000], dtype=torch.int32, device="cuda")
    q, k, v, do = (randn((n, 2, 64), torch.float16, 60 + s) for s in range(4))
    out = torch.zeros_like(q)
    lse = torch.zeros((n, 2), dtype=torch.float32, device="cuda")
    varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True, out=out, lse_buffer=lse)
    delta = torch.zeros((n, 2), dtype=torch.float32, device="cuda")
    dq, dk, dv = varlen_attention_hip_backward(do, q, k, v, q, lse.nan_to_num(0.0), cu,
                                               causal=True, delta_buffer=delta)
    torch.cuda.synchronize()
    for name, t in (("out", out), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv),
                    ("delta", delta)):
        assert torch.isnan(t).all(), f"{name} was not filled with NaN"
    # the forward derives its items here and publishes the failure in the
    # header of its workspace, which the backward passes then read
    from scree_amd.kernels.hip import attention as A

    say("case: failed schedule published by the forward -> NaN gradients")
    ws = torch.full((A.workspace_bytes(3, n, 64),), 255, dtype=torch.uint8, device="cuda")
    out2, lse2 = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True, workspace=ws)
    dq2, dk2, dv2 = varlen_attention_hip_backward(do, q, k, v, q, lse2.nan_to_num(0.0), cu,
                                                  causal=True, workspace=ws)
    torch.cuda.synchronize()
    assert ws[:16].view(torch.int32).tolist() == [0, -1, 128, 1]
    for name, t in (("out", out2), ("lse", lse2), ("dq", dq2), ("dk", dk2), ("dv", dv2)):
        assert torch.isnan(t).all(), f"{name} was not filled with NaN"


def test_backward_rejects_a_wrong_delta_buffer():
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    say("case: delta_buffer checks")
    lengths = [20, 12]
    _, cu = cu_of(lengths)
    q, k, v, do = (randn((32, 2, 32), torch.float16, 70 + s) for s in range(4))
    o, lse = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    bad = [torch.empty((32, 2), dtype=torch.float16, device="cuda"),
           torch.empty((31, 2), dtype=torch.float32, device="cuda"),
           torch.empty((2, 32), dtype=torch.float32, device="cuda").t(),
           torch.empty((32, 2), dtype=torch.float32)]
    for buf in bad:
        with pytest.raises(AssertionError, match="delta_buffer"):
            varlen_attention_hip_backward(do, q, k, v, o, lse, cu, causal=True, delta_buffer=buf)
    torch.cuda.synchronize()
