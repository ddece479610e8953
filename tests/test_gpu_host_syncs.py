"""The user-facing calls make no host synchronisation.

The reference reads ``max(seq_lens)`` with ``.item()`` before every launch
(``triton/varlen_attention.py:220-221``, ``_backward.py:320-321``) and its
``from_padded`` reads each mask row's length (``_core.py:263``).  Here the
Array-level kernels, the autograd backward and the packed <-> padded
launchers (given the sizes they cannot know on the host: ``max_len`` /
``total``) run under ``torch.cuda.set_sync_debug_mode("error")``, which
raises on any call that waits for the device.  Inputs are built, and results
checked, outside that region.
"""

import numpy as np
import pytest
import torch

import scree_amd
from oracle.attention import attention_fwd
from parity import check_close, cu_of, np64, randn, say

pytestmark = pytest.mark.gpu


@pytest.fixture
def no_sync():
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        yield
    finally:
        torch.cuda.set_sync_debug_mode("default")


def test_array_level_calls_make_no_host_sync(no_sync):
    from scree_amd.kernels import (varlen_attention, varlen_layernorm, varlen_rmsnorm,
                                   varlen_softmax)

    torch.cuda.set_sync_debug_mode("default")
    say("case: Array-level attention fwd+bwd, norms, softmax under sync debug mode")
    lengths = [5, 300, 129, 1]
    n = sum(lengths)
    off, cu = cu_of(lengths)
    qv, kv, vv, do = (randn((n, 4, 64), torch.float16, 30 + s) for s in range(4))
    qv.requires_grad_(True)
    q = scree_amd.Array(values=qv, offsets=cu)
    k = scree_amd.Array(values=kv, offsets=cu)
    v = scree_amd.Array(values=vv, offsets=cu)
    x = scree_amd.Array(values=randn((n, 256), torch.bfloat16, 40), offsets=cu)
    w = randn((256,), torch.bfloat16, 41, scale=0.02, mean=1.0)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    out = varlen_attention(q, k, v, causal=True)
    out.values.backward(do)
    y = varlen_rmsnorm(x, w)
    z = varlen_layernorm(x, w)
    s = varlen_softmax(x)
    torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert out.offsets is cu and y.offsets is cu and z.offsets is cu and s.offsets is cu
    ref, _ = attention_fwd(np64(qv), np64(kv), np64(vv), off, causal=True)
    check_close("O", np64(out.values), ref, 2e-3)
    assert qv.grad is not None and bool(torch.isfinite(qv.grad).all())


def test_padding_launchers_make_no_host_sync_given_sizes(no_sync):
    from scree_amd.kernels.hip.padding import from_padded_hip, to_padded_hip

    torch.cuda.set_sync_debug_mode("default")
    say("case: to_padded(max_len=) / from_padded(total=) under sync debug mode")
    lengths = [7, 0, 33, 2]
    n = sum(lengths)
    _, cu = cu_of(lengths)
    vals = randn((n, 3, 8), torch.float16, 50)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    padded, mask = to_padded_hip(vals, cu, max_len=max(lengths))
    back, off2 = from_padded_hip(padded, mask, total=n)
    torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert torch.equal(off2, cu)
    assert torch.equal(back, vals)


@pytest.mark.parametrize("batch", [3, 100, 2100])
def test_decreasing_offsets_fail_every_scheduler(batch):
    """Offsets that decrease somewhere but describe no more work than the host
    bound (so only an explicit check can catch them) make every scheduler --
    the wave scheduler and the forward's own derivation (up to 64
    sequences), the sorting scheduler (up to 2048), the natural-order one
    (more) -- publish a failed schedule, and every output and gradient NaN:
    the device-side check that lets the Array-level call skip a host read."""
    from scree_amd.kernels.hip import attention as A
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    n = 1000
    rng = np.random.default_rng(batch)
    off = np.sort(rng.integers(0, n + 1, size=batch + 1)).astype(np.int32)
    off[0], off[-1] = 0, n
    j = 1 + int(np.argmax(np.diff(off)[1:-1]))  # the longest inner sequence ...
    off[j + 1] = off[j] - 1  # ... ends before it starts: sequence j + 1 overlaps it
    assert off[j] > 0 and (np.diff(off) < 0).sum() == 1 and off[-1] == n
    nblk = np.maximum(np.diff(off), 0)
    assert int(((nblk + 127) // 128).sum()) <= (n + 127) // 128 + batch  # within the bound
    say(f"case: decreasing offsets B={batch} N={n}")
    cu = torch.from_numpy(off).cuda()
    ws = A.attention_schedule(cu, n, 64, True)
    assert ws[:16].view(torch.int32).tolist() == [0, -1, 128, 1]
    q, k, v, do = (randn((n, 2, 64), torch.float16, 90 + s) for s in range(4))
    out, lse = varlen_attention_hip(q, k, v, cu, causal=True, return_lse=True)
    dq, dk, dv = varlen_attention_hip_backward(do, q, k, v, q, lse.nan_to_num(0.0), cu, causal=True)
    torch.cuda.synchronize()
    for name, t in (("out", out), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.isnan(t).all(), f"{name} was not filled with NaN"
