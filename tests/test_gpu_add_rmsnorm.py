"""GPU parity of the fused residual add + RMSNorm against the oracle and the unfused path.

``h = x + r`` must equal torch's own ``x + r`` bit for bit, and ``y`` must
equal ``varlen_rmsnorm_hip(h)`` bit for bit (same arithmetic on the same
rounded row); both are also checked against the fp64 oracle with the norm
tolerances (1e-5 fp32, 1e-3 half, plus the output's rounding ``u * |ref|``).
"""

import numpy as np
import pytest
import torch

from oracle.norms import add_rmsnorm_bwd, add_rmsnorm_fwd
from parity import UNIT, check_close, np64, randn, say
from scree_amd import workloads

pytestmark = pytest.mark.gpu

ATOL = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 1e-3}
STORAGE = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}
SHAPES = [(257, 4096), (300, 128), (33, 100), (9, 4100), (5, 8192), (17, 1)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("with_w,with_dh", [(True, True), (True, False), (False, True)])
def test_add_rmsnorm_fwd_bwd(dtype, shape, with_w, with_dh):
    from scree_amd.kernels.hip import varlen_add_rmsnorm_hip_backward, varlen_rmsnorm_hip
    from scree_amd.kernels.hip.norms import add_rmsnorm_fwd as hip_fwd

    rows, dim = shape
    say(f"case: add_rmsnorm {dtype} rows={rows} dim={dim} weight={with_w} dh={with_dh}")
    x = randn((rows, dim), dtype, dim)
    r = randn((rows, dim), dtype, dim + 1, scale=0.5)
    w = randn((dim,), dtype, dim + 2, scale=0.02, mean=1.0) if with_w else None
    dy = randn((rows, dim), dtype, dim + 3)
    dh = randn((rows, dim), dtype, dim + 4) if with_dh else None
    h, y, rstd = hip_fwd(x, r, w, 1e-6, want_stats=True)
    torch.cuda.synchronize()
    assert torch.equal(h, x + r), "h differs from torch's x + r"
    assert torch.equal(y, varlen_rmsnorm_hip(h, w, eps=1e-6)), "y differs from the unfused RMSNorm"
    rh, ry, rr = add_rmsnorm_fwd(np64(x), np64(r), np64(w) if with_w else None, eps=1e-6,
                                 storage=STORAGE[dtype])
    np.testing.assert_array_equal(np64(h), rh)
    u = UNIT[dtype]
    check_close("y", np64(y), ry, ATOL[dtype], extra=np.abs(ry), unit=u)
    check_close("rstd", rstd.cpu().numpy().astype(np.float64), rr, 1e-5 * np.abs(rr).max())
    dx, dw = varlen_add_rmsnorm_hip_backward(dy, dh, h, w, eps=1e-6, rstd=rstd)
    torch.cuda.synchronize()
    rdx, rdw = add_rmsnorm_bwd(np64(dy), np64(dh) if with_dh else None, rh,
                               np64(w) if with_w else None, eps=1e-6)
    check_close("dx", np64(dx), rdx, ATOL[dtype], extra=np.abs(rdx), unit=u)
    if with_w:  # dw is stored in the weight's dtype: its own rounding is part of the bound
        check_close("dw", np64(dw), rdw, 1e-3 + 1e-4 * np.abs(rdw).max(), extra=np.abs(rdw), unit=u)


def test_add_rmsnorm_without_dh_equals_rmsnorm_backward():
    from scree_amd.kernels.hip import (varlen_add_rmsnorm_hip, varlen_add_rmsnorm_hip_backward,
                                       varlen_rmsnorm_hip_backward)

    say("case: add_rmsnorm bwd without dh == rmsnorm bwd, bf16 1000x4096")
    x = randn((1000, 4096), torch.bfloat16, 1)
    r = randn((1000, 4096), torch.bfloat16, 2)
    w = randn((4096,), torch.bfloat16, 3, scale=0.02, mean=1.0)
    dy = randn((1000, 4096), torch.bfloat16, 4)
    h, _ = varlen_add_rmsnorm_hip(x, r, w)
    a, aw = varlen_add_rmsnorm_hip_backward(dy, None, h, w)
    b, bw = varlen_rmsnorm_hip_backward(dy, h, w)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(aw, bw)


def test_add_rmsnorm_autograd_gives_both_inputs_the_gradient():
    from scree_amd.kernels.hip import varlen_add_rmsnorm_hip

    say("case: add_rmsnorm autograd fp16 300x512")
    x = randn((300, 512), torch.float16, 11).requires_grad_(True)
    r = randn((300, 512), torch.float16, 12).requires_grad_(True)
    w = randn((512,), torch.float32, 13, scale=0.02, mean=1.0).requires_grad_(True)
    gh = randn((300, 512), torch.float16, 14)
    gy = randn((300, 512), torch.float16, 15)
    h, y = varlen_add_rmsnorm_hip(x, r, w, eps=1e-6)
    (h.float() * gh.float()).sum().add((y.float() * gy.float()).sum()).backward()
    torch.cuda.synchronize()
    rh, _, _ = add_rmsnorm_fwd(np64(x), np64(r), np64(w.to(torch.float16)), storage="float16")
    rdx, rdw = add_rmsnorm_bwd(np64(gy), np64(gh), rh, np64(w.to(torch.float16)))
    u = UNIT[torch.float16]
    check_close("dx", np64(x.grad), rdx, 1e-3, extra=np.abs(rdx), unit=u)
    assert torch.equal(x.grad, r.grad)
    assert w.grad.dtype == torch.float32
    check_close("dw", np64(w.grad), rdw, 1e-3 + 1e-4 * np.abs(rdw).max())


def test_add_rmsnorm_array_api_config2_shape():
    """Config-2 shape (bf16, 64 sequences, hidden 4096) through the Array API."""
    from scree_amd import Array
    from scree_amd.kernels import varlen_add_rmsnorm, varlen_rmsnorm

    c = workloads.config2()
    say(f"case: add_rmsnorm Array API config2 N={c.total} hidden={c.hidden}")
    off = np.zeros(len(c.lengths) + 1, dtype=np.int32)
    off[1:] = np.cumsum(c.lengths)
    offsets = torch.from_numpy(off).cuda()
    x = Array(values=randn((c.total, c.hidden), torch.bfloat16, 21), offsets=offsets)
    r = randn((c.total, c.hidden), torch.bfloat16, 22)
    w = randn((c.hidden,), torch.bfloat16, 23, scale=0.02, mean=1.0)
    h, y = varlen_add_rmsnorm(x, r, w, eps=1e-6)
    torch.cuda.synchronize()
    assert h.offsets is offsets and y.offsets is offsets
    assert torch.equal(h.values, x.values + r)
    assert torch.equal(y.values, varlen_rmsnorm(h, w, eps=1e-6).values)
    with pytest.raises(ValueError):
        bad = Array(values=r, offsets=torch.from_numpy(np.array([0, c.total], dtype=np.int32)).cuda())
        varlen_add_rmsnorm(x, bad, w)
