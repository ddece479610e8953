"""GPU parity of the HIP RMSNorm / LayerNorm kernels against the oracle.

Inputs and parameters are rounded to the kernel dtype first (the reference
rounds weight/bias to x's dtype, ``triton/varlen_rmsnorm.py:79``); the oracle
runs in fp64 on those values.  Output bound: 1e-5 (fp32) or 1e-3 (half)
plus the output's own rounding, ``u * |ref|``.
"""

import numpy as np
import pytest
import torch

from oracle.norms import layernorm_bwd, layernorm_fwd, rmsnorm_bwd, rmsnorm_fwd
from parity import UNIT, check_close, np64, randn, say
from scree_amd import workloads

pytestmark = pytest.mark.gpu

ATOL = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 1e-3}

# (rows, dim): fast path, odd dims (generic path), tiny rows
SHAPES = [(257, 4096), (300, 128), (64, 8), (33, 100), (9, 4100), (5, 8192), (17, 1)]


def _inputs(rows, dim, dtype, seed):
    x = randn((rows, dim), dtype, seed)
    w = randn((dim,), dtype, seed + 1, scale=0.02, mean=1.0)
    b = randn((dim,), dtype, seed + 2, scale=0.02)
    dy = randn((rows, dim), dtype, seed + 3)
    return x, w, b, dy


def _fast_ok(dim, dtype):
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    return dim % vec == 0 and dim // vec <= 16 * 64


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("with_w", [True, False])
def test_rmsnorm_fwd_bwd(dtype, shape, with_w):
    from scree_amd.kernels.hip.norms import rmsnorm_bwd as hip_bwd, rmsnorm_fwd as hip_fwd

    rows, dim = shape
    say(f"case: rmsnorm {dtype} rows={rows} dim={dim} weight={with_w} fast={_fast_ok(dim, dtype)}")
    x, w, _, dy = _inputs(rows, dim, dtype, seed=dim)
    wk = w if with_w else None
    y, rstd = hip_fwd(x, wk, 1e-6, want_stats=True)
    torch.cuda.synchronize()
    ry, rr = rmsnorm_fwd(np64(x), np64(w) if with_w else None, eps=1e-6)
    u = UNIT[dtype]
    check_close("y", np64(y), ry, ATOL[dtype], extra=np.abs(ry), unit=u)
    check_close("rstd", rstd.cpu().numpy().astype(np.float64), rr, 1e-5 * np.abs(rr).max())
    dx, dw = hip_bwd(dy, x, wk, rstd, with_w, dw_like=torch.empty(1, dtype=torch.float32) if with_w else None)
    torch.cuda.synchronize()
    rdx, rdw = rmsnorm_bwd(np64(dy), np64(x), np64(w) if with_w else None, eps=1e-6)
    check_close("dx", np64(dx), rdx, ATOL[dtype], extra=np.abs(rdx), unit=u)
    if with_w:
        check_close("dw", np64(dw), rdw, 1e-3 + 1e-4 * np.abs(rdw).max())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("params", ["wb", "w", "b", "none"])
def test_layernorm_fwd_bwd(dtype, shape, params):
    from scree_amd.kernels.hip.norms import layernorm_bwd as hip_bwd, layernorm_fwd as hip_fwd

    rows, dim = shape
    say(f"case: layernorm {dtype} rows={rows} dim={dim} params={params} fast={_fast_ok(dim, dtype)}")
    x, w, b, dy = _inputs(rows, dim, dtype, seed=dim + 7)
    wk = w if "w" in params else None
    bk = b if "b" in params else None
    y, mean, rstd = hip_fwd(x, wk, bk, 1e-6, want_stats=True)
    torch.cuda.synchronize()
    ry, rm, rr = layernorm_fwd(np64(x), np64(w) if wk is not None else None,
                               np64(b) if bk is not None else None, eps=1e-6)
    u = UNIT[dtype]
    check_close("y", np64(y), ry, ATOL[dtype], extra=np.abs(ry), unit=u)
    check_close("mean", mean.cpu().numpy().astype(np.float64), rm, 1e-6)
    check_close("rstd", rstd.cpu().numpy().astype(np.float64), rr, 1e-5 * np.abs(rr).max())
    like = torch.empty(1, dtype=torch.float32)
    dx, dw, db = hip_bwd(dy, x, wk, mean, rstd, wk is not None, bk is not None, p_like=like)
    torch.cuda.synchronize()
    rdx, rdw, rdb = layernorm_bwd(np64(dy), np64(x), np64(w) if wk is not None else None, eps=1e-6,
                                  has_bias=bk is not None)
    check_close("dx", np64(dx), rdx, ATOL[dtype], extra=np.abs(rdx), unit=u)
    if wk is not None:
        check_close("dw", np64(dw), rdw, 1e-3 + 1e-4 * np.abs(rdw).max())
    if bk is not None:
        check_close("db", np64(db), rdb, 1e-3 + 1e-4 * np.abs(rdb).max())


def test_config2_bf16_full_size():
    """Config 2 at its full size: N=19758 x 4096 bf16, both norms, fwd + bwd."""
    from scree_amd.kernels.hip.norms import (layernorm_bwd as ln_b, layernorm_fwd as ln_f,
                                             rmsnorm_bwd as rms_b, rmsnorm_fwd as rms_f)

    c = workloads.config2()
    say(f"case: config2 rows={c.total} dim={c.hidden} bf16")
    x, w, b, dy = _inputs(c.total, c.hidden, torch.bfloat16, seed=2)
    u = UNIT[torch.bfloat16]
    x64, w64, b64, dy64 = np64(x), np64(w), np64(b), np64(dy)
    y, rstd = rms_f(x, w, c.eps, want_stats=True)
    dx, dw = rms_b(dy, x, w, rstd, True, dw_like=w)
    torch.cuda.synchronize()
    ry, _ = rmsnorm_fwd(x64, w64, eps=c.eps)
    check_close("rms y", np64(y), ry, 1e-3, extra=np.abs(ry), unit=u)
    rdx, rdw = rmsnorm_bwd(dy64, x64, w64, eps=c.eps)
    check_close("rms dx", np64(dx), rdx, 1e-3, extra=np.abs(rdx), unit=u)
    check_close("rms dw (bf16)", np64(dw), rdw, 1e-3 + 1e-4 * np.abs(rdw).max(), extra=np.abs(rdw), unit=u)
    y, mean, rstd = ln_f(x, w, b, c.eps, want_stats=True)
    dx, dw, db = ln_b(dy, x, w, mean, rstd, True, True, p_like=w)
    torch.cuda.synchronize()
    ry, _, _ = layernorm_fwd(x64, w64, b64, eps=c.eps)
    check_close("ln y", np64(y), ry, 1e-3, extra=np.abs(ry), unit=u)
    rdx, rdw, rdb = layernorm_bwd(dy64, x64, w64, eps=c.eps, has_bias=True)
    check_close("ln dx", np64(dx), rdx, 1e-3, extra=np.abs(rdx), unit=u)
    check_close("ln dw (bf16)", np64(dw), rdw, 1e-3 + 1e-4 * np.abs(rdw).max(), extra=np.abs(rdw), unit=u)
    check_close("ln db (bf16)", np64(db), rdb, 1e-3 + 1e-4 * np.abs(rdb).max(), extra=np.abs(rdb), unit=u)


def test_unaligned_input_takes_generic_path():
    from scree_amd.kernels.hip import _ffi

    say("case: unaligned x (generic path)")
    rows, dim = 40, 256
    buf = randn((rows * dim + 3,), torch.float16, 9)
    x = buf[3:].view(rows, dim)
    assert x.data_ptr() % 16 != 0
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device="cuda")
    _ffi.check(_ffi.lib().scree_rmsnorm_fwd(_ffi.ptr(x), None, _ffi.ptr(y), _ffi.ptr(rstd), rows, dim,
                                            1e-6, _ffi.DTYPE_F16, _ffi.stream_of(x)))
    torch.cuda.synchronize()
    ry, _ = rmsnorm_fwd(np64(x), None, eps=1e-6)
    check_close("y", np64(y), ry, 1e-3, extra=np.abs(ry), unit=UNIT[torch.float16])


def test_autograd_and_array_api():
    import scree_amd as scree
    from scree_amd.kernels import varlen_layernorm, varlen_rmsnorm
    from scree_amd.kernels.hip import varlen_layernorm_hip, varlen_rmsnorm_hip

    say("case: norm autograd + Array API")
    x = randn((50, 3, 64), torch.bfloat16, 1).requires_grad_(True)
    w = torch.ones(64, device="cuda", dtype=torch.float32).requires_grad_(True)
    b = torch.zeros(64, device="cuda", dtype=torch.float32).requires_grad_(True)
    dy = randn((50, 3, 64), torch.bfloat16, 2)
    y = varlen_rmsnorm_hip(x, w, eps=1e-6)
    y.backward(dy)
    assert y.shape == x.shape and y.dtype == x.dtype
    assert x.grad.shape == x.shape and w.grad.dtype == torch.float32
    rdx, rdw = rmsnorm_bwd(np64(dy), np64(x), np64(w.detach()), eps=1e-6)
    check_close("dx", np64(x.grad), rdx, 1e-3, extra=np.abs(rdx), unit=UNIT[torch.bfloat16])
    check_close("dw", np64(w.grad), rdw, 1e-3 + 1e-4 * np.abs(rdw).max())
    x.grad = None
    y = varlen_layernorm_hip(x, w, b, eps=1e-5)
    y.backward(dy)
    assert b.grad is not None and torch.isfinite(b.grad).all()
    arr = scree.pack([randn((n, 32), torch.float16, n) for n in (3, 1, 9)])
    out = varlen_rmsnorm(arr)
    assert out.offsets is arr.offsets and out.values.shape == arr.values.shape
    out = varlen_layernorm(arr)
    torch.cuda.synchronize()
    assert torch.isfinite(out.values).all()


def test_backward_deterministic():
    from scree_amd.kernels.hip.norms import layernorm_bwd as hip_bwd, layernorm_fwd as hip_fwd

    say("case: norm backward determinism")
    x, w, b, dy = _inputs(3000, 1024, torch.bfloat16, 5)
    _, mean, rstd = hip_fwd(x, w, b, 1e-6, want_stats=True)
    r1 = hip_bwd(dy, x, w, mean, rstd, True, True, p_like=w)
    r2 = hip_bwd(dy, x, w, mean, rstd, True, True, p_like=w)
    torch.cuda.synchronize()
    for a, c in zip(r1, r2):
        assert torch.equal(a, c)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_zero_rows(dtype):
    """No rows: empty outputs, and parameter gradients that are sums over no
    rows, i.e. zeros (not left unwritten)."""
    from scree_amd.kernels.hip.norms import (layernorm_bwd, layernorm_fwd, rmsnorm_bwd,
                                             rmsnorm_fwd)

    say(f"case: zero rows, dim 256, {dtype}")
    x = torch.empty((0, 256), dtype=dtype, device="cuda")
    w = randn((256,), dtype, 1, scale=0.02, mean=1.0)
    b = randn((256,), dtype, 2, scale=0.02)
    y, rstd = rmsnorm_fwd(x, w, 1e-6, True)
    assert y.shape == (0, 256) and rstd.shape == (0,)
    dx, dw = rmsnorm_bwd(torch.empty_like(x), x, w, rstd, True, dw_like=w)
    y2, mean, rstd2 = layernorm_fwd(x, w, b, 1e-6, True)
    dx2, dw2, db2 = layernorm_bwd(torch.empty_like(x), x, w, mean, rstd2, True, True, p_like=w)
    torch.cuda.synchronize()
    assert dx.shape == (0, 256) and dx2.shape == (0, 256) and y2.shape == (0, 256)
    for g in (dw, dw2, db2):
        assert g.shape == (256,) and torch.count_nonzero(g).item() == 0


def test_zero_rows_through_the_array_level_calls():
    import scree_amd
    from scree_amd.kernels import varlen_layernorm, varlen_rmsnorm, varlen_softmax

    say("case: Array-level norms and softmax on three empty sequences, with autograd")
    cu = torch.zeros(4, dtype=torch.int32, device="cuda")
    x = torch.empty((0, 64), dtype=torch.bfloat16, device="cuda", requires_grad=True)
    w = torch.ones(64, dtype=torch.bfloat16, device="cuda", requires_grad=True)
    b = torch.zeros(64, dtype=torch.bfloat16, device="cuda", requires_grad=True)
    arr = scree_amd.Array(values=x, offsets=cu)
    outs = [varlen_rmsnorm(arr, w), varlen_layernorm(arr, w, b), varlen_softmax(arr)]
    total = sum(o.values.float().sum() for o in outs)
    total.backward()
    torch.cuda.synchronize()
    assert all(o.values.shape == (0, 64) for o in outs)
    assert x.grad.shape == (0, 64)
    assert torch.count_nonzero(w.grad).item() == 0 and torch.count_nonzero(b.grad).item() == 0
