"""Pins the norm oracle (forward and closed-form backward).

* the reference's known-answer tests (``tests/test_varlen_kernels.py:78-116``);
* ``torch.nn.functional.rms_norm`` / ``layer_norm`` and their autograd;
* fp64 central finite differences;
* properties: unit RMS, zero mean / unit variance
  (``tests/test_properties.py:168-189``).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.norms import layernorm_bwd, layernorm_fwd, rmsnorm_bwd, rmsnorm_fwd


def test_reference_known_answer_layernorm():
    rng = np.random.default_rng(0)
    seqs = [rng.standard_normal((n, 8)).astype(np.float32) for n in [3, 5, 2]]
    x = np.concatenate(seqs)
    y, _, _ = layernorm_fwd(x, eps=1e-5, dtype=np.float32)
    base = (x - x.mean(-1, keepdims=True)) / np.sqrt(x.var(-1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(y, base, atol=1e-5)


def test_reference_known_answer_rmsnorm_with_and_without_weight():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal((n, 8)).astype(np.float32) for n in [3, 5, 2]])
    w = rng.standard_normal((8,)).astype(np.float32)
    y, _ = rmsnorm_fwd(x, eps=1e-6, dtype=np.float32)
    base = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(y, base, atol=1e-5)
    yw, _ = rmsnorm_fwd(x, w, eps=1e-6, dtype=np.float32)
    np.testing.assert_allclose(yw, base * w, atol=1e-5)


@pytest.mark.parametrize("shape", [(7, 16), (5, 3, 33), (1, 4096)])
def test_forward_matches_torch(shape):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(shape)
    w = rng.normal(1.0, 0.02, shape[-1])
    b = rng.normal(0.0, 0.02, shape[-1])
    y, rstd = rmsnorm_fwd(x, w, eps=1e-6)
    ref = F.rms_norm(torch.from_numpy(x), (shape[-1],), torch.from_numpy(w), eps=1e-6)
    np.testing.assert_allclose(y, ref.numpy(), atol=1e-12)
    np.testing.assert_allclose(rstd, 1 / np.sqrt((x * x).mean(-1) + 1e-6), atol=1e-12)
    y, mean, rstd = layernorm_fwd(x, w, b, eps=1e-6)
    ref = F.layer_norm(torch.from_numpy(x), (shape[-1],), torch.from_numpy(w), torch.from_numpy(b), 1e-6)
    np.testing.assert_allclose(y, ref.numpy(), atol=1e-12)
    np.testing.assert_allclose(mean, x.mean(-1), atol=1e-12)


@pytest.mark.parametrize("with_w", [False, True])
def test_rms_backward_matches_torch_autograd(with_w):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((9, 24))
    w = rng.normal(1.0, 0.1, 24) if with_w else None
    dy = rng.standard_normal((9, 24))
    dx, dw = rmsnorm_bwd(dy, x, w, eps=1e-6)
    tx = torch.from_numpy(x).requires_grad_(True)
    tw = torch.from_numpy(w).requires_grad_(True) if with_w else None
    F.rms_norm(tx, (24,), tw, eps=1e-6).backward(torch.from_numpy(dy))
    np.testing.assert_allclose(dx, tx.grad.numpy(), atol=1e-12)
    if with_w:
        np.testing.assert_allclose(dw, tw.grad.numpy(), atol=1e-12)
    else:
        assert dw is None


@pytest.mark.parametrize("with_w,with_b", [(False, False), (True, False), (True, True), (False, True)])
def test_ln_backward_matches_torch_autograd(with_w, with_b):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 2, 20))
    w = rng.normal(1.0, 0.1, 20) if with_w else None
    b = rng.normal(0.0, 0.1, 20) if with_b else None
    dy = rng.standard_normal(x.shape)
    dx, dw, db = layernorm_bwd(dy, x, w, eps=1e-5, has_bias=with_b)
    tx = torch.from_numpy(x).requires_grad_(True)
    tw = torch.from_numpy(w).requires_grad_(True) if with_w else None
    tb = torch.from_numpy(b).requires_grad_(True) if with_b else None
    F.layer_norm(tx, (20,), tw, tb, 1e-5).backward(torch.from_numpy(dy))
    np.testing.assert_allclose(dx, tx.grad.numpy(), atol=1e-12)
    if with_w:
        np.testing.assert_allclose(dw, tw.grad.numpy(), atol=1e-12)
    if with_b:
        np.testing.assert_allclose(db, tb.grad.numpy(), atol=1e-12)


def test_backward_finite_differences():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 5))
    w = rng.normal(1.0, 0.3, 5)
    b = rng.normal(0.0, 0.3, 5)
    dy = rng.standard_normal((3, 5))
    eps = 1e-6

    def fd(f, arr, idx):
        p, m = arr.copy(), arr.copy()
        p[idx] += eps
        m[idx] -= eps
        return (f(p) - f(m)) / (2 * eps)

    rdx, rdw = rmsnorm_bwd(dy, x, w, eps=1e-6)
    ldx, ldw, ldb = layernorm_bwd(dy, x, w, eps=1e-5, has_bias=True)
    for idx in [(0, 0), (1, 3), (2, 4)]:
        assert abs(fd(lambda a: (rmsnorm_fwd(a, w, 1e-6)[0] * dy).sum(), x, idx) - rdx[idx]) < 1e-7
        assert abs(fd(lambda a: (layernorm_fwd(a, w, b, 1e-5)[0] * dy).sum(), x, idx) - ldx[idx]) < 1e-7
    for j in range(5):
        assert abs(fd(lambda a: (rmsnorm_fwd(x, a, 1e-6)[0] * dy).sum(), w, j) - rdw[j]) < 1e-7
        assert abs(fd(lambda a: (layernorm_fwd(x, a, b, 1e-5)[0] * dy).sum(), w, j) - ldw[j]) < 1e-7
        assert abs(fd(lambda a: (layernorm_fwd(x, w, a, 1e-5)[0] * dy).sum(), b, j) - ldb[j]) < 1e-7


def test_properties_unit_rms_and_standardised():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((50, 64)) * 3 + 1
    y, _ = rmsnorm_fwd(x, eps=1e-6)
    np.testing.assert_allclose(np.sqrt((y * y).mean(-1)), 1.0, atol=1e-3)
    z, _, _ = layernorm_fwd(x, eps=1e-5)
    np.testing.assert_allclose(z.mean(-1), 0.0, atol=1e-10)
    np.testing.assert_allclose(z.var(-1), 1.0, atol=1e-3)


# ------------------------------------------------------ fused add + RMSNorm
from oracle.norms import add_rmsnorm_bwd, add_rmsnorm_fwd, add_rounded, round_bf16  # noqa: E402


def test_round_bf16_matches_torch_conversion():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(20000).astype(np.float32) * np.float32(3.0)
    # exact ties: bf16 value plus half an ulp, for both parities of the kept bit
    base = (np.arange(1, 257, dtype=np.uint32) << 16).view(np.float32)
    ties = (base.view(np.uint32) | 0x8000).view(np.float32)
    near = np.concatenate([x, ties, np.nextafter(ties, np.float32(np.inf)),
                           np.nextafter(ties, np.float32(-np.inf)), [0.0, -0.0, 1e-40]]).astype(np.float32)
    want = torch.from_numpy(near).to(torch.bfloat16).to(torch.float64).numpy()
    np.testing.assert_array_equal(round_bf16(near), want)


@pytest.mark.parametrize("storage,tdtype", [("float16", torch.float16), ("bfloat16", torch.bfloat16),
                                            ("float32", torch.float32)])
def test_add_rounded_matches_torch_half_addition(storage, tdtype):
    rng = np.random.default_rng(6)
    a = torch.from_numpy(rng.standard_normal(5000)).to(tdtype)
    b = torch.from_numpy(rng.standard_normal(5000) * 1e-2).to(tdtype)
    want = (a + b).to(torch.float64).numpy()
    got = add_rounded(a.to(torch.float64).numpy(), b.to(torch.float64).numpy(), storage)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("with_dh", [False, True])
def test_add_rmsnorm_matches_torch_autograd(with_dh):
    rng = np.random.default_rng(7)
    rows, d = 11, 24
    x = rng.standard_normal((rows, d))
    r = rng.standard_normal((rows, d))
    w = 1 + 0.1 * rng.standard_normal(d)
    dy = rng.standard_normal((rows, d))
    dh = rng.standard_normal((rows, d)) if with_dh else None
    h, y, rstd = add_rmsnorm_fwd(x, r, w, eps=1e-6)
    xt, rt, wt = (torch.tensor(a, requires_grad=True) for a in (x, r, w))
    ht = xt + rt
    yt = F.rms_norm(ht, (d,), wt, eps=1e-6)
    loss = (yt * torch.tensor(dy)).sum()
    if with_dh:
        loss = loss + (ht * torch.tensor(dh)).sum()
    loss.backward()
    np.testing.assert_allclose(h, ht.detach().numpy(), atol=1e-14)
    np.testing.assert_allclose(y, yt.detach().numpy(), atol=1e-12)
    dx, dw = add_rmsnorm_bwd(dy, dh, h, w, eps=1e-6)
    np.testing.assert_allclose(dx, xt.grad.numpy(), atol=1e-11)
    np.testing.assert_allclose(dx, rt.grad.numpy(), atol=1e-11)
    np.testing.assert_allclose(dw, wt.grad.numpy(), atol=1e-11)
    # the fused forward is the unfused composition
    y2, rstd2 = rmsnorm_fwd(add_rounded(x, r), w, eps=1e-6)
    np.testing.assert_array_equal(y, y2)
    np.testing.assert_array_equal(rstd, rstd2)
