"""The HIP path against the committed golden vectors (GPU).

Inputs in tests/golden/ are exactly representable in fp16 (attention) or
bf16 (norms); expected outputs come from torch's CPU fp64 library routines
(see tests/golden/make_golden.py).  Bounds are the north-star ones: O 2e-3,
dq/dk/dv 5e-3 max-abs; norms 1e-3 plus the bf16 output-rounding term.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from parity import UNIT, check_close, np64, say

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATTN = sorted(p for p in glob.glob(os.path.join(HERE, "attention_d*.npz")))
NORMS = sorted(glob.glob(os.path.join(HERE, "norms_*.npz")))


@pytest.mark.parametrize("path", ATTN, ids=lambda p: os.path.basename(p))
def test_hip_attention_matches_golden(path):
    from scree_amd.kernels.hip import varlen_attention_hip, varlen_attention_hip_backward

    g = np.load(path)
    causal = bool(g["causal"])
    say(f"case: {os.path.basename(path)} lengths={g['lengths'].tolist()}")
    dev = torch.device("cuda:0")
    q, k, v, do = (torch.from_numpy(g[n]).to(dev) for n in ("q", "k", "v", "do"))
    cu = torch.from_numpy(g["offsets"]).to(dev)
    out, lse = varlen_attention_hip(q, k, v, cu, causal=causal, return_lse=True)
    check_close("O", np64(out), g["o"].astype(np.float64), 2e-3)
    check_close("LSE", np64(lse), g["lse"].astype(np.float64), 1e-3)
    dq, dk, dv = varlen_attention_hip_backward(do, q, k, v, out, lse, cu, causal=causal)
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        check_close(name, np64(got), g[name].astype(np.float64), 5e-3)


@pytest.mark.parametrize("path", NORMS, ids=lambda p: os.path.basename(p))
def test_hip_norms_match_golden(path):
    from scree_amd.kernels.hip import varlen_layernorm_hip, varlen_rmsnorm_hip

    g = np.load(path)
    say(f"case: {os.path.basename(path)}")
    dev = torch.device("cuda:0")
    bf = torch.bfloat16
    u = UNIT[bf]
    eps = float(g["eps"])

    def leaf(name):
        return torch.from_numpy(g[name]).to(dev, bf).requires_grad_(True)

    dy = torch.from_numpy(g["dy"]).to(dev, bf)
    x, w = leaf("x"), leaf("w")
    y = varlen_rmsnorm_hip(x, w, eps)
    y.backward(dy)
    for name, got in (("rms_y", y), ("rms_dx", x.grad)):
        want = g[name].astype(np.float64)
        check_close(name, np64(got), want, 1e-3, extra=np.abs(want), unit=u)
    want = g["rms_dw"].astype(np.float64)
    check_close("rms_dw", np64(w.grad), want, 1e-3 + 1e-4 * np.abs(want).max(), extra=np.abs(want), unit=u)

    x, w, b = leaf("x"), leaf("w"), leaf("b")
    y = varlen_layernorm_hip(x, w, b, eps)
    y.backward(dy)
    for name, got in (("ln_y", y), ("ln_dx", x.grad)):
        want = g[name].astype(np.float64)
        check_close(name, np64(got), want, 1e-3, extra=np.abs(want), unit=u)
    for name, got in (("ln_dw", w.grad), ("ln_db", b.grad)):
        want = g[name].astype(np.float64)
        check_close(name, np64(got), want, 1e-3 + 1e-4 * np.abs(want).max(), extra=np.abs(want), unit=u)
