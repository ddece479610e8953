"""Generate the golden vectors in this directory.

The reference ships no golden vectors or fixtures for the varlen path, so
these are produced here from torch's own CPU library routines in float64 —
``scaled_dot_product_attention`` per sequence (with autograd for the
gradients), ``F.rms_norm`` and ``F.layer_norm`` (with autograd) — and
nothing from this repository's oracle or kernels.  Inputs are drawn so that
they are exactly representable in fp16 (attention) or bf16 (norms), so a GPU
run on the rounded inputs sees the same values.

Conventions followed (reference file:line):
  attention scale 1/sqrt(D) and causal triu mask — reference/varlen_attention.py:31-32,122-137
  LSE = natural-log logsumexp of the scaled scores — triton/varlen_attention.py:158-162
  softmax along the ragged axis per sequence — reference/varlen_softmax.py:44-61
  RMSNorm y = x / sqrt(mean(x^2) + eps) * w — reference/varlen_rmsnorm.py:58-65
  LayerNorm population variance, eps inside the sqrt — reference/varlen_layernorm.py:64-74
  offsets = [0, cumsum(L)] int32 — _core.py:137-138

Run: ``python tests/golden/make_golden.py`` (CPU only; writes *.npz here).
"""

from __future__ import annotations

import math
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def _offsets(lengths):
    off = np.zeros(len(lengths) + 1, dtype=np.int32)
    off[1:] = np.cumsum(lengths)
    return off


def _attention_case(lengths, heads, dim, causal, seed, in_dtype=np.float16):
    rng = np.random.default_rng(seed)
    n = int(sum(lengths))
    q, k, v, do = (rng.standard_normal((n, heads, dim)).astype(in_dtype) for _ in range(4))
    off = _offsets(lengths)
    tq, tk, tv, tdo = (torch.from_numpy(a.astype(np.float64)) for a in (q, k, v, do))
    tq.requires_grad_(True)
    tk.requires_grad_(True)
    tv.requires_grad_(True)
    outs, lses = [], []
    for s in range(len(lengths)):
        a, b = int(off[s]), int(off[s + 1])
        qi, ki, vi = (t[a:b].transpose(0, 1) for t in (tq, tk, tv))  # (H, L, D)
        outs.append(F.scaled_dot_product_attention(qi, ki, vi, is_causal=causal,
                                                   scale=1.0 / math.sqrt(dim)).transpose(0, 1))
        scores = (qi @ ki.transpose(-1, -2)) / math.sqrt(dim)
        if causal:
            L = b - a
            mask = torch.triu(torch.ones(L, L, dtype=torch.bool), diagonal=1)
            scores = scores.masked_fill(mask, float("-inf"))
        lses.append(torch.logsumexp(scores, dim=-1).transpose(0, 1))  # (L, H)
    o = torch.cat(outs, 0)
    lse = torch.cat(lses, 0)
    o.backward(tdo)
    return {
        "lengths": np.asarray(lengths, dtype=np.int32), "offsets": off,
        "heads": np.int32(heads), "dim": np.int32(dim), "causal": np.bool_(causal),
        "q": q, "k": k, "v": v, "do": do,
        # outputs stored in float32: ~1e-7 relative, far below every bound they check
        "o": o.detach().numpy().astype(np.float32), "lse": lse.detach().numpy().astype(np.float32),
        "dq": tq.grad.numpy().astype(np.float32), "dk": tk.grad.numpy().astype(np.float32),
        "dv": tv.grad.numpy().astype(np.float32),
    }


def _bf16_exact(a: np.ndarray) -> np.ndarray:
    """Round float64 values to the nearest bf16 (returned as float32)."""
    return torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def _norm_case(rows, dim, seed, eps):
    rng = np.random.default_rng(seed)
    x = _bf16_exact(rng.standard_normal((rows, dim)))
    w = _bf16_exact(1.0 + 0.02 * rng.standard_normal(dim))
    b = _bf16_exact(0.02 * rng.standard_normal(dim))
    dy = _bf16_exact(rng.standard_normal((rows, dim)))
    out = {"x": x, "w": w, "b": b, "dy": dy, "eps": np.float64(eps)}
    tx, tw, tb = (torch.from_numpy(a.astype(np.float64)).requires_grad_(True) for a in (x, w, b))
    tdy = torch.from_numpy(dy.astype(np.float64))
    y = F.rms_norm(tx, (dim,), tw, eps)
    y.backward(tdy)
    f32 = lambda t: t.detach().numpy().astype(np.float32)  # noqa: E731
    out.update(rms_y=f32(y), rms_dx=f32(tx.grad), rms_dw=f32(tw.grad))
    tx.grad = None
    tw.grad = None
    y = F.layer_norm(tx, (dim,), tw, tb, eps)
    y.backward(tdy)
    out.update(ln_y=f32(y), ln_dx=f32(tx.grad), ln_dw=f32(tw.grad), ln_db=f32(tb.grad))
    return out


def _softmax_case(lengths, features, seed):
    rng = np.random.default_rng(seed)
    n = int(sum(lengths))
    x = (2.0 * rng.standard_normal((n,) + features)).astype(np.float16)
    dy = rng.standard_normal((n,) + features).astype(np.float16)
    off = _offsets(lengths)
    tx = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    parts = [torch.softmax(tx[int(off[i]):int(off[i + 1])], dim=0) for i in range(len(lengths))]
    y = torch.cat(parts, 0)
    y.backward(torch.from_numpy(dy.astype(np.float64)))
    return {"lengths": np.asarray(lengths, dtype=np.int32), "offsets": off, "x": x, "dy": dy,
            "y": y.detach().numpy().astype(np.float32), "dx": tx.grad.numpy().astype(np.float32)}


def main() -> None:
    torch.manual_seed(0)
    edge = [1, 7, 33, 64, 65]  # a single token, sub-tile, tile edge +-1
    for dim in (32, 64):
        for causal in (True, False):
            case = _attention_case(edge, 1, dim, causal, seed=dim + int(causal))
            np.savez_compressed(os.path.join(HERE, f"attention_d{dim}_{'causal' if causal else 'full'}.npz"),
                                **case)
    # Config 1 slice: the first three sequences of the config-1 lengths
    # (log-normal mean 128, sigma 0.6, seed 0), one of its 4 heads, fp32 inputs.
    cfg1 = _attention_case([138, 118, 187], 1, 32, True, seed=0, in_dtype=np.float32)
    np.savez_compressed(os.path.join(HERE, "attention_cfg1_slice_causal.npz"), **cfg1)
    np.savez_compressed(os.path.join(HERE, "softmax_4x16.npz"),
                        **_softmax_case([1, 3, 0, 17, 64, 130], (4, 16), seed=7))
    np.savez_compressed(os.path.join(HERE, "norms_37x96.npz"), **_norm_case(37, 96, seed=5, eps=1e-6))
    np.savez_compressed(os.path.join(HERE, "norms_3x4096.npz"), **_norm_case(3, 4096, seed=6, eps=1e-6))


if __name__ == "__main__":
    main()
