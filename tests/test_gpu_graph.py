"""HIP-graph capture of one attention step (scheduler, forward, dQ, dK/dV),
in fp16, bf16 and fp32 (the FP32-FMA kernels).

Callers (and bench.py) may capture the launches in a graph: the kernels
allocate nothing and the library issues no memset.  Every replay must give
the eager result bit for bit, also with eager work and synchronisations
between replays and after the inputs change.
"""

import numpy as np
import pytest
import torch

from parity import cu_of, randn, say

pytestmark = pytest.mark.gpu


def _case(lengths, heads, kv_heads, dim, dtype, causal, split=False):
    from scree_amd.kernels.hip import attention as A

    n = sum(lengths)
    off, cu = cu_of(lengths)
    t = {
        "q": randn((n, heads, dim), dtype, 1), "k": randn((n, kv_heads, dim), dtype, 2),
        "v": randn((n, kv_heads, dim), dtype, 3), "do": randn((n, heads, dim), dtype, 4),
    }
    t["out"] = torch.empty_like(t["q"])
    t["lse"] = torch.empty(n, heads, device="cuda", dtype=torch.float32)
    t["delta"] = torch.empty(n, heads, device="cuda", dtype=torch.float32)
    t["dq"], t["dk"], t["dv"] = (torch.empty_like(t[x]) for x in ("q", "k", "v"))
    # split: room for the grouped-query dK/dV split (partial sums + reduce kernel)
    nbytes = (A.bwd_workspace_bytes(len(lengths), n, heads, kv_heads, dim) if split
              else A.workspace_bytes(len(lengths), n, dim))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    t["ws"] = ws

    def step():
        A.attention_schedule(cu, n, dim, causal, ws)
        A._attn_fwd(t["q"], t["k"], t["v"], cu, causal, t["out"], t["lse"], ws)
        A._attn_bwd_dq(t["do"], t["q"], t["k"], t["v"], t["out"], t["lse"], cu, causal, t["dq"],
                       t["delta"], ws)
        A._attn_bwd_dkv(t["do"], t["q"], t["k"], t["v"], t["lse"], t["delta"], cu, causal,
                        t["dk"], t["dv"], ws)

    return t, step


OUTS = ("out", "lse", "delta", "dq", "dk", "dv")


@pytest.mark.parametrize("kv_heads,split,dtype", [
    (8, False, torch.float16), (2, False, torch.float16), (2, True, torch.float16),
    (8, False, torch.bfloat16), (2, False, torch.float32)])
def test_graph_replays_match_eager(kv_heads, split, dtype):
    from scree_amd.kernels.hip import attention as A

    lengths = [300, 17, 129, 640, 1]
    say(f"case: graph replay lengths={lengths} H=8 Hkv={kv_heads} D=64 {dtype} causal split={split}")
    t, step = _case(lengths, 8, kv_heads, 64, dtype, True, split)
    if split:
        assert t["ws"].numel() > A.workspace_bytes(len(lengths), sum(lengths), 64)
    step()
    torch.cuda.synchronize()
    want = {k: t[k].clone() for k in OUTS}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rep in range(3):
        for k in OUTS:  # eager work between replays: clobber every output
            t[k].fill_(float("nan"))
        t["ws"].fill_(255)  # and the workspace: the step rebuilds the schedule
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k in OUTS:
            assert torch.equal(t[k], want[k]), f"replay {rep}: {k} differs from the eager step"
    # new inputs copied into the captured buffers: the replay follows them
    t["q"].copy_(randn(tuple(t["q"].shape), dtype, 99))
    step()
    torch.cuda.synchronize()
    want = {k: t[k].clone() for k in OUTS}
    for k in OUTS:
        t[k].zero_()
    graph.replay()
    torch.cuda.synchronize()
    for k in OUTS:
        assert torch.equal(t[k], want[k]), f"replay after input change: {k} differs"
    assert not torch.isnan(t["out"]).any()
