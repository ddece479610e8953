#!/usr/bin/env python3
"""Throughput of the HIP varlen kernel path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle-ms MS] [--no-cpu] [--only NAME]``

Primary line: causal varlen attention forward +
backward, fp16, 16 sequences summing to 12160 tokens (log-normal, sigma 0.6,
rescaled), 16 heads x head_dim 64, synthetic N(0,1) inputs already resident
in HBM.  One step = work list (the forward derives and publishes it at this
size; larger problems launch the tile scheduler) + forward (O, LSE) + dQ/Delta pass + dK/dV
pass into preallocated buffers.  K steps are replayed from HIP graphs of up
to 10 consecutive steps (graphs of one step and eager call-by-call launches
are reported beside it).  Every timed region is preceded by untimed
repetitions of exactly what it times (the same launches, or the same graph
replays) for ``--settle-ms`` milliseconds (default 50, recorded in
``config.settle_ms``): after any idle spell -- process start, or host-only
work such as graph capture -- the GPU runs its first ~10-20 ms of work up to
17 % slower while its clocks ramp up, which would otherwise land in a timed
region that lasts ~8 ms.  ``value`` is real-token causal TFLOP/s
(4*H*D*sum L(L+1)/2 forward, x3.5 for forward+backward).

Also reported (``secondary``): config 3 forward, config 4 on the reference's
fixed H100 length list, config 4 with grouped-query attention (16 query heads
on 4 K/V heads), config 5 (bf16, 32x128) forward+backward, config 2
RMSNorm / LayerNorm / fused add + RMSNorm forward and backward GB/s, varlen
softmax forward and backward and packed <-> padded conversions GB/s at the
config-2 shape (each op cycling over three input sets, so that its input is
not still cached from the previous call), the reference's 27-shape sweep (head_dim x heads x mean
length, fp16 causal, forward and forward+backward), torch's own SDPA on the same GPU for calibration (uniform
lengths with cfg4's token count), the vendor GEMM's fp16 rate on random and
on constant operands (the clock this GPU holds on real data), config 4
and config 5 run back to back for 3 s with the board's socket power and gfx
clock sampled by ``amd-smi`` (the rate at the board power limit), the
user-facing autograd step, config 1
(the reference's CPU case) on the GPU path, and per-kernel HIP-event
timings.  ``roofline`` describes the dominant kernel of the primary step;
``cpu_baseline`` times the numpy oracle (the reference's einsum call
pattern) on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_F16_TFLOPS = 2516.6   # MI355X dense fp16/bf16 MFMA, published
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, published
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


SETTLE_S = 0.05  # set from --settle-ms


def _settle(fn) -> None:
    """Untimed calls of ``fn`` (the very thing the next timed region runs)
    for SETTLE_S seconds of wall time, synchronising every 8 calls so that the
    host never runs far ahead of the GPU.  A GPU that has been idle runs its
    first ~10-20 ms of work up to 17 % slower while its clocks ramp up."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


# Input sets the HBM-bound timings cycle over (3 x 162 MB per activation).
NROT = 3


def _events_time(fn, reps: int) -> float:
    """Average milliseconds of ``fn`` over ``reps`` back-to-back calls (HIP events)."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _settle(fn)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def _graph_time(fn, reps: int, replays: int) -> float:
    """Average milliseconds of one ``fn`` when ``reps`` back-to-back calls are
    captured in a HIP graph and the graph is replayed ``replays`` times.

    The launches are the same kernels on the same preallocated buffers as the
    eager calls; the graph only removes the host's per-call launch cost (four
    ctypes calls per step otherwise keep the GPU waiting between kernels).
    Nothing the kernels do is memset or allocated inside the graph.
    """
    import torch

    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    _settle(graph.replay)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * reps)


def _graph_steps_time(fn, steps: int, chunk: int = 10) -> float:
    """Average milliseconds of one ``fn`` over exactly ``steps`` calls replayed
    from HIP graphs that hold up to ``chunk`` consecutive calls each.

    A graph launch has a fixed cost on the host and at the front of the GPU
    queue (~20 us here), so a loop of small launches is captured a few steps
    per graph, as a training loop would capture its step.  ``steps // chunk``
    replays of a ``chunk``-call graph plus one replay of a graph of the
    remainder run exactly ``steps`` calls between the two HIP events.  Each
    graph is replayed once untimed first (its upload to the device).
    """
    import torch

    chunk = max(1, min(chunk, steps))
    full, rem = divmod(steps, chunk)
    fn()
    torch.cuda.synchronize()

    def capture(n):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(n):
                fn()
        return graph

    g_full = capture(chunk) if full else None
    g_rem = capture(rem) if rem else None
    for g in (g_full, g_rem):
        if g is not None:
            g.replay()
    _settle((g_full or g_rem).replay)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(full):
        g_full.replay()
    if g_rem is not None:
        g_rem.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


class AttnCase:
    """Preallocated tensors and the four launches of one attention step."""

    def __init__(self, cfg, dtype, seed=0, kv_heads=None):
        import numpy as np
        import torch

        from scree_amd.kernels.hip import attention as A

        self.cfg, self.A = cfg, A
        dev = torch.device("cuda:0")
        n, h, d = cfg.total, cfg.heads, cfg.head_dim
        hk = h if kv_heads is None else kv_heads  # grouped-query: fewer K/V heads
        g = torch.Generator(device=dev).manual_seed(seed)
        self.q, self.k, self.v, self.do = (torch.randn(n, hh, d, device=dev, dtype=dtype, generator=g)
                                           for hh in (h, hk, hk, h))
        off = np.zeros(len(cfg.lengths) + 1, dtype=np.int32)
        off[1:] = np.cumsum(cfg.lengths)
        self.cu = torch.from_numpy(off).to(dev)
        self.out = torch.empty_like(self.q)
        self.lse = torch.empty(n, h, device=dev, dtype=torch.float32)
        self.dq, self.dk, self.dv = (torch.empty_like(t) for t in (self.q, self.k, self.v))
        self.delta = torch.empty(n, h, device=dev, dtype=torch.float32)
        # room for the grouped-query dK/dV split (just the schedule when hk == h)
        self.ws = torch.empty(A.bwd_workspace_bytes(len(cfg.lengths), n, h, hk, d), dtype=torch.uint8,
                              device=dev)

    def needs_schedule(self) -> bool:
        return self.A.needs_schedule(len(self.cfg.lengths), self.cfg.total, self.cfg.heads,
                                     self.cfg.head_dim)

    def schedule(self):
        """The work list, as the user-facing calls build it (nothing when the
        forward derives its items and publishes the list itself)."""
        self.A.prepare_workspace(self.cu, self.cfg.total, self.cfg.head_dim, self.cfg.causal,
                                 self.cfg.heads, self.ws)

    def fwd(self):
        self.A._attn_fwd(self.q, self.k, self.v, self.cu, self.cfg.causal, self.out, self.lse, self.ws)

    def bwd_dq(self):
        self.A._attn_bwd_dq(self.do, self.q, self.k, self.v, self.out, self.lse, self.cu,
                            self.cfg.causal, self.dq, self.delta, self.ws)

    def bwd_dkv(self):
        self.A._attn_bwd_dkv(self.do, self.q, self.k, self.v, self.lse, self.delta, self.cu,
                             self.cfg.causal, self.dk, self.dv, self.ws)

    def step_fwd(self):
        self.schedule()
        self.fwd()

    def step_fwd_bwd(self):
        self.schedule()
        self.fwd()
        self.bwd_dq()
        self.bwd_dkv()


def time_attention(cfg, dtype, steps, warmup, backward, per_kernel=False, kv_heads=None):
    """One step = work list (scheduler launch, or none when the forward derives
    it) + forward (+ dQ + dK/dV) on preallocated buffers.

    ``ms`` times ``steps`` steps replayed from HIP graphs of up to 10
    consecutive steps (HIP events around the replays); ``graph1_ms`` replays
    a graph of one step ``steps`` times (each step pays a graph launch);
    ``eager_ms`` times the same steps launched call by call from Python.
    Per-kernel times replay a graph of 10 launches of that kernel alone.
    """
    import torch

    case = AttnCase(cfg, dtype, kv_heads=kv_heads)
    step = case.step_fwd_bwd if backward else case.step_fwd
    for _ in range(warmup):
        step()
    eager_ms = _events_time(step, steps)
    graph1_ms = _graph_time(step, 1, steps)
    ms = _graph_steps_time(step, steps)
    flops = cfg.fwd_flops() * (3.5 if backward else 1.0)
    res = {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "eager_ms": eager_ms,
           "eager_tflops": flops / (eager_ms * 1e-3) / 1e12, "graph1_ms": graph1_ms}
    res["mfma_frac"] = res["tflops"] / PEAK_F16_TFLOPS
    if per_kernel:
        kernels = {"attn_schedule": case.schedule} if case.needs_schedule() else {}
        kernels["attn_fwd"] = case.fwd
        if backward:
            kernels.update({"attn_bwd_dq": case.bwd_dq, "attn_bwd_dkv": case.bwd_dkv})
        res["kernels_ms"] = {k: _graph_time(f, 10, max(3, steps // 5)) for k, f in kernels.items()}
    return res, case


def time_norms(cfg, steps, warmup):
    """Config-2 norms, softmax and packed <-> padded ops, bf16.  Every case
    cycles over NROT sets of inputs (each activation 162 MB, so one cycle
    reads more than the GPU's 256 MB last-level cache): a kernel that reads
    with ordinary loads would otherwise find its input still cached from the
    previous call and be credited with more than HBM bandwidth (measured:
    the softmax forward 68 us on one repeated input against 94 us cycling)."""
    import torch

    from scree_amd import workloads
    from scree_amd.kernels.hip import norms as Nm
    from scree_amd.kernels.hip import padding as Pd
    from scree_amd.kernels.hip import softmax as Sm

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(2)
    rows, dim = cfg.total, cfg.hidden
    dt = torch.bfloat16
    w = (1 + 0.02 * torch.randn(dim, device=dev, generator=g)).to(dt)
    b = (0.02 * torch.randn(dim, device=dev, generator=g)).to(dt)
    off = torch.zeros(len(cfg.lengths) + 1, dtype=torch.int32)
    off[1:] = torch.cumsum(torch.tensor(cfg.lengths, dtype=torch.int64), 0).to(torch.int32)
    cu = off.to(dev)
    max_len = max(cfg.lengths)
    sets = []
    for _ in range(NROT):
        x = torch.randn(rows, dim, device=dev, dtype=dt, generator=g)
        dy = torch.randn(rows, dim, device=dev, dtype=dt, generator=g)
        r = torch.randn(rows, dim, device=dev, dtype=dt, generator=g)
        dh = torch.randn(rows, dim, device=dev, dtype=dt, generator=g)
        _, rstd = Nm.rmsnorm_fwd(x, w, cfg.eps, True)
        _, mean, lrstd = Nm.layernorm_fwd(x, w, b, cfg.eps, True)
        h, _, hrstd = Nm.add_rmsnorm_fwd(x, r, w, cfg.eps, True)
        ys = Sm.softmax_fwd(x, cu)
        padded, pmask = Pd.to_padded_hip(x, cu, max_len=max_len)
        sets.append(dict(x=x, dy=dy, r=r, dh=dh, rstd=rstd, mean=mean, lrstd=lrstd, h=h, hrstd=hrstd,
                         ys=ys, padded=padded, pmask=pmask))
    fb = workloads.norm_fwd_bytes(rows, dim, 2, False)
    bb = workloads.norm_bwd_bytes(rows, dim, 2, False)
    lfb = workloads.norm_fwd_bytes(rows, dim, 2, True)
    lbb = workloads.norm_bwd_bytes(rows, dim, 2, True)
    # fused residual add + RMSNorm: reads x, r (and w), writes h, y; backward
    # reads dy, dh, h (and w), writes dx (and dw)
    afb = 4.0 * 2 * rows * dim + 2 * dim
    abb = 4.0 * 2 * rows * dim + 2 * 2 * dim
    y = torch.empty(rows, dim, device=dev, dtype=dt)
    nb = rows * dim * 2
    row = dim * 2
    pad_rows = len(cfg.lengths) * max_len
    eps = cfg.eps
    cases = {
        "rmsnorm_fwd": (lambda s: Nm.rmsnorm_fwd(s["x"], w, eps, True), fb),
        "rmsnorm_bwd": (lambda s: Nm.rmsnorm_bwd(s["dy"], s["x"], w, s["rstd"], True, dw_like=w), bb),
        "layernorm_fwd": (lambda s: Nm.layernorm_fwd(s["x"], w, b, eps, True), lfb),
        "layernorm_bwd": (lambda s: Nm.layernorm_bwd(s["dy"], s["x"], w, s["mean"], s["lrstd"], True, True,
                                                     p_like=w), lbb),
        "add_rmsnorm_fwd": (lambda s: Nm.add_rmsnorm_fwd(s["x"], s["r"], w, eps, True), afb),
        "add_rmsnorm_bwd": (lambda s: Nm.add_rmsnorm_bwd(s["dy"], s["dh"], s["h"], w, s["hrstd"], True,
                                                         dw_like=w), abb),
        # the two steps it replaces (torch add, then this library's RMSNorm), same algorithmic bytes
        "unfused_add_then_rmsnorm_fwd": (lambda s: Nm.rmsnorm_fwd(s["x"] + s["r"], w, eps, True), afb),
        "device_copy_same_bytes": (lambda s: y.copy_(s["x"]), 2.0 * nb),
        # varlen softmax along the ragged axis at the same shape (x: 19758 x 4096 bf16)
        "varlen_softmax_fwd": (lambda s: Sm.softmax_fwd(s["x"], cu, s["ys"]), 2.0 * nb),
        "varlen_softmax_bwd": (lambda s: Sm.softmax_bwd(s["ys"], s["dy"], cu), 3.0 * nb),
        # packed <-> padded at the same shape: (64, 829, 4096) bf16 padded batch
        "to_padded": (lambda s: Pd.to_padded_hip(s["x"], cu, max_len=max_len), rows * row + pad_rows * (row + 1)),
        "from_padded_user_call": (lambda s: Pd.from_padded_hip(s["padded"], s["pmask"]), pad_rows + 2.0 * rows * row),
        # the same call given the token count (no host read of the device total)
        "from_padded_given_total": (lambda s: Pd.from_padded_hip(s["padded"], s["pmask"], total=rows),
                                    pad_rows + 2.0 * rows * row),
    }
    out = {}
    for name, (fn, nbytes) in cases.items():
        it = [0]

        def step(fn=fn, it=it):
            fn(sets[it[0] % NROT])
            it[0] += 1

        for _ in range(warmup):
            step()
        ms = _events_time(step, steps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": ms, "GB/s": gbs, "hbm_frac": gbs / PEAK_HBM_GBS, "bytes": nbytes}
    return out


def time_sdpa_reference(heads, head_dim, batch, seqlen, steps, warmup, backend=None):
    """Calibration: torch's own fused attention on a uniform-length batch with
    the same tokens, causal fp16, forward + backward; ``backend`` None is the
    default SDPA dispatch (flash attention on this build), else the name of a
    ``torch.nn.attention.SDPBackend``."""
    import contextlib

    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    shape = (batch, heads, seqlen, head_dim)
    q, k, v, do = (torch.randn(*shape, device=dev, dtype=torch.float16, generator=g) for _ in range(4))
    for t in (q, k, v):
        t.requires_grad_(True)

    ctx = (lambda: contextlib.nullcontext()) if backend is None else (
        lambda: sdpa_kernel(getattr(SDPBackend, backend)))

    def step():
        with ctx():
            o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        o.backward(do)

    for _ in range(warmup):
        step()
    ms = _events_time(step, steps)
    from scree_amd.workloads import attn_fwd_flops
    flops = 3.5 * attn_fwd_flops([seqlen] * batch, heads, head_dim, True)
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12}


def _read_power():
    """(socket power W, gfx clock MHz) of GPU 0 from ``amd-smi`` run as a child
    process, or None where the tool or the fields are missing."""
    import re
    import subprocess

    try:
        r = subprocess.run(["amd-smi", "metric", "-p", "-c"], capture_output=True, text=True, timeout=10)
    except (OSError, subprocess.SubprocessError):
        return None
    pw = re.search(r"SOCKET_POWER:\s*(\d+(?:\.\d+)?)\s*W", r.stdout)
    ck = re.search(r"GFX_0:\s*\n\s*CLK:\s*(\d+)\s*MHz", r.stdout)
    if not pw or not ck:
        return None
    return float(pw.group(1)), float(ck.group(1))


def time_sustained(fn, steps_per_call, seconds=3.0):
    """Milliseconds per step of ``fn`` (``steps_per_call`` steps per call)
    launched back to back for ``seconds``, with the board's socket power and
    the gfx clock sampled beside it (medians over the samples after the first
    half second).  Short timed regions run at a higher clock than this: the
    GPU's power management lets the clock down over the first seconds of
    load, to hold the board power limit."""
    import threading

    import torch

    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            s = _read_power()
            if s is None:
                return
            samples.append((time.perf_counter(), *s))

    fn()
    torch.cuda.synchronize()
    th = threading.Thread(target=sampler, daemon=True)
    t0 = time.perf_counter()
    th.start()
    n = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
        n += 4
    dt = time.perf_counter() - t0
    stop.set()
    th.join(timeout=15)
    late = [s for s in samples if s[0] - t0 > 0.5]
    return {"seconds": round(dt, 2), "steps": n * steps_per_call,
            "ms_per_step": round(dt * 1e3 / (n * steps_per_call), 4),
            "socket_power_W": statistics.median(s[1] for s in late) if late else None,
            "gfx_clock_MHz": statistics.median(s[2] for s in late) if late else None,
            "power_samples": len(late)}


def time_gemm_calibration(n=8192, reps=200):
    """Calibration: the vendor GEMM (``torch.matmul``, ROCm's BLAS) on fp16
    n x n by n x n, once with N(0,1) operands and once with all-ones operands.

    The same instruction stream draws different power on different data: the
    GPU holds its top clock on constant operands and lowers it on random
    ones, so the random-operand rate is the dense matrix rate this GPU
    sustains on real data, beside the published peak the roofline uses."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)
    out = {}
    for name, init in (("random", lambda: torch.randn(n, n, device=dev, dtype=torch.float16, generator=g)),
                       ("ones", lambda: torch.ones(n, n, device=dev, dtype=torch.float16))):
        a, b = init(), init()
        c = torch.empty(n, n, device=dev, dtype=torch.float16)
        fn = lambda: torch.matmul(a, b, out=c)  # noqa: E731
        fn()
        ms = _events_time(fn, reps)
        tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        out[name] = {"ms": round(ms, 4), "tflops": round(tf, 1), "frac_of_published_peak": round(tf / PEAK_F16_TFLOPS, 4)}
        del a, b, c
    return out


def time_config1_gpu(steps, warmup):
    """Config 1 (the reference's CPU plumbing case) on the GPU path.

    Config 1 is stated in fp32: attention runs in fp32 on the fp32 kernels
    (what the Array-level call takes fp32 arrays to; the reference's GPU
    launcher rejects fp32, ``triton/varlen_attention.py:215``) and, for
    comparison, in fp16 on the matrix-instruction kernels, on the same
    lengths and 4 heads x head_dim 32 (causal, forward and forward+backward);
    RMSNorm runs in fp32 on the packed tokens as (tokens, 128) rows with
    gamma = 1, the reference's own reshaping
    (``benchmarks/bench_throughput.py:122``).
    """
    import torch

    from scree_amd import workloads
    from scree_amd.kernels.hip import norms as Nm

    lengths = workloads.config1_lengths()
    out = {"tokens": int(sum(lengths))}
    for name, dt in (("fp32", torch.float32), ("fp16", torch.float16)):
        for bwd in (False, True):
            cfg = workloads.AttnConfig("cfg1_attn_gpu", lengths, 4, 32, name, True, bwd)
            r, _ = time_attention(cfg, dt, steps, warmup, backward=bwd)
            out[f"attn_causal_{name}_fwd_bwd" if bwd else f"attn_causal_{name}_fwd"] = {
                "us": round(r["ms"] * 1e3, 2), "tflops": round(r["tflops"], 3)}
    dev = torch.device("cuda:0")
    x = torch.randn(out["tokens"], 128, device=dev, dtype=torch.float32,
                    generator=torch.Generator(device=dev).manual_seed(3))
    w = torch.ones(128, device=dev, dtype=torch.float32)
    for _ in range(warmup):
        Nm.rmsnorm_fwd(x, w, 1e-6, False)
    ms = _events_time(lambda: Nm.rmsnorm_fwd(x, w, 1e-6, False), steps)
    nbytes = workloads.norm_fwd_bytes(out["tokens"], 128, 4, False)
    out["rmsnorm_fp32_x128_fwd"] = {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    return out


def time_shape_sweep(steps, warmup):
    """The reference's 27-shape sweep (``benchmarks/modal_multishape_sweep.py:64-69``):
    head_dim 32/64/128 x heads 4/8/16 x mean length 256/1024/2048, 16
    sequences, log-normal sigma 0.6 (seed 0, ``max(1, int(x))``, no clip),
    causal fp16.  Each row: forward and forward+backward steps (work list
    included) on preallocated buffers, replayed from HIP graphs of up to 10
    steps, real-token causal TFLOP/s and fraction of the dense fp16 peak."""
    import torch

    from scree_amd import workloads

    rows = []
    for head_dim in (32, 64, 128):
        for heads in (4, 8, 16):
            for mean_len in (256, 1024, 2048):
                lengths = workloads.lognormal_lengths(16, mean_len, 0.6, seed=0, lo=1)
                cfg = workloads.AttnConfig(f"sweep_d{head_dim}_h{heads}_m{mean_len}", lengths, heads,
                                           head_dim, "fp16", True, True)
                case = AttnCase(cfg, torch.float16)
                row = {"head_dim": head_dim, "heads": heads, "mean_len": mean_len,
                       "tokens": cfg.total}
                for tag, step, mult in (("fwd", case.step_fwd, 1.0), ("fwd_bwd", case.step_fwd_bwd, 3.5)):
                    for _ in range(warmup):
                        step()
                    ms = _graph_steps_time(step, steps)
                    tf = cfg.fwd_flops() * mult / (ms * 1e-3) / 1e12
                    row[f"{tag}_ms"] = round(ms, 4)
                    row[f"{tag}_tflops"] = round(tf, 1)
                    row[f"{tag}_mfma_frac"] = round(tf / PEAK_F16_TFLOPS, 4)
                rows.append(row)
                del case
                log(f"sweep d{head_dim} h{heads} m{mean_len}: fwd {row['fwd_ms']:.4f} ms "
                    f"{row['fwd_tflops']:.0f} TF/s, fwd+bwd {row['fwd_bwd_ms']:.4f} ms "
                    f"{row['fwd_bwd_tflops']:.0f} TF/s")
    return rows


def time_autograd_step(cfg, dtype, steps, warmup):
    """User-facing path: autograd Function forward + backward (allocations included)."""
    import numpy as np
    import torch

    from scree_amd.kernels.hip import varlen_attention_hip_autograd

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    n, h, d = cfg.total, cfg.heads, cfg.head_dim
    q, k, v, do = (torch.randn(n, h, d, device=dev, dtype=dtype, generator=g) for _ in range(4))
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    off = np.zeros(len(cfg.lengths) + 1, dtype=np.int32)
    off[1:] = np.cumsum(cfg.lengths)
    cu = torch.from_numpy(off).to(dev)

    def step():
        # grads start empty each step, as after optimizer.zero_grad() and as in
        # the reference's loop, which builds fresh leaves per iteration
        # (benchmarks/modal_autograd_bench.py:125-131); otherwise backward adds
        # into .grad (three extra elementwise kernels over q, k and v)
        q.grad = k.grad = v.grad = None
        out = varlen_attention_hip_autograd(q, k, v, cu, causal=cfg.causal)
        out.backward(do)

    for _ in range(warmup):
        step()
    ms = _events_time(step, steps)
    return {"ms": ms, "tflops": cfg.fwd_flops() * 3.5 / (ms * 1e-3) / 1e12}


def _cpu_median(fn, warmup=2, iters=5) -> float:
    """Median seconds of ``fn`` (time.perf_counter), after ``warmup`` untimed calls."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(cfg, heads_sample=1, warmup=2, iters=5):
    """The oracle (reference numpy einsum path, fp32, single-threaded) on a head sample."""
    import numpy as np

    from oracle.attention import attention_bwd, attention_fwd
    from scree_amd import workloads

    rng = np.random.default_rng(0)
    n, d = cfg.total, cfg.head_dim
    q, k, v, do = (rng.standard_normal((n, heads_sample, d)).astype(np.float32) for _ in range(4))
    off = np.zeros(len(cfg.lengths) + 1, dtype=np.int32)
    off[1:] = np.cumsum(cfg.lengths)

    def run():
        o, lse = attention_fwd(q, k, v, off, causal=cfg.causal, dtype=np.float32, impl="einsum")
        attention_bwd(do, q, k, v, o, lse, off, causal=cfg.causal, dtype=np.float32, impl="einsum")

    sec = _cpu_median(run, warmup, iters)
    flops = 3.5 * workloads.attn_fwd_flops(cfg.lengths, heads_sample, d, cfg.causal)
    return {
        "value": flops / sec / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"config 4 forward+backward on {heads_sample} of {cfg.heads} heads (all "
                   f"{len(cfg.lengths)} sequences, {n} tokens), fp32 numpy einsum as in the "
                   f"reference's numpy branch (backward: closed-form restatement); median of "
                   f"{iters} after {warmup} warmup; {sec * 1e3:.0f} ms per sample step; host "
                   f"os.cpu_count()={os.cpu_count()}, affinity={len(os.sched_getaffinity(0))}; "
                   "einsum without optimize is single-threaded"),
    }


def cpu_plumbing():
    """Config 1 on the CPU oracle (the reference's own CPU case), plus a config 2 RMSNorm sample."""
    import numpy as np

    from oracle.attention import attention_fwd
    from oracle.norms import rmsnorm_fwd
    from scree_amd import workloads

    lengths = workloads.config1_lengths()
    n = int(sum(lengths))
    off = np.zeros(len(lengths) + 1, dtype=np.int32)
    off[1:] = np.cumsum(lengths)
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((n, 4, 32)).astype(np.float32) for _ in range(3))
    out = {"cfg1_tokens": n}
    for causal in (False, True):
        sec = _cpu_median(lambda: attention_fwd(q, k, v, off, causal=causal, dtype=np.float32,
                                                impl="einsum"))
        out[f"cfg1_attn_causal_{causal}_ms"] = round(sec * 1e3, 3)
    x128 = rng.standard_normal((n, 128)).astype(np.float32)
    sec = _cpu_median(lambda: rmsnorm_fwd(x128, None, 1e-6, dtype=np.float32))
    out["cfg1_rmsnorm_1980x128_ms"] = round(sec * 1e3, 3)
    cfg2 = workloads.config2()
    rows = 2048  # row sample of config 2 (19758 x 4096), fp32 numpy
    xs = rng.standard_normal((rows, cfg2.hidden)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(cfg2.hidden)).astype(np.float32)
    sec = _cpu_median(lambda: rmsnorm_fwd(xs, w, cfg2.eps, dtype=np.float32))
    out["cfg2_rmsnorm_fwd_cpu_GBps"] = round(workloads.norm_fwd_bytes(rows, cfg2.hidden, 4, False)
                                             / sec / 1e9, 2)
    out["cfg2_rmsnorm_fwd_cpu_sample"] = f"{rows} of {cfg2.total} rows, fp32, 1 core"
    return out


def load_traffic(kernel: str, workload: str):
    try:
        with open(TRAFFIC_FILE) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    ent = data.get(workload, {}).get(kernel)
    return None if ent is None else ent.get("hbm_bytes_per_launch")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--primary-only", action="store_true", help="skip the secondary configs")
    ap.add_argument("--no-sweep", action="store_true", help="skip the 27-shape sweep")
    ap.add_argument("--settle-ms", type=float, default=50.0, metavar="MS",
                    help="untimed repetitions of each timed region's launches before it (0: none)")
    ap.add_argument("--only", choices=["cfg5"], default=None,
                    help="time one secondary workload alone and print its figures (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the varlen "
              "path has no multi-GPU mode. Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from scree_amd import workloads
    from scree_amd.kernels.hip import _ffi

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    _ffi.lib()  # raise now if the library is missing
    torch.cuda.set_device(0)
    fp16 = torch.float16
    global SETTLE_S
    SETTLE_S = max(0.0, args.settle_ms) * 1e-3
    if args.only == "cfg5":
        cfg5 = workloads.config5()
        r, _ = time_attention(cfg5, torch.bfloat16, args.steps, args.warmup, backward=True,
                              per_kernel=True)
        print(json.dumps({"workload": cfg5.name, "ms": round(r["ms"], 4), "tflops": round(r["tflops"], 2),
                          "mfma_frac": round(r["mfma_frac"], 4),
                          "kernels_us": {k: round(v * 1e3, 1) for k, v in r["kernels_ms"].items()}}),
              flush=True)
        return 0

    cfg4 = workloads.config4()
    log(f"primary: {cfg4.name} lengths={cfg4.lengths}")
    prim, case4 = time_attention(cfg4, fp16, args.steps, args.warmup, backward=True, per_kernel=True)
    log(f"primary: {prim['ms']:.4f} ms/step, {prim['tflops']:.1f} TFLOP/s "
        f"(one-step graphs: {prim['graph1_ms']:.4f}, eager launches: {prim['eager_ms']:.4f} ms/step)")

    # roofline of the dominant kernel: algorithmic FLOPs it owns / its launch time
    f_fwd = cfg4.fwd_flops()
    owned = {"attn_schedule": 0.0, "attn_fwd": f_fwd, "attn_bwd_dq": 0.5 * f_fwd,
             "attn_bwd_dkv": 2.0 * f_fwd}
    kms = prim["kernels_ms"]
    dom = max(kms, key=kms.get)
    achieved = owned[dom] / (kms[dom] * 1e-3) / 1e12
    roofline = {
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": PEAK_F16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_F16_TFLOPS, 4),
        "traffic": load_traffic(dom, "cfg4"),
        "kernel": dom,
        "avg_launch_us": round(kms[dom] * 1e3, 2),
        "algorithmic_flops_per_launch": owned[dom],
    }

    secondary = {"cfg4_kernels_us": {k: round(v * 1e3, 2) for k, v in kms.items()},
                 "cfg4_eager_launches": {"ms": round(prim["eager_ms"], 4),
                                         "tflops": round(prim["eager_tflops"], 2)},
                 "cfg4_one_step_graphs": {"ms": round(prim["graph1_ms"], 4),
                                          "tflops": round(cfg4.fwd_flops() * 3.5 / (prim["graph1_ms"] * 1e-3)
                                                          / 1e12, 2)}}
    if not args.primary_only:
        g4 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g4):
            for _ in range(10):
                case4.step_fwd_bwd()
        secondary["cfg4_sustained_3s"] = time_sustained(g4.replay, 10)
        log(f"cfg4 sustained: {secondary['cfg4_sustained_3s']}")
        del g4
        small = max(3, args.steps // 2)
        cfg3 = workloads.config3()
        r, _ = time_attention(cfg3, fp16, args.steps, args.warmup, backward=False, per_kernel=True)
        secondary["cfg3_fwd"] = {"ms": round(r["ms"], 4), "tflops": round(r["tflops"], 2),
                                 "mfma_frac": round(r["mfma_frac"], 4),
                                 "kernels_us": {k: round(v * 1e3, 2) for k, v in r["kernels_ms"].items()}}
        log(f"cfg3 fwd: {r['ms']:.4f} ms {r['tflops']:.1f} TFLOP/s")
        for name, c, bwd in (("cfg3_fwd_fixed_h100_list", workloads.config3(fixed=True), False),
                             ("cfg4_fwd_bwd_fixed_h100_list", workloads.config4(fixed=True), True)):
            r, _ = time_attention(c, fp16, args.steps, args.warmup, backward=bwd)
            secondary[name] = {"ms": round(r["ms"], 4), "tflops": round(r["tflops"], 2),
                               "mfma_frac": round(r["mfma_frac"], 4)}
            log(f"{name}: {r['ms']:.4f} ms {r['tflops']:.1f} TFLOP/s")
        au = time_autograd_step(cfg4, fp16, args.steps, args.warmup)
        secondary["cfg4_autograd_user_call"] = {"ms": round(au["ms"], 4), "tflops": round(au["tflops"], 2)}
        secondary["cfg1_gpu"] = time_config1_gpu(args.steps, args.warmup)
        log(f"cfg1 on the GPU: {secondary['cfg1_gpu']}")
        cfg5 = workloads.config5()
        r, case5 = time_attention(cfg5, torch.bfloat16, small, 2, backward=True, per_kernel=True)
        secondary["cfg5_fwd_bwd_bf16"] = {"ms": round(r["ms"], 3), "tflops": round(r["tflops"], 2),
                                          "mfma_frac": round(r["mfma_frac"], 4),
                                          "kernels_us": {k: round(v * 1e3, 1) for k, v in r["kernels_ms"].items()},
                                          "sustained_3s": time_sustained(case5.step_fwd_bwd, 1)}
        del case5
        log(f"cfg5: {r['ms']:.3f} ms {r['tflops']:.1f} TFLOP/s")
        gq = workloads.config4()
        gq.name = "cfg4_gqa_16q_4kv"
        r, _ = time_attention(gq, fp16, args.steps, args.warmup, backward=True, kv_heads=4)
        secondary["cfg4_gqa_16q_heads_4kv_heads"] = {"ms": round(r["ms"], 4),
                                                      "tflops": round(r["tflops"], 2),
                                                      "mfma_frac": round(r["mfma_frac"], 4)}
        log(f"cfg4 GQA 16q/4kv: {r['ms']:.4f} ms {r['tflops']:.1f} TFLOP/s")
        uni = workloads.AttnConfig("uniform_16x760_fp16_16x64", [760] * 16, 16, 64, "fp16", True, True)
        ours, _ = time_attention(uni, fp16, args.steps, args.warmup, backward=True)
        ref = time_sdpa_reference(16, 64, 16, 760, args.steps, args.warmup)
        eff = time_sdpa_reference(16, 64, 16, 760, args.steps, args.warmup, backend="EFFICIENT_ATTENTION")
        secondary["vendor_calibration_uniform_16x760"] = {
            "what": "causal fp16 fwd+bwd, 16 seqs x 760 tokens (12160, as cfg4), 16x64: this "
                    "library's step vs torch.nn.functional.scaled_dot_product_attention (default "
                    "ROCm dispatch, which is flash attention on this build, and the memory-"
                    "efficient backend; padded batch of equal lengths) on the same GPU",
            "ours_ms": round(ours["ms"], 4), "ours_tflops": round(ours["tflops"], 2),
            "torch_sdpa_ms": round(ref["ms"], 4), "torch_sdpa_tflops": round(ref["tflops"], 2),
            "torch_sdpa_efficient_ms": round(eff["ms"], 4),
            "torch_sdpa_efficient_tflops": round(eff["tflops"], 2)}
        log(f"calibration 16x760: ours {ours['tflops']:.0f} TF/s, torch SDPA {ref['tflops']:.0f} TF/s "
            f"(efficient backend {eff['tflops']:.0f})")
        gm = time_gemm_calibration()
        secondary["vendor_gemm_fp16_8192"] = {
            "what": "torch.matmul fp16 8192x8192x8192, 200 back-to-back calls after the settle, "
                    "N(0,1) operands vs all-ones operands (same kernels; the GPU lowers its "
                    "clock on random data)", **gm}
        log(f"vendor GEMM fp16 8192^3: random {gm['random']['tflops']:.0f} TF/s, ones {gm['ones']['tflops']:.0f} TF/s")
        if not args.no_sweep:
            secondary["reference_shape_sweep_fp16_causal"] = time_shape_sweep(20, 3)
        nr = time_norms(workloads.config2(), args.steps, args.warmup)
        secondary["cfg2_norms_bf16"] = {k: {"us": round(v["ms"] * 1e3, 2), "GB/s": round(v["GB/s"], 1),
                                            "hbm_frac": round(v["hbm_frac"], 4)} for k, v in nr.items()}
        log("cfg2: " + ", ".join(f"{k} {v['GB/s']:.0f} GB/s" for k, v in nr.items()))

    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline(cfg4)
        log(f"cpu: {cpu['value'] * 1e3:.3f} GFLOP/s")
        secondary["cpu_plumbing"] = cpu_plumbing()
        log(f"cpu plumbing: {secondary['cpu_plumbing']}")

    line = {
        "metric": "causal varlen attn fwd & fwd+bwd TFLOP/s, MFMA %; varlen RMSNorm HBM GB/s",
        "value": round(prim["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(prim["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1), resident in HBM",
        "config": {
            "workload": ("cfg4: causal varlen attention forward+backward (fwd with its work list + dQ + dK/dV), "
                         f"fp16, {len(cfg4.lengths)} seqs, {cfg4.total} tokens (log-normal sigma 0.6 "
                         f"rescaled), {cfg4.heads} heads x head_dim {cfg4.head_dim}"),
            "lengths": cfg4.lengths,
            "mfma_frac": round(prim["mfma_frac"], 4),
            "launch": "K steps replayed from HIP graphs of up to 10 consecutive steps (graphs of "
                      "one step: secondary.cfg4_one_step_graphs; eager per-call launches: "
                      "secondary.cfg4_eager_launches)",
            "settle_ms": SETTLE_S * 1e3,
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
