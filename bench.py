#!/usr/bin/env python3
"""Benchmark of the torch_gcu PrivateUse1 op path on one MI355X.

A step is one pass of BASELINE config 2 (row reductions and softmax) over one
batch of synthetic input already resident in HBM:
    sum(-1), amax(-1), log_softmax(-1) of bf16 logits [8192, 32000] N(0, 4)
    mean(0) of fp32 [16384, 4096] N(0, 1)
all through the gfx950 kernels.  `value` is the step's algorithmic bytes
(unique inputs read once + outputs written once) divided by the step time,
in GB/s.  Two input sets alternate between steps so the 256 MiB MALL cannot
serve a re-read.

The same JSON line carries
  roofline      the dominant kernel (log_softmax) timed per launch with HIP
                events on the stream it runs on, against 8 TB/s; `traffic`
                is the HBM bytes per launch that the committed rocprofv3
                counter runs measured (profiles/log_softmax_config2_traffic.md);
  cpu_baseline  CPU ATen (the reference's fallback path, run through
                oracle.aten) on a bounded row sample of the same workload;
  ops           every other measured op of configs 1 and 3 (GB/s, fraction
                of HBM peak), each with its own rotation of input sets.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-ops]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "torch-gcu_amd"))

HBM_PEAK_GBS = 8000.0
# PCIe 5.0 x16 (32 GT/s x 16 lanes, 128b/130b): the MI355X host link, per direction
PCIE5_X16_GBS = 63.0
CAL_COPY_BYTES = 512 * 2**20
METRIC = "HBM GB/s (elementwise/norm), MFMA TFLOPS (addmm/int8), decoder-layer tok/s"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-ops", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--section", choices=sorted(SECTIONS),
                    help="time one group of op lines only (one JSON line per op, no headline "
                         "step): the command a counter profile of those kernels runs")
    return ap.parse_args()


class EventTimer:
    """Accumulates device time of launches on the current stream."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []

    def __enter__(self):
        self.s = self.torch.cuda.Event(enable_timing=True)
        self.e = self.torch.cuda.Event(enable_timing=True)
        self.s.record()
        return self

    def __exit__(self, *a):
        self.e.record()
        self.pairs.append((self.s, self.e))

    def total_ms(self):
        self.torch.cuda.synchronize()
        return sum(s.elapsed_time(e) for s, e in self.pairs)


def config2_alg_bytes(rows=8192, vocab=32000, mrows=16384, mcols=4096):
    x = rows * vocab * 2
    return {
        "sum": x + rows * 2,
        "amax": x + rows * 2,
        "log_softmax": 2 * x,
        "mean": mrows * mcols * 4 + mcols * 4,
    }


def run_config2(torch, _abi, synthetic, steps, warmup):
    log("bench: generating config 2 inputs (2 sets)")
    sets = []
    for k in range(2):
        c = synthetic.config2()
        if k == 1:  # a second, different set for MALL rotation
            c = {"logits": c["logits"].flip(0).contiguous(), "m": c["m"].flip(0).contiguous()}
        sets.append({"logits": c["logits"].cuda(), "m": c["m"].cuda()})
    rows, vocab = sets[0]["logits"].shape
    outs = {
        "sum": torch.empty(rows, dtype=torch.bfloat16, device="cuda"),
        "amax": torch.empty(rows, dtype=torch.bfloat16, device="cuda"),
        "log_softmax": torch.empty(rows, vocab, dtype=torch.bfloat16, device="cuda"),
        "mean": torch.empty(sets[0]["m"].shape[1], dtype=torch.float32, device="cuda"),
    }
    # the same inputs on the gcu device, for the step through the dispatcher
    gsets = [{"logits": st["logits"].cpu().to("gcu"), "m": st["m"].cpu().to("gcu")}
             for st in sets]
    timers = {k: EventTimer(torch) for k in outs}
    # one plain 512 MiB device copy (untimed): under rocprofv3 --pmc its
    # FETCH_SIZE / WRITE_SIZE calibrate the counters against known bytes
    cal = torch.empty(CAL_COPY_BYTES // 2, dtype=torch.int16, device="cuda")
    _abi.copy_(torch.empty_like(cal), cal)
    del cal

    def step(i, timed):
        s = sets[i % 2]
        if timed:
            with timers["sum"]:
                _abi.sum_(outs["sum"], s["logits"], [-1])
            with timers["amax"]:
                _abi.amax(outs["amax"], s["logits"], [-1])
            with timers["log_softmax"]:
                _abi.log_softmax(outs["log_softmax"], s["logits"], -1)
            with timers["mean"]:
                _abi.mean(outs["mean"], s["m"], [0])
        else:
            _abi.sum_(outs["sum"], s["logits"], [-1])
            _abi.amax(outs["amax"], s["logits"], [-1])
            _abi.log_softmax(outs["log_softmax"], s["logits"], -1)
            _abi.mean(outs["mean"], s["m"], [0])

    def dispatch_step(i):
        # the PrivateUse1 path: torch ops on gcu tensors, through the
        # generated wrappers into the same kernels
        s = gsets[i % 2]
        torch.sum(s["logits"], -1)
        torch.amax(s["logits"], -1)
        torch.log_softmax(s["logits"], -1)
        torch.mean(s["m"], 0)

    for i in range(warmup):
        step(i, False)
        dispatch_step(i)
    torch.cuda.synchronize()
    torch.gcu.synchronize()
    log(f"bench: warmup done ({warmup} steps), timing {steps} steps")
    # whole-job wall time of exactly `steps` steps, through the dispatcher
    t0 = time.perf_counter()
    for i in range(steps):
        dispatch_step(i)
    torch.gcu.synchronize()
    wall = time.perf_counter() - t0
    # the same steps called through the C ABI directly
    t0 = time.perf_counter()
    for i in range(steps):
        step(i, False)
    torch.cuda.synchronize()
    wall_abi = time.perf_counter() - t0
    # host cost of one dispatched op: the enqueue loop timed while a spin
    # kernel holds the device (gcu's default stream is the null stream the
    # spin runs on), so the host never waits on it
    hold_device(torch)
    t0 = time.perf_counter()
    for i in range(steps):
        dispatch_step(i)
    host_us = (time.perf_counter() - t0) / (4 * steps) * 1e6
    torch.gcu.synchronize()
    torch.cuda.synchronize()
    # per-kernel device time: the same steps again with HIP events around each
    # launch, queued behind a spin kernel so no host launch gap is counted
    hold_device(torch)
    for i in range(steps):
        step(i, True)
    torch.cuda.synchronize()
    per_op_ms = {k: t.total_ms() / steps for k, t in timers.items()}
    return wall, wall_abi, host_us, per_op_ms


TRAFFIC_PROFILE = os.path.join(REPO, "profiles", "log_softmax_config2_traffic.md")


def committed_traffic():
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (copy-calibrated), or None."""
    import re

    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch = (\d+)", text)
    return int(m.group(1)) if m else None


def cpu_model():
    """The host CPU's model name (the first `model name` of /proc/cpuinfo,
    what lscpu prints)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_time(fn, min_s=0.6, max_n=50):
    """Mean wall time of fn on the host after one warm-up call."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= min_s or n >= max_n:
            return el / n


def cpu_config_ops(torch, synthetic):
    """CPU ATen (the reference's fallback path) on every config op of the
    bench, on bounded samples of the same workloads: {op name: record}.
    Fused ops without a reference op (RMSNorm, RoPE, SiLU-mul, int8 linear)
    run as their fp32 closed forms (oracle.aten)."""
    from oracle import aten
    from torch_gcu.utils import decoder_layer as dl

    log("bench: CPU ATen per config")
    thr = torch.get_num_threads()
    out = {}

    def rec(name, sec, sample, alg=None, flops=None, tokens=None):
        r = {"ms": round(sec * 1e3, 3), "threads": thr, "sample": sample}
        if alg is not None:
            r["GB/s"] = round(alg / sec / 1e9, 2)
        if flops is not None:
            r["TFLOP/s"] = round(flops / sec / 1e12, 4)
        if tokens is not None:
            r["tok/s"] = round(tokens / sec, 1)
        out[name] = r

    c1 = synthetic.config1()
    rec("c1.mul [4096,4096]x[4096] f32", cpu_time(lambda: aten.mul(c1["a"], c1["b"])),
        "full size", alg=4096 * 4096 * 8 + 4096 * 4)
    rec("c1.add [4096,4096]+0.5 f32", cpu_time(lambda: aten.add(c1["a"], 0.5)), "full size",
        alg=4096 * 4096 * 8)
    rec("c1.index_select int64 [1048576,8] x 262144",
        cpu_time(lambda: aten.index_select(c1["table"], 0, c1["idx"])), "full size", alg=35651584)
    del c1
    T = 2048  # 1/8 of config 3's 16384 tokens
    c3 = synthetic.config3(tokens=T)
    rec("c3.rms_norm bf16 [16384,4096]", cpu_time(lambda: aten.rms_norm(c3["x"], c3["w"], 1e-6)),
        f"{T} of 16384 rows", alg=T * 4096 * 4 + 8192)
    rec("c3.rope q,k bf16 [16384,32,128]",
        cpu_time(lambda: (aten.rope(c3["q"], c3["pos"], 1e4), aten.rope(c3["k"], c3["pos"], 1e4))),
        f"{T} of 16384 tokens", alg=4 * T * 32 * 128 * 2)
    rec("c3.silu_mul bf16 [16384,11008]", cpu_time(lambda: aten.silu_mul(c3["gate"], c3["up"])),
        f"{T} of 16384 rows", alg=3 * T * 11008 * 2)
    del c3
    gen = torch.Generator().manual_seed(20261204)
    M = 1024  # 1/8 of config 4's 8192 rows
    A = (torch.randn(M, 4096, generator=gen) * 0.02).bfloat16()
    B = (torch.randn(4096, 4096, generator=gen) * 0.02).bfloat16()
    bias = (torch.randn(4096, generator=gen) * 0.02).bfloat16()
    sec = cpu_time(lambda: torch.addmm(bias, A, B))
    for lay in ("B row-major [K,N]", "B = W^T, K-contiguous"):
        rec(f"c4.addmm bf16 M8192 N4096 K4096 ({lay})", sec, f"CPU ATen bf16 addmm, M={M} rows",
            flops=2 * M * 4096 * 4096)
    W = torch.randint(-127, 128, (11008, 4096), generator=gen, dtype=torch.int8)
    sc = torch.rand(11008, generator=gen) * 0.009 + 0.001
    for Mi in (16, 256, 4096):
        m = min(Mi, 512)
        x = torch.randn(m, 4096, generator=gen).bfloat16()
        rec(f"c4.int8_linear M={Mi} W int8 [11008,4096]",
            cpu_time(lambda: aten.int8_linear(x, W, sc)),
            f"fp32 closed form, M={m} rows" + ("" if m == Mi else f" of {Mi}"),
            flops=2 * m * 11008 * 4096)
    del A, B, W
    cfg = dl.LayerConfig()
    w = dl.init_weights(cfg)
    ids = torch.randint(0, cfg.vocab, (1, 2048), generator=gen)
    sec = cpu_time(lambda: dl.forward(w, ids, cfg), min_s=1.0, max_n=3)
    for name in ("eager", "gcugraph replay"):
        rec(f"c5.decoder_layer fwd B8xS2048 ({name})", sec,
            "CPU ATen bf16 layer on 1 of the 8 sequences (2048 tokens)", tokens=2048)
    return out


def cpu_baseline(torch, synthetic, seconds):
    """CPU ATen on a row sample of config 2 (same distributions and seeds)."""
    from oracle import aten

    # 131 MB of logits and 67 MB of fp32: larger than the host's caches
    rows, mrows = 2048, 4096
    c = synthetic.config2(rows=rows, mrows=mrows)
    ab = config2_alg_bytes(rows=rows, mrows=mrows)
    total = sum(ab.values())
    # warm up once, then repeat until the budget is spent
    aten.sum_(c["logits"], -1)
    aten.amax(c["logits"], -1)
    aten.log_softmax(c["logits"], -1)
    aten.mean(c["m"], 0)
    n, t0 = 0, time.perf_counter()
    while True:
        aten.sum_(c["logits"], -1)
        aten.amax(c["logits"], -1)
        aten.log_softmax(c["logits"], -1)
        aten.mean(c["m"], 0)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {
        "value": round(total * n / el / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "cpu_count": os.cpu_count(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"CPU ATen (the reference's CPU fallback path, via oracle.aten) running "
                   f"sum/amax/log_softmax on bf16 [{rows},32000] and mean(0) on fp32 "
                   f"[{mrows},4096], {n} passes in {el:.1f} s"),
    }


MFMA_BF16_PEAK_TFLOPS = 2500.0


def hold_device(torch, ms=20.0):
    """Keeps the stream busy for about `ms` with a spin kernel, so the launches
    enqueued right after it reach the device back to back: the timed region
    then measures device time, not the host's per-call launch cost."""
    torch.cuda._sleep(int(ms * 2.4e6))  # the spin counts shader clocks (~2.4 GHz)


def bench_op(torch, name, sets, fn, alg_bytes, iters=30, flops=None, bound="hbm", warm_ms=None):
    """Per-launch device time of fn over rotating input sets (HIP events on
    the stream the ops run on; the launches are queued behind a spin kernel,
    and `host_bound` reports whether the device caught up with the host).

    MFMA-bound ops (flops given) are timed at their sustained clock: about
    `warm_ms` (default 25 ms) of untimed launches of the same op run right
    before the timed ones, in the same queue.  The chip raises its clock over
    the first few milliseconds of a burst of matrix work (a GEMM's first
    3-5 ms run 10-15 % slower than the next ones), and a training or serving
    loop runs at the sustained rate."""
    for s in sets[:2]:
        fn(s)
    torch.cuda.synchronize()
    st = torch.cuda.Event(enable_timing=True)
    en = torch.cuda.Event(enable_timing=True)
    warm = 0
    if warm_ms is None:
        warm_ms = 25.0 if flops is not None else 0.0
    if warm_ms > 0:
        # one untimed probe launch gives the per-launch time to size the warm-up
        st.record()
        fn(sets[0])
        en.record()
        torch.cuda.synchronize()
        warm = min(2000, int(warm_ms / max(st.elapsed_time(en), 1e-3)) + 1)
    hold_device(torch)
    for i in range(warm):
        fn(sets[i % len(sets)])
    st.record()
    for i in range(iters):
        fn(sets[i % len(sets)])
    en.record()
    host_bound = st.query()  # the device reached the start before all launches were queued
    torch.cuda.synchronize()
    ms = st.elapsed_time(en) / iters
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    r = {"op": name, "ms": round(ms, 4), "GB/s": round(gbs, 1),
         "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "alg_bytes": alg_bytes}
    if host_bound:
        r["host_bound"] = True
    if flops is not None:
        tf = flops / (ms * 1e-3) / 1e12
        r.update({"TFLOP/s": round(tf, 1), "frac_mfma_bf16": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                  "flops": flops, "bound": bound})
    return r


def gemm_ops(torch, _abi):
    """Config 4: bf16 addmm M8192 N4096 K4096 and the int8 weight-only linear
    (W int8 [11008, 4096], fp32 scales) at M = 16, 256, 4096."""
    res = []
    log("bench: config 4 ops")
    gen = torch.Generator().manual_seed(20261204)
    M, N, K = 8192, 4096, 4096
    A = [(torch.randn(M, K, generator=gen) * 0.02).bfloat16().cuda() for _ in range(2)]
    B = [(torch.randn(K, N, generator=gen) * 0.02).bfloat16().cuda() for _ in range(2)]
    bias = (torch.randn(N, generator=gen) * 0.02).bfloat16().cuda()
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    sets = [{"a": A[i], "b": B[i]} for i in range(2)]
    res.append(bench_op(torch, "c4.addmm bf16 M8192 N4096 K4096 (B row-major [K,N])", sets,
                        lambda s: _abi.addmm(out, bias, s["a"], s["b"]),
                        (M * K + K * N + M * N) * 2 + N * 2, iters=10, flops=2 * M * N * K,
                        bound="mfma"))
    Bt = [b.t().contiguous().t() for b in B]  # the nn.Linear layout: W [N, K], B = W^T
    sets = [{"a": A[i], "b": Bt[i]} for i in range(2)]
    res.append(bench_op(torch, "c4.addmm bf16 M8192 N4096 K4096 (B = W^T, K-contiguous)", sets,
                        lambda s: _abi.addmm(out, bias, s["a"], s["b"]),
                        (M * K + K * N + M * N) * 2 + N * 2, iters=10, flops=2 * M * N * K,
                        bound="mfma"))
    del A, B, Bt, out, sets
    N, K = 11008, 4096
    # 13 weight copies (586 MB) rotated, past the 256 MiB MALL: every launch
    # streams its weight from HBM
    W = [torch.randint(-127, 128, (N, K), generator=gen, dtype=torch.int8).cuda()]
    W += [W[0].roll(k, 0) for k in range(1, 13)]
    scales = (torch.rand(N, generator=gen) * 0.009 + 0.001).cuda()
    for M in (16, 256, 4096):
        x = torch.randn(M, K, generator=gen).bfloat16().cuda()
        o = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        sets = [{"w": w} for w in W]
        alg = N * K + N * 4 + M * K * 2 + M * N * 2
        res.append(bench_op(torch, f"c4.int8_linear M={M} W int8 [11008,4096]", sets,
                            lambda s: _abi.int8_linear(o, x, s["w"], scales), alg,
                            iters=20 if M < 4096 else 10, flops=2 * M * N * K,
                            bound="hbm" if M == 16 else "mfma"))
    del W
    # addmv (the GEMV behind mv / matmul(2-D, 1-D)): bf16 [11008, 4096] x [4096]
    # plus a [11008] bias, eight matrices rotated (360 MiB, past the MALL)
    mats = [(torch.randn(N, K, generator=gen) * 0.02).bfloat16().cuda() for _ in range(8)]
    vec = torch.randn(K, generator=gen).bfloat16().cuda()
    vb = torch.randn(N, generator=gen).bfloat16().cuda()
    vo = torch.empty(N, dtype=torch.bfloat16, device="cuda")
    res.append(bench_op(torch, "f2.addmv bf16 [11008,4096] x [4096]", [{"m": m} for m in mats],
                        lambda s: _abi.addmv(vo, vb, s["m"], vec), N * K * 2 + K * 2 + 2 * N * 2,
                        iters=40, flops=2 * N * K, bound="hbm"))
    return res


def other_ops(torch, _abi, synthetic):
    res = config1_ops(torch, _abi, synthetic)
    res.extend(config3_ops(torch, _abi, synthetic))
    res.extend(gemm_ops(torch, _abi))
    res.extend(transfer_ops(torch, _abi))
    res.extend(attention_ops(torch, _abi))
    res.extend(decoder_ops(torch))
    return res


def config1_ops(torch, _abi, synthetic):
    """Config 1: f32 broadcast mul and scalar add [4096, 4096], int64
    index_select of 262144 rows from a [1048576, 8] table."""
    res = []
    log("bench: config 1 ops")
    c1 = synthetic.config1()
    a, b = c1["a"].cuda(), c1["b"].cuda()
    sets = [{"a": a if k == 0 else a.roll(k, 0), "o": torch.empty_like(a)} for k in range(5)]
    res.append(bench_op(torch, "c1.mul [4096,4096]x[4096] f32", sets,
                        lambda s: _abi.mul(s["o"], s["a"], b), 4096 * 4096 * 8 + 4096 * 4))
    res.append(bench_op(torch, "c1.add [4096,4096]+0.5 f32", sets,
                        lambda s: _abi.add(s["o"], s["a"], 0.5), 4096 * 4096 * 8))
    del sets
    table, idx = c1["table"].cuda(), c1["idx"].cuda()
    tsets = [{"t": table if k == 0 else table.roll(k, 0), "o": torch.empty(idx.numel(), 8, dtype=torch.int64, device="cuda")}
             for k in range(8)]
    res.append(bench_op(torch, "c1.index_select int64 [1048576,8] x 262144", tsets,
                        lambda s: _abi.index_select(s["o"], s["t"], 0, idx), 35651584))
    del tsets, table
    return res


def config3_ops(torch, _abi, synthetic):
    """Config 3: RMSNorm, RoPE on q and k, SiLU-mul at the Llama-7B token
    shapes."""
    res = []
    log("bench: config 3 ops")
    c3 = synthetic.config3()
    x, w = c3["x"].cuda(), c3["w"].cuda()
    xs = [{"x": x if k == 0 else x.roll(k, 0), "o": torch.empty_like(x)} for k in range(3)]
    res.append(bench_op(torch, "c3.rms_norm bf16 [16384,4096]", xs,
                        lambda s: _abi.rms_norm(s["o"], s["x"], w, 1e-6), 268443648))
    del xs, x
    q, k, pos = c3["q"].cuda(), c3["k"].cuda(), c3["pos"].cuda()
    # three distinct (q, k) sets (768 MiB of input) rotated, past the MALL
    qs = [{"q": q.roll(j, 0), "k": k.roll(j, 0), "qo": torch.empty_like(q),
           "ko": torch.empty_like(k)} for j in range(3)]
    res.append(bench_op(torch, "c3.rope q,k bf16 [16384,32,128]", qs,
                        lambda s: _abi.rope(s["qo"], s["ko"], s["q"], s["k"], pos, 10000.0),
                        536870912))
    del qs, q, k
    gt, up = c3["gate"].cuda(), c3["up"].cuda()
    gs = [{"g": gt, "u": up, "o": torch.empty_like(gt)}, {"g": up, "u": gt, "o": torch.empty_like(gt)}]
    res.append(bench_op(torch, "c3.silu_mul bf16 [16384,11008]", gs,
                        lambda s: _abi.silu_mul(s["o"], s["g"], s["u"]), 1082130432))
    del gs, gt, up, c3
    return res


def transfer_ops(torch, _abi):
    """The copy and transfer step around the ops: cat (a KV-cache append and
    the rotate-half halves), a dtype-cast and a transposing device copy, and
    host <-> device copies through the gcu device from pinned (caching host
    allocator) and pageable memory."""
    res = []
    log("bench: copy and transfer")
    gen = torch.Generator().manual_seed(20261207)
    B, H, S, D = 8, 32, 2048, 128
    kv = [[torch.randn(B, H, S, D, generator=gen).bfloat16().cuda() for _ in range(2)]
          for _ in range(2)]
    out = torch.empty(B, H, 2 * S, D, dtype=torch.bfloat16, device="cuda")
    res.append(bench_op(torch, "f3.cat bf16 2x[8,32,2048,128] dim 2", [{"x": x} for x in kv],
                        lambda s: _abi.cat(out, s["x"], 2), 2 * out.numel() * 2, iters=20))
    del kv, out
    halves = [[torch.randn(16384 * 32, 64, generator=gen).bfloat16().cuda() for _ in range(2)]
              for _ in range(2)]
    out = torch.empty(16384 * 32, 128, dtype=torch.bfloat16, device="cuda")
    res.append(bench_op(torch, "f3.cat bf16 2x[524288,64] dim -1 (128-byte rows)",
                        [{"x": x} for x in halves], lambda s: _abi.cat(out, s["x"], 1),
                        2 * out.numel() * 2, iters=20))
    del halves, out
    n = 8192
    src = [torch.randn(n, n, generator=gen).cuda() for _ in range(2)]
    o16 = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")
    res.append(bench_op(torch, "f3.copy f32 -> bf16 [8192,8192]", [{"x": x} for x in src],
                        lambda s: _abi.copy_(o16, s["x"]), n * n * 6, iters=20))
    src16 = [x.bfloat16() for x in src]
    del src
    res.append(bench_op(torch, "f3.copy bf16 transpose [8192,8192]", [{"x": x.t()} for x in src16],
                        lambda s: _abi.copy_(o16, s["x"]), n * n * 4, iters=20))
    del src16, o16
    res.extend(host_transfer_ops(torch))
    res.extend(optimizer_ops(torch, _abi))
    res.extend(backward_ops(torch, _abi))
    return res


def backward_ops(torch, _abi):
    """The training-side backward ops at the shapes of configs 2 and 3:
    silu_backward bf16 [16384, 11008], log_softmax backward bf16
    [8192, 32000], layer-norm backward bf16 [16384, 4096] with all three
    gradients (two reads and one write per element, plus the weight and the
    column sums)."""
    log("bench: backward ops")
    gen = torch.Generator().manual_seed(20261209)
    res = []
    M, N = 16384, 11008
    sets = [{"dy": torch.randn(M, N, generator=gen).bfloat16().cuda(),
             "x": torch.randn(M, N, generator=gen).bfloat16().cuda()} for _ in range(2)]
    o = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    res.append(bench_op(torch, "f4.silu_backward bf16 [16384,11008]", sets,
                        lambda s: _abi.silu_backward(o, s["dy"], s["x"]), M * N * 6))
    del sets, o
    M, N = 8192, 32000
    sets = []
    for _ in range(2):
        x = torch.randn(M, N, generator=gen).bfloat16().cuda()
        sets.append({"dy": torch.randn(M, N, generator=gen).bfloat16().cuda(),
                     "y": torch.log_softmax(x.float(), -1).bfloat16()})
        del x
    o = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    res.append(bench_op(torch, "f4.log_softmax_backward bf16 [8192,32000]", sets,
                        lambda s: _abi.log_softmax_backward(o, s["dy"], s["y"], -1), M * N * 6))
    del sets, o
    M, N = 16384, 4096
    w = torch.randn(N, generator=gen).bfloat16().cuda()
    sets = []
    for _ in range(2):
        x = torch.randn(M, N, generator=gen).bfloat16().cuda()
        mean = x.float().mean(-1, keepdim=True)
        rstd = torch.rsqrt(x.float().var(-1, unbiased=False, keepdim=True) + 1e-5)
        sets.append({"dy": torch.randn(M, N, generator=gen).bfloat16().cuda(), "x": x,
                     "mean": mean, "rstd": rstd})
    dx = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    mo = torch.empty(M, 1, dtype=torch.bfloat16, device="cuda")
    ro = torch.empty(M, 1, dtype=torch.bfloat16, device="cuda")
    res.append(bench_op(torch, "f4.layer_norm fwd bf16 [16384,4096] (out, mean, rstd)", sets,
                        lambda s: _abi.layer_norm(dx, mo, ro, s["x"], w, w, N, 1e-5),
                        M * N * 4 + M * 4 + N * 4))
    dw, db = torch.empty_like(w), torch.empty_like(w)
    res.append(bench_op(torch, "f4.layer_norm_backward bf16 [16384,4096] (dx, dgamma, dbeta)", sets,
                        lambda s: _abi.layer_norm_backward(dx, dw, db, s["dy"], s["x"], s["mean"],
                                                           s["rstd"], w, N),
                        M * N * 6 + M * 8 + N * 6))
    return res


def optimizer_ops(torch, _abi):
    """One fused AdamW step over the fp32 parameters of one Llama-7B decoder
    layer (q, k, v, o [4096, 4096], gate and up [11008, 4096], down
    [4096, 11008], two norm weights [4096]: 202 M elements); per element 4
    reads and 3 writes of 4 bytes."""
    log("bench: fused AdamW")
    gen = torch.Generator().manual_seed(20261208)
    shapes = [(4096, 4096)] * 4 + [(11008, 4096)] * 2 + [(4096, 11008), (4096,), (4096,)]
    lists = [[torch.randn(s, generator=gen).cuda() for s in shapes] for _ in range(2)]
    grads = [torch.randn(s, generator=gen).cuda() * 1e-3 for s in shapes]
    m = [torch.zeros(s, device="cuda") for s in shapes]
    v = [torch.zeros(s, device="cuda") for s in shapes]
    steps = [torch.ones((), device="cuda") for _ in shapes]
    n = sum(int(torch.Size(s).numel()) for s in shapes)
    hp = dict(lr=1e-4, beta1=0.9, beta2=0.95, weight_decay=0.1, eps=1e-8)
    return [bench_op(torch, "f4.fused_adamw fp32, one Llama-7B layer (202M params)",
                     [{"p": p} for p in lists],
                     lambda s: _abi.fused_adamw(s["p"], grads, m, v, [], steps, **hp),
                     n * 4 * 7, iters=10)]


def host_transfer_ops(torch, nbytes=256 << 20, iters=8):
    """PCIe copies of 256 MiB through the gcu device: wall time per copy over
    `iters` back-to-back copies (synchronised once), against the published
    PCIe 5.0 x16 rate of the MI355X host link."""
    import torch_gcu  # noqa: F401

    res = []
    n = nbytes // 4
    d = torch.empty(n, device="gcu")
    pinned = torch.randn(n).pin_memory()
    pageable = torch.randn(n)
    back = torch.empty(n, pin_memory=True)
    cases = [("f3.h2d pinned non_blocking 256 MiB", lambda: d.copy_(pinned, non_blocking=True)),
             ("f3.h2d pageable 256 MiB", lambda: d.copy_(pageable)),
             ("f3.d2h pinned non_blocking 256 MiB", lambda: back.copy_(d, non_blocking=True))]
    for name, fn in cases:
        fn()
        torch.gcu.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.gcu.synchronize()
        sec = (time.perf_counter() - t0) / iters
        gbs = nbytes / sec / 1e9
        res.append({"op": name, "ms": round(sec * 1e3, 3), "GB/s": round(gbs, 1),
                    "frac_pcie5_x16": round(gbs / PCIE5_X16_GBS, 4), "alg_bytes": nbytes})
    assert torch.equal(back, pageable), "round trip through the device"
    return res


def attention_ops(torch, _abi):
    """Config 5's attention alone: causal SDPA forward, q/k/v bf16
    [8, 32, 2048, 128], through the flash kernel."""
    log("bench: config 5 attention")
    gen = torch.Generator().manual_seed(20261206)
    B, H, S, D = 8, 32, 2048, 128
    sets = []
    for _ in range(2):
        q, k, v = (torch.randn(B, H, S, D, generator=gen).bfloat16().cuda() for _ in range(3))
        sets.append({"q": q, "k": k, "v": v})
    out = torch.empty(B, H, S, D, dtype=torch.bfloat16, device="cuda")
    flops = 4 * B * H * D * (S * (S + 1) // 2)
    return [bench_op(torch, "c5.sdpa causal bf16 [8,32,2048,128]", sets,
                     lambda s: _abi.flash_attention_fwd(out, None, s["q"], s["k"], s["v"], True),
                     4 * B * H * S * D * 2, iters=10, flops=flops, bound="mfma")]


def decoder_ops(torch, steps=5):
    """Config 5: Llama-7B-shaped decoder layer forward, batch 8 x seq 2048,
    random-init bf16 weights, through the gcu PrivateUse1 ops: eager, then a
    GCUGraph replay of the same layer; tokens/s and allocator peak/reserved."""
    import torch_gcu  # noqa: F401
    from torch_gcu.utils import decoder_layer as dl

    log("bench: config 5 decoder layer")
    cfg = dl.LayerConfig()
    B, S = 8, 2048
    w = {k: v.to("gcu") for k, v in dl.init_weights(cfg).items()}
    gen = torch.Generator().manual_seed(20261205)
    ids = torch.randint(0, cfg.vocab, (B, S), generator=gen).to("gcu")
    pos = dl.positions(B, S, "gcu")
    flops = dl.flops(cfg, B, S)
    for _ in range(4):  # about 25 ms of warm-up: the sustained clock of matrix work
        dl.forward(w, ids, cfg, pos)
    torch.gcu.synchronize()
    torch.gcu.reset_peak_memory_stats()
    t0 = time.perf_counter()
    for _ in range(steps):
        dl.forward(w, ids, cfg, pos)
    torch.gcu.synchronize()
    eager_s = (time.perf_counter() - t0) / steps
    peak = torch.gcu.max_memory_allocated()
    reserved = torch.gcu.memory_reserved()
    graph = torch.gcu.GCUGraph()
    with torch.gcu.graph(graph):
        dl.forward(w, ids, cfg, pos)
    # the same warm-up as eager: the capture leaves the GPU idle and the clock
    # falls; a kernel trace showed the first replays at 7.98, 7.22, 6.79 ms
    # and eager's first passes at 7.58, 7.23, 6.95 ms before both settle
    for _ in range(4):
        graph.replay()
    torch.gcu.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.gcu.synchronize()
    graph_s = (time.perf_counter() - t0) / steps
    graph.reset()
    tokens = B * S
    out = []
    for name, sec in [("eager", eager_s), ("gcugraph replay", graph_s)]:
        tf = flops / sec / 1e12
        out.append({"op": f"c5.decoder_layer fwd B8xS2048 ({name})", "ms": round(sec * 1e3, 3),
                    "tok/s": round(tokens / sec, 1), "TFLOP/s": round(tf, 1),
                    "frac_mfma_bf16": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "flops": flops,
                    "alloc_peak_bytes": peak, "alloc_reserved_bytes": reserved})
    return out


SECTIONS = {
    "config1": lambda torch, _abi: config1_ops(torch, _abi, _synthetic()),
    "config3": lambda torch, _abi: config3_ops(torch, _abi, _synthetic()),
    "gemm": lambda torch, _abi: gemm_ops(torch, _abi),
    "attention": lambda torch, _abi: attention_ops(torch, _abi),
    "transfer": lambda torch, _abi: transfer_ops(torch, _abi),
    "backward": lambda torch, _abi: backward_ops(torch, _abi),
    "decoder": lambda torch, _abi: decoder_ops(torch),
}


def _synthetic():
    from torch_gcu.utils import synthetic

    return synthetic


def run_section(name):
    import torch

    from torch_gcu import _abi

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.init()
    _abi.install_workspace()
    import torch_gcu  # noqa: F401

    # one plain 512 MiB device copy (untimed): under rocprofv3 --pmc its
    # FETCH_SIZE / WRITE_SIZE calibrate the counters against known bytes
    cal = torch.empty(CAL_COPY_BYTES // 2, dtype=torch.int16, device="cuda")
    _abi.copy_(torch.empty_like(cal), cal)
    del cal
    for r in SECTIONS[name](torch, _abi):
        print(json.dumps(r), flush=True)
    return 0


def main():
    args = parse()
    if args.section:
        return run_section(args.section)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); every GPU box "
              "in this setup has one MI355X.  Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch

    from torch_gcu import _abi
    from torch_gcu.utils import synthetic

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.init()
    _abi.install_workspace()
    props = torch.cuda.get_device_properties(0)
    log(f"bench: device {props.name}, {props.multi_processor_count} CUs")

    import torch_gcu  # noqa: F401  (the gcu device for the dispatcher path)

    wall, wall_abi, host_us, per_op_ms = run_config2(torch, _abi, synthetic, args.steps,
                                                     args.warmup)
    ab = config2_alg_bytes()
    total_bytes = sum(ab.values())
    ms_per_step = wall * 1e3 / args.steps
    value = total_bytes / (wall / args.steps) / 1e9
    ls_ms = per_op_ms["log_softmax"]
    achieved = ab["log_softmax"] / (ls_ms * 1e-3) / 1e9
    per_op = {k: {"ms": round(v, 4), "GB/s": round(ab[k] / (v * 1e-3) / 1e9, 1),
                  "frac_hbm": round(ab[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
              for k, v in per_op_ms.items()}
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded CPU generators of BASELINE config 2, copied to HBM)",
        "config": {"workload": "config2: sum/amax/log_softmax over bf16 [8192,32000] + "
                               "mean(0) over fp32 [16384,4096]",
                   "path": "torch.sum/amax/log_softmax/mean on gcu tensors (PrivateUse1 "
                           "dispatcher -> generated wrappers -> C ABI -> gfx950 kernels)",
                   "alg_bytes_per_step": total_bytes, "per_op": per_op,
                   "c_abi_ms_per_step": round(wall_abi * 1e3 / args.steps, 4),
                   "host_us_per_dispatched_op": round(host_us, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": committed_traffic(),
                     "traffic_source": "profiles/log_softmax_config2_traffic.md (rocprofv3 "
                                       "FETCH_SIZE + WRITE_SIZE, scaled by a 512 MiB copy)",
                     "kernel": "softmax_reg_kernel (log_softmax)",
                     "alg_bytes_per_launch": ab["log_softmax"],
                     "avg_launch_ms": round(ls_ms, 4)},
    }
    if not args.no_ops:
        line["ops"] = other_ops(torch, _abi, synthetic)
    if not args.no_cpu:
        log("bench: CPU baseline")
        line["cpu_baseline"] = cpu_baseline(torch, synthetic, args.cpu_seconds)
        if not args.no_ops:
            cpu_ops = cpu_config_ops(torch, synthetic)
            for r in line["ops"]:
                if r["op"] in cpu_ops:
                    r["cpu_aten"] = cpu_ops[r["op"]]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
