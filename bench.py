"""Benchmark of the Q4_G64 path on one MI355X.

Headline (`value`): the fused Qwen2.5-3B-shaped MLP decode step of config 1 at
B = 1 -- h += down(silu(gate h) * up h) with gate/up [11008, 2048] and down
[2048, 11008] Q4_G64 -- as algorithmic HBM GB/s: (3 x 12,681,216 B of weights
+ 8,192 B of h) per step / time per step.  Steps rotate over distinct weight
copies totalling > 1 GB so that the 256 MB MALL cannot serve them; the step
sequence is captured once in a HIP graph and replayed.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
       python bench.py --profile prefill|few|gemv   (short eager run for rocprofv3 counter passes)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "kriya-rt_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "Q4 GEMV HBM GB/s (% of peak); decode tok/s @3B shape; prefill GEMM MFMA util"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16/fp16
Q4_BYTES = lambda n, k: n * k // 2 + n * (k // 64) * 4  # noqa: E731  nibbles + bf16 scale + bf16 bias


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Rotation:
    """`copies` distinct device copies of a list of Q4 weights (copy 0 = the seeded data)."""

    def __init__(self, kq, torch, planars, copies):
        self.sets = []
        base = [kq.Q4Matrix.from_numpy(*p) for p in planars]
        gen = torch.Generator(device="cuda")
        gen.manual_seed(1234)
        for c in range(copies):
            if c == 0:
                self.sets.append(base)
                continue
            ms = []
            for b in base:
                qw = torch.randint(-(2 ** 31), 2 ** 31 - 1, b.qw.shape, dtype=torch.int32, device="cuda",
                                   generator=gen)
                ms.append(kq.Q4Matrix(qw, b.scales.clone(), b.biases.clone()))
            self.sets.append(ms)

    def __len__(self):
        return len(self.sets)


def graph_time_per_step(torch, fn, nsteps, replays, warmup_replays=2):
    """Capture fn(i) for i < nsteps in one HIP graph; return seconds per step over `replays` replays."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(min(nsteps, 3)):  # eager warm-up outside capture
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(nsteps):
            fn(i)
    for _ in range(warmup_replays):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e-3 / (replays * nsteps)


# A bounded spin kernel (torch.cuda._sleep) holds the stream while the host enqueues a chain of launches, so the
# GPU then runs them back to back with no host gaps.  ~50 M shader cycles is ~20 ms at MI355X clocks, far more than
# the host needs to enqueue CHAIN_LAUNCHES launches (longer chains hold proportionally longer).
HOLD_CYCLES = 50_000_000
CHAIN_LAUNCHES = 640  # launches per timed chain (the host queues them in a few ms)


def chain_time_per_launch(torch, fn, n, reps=3):
    """Average duration of one launch of fn(i): n eager launches fn(0) .. fn(n - 1) are queued behind a bounded spin
    kernel and bracketed by two HIP events on the launch stream; the median over `reps` chains of elapsed / n.
    rocprofv3 --kernel-trace reports the same average duration for the kernel (within ~1 %), whereas replays of a
    HIP graph of the chain run a few per cent apart from it.  A chain whose hold ended before the host had queued
    it is run again behind a hold twice as long (up to 16x: a profiler slows the host's launches several-fold).
    Returns (seconds per launch, starved) where starved is True if a chain was still not fully queued when its
    hold ended (then host gaps may be included)."""
    for i in range(min(n, 3)):
        fn(i)
    torch.cuda.synchronize()
    times, starved = [], False
    hold = HOLD_CYCLES * max(1, -(-n // CHAIN_LAUNCHES))
    for _ in range(reps):
        for attempt in range(5):  # a slow host (e.g. under a profiler) gets a longer hold, up to 16x
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(hold)
            a.record()
            for i in range(n):
                fn(i)
            b.record()
            short = a.query()  # the hold already ended: the GPU may have waited for the host
            torch.cuda.synchronize()
            if not short or attempt == 4:
                break
            hold *= 2
        starved |= short
        times.append(a.elapsed_time(b) * 1e-3 / n)
    return float(np.median(times)), starved


def graph_time_exact(torch, fn, steps, warmup):
    """The contract's timed region: `warmup` untimed steps, then EXACTLY `steps` steps fn(0) .. fn(steps - 1)
    captured in one HIP graph and replayed once, bracketed by device synchronisations.  Returns seconds per
    step."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(max(warmup, 1)):  # eager warm-up outside capture
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    g.replay()  # the first replay uploads the graph: untimed
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e-3 / steps


def bench_mlp(kq, torch, synth, B, copies, steps, warmup):
    """Config 1: fused MLP decode at batch B.  Returns a dict of measurements."""
    H, I = synth.HIDDEN, synth.INTER
    planars = [synth.q4_weight(I, H, 1001), synth.q4_weight(I, H, 1002), synth.q4_weight(H, I, 1003)]
    rot = Rotation(kq, torch, planars, copies)
    h = torch.from_numpy(synth.bf16_normal((B, H), 1010 + B).view(np.int16)).cuda().view(torch.bfloat16)
    ws = kq.mlp_workspace(B, H, I)
    xs = h.clone()  # MLP input (bf16); h is the residual stream updated in place

    def step(i):
        g, u, d = rot.sets[i % len(rot)]
        kq.mlp(g, u, d, h, x=xs, workspace=ws)

    nsteps = len(rot)
    replays = max(1, steps // nsteps)
    warm = max(1, warmup // nsteps)
    t_step = graph_time_exact(torch, step, steps, warmup)  # exactly `steps` steps in the timed region
    weight_bytes = 3 * Q4_BYTES(I, H)
    alg_bytes = weight_bytes + 2 * 2 * B * H  # weights + h read + h write
    out = {"B": B, "s_per_step": t_step, "alg_bytes": alg_bytes, "gbs": alg_bytes / t_step / 1e9, "steps": steps}

    # per-kernel average durations (each kernel alone over the rotating copies, as an eager chain behind a hold)
    act = torch.empty((B, I), dtype=torch.bfloat16, device="cuda")

    def gate_up(i):
        g, u, _ = rot.sets[i % len(rot)]
        kq.gate_up_act(g, u, xs, out=act)

    def down(i):
        _, _, d = rot.sets[i % len(rot)]
        kq.q4_linear(d, act, y=h, accumulate=True)

    chain = max(steps, CHAIN_LAUNCHES)
    t_gu, st_gu = chain_time_per_launch(torch, gate_up, chain)
    out["kernels"] = {"gate_up_act": {"s": t_gu, "alg_bytes": 2 * Q4_BYTES(I, H) + 2 * B * H + 2 * B * I,
                                      "graph_s": graph_time_per_step(torch, gate_up, nsteps, replays, warm),
                                      "starved": st_gu}}
    if B == 1:  # m = 1: the down projection is one launch of its own (the GEMV with accumulate)
        t_dn, st_dn = chain_time_per_launch(torch, down, chain)
        out["kernels"]["down_acc"] = {"s": t_dn, "alg_bytes": Q4_BYTES(H, I) + 2 * B * I + 4 * B * H,
                                      "graph_s": graph_time_per_step(torch, down, nsteps, replays, warm),
                                      "starved": st_dn}
    for k in out["kernels"].values():
        k["gbs"] = k["alg_bytes"] / k["s"] / 1e9
    return out


def bench_mlp_tp_share(kq, torch, synth, B, tp, copies, steps, warmup):
    """One GPU's share of config 1's MLP under tp-way tensor parallelism: gate/up rows [0, I/tp) (column-
    parallel) and the down projection's K columns [0, I/tp) (row-parallel, whole 64-groups), the share's f32
    partial [B, H] accumulated into a buffer the all-reduce would sum.  Exactly `steps` steps in one graph, as
    the headline; the all-reduce itself is not run (one GPU)."""
    H, I = synth.HIDDEN, synth.INTER
    Is = I // tp
    assert Is % 64 == 0, "shards must be whole 64-groups"
    g, u, d = synth.q4_weight(I, H, 1001), synth.q4_weight(I, H, 1002), synth.q4_weight(H, I, 1003)
    rows = lambda p: tuple(np.ascontiguousarray(a[:Is]) for a in p)  # noqa: E731
    cols = (np.ascontiguousarray(d[0][:, :Is // 8]), np.ascontiguousarray(d[1][:, :Is // 64]),
            np.ascontiguousarray(d[2][:, :Is // 64]))
    rot = Rotation(kq, torch, [rows(g), rows(u), cols], copies)
    x = torch.from_numpy(synth.bf16_normal((B, H), 1010 + B).view(np.int16)).cuda().view(torch.bfloat16)
    part = torch.zeros((B, H), dtype=torch.float32, device="cuda")
    ws = kq.mlp_workspace(B, H, Is)

    def step(i):
        gs, us, ds = rot.sets[i % len(rot)]
        kq.mlp(gs, us, ds, part, x=x, workspace=ws)

    t = graph_time_exact(torch, step, steps, warmup)
    alg = 3 * Q4_BYTES(Is, H) + 2 * B * H + 2 * 4 * B * H  # weights + x + the f32 partial read and written
    return {"tp": tp, "B": B, "gate_up_rows": Is, "down_k": Is, "step_us": round(t * 1e6, 3),
            "alg_bytes": alg, "gbs": round(alg / t / 1e9, 1), "frac_hbm": round(alg / t / 1e9 / HBM_PEAK_GBS, 4)}


def stream_floor(kq, torch, nbytes, copies, steps, warmup):
    """Seconds per plain read of nbytes (kr_stream_read: one 16-byte non-temporal load per thread) over
    `copies` rotating buffers, timed like the kernels: the floor for a read of that size on this GPU."""
    n = (nbytes + 15) // 16 * 16
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    bufs = [torch.randint(-(2 ** 31), 2 ** 31 - 1, (n // 4,), dtype=torch.int32, device="cuda", generator=gen)
            for _ in range(copies)]
    hits = torch.zeros(int(kq.lib().kr_stream_read_pieces(n)), dtype=torch.int32, device="cuda")

    def rd(i):
        kq.stream_read(bufs[i % copies], hits=hits)

    t, _ = chain_time_per_launch(torch, rd, max(steps, CHAIN_LAUNCHES))
    del bufs
    return t


def bench_gemv_cfg0(kq, torch, synth, copies, steps, warmup):
    N, K = 11008, 2048
    rot = Rotation(kq, torch, [synth.q4_weight(N, K, 0)], copies)
    x = torch.from_numpy(synth.bf16_normal((1, K), 1).view(np.int16)).cuda().view(torch.bfloat16)
    y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")

    def step(i):
        kq.q4_linear(rot.sets[i % len(rot)][0], x, y=y)

    nsteps = len(rot)
    t = graph_time_per_step(torch, step, nsteps, max(1, steps // nsteps), max(1, warmup // nsteps))
    alg = Q4_BYTES(N, K) + 2 * K + 2 * N
    return {"s_per_step": t, "alg_bytes": alg, "gbs": alg / t / 1e9, "problems": nsteps}


def bench_prefill_cfg2(kq, torch, synth, copies, steps):
    """Config 2: the seven projections of one layer at M = 512: q/k/v in one launch, o accumulated into the
    residual, and the MLP entry point (gate/up + SwiGLU, then down accumulated into the residual)."""
    M, H, I, KV = 512, 2048, 11008, 256
    shapes = [(H, H), (KV, H), (KV, H), (H, H), (I, H), (I, H), (H, I)]  # q k v o gate up down
    planars = [synth.q4_weight(n, k, 2000 + i) for i, (n, k) in enumerate(shapes)]
    rot = Rotation(kq, torch, planars, copies)
    x = torch.from_numpy(synth.bf16_normal((M, H), 2100).view(np.int16)).cuda().view(torch.bfloat16)
    qo = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    ko = torch.empty((M, KV), dtype=torch.bfloat16, device="cuda")
    vo = torch.empty((M, KV), dtype=torch.bfloat16, device="cuda")
    h = x.clone()  # residual stream: the o and down projections accumulate into it, as in a layer
    ws = kq.mlp_workspace(M, H, I)

    def layer(i):
        q, k, v, o, g, u, d = rot.sets[i % len(rot)]
        kq.qkv(q, k, v, x, out_dtype=kq.DTYPE_BF16, outs=(qo, ko, vo))
        kq.q4_linear(o, x, y=h, accumulate=True)
        kq.mlp(g, u, d, h, x=x, workspace=ws)  # gate/up + SwiGLU, then down into h (split K via the workspace)

    t = graph_time_per_step(torch, layer, len(rot), max(1, steps // (8 * len(rot))), 1)
    flops = sum(2 * M * n * k for n, k in shapes)
    tflops = flops / t / 1e12
    return {"us": round(t * 1e6, 2), "tflops": round(tflops, 1), "mfma_util": round(tflops / MFMA_PEAK_TFLOPS, 4),
            "flops_per_layer": flops, "m": M}


def bench_decode_cfg3(torch, B, steps):
    """Config 3: one greedy decode step of the 36-layer model at context 512, batch B."""
    from kriya_q4.qwen_decode import QWEN25_3B, QwenQ4Decoder
    m = QwenQ4Decoder(QWEN25_3B, batch=B, ctx=512, seed=3000 + B)
    nsteps = 4
    t = graph_time_per_step(torch, lambda i: m.step(), nsteps, max(1, steps // nsteps), 1)
    bytes_step = QWEN25_3B.q4_bytes_per_step() + B * 36 * 513 * 2 * 256 * 2  # weights + KV read
    out = {"B": B, "step_us": round(t * 1e6, 1), "tok_s": round(B / t, 1),
           "gbs": round(bytes_step / t / 1e9, 1), "frac_hbm": round(bytes_step / t / 1e9 / HBM_PEAK_GBS, 4)}
    del m
    torch.cuda.empty_cache()
    return out


def bench_moe_cfg4(kq, torch, synth, copies, steps):
    """Config 4: one MoE layer (60 experts, top-4, hidden 2048, inter 1408) at T = 1 and T = 64."""
    E, K, H, I = 60, 4, 2048, 1408
    planars = [synth.q4_weight(E * I, H, 4001), synth.q4_weight(E * I, H, 4002), synth.q4_weight(E * H, I, 4003)]
    rot = Rotation(kq, torch, planars, copies)
    res = {}
    for T in (1, 64):
        x = torch.from_numpy(synth.bf16_normal((T, H), 4004).view(np.int16)).cuda().view(torch.bfloat16)
        logits = torch.from_numpy(synth.f32_normal((T, E), 4005)).cuda()
        r = kq.MoeRoute(T, E, K)
        ws = kq.moe_workspace(T, K, H, I)
        y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        kq.moe_route(logits, K, True, out=r)
        torch.cuda.synchronize()
        active = int((r.counts > 0).sum().item())

        def step(i):  # routing from the logits, then the experts (kr_q4_moe_route_experts)
            g, u, d = rot.sets[i % len(rot)]
            kq.moe_route_experts(g, u, d, E, x, logits, K, True, out=r, y=y, workspace=ws)

        def experts(i):
            g, u, d = rot.sets[i % len(rot)]
            kq.moe_experts(g, u, d, E, x, r, y=y, workspace=ws)

        t = graph_time_per_step(torch, step, len(rot), max(1, steps // (4 * len(rot))), 1)
        te = graph_time_per_step(torch, experts, len(rot), max(1, steps // (4 * len(rot))), 1)
        wbytes = active * 3 * Q4_BYTES(I, H)
        res[f"T{T}"] = {"active_experts": active, "step_us": round(t * 1e6, 2), "experts_us": round(te * 1e6, 2),
                        "tok_s": round(T / t, 1), "experts_gbs": round(wbytes / te / 1e9, 1),
                        "experts_frac_hbm": round(wbytes / te / 1e9 / HBM_PEAK_GBS, 4),
                        "tflops": round(2 * T * K * 3 * I * H / te / 1e12, 2)}
    return res


def host_cores():
    """(os.cpu_count(), CPUs this process may run on)."""
    n = os.cpu_count() or 1
    try:
        return n, len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return n, n


def _median_time(fn, budget_s, min_runs=10, warm=3):
    """3 warm-up calls, then at least `min_runs` timed calls and at least `budget_s` seconds; median."""
    for _ in range(warm):
        fn()
    times = []
    t0 = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t0 < budget_s and len(times) < 10000):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return float(np.median(times)), len(times), time.perf_counter() - t0


def cpu_baseline(synth, budget_s=3.0):
    """The reference CPU path as its tests define it -- dequantize_q4_group64_to_f32 (quantizer.rs:112-126),
    then a sequential f32 dot per row (test_shader_compile.rs:592-595) -- restated in C (oracle/kr_oracle.c),
    timed on this host: config 1 B = 1 (the headline's unit) and config 0, on the CPUs this process may use
    (at most 16, the CPU share of one GPU on the box) and on one core, plus the upper bound that dots
    weights dequantised once beforehand."""
    import oracle

    nproc, aff = host_cores()
    threads = max(1, min(aff, 16))
    H, I = synth.HIDDEN, synth.INTER
    variants = {}
    # config 0: one GEMV 11008 x 2048
    W0 = oracle.Q4Planar(*synth.q4_weight(11008, 2048, 0))
    x0 = synth.bf16_normal((1, 2048), 1)
    b0 = Q4_BYTES(11008, 2048) + 2 * 2048 + 2 * 11008
    for name, th in (("cfg0_faithful", threads), ("cfg0_faithful_1core", 1)):
        med, n, el = _median_time(lambda: oracle.q4_matmul(W0, x0, threads=th), budget_s)
        variants[name] = {"us": round(med * 1e6, 1), "gbs": round(b0 / med / 1e9, 3), "threads": th, "runs": n,
                          "seconds": round(el, 1)}
    w0f = oracle.dequant_planar(W0)
    x0f = oracle.bf16_to_f32(x0)
    med, n, el = _median_time(lambda: oracle.f32_matmul(w0f, x0f, threads=threads), budget_s)
    variants["cfg0_predequantised_upper_bound"] = {"us": round(med * 1e6, 1), "gbs": round(b0 / med / 1e9, 3),
                                                   "threads": threads, "runs": n, "seconds": round(el, 1),
                                                   "note": "dot only; bytes counted as Q4 for comparison"}
    del w0f
    # config 1 B = 1: the fused MLP step (the headline workload)
    g = oracle.Q4Planar(*synth.q4_weight(I, H, 1001))
    u = oracle.Q4Planar(*synth.q4_weight(I, H, 1002))
    d = oracle.Q4Planar(*synth.q4_weight(H, I, 1003))
    x = synth.bf16_normal((1, H), 1011)
    alg = 3 * Q4_BYTES(I, H) + 4 * H
    med, n, el = _median_time(lambda: oracle.q4_mlp(g, u, d, x, threads=threads), 2 * budget_s)
    variants["cfg1_B1_faithful"] = {"us": round(med * 1e6, 1), "gbs": round(alg / med / 1e9, 3), "threads": threads,
                                    "runs": n, "seconds": round(el, 1)}
    total = sum(v["seconds"] for v in variants.values())
    return {"value": variants["cfg1_B1_faithful"]["gbs"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"cfg1 B=1 MLP step, median of {variants['cfg1_B1_faithful']['runs']} calls "
                      f"({variants['cfg1_B1_faithful']['seconds']} s): dequantize_q4_group64_to_f32 + sequential "
                      f"f32 dot, C restatement (oracle/kr_oracle.c) on {threads} threads; {total:.1f} s of CPU "
                      f"timing in all variants",
            "host_nproc": nproc, "host_affinity_cpus": aff, "variants": variants}


def measured_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE runs scaled by a plain copy's counters), or None."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic_q4_gemv_cfg1_B1.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch="):
                return int(line.split("=", 1)[1])
    except OSError:
        pass
    return None


def copy_calibration(torch):
    """A plain device copy of known size (4 x 256 MiB) to scale the PMC byte counters."""
    a = torch.empty(256 * 1024 * 1024 // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    log("copied 4 x 256 MiB")


def profile_run(kq, torch, synth, what, reps=8):
    """Short eager runs for rocprofv3 counter passes (--profile): each workload's launches `reps` times on two
    weight copies (few dispatches, so every counter pass stays short).
      prefill: cfg2's layer at M = 512 (q/k/v in one launch, o accumulated, gate/up + SwiGLU, split-K down);
      few:     cfg1's MLP at B = 16 (few-token gate/up, down with the in-launch split-K reduction) and cfg4's
               grouped experts at T = 64;
      gemv:    cfg1's MLP at B = 1 (the headline kernels) and cfg0's GEMV."""
    H, I, KV = synth.HIDDEN, synth.INTER, 256
    if what == "prefill":
        M = 512
        shapes = [(H, H), (KV, H), (KV, H), (H, H), (I, H), (I, H), (H, I)]
        rot = Rotation(kq, torch, [synth.q4_weight(n, k, 2000 + i) for i, (n, k) in enumerate(shapes)], 2)
        x = torch.from_numpy(synth.bf16_normal((M, H), 2100).view(np.int16)).cuda().view(torch.bfloat16)
        qo = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        ko = torch.empty((M, KV), dtype=torch.bfloat16, device="cuda")
        vo = torch.empty_like(ko)
        h = x.clone()
        ws = kq.mlp_workspace(M, H, I)
        for i in range(reps):
            q, k, v, o, g, u, d = rot.sets[i % 2]
            kq.qkv(q, k, v, x, out_dtype=kq.DTYPE_BF16, outs=(qo, ko, vo))
            kq.q4_linear(o, x, y=h, accumulate=True)
            kq.mlp(g, u, d, h, x=x, workspace=ws)
    elif what in ("few", "gemv"):
        B = 16 if what == "few" else 1
        rot = Rotation(kq, torch, [synth.q4_weight(I, H, 1001), synth.q4_weight(I, H, 1002),
                                   synth.q4_weight(H, I, 1003)], 2)
        h = torch.from_numpy(synth.bf16_normal((B, H), 1010 + B).view(np.int16)).cuda().view(torch.bfloat16)
        xs = h.clone()
        ws = kq.mlp_workspace(B, H, I)
        for i in range(reps):
            g, u, d = rot.sets[i % 2]
            kq.mlp(g, u, d, h, x=xs, workspace=ws)
        if what == "gemv":  # config 0: one GEMV 11008 x 2048 into bf16
            rot0 = Rotation(kq, torch, [synth.q4_weight(11008, 2048, 0)], 2)
            x0 = torch.from_numpy(synth.bf16_normal((1, 2048), 1).view(np.int16)).cuda().view(torch.bfloat16)
            y0 = torch.empty((1, 11008), dtype=torch.bfloat16, device="cuda")
            for i in range(reps):
                kq.q4_linear(rot0.sets[i % 2][0], x0, y=y0)
        if what == "few":
            E, K, T, Im = 60, 4, 64, 1408
            mrot = Rotation(kq, torch, [synth.q4_weight(E * Im, H, 4001), synth.q4_weight(E * Im, H, 4002),
                                        synth.q4_weight(E * H, Im, 4003)], 2)
            x = torch.from_numpy(synth.bf16_normal((T, H), 4004).view(np.int16)).cuda().view(torch.bfloat16)
            logits = torch.from_numpy(synth.f32_normal((T, E), 4005)).cuda()
            r = kq.moe_route(logits, K, True)
            y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
            mws = kq.moe_workspace(T, K, H, Im)
            for i in range(reps):
                g, u, d = mrot.sets[i % 2]
                kq.moe_experts(g, u, d, E, x, r, y=y, workspace=mws)
    else:
        raise SystemExit(f"--profile: unknown workload {what!r} (prefill, few, gemv)")
    torch.cuda.synchronize()
    log(f"profile run '{what}' done ({reps} repetitions)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--copies", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 4 x 256 MiB device copy (PMC byte-counter calibration)")
    ap.add_argument("--profile", choices=["prefill", "few", "gemv"],
                    help="only a short eager run of one workload, for rocprofv3 counter passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              f"(multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)

    import torch

    import kriya_q4 as kq
    from kriya_q4 import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.calibrate_copy:
        copy_calibration(torch)
        return
    kq.lib()
    if args.profile:
        profile_run(kq, torch, synth, args.profile)
        return
    log(f"device {torch.cuda.get_device_name(0)}")

    log("cfg1 B=1 (headline)")
    head = bench_mlp(kq, torch, synth, 1, args.copies, args.steps, args.warmup)
    dom = head["kernels"]["gate_up_act"]
    result = {
        "metric": METRIC,
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(head["s_per_step"] * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_g64 weights x bf16 activations, f32 accumulation",
        "data": f"synthetic: seeded SplitMix64 weights (config-0 distribution), {args.copies} rotating weight "
                f"copies ({args.copies * 3 * Q4_BYTES(11008, 2048) / 1e9:.2f} GB) so HBM, not MALL, serves them",
        "config": {"workload": "cfg1_fused_mlp_decode_B1", "hidden": 2048, "intermediate": 11008, "batch": 1,
                   "weights": "Q4_G64 gate/up [11008,2048], down [2048,11008]",
                   "launches_per_step": 2, "graph": "HIP graph replay"},
        "roofline": {"bound": "hbm",
                     "kernel": "kr::q4_gemv_wave_kernel<2, 1, 5, false, false> (gate+up+SiLU fused, m=1)",
                     "achieved": round(dom["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": "profiles/pmc_traffic_q4_gemv_cfg1_B1.md (rocprofv3 FETCH_SIZE/WRITE_SIZE, "
                                       "copy-calibrated)",
                     "alg_bytes_per_launch": dom["alg_bytes"], "avg_launch_us": round(dom["s"] * 1e6, 3),
                     "timing": "HIP events around an eager chain of launches over the rotating copies, queued "
                               "behind a bounded spin kernel (the duration rocprofv3 --kernel-trace reports)",
                     "chain_starved": dom["starved"],
                     "graph_interval_us": round(dom["graph_s"] * 1e6, 3)},
        "cpu_baseline": None,
    }
    log("streaming floor (plain reads of the same byte counts)")
    floors = {k: stream_floor(kq, torch, v["alg_bytes"], args.copies, args.steps, args.warmup)
              for k, v in head["kernels"].items()}
    result["roofline"]["stream_floor_us"] = round(floors["gate_up_act"] * 1e6, 3)
    result["roofline"]["frac_of_stream_floor"] = round(floors["gate_up_act"] / dom["s"], 4)
    extra = {"cfg1_B1": {"step_us": round(head["s_per_step"] * 1e6, 3), "gbs": round(head["gbs"], 1),
                         "frac_hbm": round(head["gbs"] / HBM_PEAK_GBS, 4),
                         "kernels_us": {k: round(v["s"] * 1e6, 3) for k, v in head["kernels"].items()},
                         "kernels_graph_interval_us": {k: round(v["graph_s"] * 1e6, 3)
                                                       for k, v in head["kernels"].items()},
                         "kernels_gbs": {k: round(v["gbs"], 1) for k, v in head["kernels"].items()},
                         "stream_floor_us": {k: round(v * 1e6, 3) for k, v in floors.items()}}}
    if not args.quick:
        log("cfg0 GEMV")
        g0 = bench_gemv_cfg0(kq, torch, synth, args.copies * 3, args.steps, args.warmup)
        extra["cfg0_gemv"] = {"us": round(g0["s_per_step"] * 1e6, 3), "gbs": round(g0["gbs"], 1),
                              "frac_hbm": round(g0["gbs"] / HBM_PEAK_GBS, 4)}
        result["sustained"] = {"what": f"cfg0 GEMV over {g0['problems']} distinct weight matrices in one HIP graph "
                                       f"(sum of algorithmic bytes / wall time)", "problems": g0["problems"],
                               "gbs": round(g0["gbs"], 1), "frac_hbm": round(g0["gbs"] / HBM_PEAK_GBS, 4)}
        for B in (4, 16):
            log(f"cfg1 B={B}")
            r = bench_mlp(kq, torch, synth, B, args.copies, args.steps, args.warmup)
            gu = r["kernels"]["gate_up_act"]["s"]
            extra[f"cfg1_B{B}"] = {"step_us": round(r["s_per_step"] * 1e6, 3), "gbs": round(r["gbs"], 1),
                                   "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4),
                                   "tok_s": round(B / r["s_per_step"], 1),
                                   "kernels_us": {"gate_up_act": round(gu * 1e6, 3),
                                                  "down_acc (step - gate_up)": round((r["s_per_step"] - gu) * 1e6, 3)}}
        log("cfg1 one GPU's share under 4-way tensor parallelism")
        extra["cfg1_tp4_share"] = {f"B{B}": bench_mlp_tp_share(kq, torch, synth, B, 4, args.copies * 4,
                                                                 args.steps, args.warmup) for B in (1, 16)}
        log("cfg2 prefill M=512")
        extra["cfg2_prefill_M512"] = bench_prefill_cfg2(kq, torch, synth, 24, args.steps)  # 24 x 43.4 MB
        log("cfg4 MoE")
        extra["cfg4_moe"] = bench_moe_cfg4(kq, torch, synth, 4, args.steps)
        for B in (1, 16):
            log(f"cfg3 decode B={B}")
            extra[f"cfg3_decode_B{B}"] = bench_decode_cfg3(torch, B, min(args.steps, 200))
    result["extra"] = extra
    if not args.no_cpu:
        log("cpu baseline (oracle: cfg0 and cfg1 B=1, all allowed cores and one core, pre-dequantised bound)")
        result["cpu_baseline"] = cpu_baseline(synth)
        result["cpu_baseline"]["gpu_over_cpu"] = round(result["value"] / result["cpu_baseline"]["value"], 1)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
