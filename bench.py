#!/usr/bin/env python3
"""Benchmark of the engine-mlx attention hot path on one MI355X.

Headline workload (the metric's decode half): Qwen3-8B-shape batched decode
step, batch 32, 32 query / 8 KV heads, head_dim 128, bf16 static cache of
capacity 8192 per sequence, valid lengths uniform in [512, 8192] (seed 1234).
One step = the pre-attention for one new token per sequence (q/k RMSNorm,
RoPE, K/V written at offset len-1) and decode attention over len positions,
issued as one fused ema_decode_step call. value = algorithmic bytes of the
step / step time.

The other shapes are measured after it and reported under "secondary"
(prefill TFLOP/s for the metric's prefill half, the remaining configurations).
Inputs are synthetic (seeded normal), already resident in HBM.

python bench.py [--steps K] [--warmup W] [--only primary] [--no-cpu-baseline] [--calibrate-copy]

--calibrate-copy first copies 1 GiB device-to-device (torch), so a FETCH_SIZE /
WRITE_SIZE counter profile of the same command holds a copy kernel of known
size to scale the counters by.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "engine-mlx_amd"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
METRIC = "decode attn GB/s (% of 8 TB/s) + prefill attn TFLOP/s, Qwen3-8B shapes"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--only", choices=["all", "primary", "prefill", "decode_long", "decode_b1", "prefill_chunk", "fp8",
                                      "fp8_tail", "fp8_prefill", "int4", "gdn", "gdn_step", "qmm", "prefill_1p7b",
                                      "pre"],
                   default="all")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--calibrate-copy", action="store_true")
    return p.parse_args()


class Ctx:
    def __init__(self):
        import torch

        self.torch = torch
        self.dev = torch.device("cuda:0")
        self.gen = torch.Generator(device=self.dev)
        self.gen.manual_seed(2024)

    def randn(self, shape, mean=0.0, std=1.0):
        t = self.torch.randn(shape, generator=self.gen, device=self.dev, dtype=self.torch.float32)
        return (t * std + mean).to(self.torch.bfloat16)

    def i32(self, values):
        return self.torch.tensor(list(map(int, values)), dtype=self.torch.int32, device=self.dev)


def time_calls(torch, fn, steps, warmup):
    """Average ms per call of fn(): `steps` calls captured in one HIP graph; the graph is
    replayed for about half a second first (so the clocks reach the level they hold
    under sustained load of this kernel), then five replays are timed with HIP events on
    the replay stream and the median is returned, so host launch cost is not in the
    figure."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(steps):
                fn()
    torch.cuda.synchronize()
    times = []
    with torch.cuda.stream(stream):
        t_warm = time.perf_counter() + 0.5
        n_warm = 0
        while n_warm < 3 or time.perf_counter() < t_warm:
            graph.replay()  # warm replays (clocks settle under sustained load)
            stream.synchronize()
            n_warm += 1
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            e1.synchronize()
            times.append(e0.elapsed_time(e1) / steps)
    torch.cuda.synchronize()
    return sorted(times)[len(times) // 2]  # median of 5 timed replays


# ---------------------------------------------------------------- decode
def decode_bytes(lengths, Hq, Hkv, D):
    B = len(lengths)
    return sum(2 * Hkv * int(L) * D * 2 for L in lengths) + 2 * B * Hq * D * 2


def pre_bytes(B, T, Hq, Hkv, D):
    return B * T * ((Hq + 2 * Hkv) * D * 2 + Hq * D * 2 + 2 * Hkv * D * 2)


def primary(ctx, ema, args):
    torch = ctx.torch
    import numpy as np

    B, Hq, Hkv, D, cap = 32, 32, 8, 128, 8192
    lengths = np.random.default_rng(1234).integers(512, 8193, size=B)
    off = lengths - 1
    log(f"[bench] decode step B={B} {Hq}q/{Hkv}kv D={D} cap={cap} sum(L)={int(lengths.sum())}")
    cache = ema.StaticCache(B, Hkv, cap, D, k=ctx.randn((B, Hkv, cap, D)), v=ctx.randn((B, Hkv, cap, D)))
    qkv = ctx.randn((B, 1, (Hq + 2 * Hkv) * D))
    qw = ctx.randn((D,), 1.0, 0.02)
    kw = ctx.randn((D,), 1.0, 0.02)
    off_d, len_d = ctx.i32(off), ctx.i32(lengths)
    q = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=ctx.dev)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    scale = 1.0 / math.sqrt(D)

    def step():
        ema.decode_step(qkv2d, qw, kw, 1e-6, 1e6, off_d, Hq, cache, cap, scale, out=out, workspace=ws)

    qkv2d = qkv.reshape(B, -1)
    # untimed: about half a second of steps (clocks settle under sustained load), then the
    # W warmup steps
    t_warm = time.perf_counter() + 0.5
    while time.perf_counter() < t_warm:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # One step is one ema_decode_step call (two kernels on this stream), so the
    # events around the K timed steps also give the call's average duration.
    K = args.steps
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        step()
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = t0.elapsed_time(t1) / K
    ms_call = ms_step
    ab = decode_bytes(lengths, Hq, Hkv, D)
    sb = ab + pre_bytes(B, 1, Hq, Hkv, D)
    res = {
        "lengths_sum": int(lengths.sum()), "step_bytes": sb, "attn_bytes": ab,
        "ms_per_step": ms_step, "call_ms": ms_call, "wall_s": wall,
        "step_gbs": sb / (ms_step * 1e-3) / 1e9, "call_gbs": sb / (ms_call * 1e-3) / 1e9,
    }
    log(f"[bench] fused decode step {ms_step*1e3:.1f} us per step ({res['step_gbs']:.0f} GB/s); "
        f"per call {ms_call*1e3:.1f} us ({res['call_gbs']:.0f} GB/s, {res['call_gbs']/HBM_PEAK_GBS:.1%} of HBM)")
    # q of the last step, for the CPU baseline (same inputs the GPU attended with)
    ema.pre_attention(qkv, qw, kw, 1e-6, 1e6, off_d, Hq, cache, q_out=q)
    torch.cuda.synchronize()
    state = dict(cache=cache, q=q, lengths=lengths, Hq=Hq, Hkv=Hkv, D=D, cap=cap, scale=scale, bytes=ab)
    return res, state


def cpu_baseline(state, seconds):
    """The oracle's f32 SDPA (MLX CPU-stream arithmetic, OpenMP) on the same decode workload."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import torch

    cache = state["cache"]
    kc = cache.k.view(torch.int16).cpu().numpy().view(np.uint16)
    vc = cache.v.view(torch.int16).cpu().numpy().view(np.uint16)
    q = state["q"].view(torch.int16).cpu().numpy().view(np.uint16)
    L = np.asarray(state["lengths"], np.int32)
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t = time.perf_counter()
        oracle.sdpa(q, kc, vc, L, state["scale"], False, precision=1)
        times.append(time.perf_counter() - t)
        if time.perf_counter() > t_end or len(times) >= 20:
            break
    med = statistics.median(times)
    return {
        "value": state["bytes"] / med / 1e9, "unit": "GB/s", "cores": oracle.num_threads(), "kind": "port",
        "sample": f"the full batch-32 decode attention (same lengths, {len(times)} runs, median {med*1e3:.1f} ms): "
                  "oracle f32 SDPA, bf16 inputs, OpenMP over (sequence, kv head)",
    }


def cpu_baseline_b1(seconds):
    """The oracle's f32 SDPA (OpenMP) on the batch-1 Qwen3-1.7B-shape decode attention:
    16 query / 8 kv heads, head_dim 128, cache capacity 4096 with 1024 valid positions,
    q/K/V ~ N(0,1) from seeds, scale 1/sqrt(128)."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    B, Hq, Hkv, D, cap, L = 1, 16, 8, 128, 4096, 1024
    q = oracle.normal_bf16((B, Hq, 1, D), seed=11)
    kc = oracle.normal_bf16((B, Hkv, cap, D), seed=12)
    vc = oracle.normal_bf16((B, Hkv, cap, D), seed=13)
    lens = np.full(B, L, np.int32)
    by = decode_bytes([L], Hq, Hkv, D)
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t = time.perf_counter()
        oracle.sdpa(q, kc, vc, lens, 1.0 / math.sqrt(D), False, precision=1)
        times.append(time.perf_counter() - t)
        if time.perf_counter() > t_end or len(times) >= 2000:
            break
    med = statistics.median(times)
    return {
        "value": by / med / 1e9, "unit": "GB/s", "cores": oracle.num_threads(), "kind": "port",
        "us_per_call": med * 1e6, "workload": "decode_B1_16q8kv_L1024_cap4096",
        "sample": f"the batch-1 decode attention, L 1024 of cap 4096 ({len(times)} runs, median "
                  f"{med*1e6:.0f} us): oracle f32 SDPA, bf16 inputs, OpenMP over (sequence, kv head)",
    }


# ------------------------------------------------------------- secondary
def prefill_flops(Hq, D, T, off):
    return 4 * Hq * D * (T * off + T * (T + 1) // 2)


def profiled_counters():
    """Counter readings of the kernels as profiled (rocprofv3 runs of this script's
    workloads, recorded in profiles/*.md as `bench_counters: {json}` lines, one per
    workload): matrix-pipe busy fraction at 2.4 GHz, executed MFMA flops over algorithmic
    flops, and HBM bytes per call (FETCH_SIZE x 2 + WRITE_SIZE, the copy-kernel
    calibration). Keyed by workload name; each entry names its profile file."""
    found = {}
    pdir = os.path.join(ROOT, "profiles")
    try:
        names = sorted(os.listdir(pdir))
    except OSError:
        return found
    for name in names:
        if not name.endswith(".md"):
            continue
        for line in open(os.path.join(pdir, name)):
            if line.startswith("bench_counters:"):
                rec = json.loads(line.split(":", 1)[1])
                rec["counter_source"] = "profiles/" + name
                found[rec.pop("workload")] = rec
    return found


def prefill_roofline(name, tf, fl):
    roof = {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / BF16_PEAK_TFLOPS, 4), "flops_per_call": fl}
    rec = profiled_counters().get(name)
    if rec:
        roof.update(rec)
    return roof


def bench_prefill(ctx, ema, name, B, Hq, Hkv, D, cap, T, off, steps=20):
    torch = ctx.torch
    cache = ema.StaticCache(B, Hkv, cap, D, k=ctx.randn((B, Hkv, cap, D)), v=ctx.randn((B, Hkv, cap, D)))
    q = ctx.randn((B, Hq, T, D))
    qo = ctx.i32([off] * B)
    out = torch.empty((B, T, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ms = time_calls(torch, lambda: ema.prefill_attention(q, cache, qo, causal=True, out=out), steps, 5)
    fl = B * prefill_flops(Hq, D, T, off)
    tf = fl / (ms * 1e-3) / 1e12
    log(f"[bench] {name}: {ms*1e3:.1f} us, {tf:.1f} TFLOP/s ({tf/BF16_PEAK_TFLOPS:.1%} of bf16 peak)")
    return {"workload": name, "us": ms * 1e3, "tflops": tf, "frac_of_peak": tf / BF16_PEAK_TFLOPS, "flops": fl,
            "roofline": prefill_roofline(name, tf, fl)}


def bench_decode(ctx, ema, name, B, Hq, Hkv, D, cap, lengths, steps=20):
    torch = ctx.torch
    cache = ema.StaticCache(B, Hkv, cap, D, k=ctx.randn((B, Hkv, cap, D)), v=ctx.randn((B, Hkv, cap, D)))
    q = ctx.randn((B, Hq, D))
    ld = ctx.i32(lengths)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    ms = time_calls(torch, lambda: ema.decode_attention(q, cache, ld, int(max(lengths)), out=out, workspace=ws),
                    steps, 5)
    by = decode_bytes(lengths, Hq, Hkv, D)
    gbs = by / (ms * 1e-3) / 1e9
    log(f"[bench] {name}: {ms*1e3:.1f} us, {gbs:.0f} GB/s ({gbs/HBM_PEAK_GBS:.1%} of HBM)")
    return {"workload": name, "us": ms * 1e3, "gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "bytes": by}


def bench_decode_pair(ctx, ema, name, steps=20):
    """The same batch-32 step as two calls: ema_pre_attention (T=1) + ema_decode_attention."""
    import numpy as np

    torch = ctx.torch
    B, Hq, Hkv, D, cap = 32, 32, 8, 128, 8192
    lengths = np.random.default_rng(1234).integers(512, 8193, size=B)
    cache = ema.StaticCache(B, Hkv, cap, D, k=ctx.randn((B, Hkv, cap, D)), v=ctx.randn((B, Hkv, cap, D)))
    qkv = ctx.randn((B, 1, (Hq + 2 * Hkv) * D))
    qw, kw = ctx.randn((D,), 1.0, 0.02), ctx.randn((D,), 1.0, 0.02)
    off_d, len_d = ctx.i32(lengths - 1), ctx.i32(lengths)
    q = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=ctx.dev)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)

    def pair():
        ema.pre_attention(qkv, qw, kw, 1e-6, 1e6, off_d, Hq, cache, q_out=q)
        ema.decode_attention(q, cache, len_d, cap, out=out, workspace=ws)

    ms = time_calls(torch, pair, steps, 5)
    ms_attn = time_calls(torch, lambda: ema.decode_attention(q, cache, len_d, cap, out=out, workspace=ws), steps, 5)
    by = decode_bytes(lengths, Hq, Hkv, D)
    sb = by + pre_bytes(B, 1, Hq, Hkv, D)
    log(f"[bench] {name}: step {ms*1e3:.1f} us ({sb/(ms*1e-3)/1e9:.0f} GB/s); decode attention alone "
        f"{ms_attn*1e3:.1f} us ({by/(ms_attn*1e-3)/1e9:.0f} GB/s)")
    return {"workload": name, "us": ms * 1e3, "gbs": sb / (ms * 1e-3) / 1e9, "attn_us": ms_attn * 1e3,
            "attn_gbs": by / (ms_attn * 1e-3) / 1e9, "frac_of_peak": by / (ms_attn * 1e-3) / 1e9 / HBM_PEAK_GBS}


def fp8_cache(ctx, ema, B, Hkv, cap, D, n_rot=0):
    """FP8 cache of random finite E4M3FN codes with block exponents in {-8, -7} (values of
    N(0,1) size); with n_rot = 64 the last 64 dims of each row are N(0,1) bf16 values."""
    torch = ctx.torch

    def codes():
        c = torch.randint(0, 254, (B, Hkv, cap, D - n_rot), generator=ctx.gen, device=ctx.dev, dtype=torch.int32)
        c = (c + (c >= 0x7F).to(torch.int32)).to(torch.uint8)  # no NaN codes
        if not n_rot:
            return c
        tail = ctx.randn((B, Hkv, cap, n_rot)).view(torch.uint8)
        return torch.cat([c, tail], dim=-1).contiguous()

    def exps():
        e = torch.randint(-8, -6, (B, Hkv, cap, D // 64), generator=ctx.gen, device=ctx.dev,
                          dtype=torch.int32).to(torch.int8)
        if n_rot:
            e[..., 1] = 0
        return e

    return ema.StaticCache(B, Hkv, cap, D, dtype="fp8", n_rot=n_rot, k=codes(), v=codes(), k_exp=exps(),
                           v_exp=exps())


def fp8_decode_bytes(lengths, Hq, Hkv, D, n_rot=0):
    """K and V rows (codes, and the bf16 tail with n_rot) + block exponents of the valid
    rows, q in, out."""
    B = len(lengths)
    return sum(2 * Hkv * int(L) * (D + n_rot + D // 64) for L in lengths) + 2 * B * Hq * D * 2


def bench_fp8_step(ctx, ema, name, steps=20, n_rot=0):
    """The batch-32 Qwen3-8B-shape decode step (fused ema_decode_step) over an FP8 cache."""
    import numpy as np

    torch = ctx.torch
    B, Hq, Hkv, D, cap = 32, 32, 8, 128, 8192
    lengths = np.random.default_rng(1234).integers(512, 8193, size=B)
    cache = fp8_cache(ctx, ema, B, Hkv, cap, D, n_rot)
    qkv = ctx.randn((B, (Hq + 2 * Hkv) * D))
    qw, kw = ctx.randn((D,), 1.0, 0.02), ctx.randn((D,), 1.0, 0.02)
    off_d = ctx.i32(lengths - 1)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    ms = time_calls(torch, lambda: ema.decode_step(qkv, qw, kw, 1e-6, 1e6, off_d, Hq, cache, cap, out=out,
                                                   workspace=ws), steps, 5)
    by = (fp8_decode_bytes(lengths, Hq, Hkv, D, n_rot) + B * (Hq + 2 * Hkv) * D * 2
          + B * Hkv * 2 * (D + n_rot + D // 64))
    gbs = by / (ms * 1e-3) / 1e9
    log(f"[bench] {name}: step {ms*1e3:.1f} us, {gbs:.0f} GB/s ({gbs/HBM_PEAK_GBS:.1%} of HBM)")
    return {"workload": name, "us": ms * 1e3, "gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "bytes": by}


def bench_fp8_decode(ctx, ema, name, B, Hq, Hkv, D, cap, lengths, steps=20, n_rot=0):
    torch = ctx.torch
    cache = fp8_cache(ctx, ema, B, Hkv, cap, D, n_rot)
    q = ctx.randn((B, Hq, D))
    ld = ctx.i32(lengths)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    ms = time_calls(torch, lambda: ema.decode_attention(q, cache, ld, int(max(lengths)), out=out, workspace=ws),
                    steps, 5)
    by = fp8_decode_bytes(lengths, Hq, Hkv, D, n_rot)
    gbs = by / (ms * 1e-3) / 1e9
    log(f"[bench] {name}: {ms*1e3:.1f} us, {gbs:.0f} GB/s ({gbs/HBM_PEAK_GBS:.1%} of HBM)")
    return {"workload": name, "us": ms * 1e3, "gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "bytes": by}


def int4_cache(ctx, ema, B, Hkv, cap, D):
    """int4 affine cache of random codes with group scales near 0.3 and biases near -2.2
    (values of N(0,1) size)."""
    torch = ctx.torch

    def words():
        return torch.randint(-2 ** 31, 2 ** 31 - 1, (B, Hkv, cap, D // 8), generator=ctx.gen, device=ctx.dev,
                             dtype=torch.int64).to(torch.int32)

    def meta(mean, std):
        return ctx.randn((B, Hkv, cap, D // 64), mean, std)

    return ema.StaticCache(B, Hkv, cap, D, dtype="int4", k=words(), v=words(), k_scales=meta(0.3, 0.05),
                           k_biases=meta(-2.2, 0.1), v_scales=meta(0.3, 0.05), v_biases=meta(-2.2, 0.1))


def int4_decode_bytes(lengths, Hq, Hkv, D):
    """K and V codes + bf16 group scales and biases of the valid rows, q in, out."""
    B = len(lengths)
    return sum(2 * Hkv * int(L) * (D // 2 + 4 * (D // 64)) for L in lengths) + 2 * B * Hq * D * 2


def bench_int4_decode(ctx, ema, name, B, Hq, Hkv, D, cap, lengths, steps=20):
    torch = ctx.torch
    cache = int4_cache(ctx, ema, B, Hkv, cap, D)
    q = ctx.randn((B, Hq, D))
    ld = ctx.i32(lengths)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    ms = time_calls(torch, lambda: ema.decode_attention(q, cache, ld, int(max(lengths)), out=out, workspace=ws),
                    steps, 5)
    by = int4_decode_bytes(lengths, Hq, Hkv, D)
    gbs = by / (ms * 1e-3) / 1e9
    log(f"[bench] {name}: {ms*1e3:.1f} us, {gbs:.0f} GB/s ({gbs/HBM_PEAK_GBS:.1%} of HBM)")
    return {"workload": name, "us": ms * 1e3, "gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "bytes": by}


def bench_int4_step(ctx, ema, name, steps=20):
    """The batch-32 Qwen3-8B-shape decode step (fused ema_decode_step) over an int4 cache."""
    import numpy as np

    torch = ctx.torch
    B, Hq, Hkv, D, cap = 32, 32, 8, 128, 8192
    lengths = np.random.default_rng(1234).integers(512, 8193, size=B)
    cache = int4_cache(ctx, ema, B, Hkv, cap, D)
    qkv = ctx.randn((B, (Hq + 2 * Hkv) * D))
    qw, kw = ctx.randn((D,), 1.0, 0.02), ctx.randn((D,), 1.0, 0.02)
    off_d = ctx.i32(lengths - 1)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ws = ema.decode_workspace(B, Hq, Hkv, D, cap)
    ms = time_calls(torch, lambda: ema.decode_step(qkv, qw, kw, 1e-6, 1e6, off_d, Hq, cache, cap, out=out,
                                                   workspace=ws), steps, 5)
    by = (int4_decode_bytes(lengths, Hq, Hkv, D) + B * (Hq + 2 * Hkv) * D * 2 +
          B * Hkv * 2 * (D // 2 + 4 * (D // 64)))
    gbs = by / (ms * 1e-3) / 1e9
    log(f"[bench] {name}: step {ms*1e3:.1f} us, {gbs:.0f} GB/s ({gbs/HBM_PEAK_GBS:.1%} of HBM)")
    return {"workload": name, "us": ms * 1e3, "gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "bytes": by}


def bench_fp8_prefill(ctx, ema, name, B, Hq, Hkv, D, cap, T, off, steps=20):
    """Prefill over an FP8 cache: decode of the attended rows into the bf16 workspace + the
    bf16 prefill, per call."""
    torch = ctx.torch
    cache = fp8_cache(ctx, ema, B, Hkv, cap, D)
    q = ctx.randn((B, Hq, T, D))
    qo = ctx.i32([off] * B)
    out = torch.empty((B, T, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    kv = off + T
    ws = torch.empty(ema.prefill_workspace_size(cache, kv), dtype=torch.uint8, device=ctx.dev)
    ms = time_calls(torch, lambda: ema.prefill_attention(q, cache, qo, causal=True, out=out, max_kv_len=kv,
                                                         workspace=ws), steps, 5)
    fl = B * prefill_flops(Hq, D, T, off)
    tf = fl / (ms * 1e-3) / 1e12
    log(f"[bench] {name}: {ms*1e3:.1f} us, {tf:.1f} TFLOP/s ({tf/BF16_PEAK_TFLOPS:.1%} of bf16 peak)")
    return {"workload": name, "us": ms * 1e3, "tflops": tf, "frac_of_peak": tf / BF16_PEAK_TFLOPS, "flops": fl}


def bench_prefill_layer(ctx, ema, name, dtype, B, Hq, Hkv, D, cap, T, steps=20, prefill_only=False):
    """A fresh prefill chunk (offset 0) as a layer runs it: ema_pre_attention (norms, RoPE,
    the K/V rows written into the cache) + causal prefill. FP8 cache: ema_pre_attention_ws
    also writes the chunk's decoded rows into the prefill's bf16 copy, and the prefill
    (EMA_PREFILL_ROWS_DECODED, keys the chunk's own) runs no decode pass. prefill_only:
    time the prefill call alone, with the copy filled once beforehand."""
    torch = ctx.torch
    fp8 = dtype == "fp8"
    cache = ema.StaticCache(B, Hkv, cap, D, dtype=dtype)
    qkv = ctx.randn((B, T, (Hq + 2 * Hkv) * D))
    qw, kw = ctx.randn((D,), 1.0, 0.02), ctx.randn((D,), 1.0, 0.02)
    off = ctx.i32([0] * B)
    q = torch.empty((B, Hq, T, D), dtype=torch.bfloat16, device=ctx.dev)
    out = torch.empty((B, T, Hq * D), dtype=torch.bfloat16, device=ctx.dev)
    ws = torch.empty(ema.prefill_workspace_size(cache, T), dtype=torch.uint8, device=ctx.dev) if fp8 else None
    pre_kw = {"prefill_workspace": ws, "max_kv_len": T} if fp8 else {}
    att_kw = {"max_kv_len": T, "workspace": ws, "rows_decoded": True, "chunk_only": True} if fp8 else {}

    def pre():
        ema.pre_attention(qkv, qw, kw, 1e-6, 1e6, off, Hq, cache, q_out=q, **pre_kw)

    def att():
        ema.prefill_attention(q, cache, off, causal=True, out=out, **att_kw)

    if prefill_only:
        pre()
        ms = time_calls(torch, att, steps, 5)
    else:
        ms = time_calls(torch, lambda: (pre(), att()), steps, 5)
    fl = B * prefill_flops(Hq, D, T, 0)
    tf = fl / (ms * 1e-3) / 1e12
    log(f"[bench] {name}: {ms*1e3:.1f} us, {tf:.1f} TFLOP/s of the attention ({tf/BF16_PEAK_TFLOPS:.1%} of bf16 peak)")
    return {"workload": name, "us": ms * 1e3, "tflops": tf, "frac_of_peak": tf / BF16_PEAK_TFLOPS, "flops": fl}


def gdn_bytes(B, T, Hk, Hv, Dk, Dv, act=2):
    """State read + write, q/k/v in, y out, g/beta in."""
    return 8 * B * Hv * Dv * Dk + act * B * T * (2 * Hk * Dk + 2 * Hv * Dv) + 8 * B * T * Hv


def qmm_bytes(M, N, K, gs, bits, act=2):
    """Packed weights, scales and biases, x in, y out: each read or written once."""
    return N * K * bits // 8 + 2 * act * N * (K // gs) + act * M * K + act * M * N


def bench_qmm(ctx, ema, name, M, N, K, gs=64, bits=4, steps=48, min_set_bytes=300 << 20):
    """Affine-quantised projection (ema_quantized_matmul) y[M, N] = x W^T, bf16 activations.
    As in a decode step, each call reads another layer's weights: the calls cycle over
    enough distinct weight sets (over 300 MB, more than the 256 MB last-level cache)
    that every call streams its weights from HBM."""
    torch = ctx.torch
    per = N * K * bits // 8 + 4 * N * (K // gs)
    L = max(1, min(steps, -(-min_set_bytes // per)))
    words = K * bits // 32
    sets = []
    for _ in range(L):
        w = torch.randint(-2**31, 2**31 - 1, (N, words), dtype=torch.int32, device=ctx.dev, generator=ctx.gen)
        sc = (torch.rand((N, K // gs), device=ctx.dev, generator=ctx.gen) * 0.004 + 0.001).to(torch.bfloat16)
        bi = (torch.rand((N, K // gs), device=ctx.dev, generator=ctx.gen) * 0.04 - 0.02).to(torch.bfloat16)
        sets.append((w, sc, bi))
    x = ctx.randn((M, K))
    y = torch.empty((M, N), dtype=torch.bfloat16, device=ctx.dev)
    it = [0]

    def call():
        w, sc, bi = sets[it[0] % L]
        it[0] += 1
        ema.quantized_matmul(x, w, sc, bi, group_size=gs, bits=bits, out=y)

    ms = time_calls(torch, call, steps, 2 * L)
    by = qmm_bytes(M, N, K, gs, bits)
    gbs = by / (ms * 1e-3) / 1e9
    tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    log(f"[bench] {name}: {ms*1e3:.2f} us, {gbs:.0f} GB/s ({gbs/HBM_PEAK_GBS:.1%} of HBM), {tf:.1f} TFLOP/s "
        f"({L} weight sets)")
    return {"workload": name, "us": ms * 1e3, "gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "bytes": by,
            "tflops": tf, "weight_sets": L}


def bench_gdn(ctx, ema, name, B, T, Hk, Hv, Dk, Dv, steps=20, workspace=False):
    """Gated DeltaNet scan (ema_gdn_scan, or ema_gdn_scan_ws with a workspace: the WY form),
    bf16 activations, f32 state updated in place (bounded: unit keys, g and beta in (0, 1))."""
    torch = ctx.torch
    q = ctx.randn((B, T, Hk, Dk), 0.0, 1.0 / Dk)
    k = ctx.randn((B, T, Hk, Dk), 0.0, 1.0)
    k = (k.float() / k.float().norm(dim=-1, keepdim=True)).to(torch.bfloat16).contiguous()
    v = ctx.randn((B, T, Hv, Dv))
    g = torch.rand((B, T, Hv), device=ctx.dev) * 0.5 + 0.5
    beta = torch.rand((B, T, Hv), device=ctx.dev)
    S = torch.randn((B, Hv, Dv, Dk), device=ctx.dev) * 0.5
    y = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=ctx.dev)
    ws = ema.gdn_workspace(B, T, Hk, Hv, Dk, Dv) if workspace else None
    ms = time_calls(torch, lambda: ema.gdn_scan(q, k, v, g, beta, S, y=y, workspace=ws), steps, 5)
    by = gdn_bytes(B, T, Hk, Hv, Dk, Dv)
    gbs = by / (ms * 1e-3) / 1e9
    tok = B * T / (ms * 1e-3)
    log(f"[bench] {name}: {ms*1e3:.1f} us, {gbs:.0f} GB/s ({gbs/HBM_PEAK_GBS:.1%} of HBM), {tok:.3g} tokens/s")
    return {"workload": name, "us": ms * 1e3, "gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "bytes": by,
            "tokens_per_s": tok}


def bench_pre(ctx, ema, name, T, Hq, Hkv, D, cap, steps=20):
    torch = ctx.torch
    cache = ema.StaticCache(1, Hkv, cap, D)
    # qkv = x W for x [T, 2048] ~ N(0,1), W ~ N(0, 1/sqrt(2048)): the projection is outside the path
    x = ctx.randn((T, 2048))
    w = ctx.randn((2048, (Hq + 2 * Hkv) * D), 0.0, 1.0 / math.sqrt(2048))
    qkv = (x @ w).reshape(1, T, -1).contiguous()
    qw, kw = ctx.randn((D,), 1.0, 0.02), ctx.randn((D,), 1.0, 0.02)
    off = ctx.i32([0])
    q = torch.empty((1, Hq, T, D), dtype=torch.bfloat16, device=ctx.dev)
    ms = time_calls(torch, lambda: ema.pre_attention(qkv, qw, kw, 1e-6, 1e6, off, Hq, cache, q_out=q), steps, 5)
    by = pre_bytes(1, T, Hq, Hkv, D)
    gbs = by / (ms * 1e-3) / 1e9
    log(f"[bench] {name}: {ms*1e3:.1f} us, {gbs:.0f} GB/s")
    return {"workload": name, "us": ms * 1e3, "gbs": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS, "bytes": by}


def profiled_traffic():
    """HBM bytes per ema_decode_step call measured by the FETCH_SIZE / WRITE_SIZE
    counter runs recorded in profiles/decode_step_b32_qwen3_8b.md (None if absent)."""
    path = os.path.join(ROOT, "profiles", "decode_step_b32_qwen3_8b.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_call:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for {max(args.gpus, world)}); the attention path here is "
              "single-GPU and has no multi-GPU mode.", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    import ema_attn as ema

    ema.lib()
    ctx = Ctx()
    if args.calibrate_copy:  # a copy kernel of known size (1 GiB read + 1 GiB write)
        src = torch.ones(1 << 29, dtype=torch.int16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    res, state = primary(ctx, ema, args)
    secondary = []
    if args.only in ("all", "prefill"):
        secondary.append(bench_prefill(ctx, ema, "prefill_causal_T2048_32q8kv_qwen3_8b", 1, 32, 8, 128, 4096, 2048, 0))
    if args.only in ("all", "prefill_1p7b"):
        secondary.append(bench_prefill(ctx, ema, "prefill_causal_T2048_16q8kv_qwen3_1p7b", 1, 16, 8, 128, 4096, 2048, 0))
    if args.only in ("all", "pre"):
        secondary.append(bench_pre(ctx, ema, "pre_attention_T2048_16q8kv", 2048, 16, 8, 128, 4096))
    if args.only == "all":
        secondary.append(bench_decode_pair(ctx, ema, "decode_B32_32q8kv_unfused_pre_attention_plus_attention"))
    if args.only in ("all", "decode_b1"):
        secondary.append(bench_decode(ctx, ema, "decode_B1_16q8kv_L1024_cap4096", 1, 16, 8, 128, 4096, [1024]))
    if args.only in ("all", "decode_long"):
        secondary.append(bench_decode(ctx, ema, "decode_B8_32q4kv_L32768", 8, 32, 4, 128, 32768, [32768] * 8))
    if args.only in ("all", "prefill_chunk"):
        secondary.append(bench_prefill(ctx, ema, "prefill_chunk_off14336_T2048_64q8kv", 1, 64, 8, 128, 16384, 2048,
                                       14336, steps=10))
    if args.only in ("all", "fp8"):
        secondary.append(bench_fp8_step(ctx, ema, "decode_step_B32_32q8kv_fp8_cache"))
        secondary.append(bench_fp8_decode(ctx, ema, "decode_B8_32q4kv_L32768_fp8_cache", 8, 32, 4, 128, 32768,
                                          [32768] * 8))
    if args.only in ("all", "fp8", "fp8_prefill"):
        secondary.append(bench_fp8_prefill(ctx, ema, "prefill_causal_T2048_32q8kv_fp8_cache", 1, 32, 8, 128, 4096,
                                           2048, 0))
        # the chunk's rows decoded by pre-attention: the prefill call runs no decode pass
        secondary.append(bench_prefill_layer(ctx, ema, "prefill_causal_T2048_32q8kv_fp8_cache_rows_from_pre_attention",
                                             "fp8", 1, 32, 8, 128, 4096, 2048, prefill_only=True))
        for dt in ("bf16", "fp8"):
            secondary.append(bench_prefill_layer(ctx, ema, f"pre_attention_plus_prefill_T2048_32q8kv_{dt}_cache", dt, 1,
                                                 32, 8, 128, 4096, 2048))
    if args.only in ("all", "fp8", "fp8_tail"):
        # Fp8Cache::new(128, 64): dims 64..127 of each row kept as bf16
        secondary.append(bench_fp8_step(ctx, ema, "decode_step_B32_32q8kv_fp8_cache_rope_tail64", n_rot=64))
        secondary.append(bench_fp8_decode(ctx, ema, "decode_B8_32q4kv_L32768_fp8_cache_rope_tail64", 8, 32, 4, 128,
                                          32768, [32768] * 8, n_rot=64))
    if args.only in ("all", "int4"):
        secondary.append(bench_int4_step(ctx, ema, "decode_step_B32_32q8kv_int4_cache"))
        secondary.append(bench_int4_decode(ctx, ema, "decode_B8_32q4kv_L32768_int4_cache", 8, 32, 4, 128, 32768,
                                           [32768] * 8))
    if args.only in ("all", "gdn", "gdn_step"):
        # Gated DeltaNet layer of Qwen3-Next shape: 16 key / 32 value heads, head dims 128
        secondary.append(bench_gdn(ctx, ema, "gdn_decode_step_B32_16k32v_dk128_dv128", 32, 1, 16, 32, 128, 128))
    if args.only in ("all", "gdn"):
        secondary.append(bench_gdn(ctx, ema, "gdn_scan_T2048_B1_16k32v_dk128_dv128", 1, 2048, 16, 32, 128, 128,
                                   steps=10, workspace=True))
        secondary.append(bench_gdn(ctx, ema, "gdn_scan_T2048_B1_16k32v_dk128_dv128_no_workspace", 1, 2048, 16, 32,
                                   128, 128, steps=5))
    if args.only in ("all", "qmm"):
        # affine-quantised projections around the attention path (MLX 4-bit, group 64):
        # Qwen3-8B q|k|v (4096 -> 6144) and o_proj (4096 -> 4096) per decode step
        secondary.append(bench_qmm(ctx, ema, "qmatmul_qkv_M32_K4096_N6144_4bit_g64", 32, 6144, 4096))
        secondary.append(bench_qmm(ctx, ema, "qmatmul_qkv_M1_K4096_N6144_4bit_g64", 1, 6144, 4096))
        secondary.append(bench_qmm(ctx, ema, "qmatmul_o_proj_M32_K4096_N4096_4bit_g64", 32, 4096, 4096))
        secondary.append(bench_qmm(ctx, ema, "qmatmul_qkv_M32_K4096_N6144_8bit_g64", 32, 6144, 4096, bits=8))
        secondary.append(bench_qmm(ctx, ema, "qmatmul_qkv_prefill_M2048_K2048_N4096_4bit_g64", 2048, 4096, 2048,
                                   steps=8))
    cpu = cpu_b1 = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle f32 SDPA on the host)")
        cpu = cpu_baseline(state, args.cpu_seconds)
        log(f"[bench] CPU baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads")
        cpu_b1 = cpu_baseline_b1(min(args.cpu_seconds, 3.0))
        log(f"[bench] CPU baseline, batch-1 decode: {cpu_b1['us_per_call']:.0f} us per call, "
            f"{cpu_b1['value']:.2f} GB/s on {cpu_b1['cores']} threads")
    line = {
        "metric": METRIC,
        "value": round(res["step_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) q/K/V and qkv, norm weights 1+N(0,0.02), lengths U[512,8192] seed 1234",
        "config": {
            "workload": "qwen3_8b_batched_decode_step: pre-attention (T=1) + decode attention (fused ema_decode_step)",
            "batch": 32, "n_heads": 32, "n_kv_heads": 8, "head_dim": 128, "capacity": 8192,
            "lengths_sum": res["lengths_sum"], "parallelism": "single_gpu",
        },
        "roofline": {
            "bound": "hbm", "kernel": "ema_decode_step (decode_kernel<fused> + decode_merge_kernel)",
            "achieved": round(res["call_gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(res["call_gbs"] / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(),
            "traffic_source": "FETCH_SIZE/WRITE_SIZE runs, profiles/decode_step_b32_qwen3_8b.md",
            "call_us": round(res["call_ms"] * 1e3, 2), "call_bytes": res["step_bytes"],
        },
        "cpu_baseline": cpu,
        "cpu_baseline_decode_b1": cpu_b1,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
