#!/usr/bin/env python3
"""Benchmark: MoE-layer decode tokens/s + achieved HBM GB/s on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload (the headline metric: config 3 at T = 8): one step is one
decode MoE layer over T = 8 tokens — router (f32 [64,1280]), top-6 with
renormalised gates, 64 int8 experts (gate/up [896,1280], down [1280,896],
per-row f32 scales), SwiGLU, slot-order combine. Inputs are resident in HBM
before timing. To measure HBM rather than the 256 MB Infinity Cache, the
timed steps rotate over --copies distinct layers (each with its own router
and its own copy of the expert weights; 220 MB each), like consecutive
decoder layers. Synthetic seeded data (no checkpoint).

Other workloads (--workload): lm_head (config 2), lm_head_sample (config 2
with the no-repeat-ngram ban and history append fused in), igemm (config 1),
rswa (config 5), moe_prefill_i4 (config 4). Each prints ONE JSON line with `roofline` (dominant kernel,
algorithmic bytes / HIP-event-timed average launch) and, at N = 1,
`cpu_baseline` (the reference's x86 int8 tier restated in C, oracle/,
timed on a bounded sample on this host).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
H, I, E, K = 1280, 896, 64, 6


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cpu() -> dict:
    """The host the CPU baseline ran on: logical CPUs (nproc) and the model
    string from /proc/cpuinfo."""
    model = "unknown"
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


TRAFFIC_NOTE = ("stored: profiles/traffic.json, rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs scaled by a 512 MiB "
                "copy; null when the kernel's source changed since it was measured")


def traffic_for(kernel: str, workload: str):
    """HBM bytes per launch measured with rocprofv3 --pmc: FETCH_SIZE and
    WRITE_SIZE (one run each) scaled by what the same counters read for a
    512 MiB device-to-device copy (profiles/traffic.json, written by
    rocprof_summary.py traffic). A stored value is returned only
    while the hash of the kernel source it was measured on matches the file
    as it is now; otherwise (or if not recorded) None."""
    from rocprof_summary import source_sha16

    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        rec = json.loads(f.read_text()).get(f"{kernel}@{workload}")
    except (OSError, ValueError):
        return None
    if rec is None or "source" not in rec or not (ROOT / rec["source"]).exists():
        return None
    if source_sha16(ROOT / rec["source"]) != rec.get("source_sha256_16"):
        return None
    return rec.get("bytes_per_dispatch")


STAT_STEPS = 100  # the per-kernel statistics pass runs at least this many steps
STAT_GROUPS = 100  # step statistics: this many samples ...
STEPS_PER_MARK = 10  # ... each the mean of this many consecutive steps between two marks


def timed(ctx, step, steps: int):
    """Three passes over the same steps.

    1. Throughput: exactly `steps` steps between two device synchronisations
       (wall clock); `value` and `ms_per_step` come from this pass.
    2. Per-kernel HIP events over max(steps, STAT_STEPS) steps. The events
       ride in each kernel's dispatch packet (hipExtLaunchKernelGGL), so they
       time the kernel's own execution (they agree with rocprofv3's kernel
       trace); their completion signals slow the step as a whole, which is why
       throughput comes from pass 1. Per launch: mean, min, median, p90.
    3. Step marks: an event recorded on the stream after every
       STEPS_PER_MARK steps, STAT_GROUPS + 1 marks. Each sample is the
       GPU-clock time between two marks over STEPS_PER_MARK (a mark per
       step would add its own ~2 us to every sample), summarised as min /
       median / p90 / CoV (the reference's statistics, perf_harness.rs:
       186-282, nearest-rank percentiles)."""
    ctx.device_synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    ctx.device_synchronize()
    el = time.perf_counter() - t0
    log(f"timed pass: {steps} steps in {el * 1e3:.3f} ms")
    n_stat = max(steps, STAT_STEPS)
    ctx.prof_reset()
    ctx.prof_enable(True)
    for i in range(n_stat):
        step(i)
    prof = ctx.prof_read()
    ctx.prof_enable(False)
    kernels = {k: round(v["ms"] / max(v["count"], 1) * 1e3, 3) for k, v in prof.items()}
    ctx.device_synchronize()
    log(f"per-kernel pass: {n_stat} steps")
    ctx.mark()
    for g in range(STAT_GROUPS):
        for i in range(STEPS_PER_MARK):
            step(g * STEPS_PER_MARK + i)
        ctx.mark()
    group_ms = ctx.marks_read()
    log(f"step-statistics pass: {STAT_GROUPS} x {STEPS_PER_MARK} steps")
    st = sample_stats([v * 1e-3 / STEPS_PER_MARK for v in group_ms], scale=1e6, unit="us")
    st["steps_per_sample"] = STEPS_PER_MARK
    return el, prof, kernels, st


def set_stat_sizes(stat_steps: int, stat_groups: int) -> None:
    """Sizes of timed()'s statistics passes (small for counter runs, where
    every dispatch is slow)."""
    global STAT_STEPS, STAT_GROUPS
    STAT_STEPS, STAT_GROUPS = max(1, stat_steps), max(1, stat_groups)


def nearest_rank(sorted_asc, q: float) -> float:
    """perf_harness.rs:276-282: rank = ceil(q * n) clamped to [1, n]."""
    n = len(sorted_asc)
    rank = min(max(int(np.ceil(q * n)), 1), n)
    return sorted_asc[rank - 1]


def sample_stats(secs, scale: float = 1e3, unit: str = "ms") -> dict:
    """perf_harness.rs:186-263 SampleStats over per-iteration seconds: n,
    min (best-of-N), p50, p90 (nearest rank), mean and the coefficient of
    variation in percent (sample standard deviation / mean), in `unit`."""
    v = sorted(secs)
    n = len(v)
    mean = sum(v) / n
    var = sum((x - mean) ** 2 for x in v) / (n - 1) if n > 1 else 0.0
    return {"n": n, "unit": unit, "min": round(v[0] * scale, 3), "p50": round(nearest_rank(v, 0.5) * scale, 3),
            "p90": round(nearest_rank(v, 0.9) * scale, 3), "mean": round(mean * scale, 3),
            "cv_pct": round(100.0 * var ** 0.5 / mean, 2) if mean > 0 else 0.0}


def launch_stats(prof: dict, name: str) -> dict:
    """Median, p90 and minimum launch time (us) of one profiled scope."""
    g = prof.get(name) or {}
    if not g.get("count"):
        return {}
    return {"p50_launch_us": round(g["p50_ms"] * 1e3, 3), "p90_launch_us": round(g["p90_ms"] * 1e3, 3),
            "min_launch_us": round(g["min_ms"] * 1e3, 3), "launches_timed": g["count"]}


def cpu_stats(call, units_per_call: float, unit: str, seconds: float, min_iters: int = 3,
              max_iters: int = 100000) -> dict:
    """The CPU baseline's timing, after the reference's bench harness
    (perf_harness.rs:186-263): one warm-up call discarded, then one
    wall-clock sample per call until `seconds` have passed (at least
    `min_iters` calls). `value` is the throughput of the median call; `best`
    that of the fastest (best-of-N); the per-call times' p50 / p90 / min and
    CoV are kept beside them."""
    call()
    secs = []
    t_end = time.perf_counter() + seconds
    while len(secs) < max_iters and (len(secs) < min_iters or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        call()
        secs.append(time.perf_counter() - t0)
    st = sample_stats(secs)
    return {"value": round(units_per_call / (st["p50"] * 1e-3), 2), "unit": unit,
            "best": round(units_per_call / (st["min"] * 1e-3), 2), "call_ms": st,
            "cov_pct": st["cv_pct"], "calls": len(secs), "seconds": round(sum(secs), 2)}


def kernel_us(prof: dict, name: str) -> float:
    g = prof.get(name)
    if not g or not g["count"]:
        return float("nan")
    return g["ms"] / g["count"] * 1e3


# ---------------------------------------------------------------------------
# config 3: MoE decode
# ---------------------------------------------------------------------------

def make_moe_host(seed: int):
    from franken_ocr_amd import synth

    router = synth.f32_normal(synth.seed_of(seed), E * H, 0.0, 0.02).reshape(E, H)
    wg = synth.int8_uniform(synth.seed_of(seed + 1), E * I * H)
    wu = synth.int8_uniform(synth.seed_of(seed + 2), E * I * H)
    wd = synth.int8_uniform(synth.seed_of(seed + 3), E * H * I)
    sg = synth.f32_uniform(synth.seed_of(seed + 4), E * I, 1e-3, 2e-2)
    su = synth.f32_uniform(synth.seed_of(seed + 5), E * I, 1e-3, 2e-2)
    sd = synth.f32_uniform(synth.seed_of(seed + 6), E * H, 1e-3, 2e-2)
    return router, wg, sg, wu, su, wd, sd


def bench_moe(args, ctx):
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import MoeLayer

    T = args.tokens
    log(f"moe_decode: T={T}, {args.copies} layer copies, generating weights")
    base = make_moe_host(100)
    layers = []
    for c in range(args.copies):
        router = synth.f32_normal(synth.seed_of(1000 + c), E * H, 0.0, 0.02).reshape(E, H)
        layers.append(MoeLayer(H, I, E, K, router, *base[1:], ctx=ctx))
    hidden = synth.f32_normal(synth.seed_of(50), T * H).reshape(T, H)
    dx = ctx.to_device(hidden)
    dout = ctx.empty((T, H), np.float32)
    idx_bufs = [ctx.empty((T, K), np.uint32) for _ in layers]
    gate_bufs = [ctx.empty((T, K), np.float32) for _ in layers]

    def step(i):
        j = i % len(layers)
        layers[j].decode(dx, dout, idx_bufs[j], gate_bufs[j], norm_topk=True, routed_scale=1.0, check_route=False)

    for i in range(args.warmup):
        step(i)
    for j in range(len(layers)):  # every copy routes once before its experts are counted
        step(j)
    ctx.device_synchronize()
    # distinct experts actually routed, per copy (for algorithmic bytes)
    U = [len(np.unique(b.numpy())) for b in idx_bufs]
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    tok_s = T * args.steps / el

    mean_u = float(np.mean([U[i % len(U)] for i in range(args.steps)]))
    pairs = T * K
    gate_up_bytes = mean_u * 2 * (I * H + I * 4) + T * H + T * 4 + pairs * I * 4
    layer_bytes = mean_u * (3 * I * H + 2 * I * 4 + H * 4) + E * H * 4 + 2 * T * H * 4
    gu_ms = kernel_us(prof, "moe_gate_up") * 1e-3
    achieved = gate_up_bytes / (gu_ms * 1e-3) / 1e9
    layer_gbs = layer_bytes / (ms * 1e-3) / 1e9
    log(f"U per copy {U}; per-kernel avg us {kernels}")
    return {
        "metric": "MoE-layer decode tokens/s + achieved HBM GB/s (% of 8 TB/s peak), 1 GPU",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "ms_per_step": round(ms, 5),
        "dtype": "int8",
        "config": {"workload": "moe_decode", "tokens": T, "hidden": H, "inter": I, "experts": E, "top_k": K,
                   "norm_topk": True, "layer_copies_rotated": args.copies, "distinct_experts_mean": mean_u},
        # the dominant kernel's roofline, and beside it the whole layer's (the
        # metric and the >= 60% target are layer-level: every byte of the step
        # over the step's wall-clock time, route and kernel boundaries included)
        "roofline": {"bound": "hbm", "kernel": "moe_gate_up", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for("moe_gate_up", "moe_decode_t%d" % T), "traffic_note": TRAFFIC_NOTE,
                     "algorithmic_bytes_per_launch": int(gate_up_bytes), "avg_launch_us": round(gu_ms * 1e3, 3),
                     **launch_stats(prof, "moe_gate_up"),
                     "layer_achieved": round(layer_gbs, 1), "layer_frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                     "layer_algorithmic_bytes_per_step": int(layer_bytes),
                     "layer_frac_at_p50_step": round(layer_bytes / (sstats["p50"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        "layer_roofline": {"achieved": round(layer_gbs, 1), "unit": "GB/s", "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                           "algorithmic_bytes_per_step": int(layer_bytes)},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": (hidden, layers[0], base),
    }


def cpu_moe(args, inputs):
    from oracle import pyoracle
    from franken_ocr_amd import synth

    hidden, layer0, base = inputs
    router = synth.f32_normal(synth.seed_of(1000), E * H, 0.0, 0.02).reshape(E, H)
    _, wg, sg, wu, su, wd, sd = base
    L = pyoracle.lib()
    tier = L.cpu_detect_tier()
    T = hidden.shape[0]
    out = np.zeros(T * H, np.float32)
    idx = np.zeros(T * K, np.uint32)
    gates = np.zeros(T * K, np.float32)
    P = pyoracle.p
    args_c = [P(np.ascontiguousarray(hidden)), T, H, I, E, K, P(router), P(wg), P(sg), P(wu), P(su), P(wd), P(sd),
              1, 1.0, P(out), P(idx), P(gates)]
    res = cpu_stats(lambda: L.cpu_moe_decode(tier, *args_c), T, "tokens/s", args.cpu_seconds)
    st, want, want_idx, _ = pyoracle.moe_decode(hidden, router, wg, sg, wu, su, wd, sd, E, K, I, norm_topk=True)
    same = st == 0 and np.array_equal(out, want.reshape(-1)) and np.array_equal(idx, want_idx.reshape(-1))
    res.update({"cores": min(K, os.cpu_count() or 1), "kind": "port", "tier": L.cpu_tier_feature(tier).decode(),
                "matches_oracle": bool(same),
                "sample": f"MoE decode steps of T={T} tokens (first layer copy); top-{K} experts as concurrent "
                          f"single-thread tasks, tokens sequential (decoder.rs:2231-2252)"})
    return res


# ---------------------------------------------------------------------------
# config 2: LM head GEMV + argmax
# ---------------------------------------------------------------------------

def bench_lm_head(args, ctx, sampler=False):
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import QInt8, lm_head_i8, lm_head_sample_i8

    M, N, Kd = args.tokens, 129280, 1280
    log(f"lm_head: M={M}, {args.copies} weight copies, fused sampler={sampler}")
    w = synth.int8_uniform(synth.seed_of(20), N * Kd)
    s = synth.f32_uniform(synth.seed_of(21), N, 1e-3, 2e-2)
    heads = [QInt8(w, s, N, Kd, ctx) for _ in range(args.copies)]
    x = synth.f32_normal(synth.seed_of(22), M * Kd).reshape(M, Kd)
    dx = ctx.to_device(x)
    dl = ctx.empty((M, N), np.float32)
    da = ctx.empty((M,), np.uint32)
    if sampler:
        # each stream starts with 128 generated tokens; every step bans over the
        # 35-gram / 128-token window and appends its token on the device
        cap = 128 + args.warmup + args.steps
        hist = np.zeros((M, cap), np.uint32)
        hist[:, :128] = synth.int_uniform(synth.seed_of(23), M * 128, 0, N - 1).reshape(M, 128)
        dh, dlen = ctx.to_device(hist), ctx.to_device(np.full(M, 128, np.uint32))

    def step(i):
        if sampler:
            lm_head_sample_i8(heads[i % len(heads)], dx, da, dh, dlen, 35, 128, append=True, logits=dl)
        else:
            lm_head_i8(heads[i % len(heads)], dx, da, dl)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    g_ms = kernel_us(prof, "lm_head_gemv") * 1e-3
    gemv_bytes = N * Kd + N * 4 + M * Kd + M * 4 + M * N * 4
    total_bytes = gemv_bytes + M * Kd * 4 + M * 4
    achieved = gemv_bytes / (g_ms * 1e-3) / 1e9
    log(f"per-kernel avg us {kernels}")
    metric = ("LM-head int8 GEMV + no-repeat-ngram ban + argmax + history append tokens/s (129280x1280, 35-gram, "
              "window 128), 1 GPU" if sampler else "LM-head int8 GEMV + argmax tokens/s (129280x1280), 1 GPU")
    cfg = {"workload": "lm_head_sample" if sampler else "lm_head", "rows": M, "vocab": N, "hidden": Kd,
           "weight_copies_rotated": args.copies}
    if sampler:
        cfg.update({"no_repeat_ngram_size": 35, "ngram_window": 128, "history_start_len": 128})
    return {
        "metric": metric,
        "value": round(M * args.steps / el, 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "dtype": "int8",
        "config": cfg,
        "roofline": {"bound": "hbm", "kernel": "lm_head_gemv", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for("lm_head_gemv", f"lm_head_m{M}"), "traffic_note": TRAFFIC_NOTE,
                     "algorithmic_bytes_per_launch": int(gemv_bytes), "avg_launch_us": round(g_ms * 1e3, 3), **launch_stats(prof, "lm_head_gemv")},
        "step_achieved_gbs": round(total_bytes / (ms * 1e-3) / 1e9, 1),
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": (x, w, s),
    }


def cpu_lm_head(args, inputs):
    from oracle import pyoracle

    x, w, s = inputs
    L = pyoracle.lib()
    tier = L.cpu_detect_tier()
    M, N, Kd = x.shape[0], 129280, 1280
    logits = np.zeros(M * N, np.float32)
    am = np.zeros(M, np.uint32)
    P = pyoracle.p
    res = cpu_stats(lambda: L.cpu_lm_head_i8(tier, P(x), M, P(w), P(s), N, Kd, P(logits), P(am)), M, "tokens/s",
                    args.cpu_seconds)
    want_l, want_a = pyoracle.lm_head_i8(x, w, s, N, Kd)
    same = np.array_equal(logits, want_l.reshape(-1)) and np.array_equal(am, want_a)
    res.update({"cores": int(L.cpu_threads()), "kind": "port", "tier": L.cpu_tier_feature(tier).decode(),
                "matches_oracle": bool(same),
                "sample": f"LM-head GEMV+argmax calls of M={M} rows; 64-row blocks over all threads "
                          f"(decoder.rs:1621-1640)"})
    return res


# ---------------------------------------------------------------------------
# config 1: single igemm at the gate-proj shape
# ---------------------------------------------------------------------------

IGEMM_SETS = 8  # distinct 64-expert weight sets (8 x 73.4 MB = 587 MB, over twice the 256 MB MALL)


def igemm_weight_sets(ctx, N, Kd):
    """IGEMM_SETS device copies of 64 experts' gate-proj weights (one seeded
    host set uploaded to distinct allocations: the Infinity Cache holds lines
    by address, so every copy is read from HBM once the rotation has cycled)."""
    from franken_ocr_amd import synth

    w = synth.int8_uniform(synth.seed_of(1), 64 * N * Kd)
    return w, [ctx.to_device(w) for _ in range(IGEMM_SETS)]


def bench_igemm(args, ctx):
    from franken_ocr_amd import _abi, synth

    M, N, Kd = args.tokens, 896, 1280
    w, sets = igemm_weight_sets(ctx, N, Kd)
    copies = 64 * len(sets)  # distinct 1.15 MB gate-proj matrices, rotated
    log(f"igemm: M={M}, {copies} distinct weight matrices ({copies * N * Kd / 1e6:.0f} MB) rotated")
    a = synth.int8_uniform(synth.seed_of(2), M * Kd)
    da = ctx.to_device(a)
    dout = ctx.empty((M, N), np.int32)

    def step(i):
        c = i % copies
        _abi.call("focr_hip_igemm_s8s8_dev", ctx.handle, da.c_ptr, sets[c % len(sets)].offset((c // len(sets)) * N * Kd),
                  M, Kd, N, dout.c_ptr)

    for i in range(max(args.warmup, copies)):  # every matrix once: the timed pass starts from a cycled MALL
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    g_ms = kernel_us(prof, "igemm_i8") * 1e-3
    nbytes = N * Kd + M * Kd + 2 * M * N * 4
    achieved = nbytes / (g_ms * 1e-3) / 1e9
    return {
        "metric": "int8 igemm (gate-proj 896x1280) launches/s, 1 GPU",
        "value": round(args.steps / el, 1), "unit": "launches/s", "ms_per_step": round(el / args.steps * 1e3, 5),
        "dtype": "int8", "config": {"workload": "igemm", "m": M, "n": N, "k": Kd, "weight_copies_rotated": copies,
                                    "rotated_weight_bytes": copies * N * Kd},
        "roofline": {"bound": "hbm", "kernel": "igemm_i8", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for("igemm_i8", f"igemm_m{M}"), "traffic_note": TRAFFIC_NOTE,
                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(g_ms * 1e3, 3),
                     **launch_stats(prof, "igemm_i8")},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": (a, w[: N * Kd]),
    }


def bench_igemm_batched(args, ctx):
    """cfg1 batched: 64 distinct experts' gate projections (896 x 1280 each,
    73.4 MB) in one launch, each against its own M activation rows, i32 out
    accumulated (+=). The timed launches rotate over IGEMM_SETS distinct
    64-expert weight sets (587 MB), so the weights come from HBM."""
    from franken_ocr_amd import _abi, synth

    M, N, Kd, B = args.tokens, 896, 1280, 64
    w, sets = igemm_weight_sets(ctx, N, Kd)
    log(f"igemm_batched: M={M}, {B} instances per launch, {len(sets)} weight sets rotated")
    a = synth.int8_uniform(synth.seed_of(3), B * M * Kd)
    da = ctx.to_device(a)
    dout = ctx.to_device(np.zeros(B * M * N, np.int32))

    def step(i):
        _abi.call("focr_hip_igemm_s8s8_batched_dev", ctx.handle, da.c_ptr, sets[i % len(sets)].c_ptr, B, M, Kd, N,
                  dout.c_ptr)

    for i in range(max(args.warmup, len(sets))):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    g_us = kernel_us(prof, "igemm_i8_batched")
    nbytes = B * (N * Kd + M * Kd + 2 * M * N * 4)
    achieved = nbytes / (g_us * 1e-6) / 1e9
    return {
        "metric": "int8 igemm, 64 experts' gate-proj (896x1280) in one launch, launches/s, 1 GPU",
        "value": round(args.steps / el, 1), "unit": "launches/s", "ms_per_step": round(el / args.steps * 1e3, 5),
        "dtype": "int8", "config": {"workload": "igemm_batched", "m": M, "n": N, "k": Kd, "instances": B,
                                    "weight_bytes": B * N * Kd, "weight_sets_rotated": len(sets)},
        "roofline": {"bound": "hbm", "kernel": "igemm_i8_batched", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for("igemm_i8_batched", f"igemm_batched_m{M}"), "traffic_note": TRAFFIC_NOTE,
                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(g_us, 3),
                     **launch_stats(prof, "igemm_i8_batched")},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": (a, w, M),
    }


def cpu_igemm(args, inputs):
    from oracle import pyoracle

    a, w = inputs
    L = pyoracle.lib()
    tier = L.cpu_detect_tier()
    M, N, Kd = args.tokens, 896, 1280
    out = np.zeros(M * N, np.int32)
    P = pyoracle.p
    res = cpu_stats(lambda: L.cpu_igemm_s8s8(tier, P(a), P(w), M, Kd, N, P(out)), 1, "launches/s", args.cpu_seconds)
    want = pyoracle.igemm_s8s8(a, w, M, Kd, N)
    got = np.zeros(M * N, np.int32)
    L.cpu_igemm_s8s8(tier, P(a), P(w), M, Kd, N, P(got))
    res.update({"cores": 1, "kind": "port", "tier": L.cpu_tier_feature(tier).decode(),
                "matches_oracle": bool(np.array_equal(got, want)),
                "sample": f"single-thread igemm_s8s8 calls at M={M} (the tier kernel is single-threaded, x86.rs)"})
    return res


def cpu_igemm_batched(args, inputs):
    from oracle import pyoracle

    a, w, M = inputs
    L = pyoracle.lib()
    tier = L.cpu_detect_tier()
    N, Kd, B = 896, 1280, 64
    out = np.zeros(B * M * N, np.int32)
    P = pyoracle.p
    res = cpu_stats(lambda: L.cpu_igemm_s8s8_batched(tier, P(a), P(w), B, M, Kd, N, P(out)), 1, "launches/s",
                    args.cpu_seconds)
    got = np.zeros(B * M * N, np.int32)
    L.cpu_igemm_s8s8_batched(tier, P(a), P(w), B, M, Kd, N, P(got))
    same = all(np.array_equal(got[i * M * N:(i + 1) * M * N],
                              pyoracle.igemm_s8s8(a[i * M * Kd:(i + 1) * M * Kd], w[i * N * Kd:(i + 1) * N * Kd],
                                                  M, Kd, N)) for i in (0, B - 1))
    res.update({"cores": int(L.cpu_threads()), "kind": "port", "tier": L.cpu_tier_feature(tier).decode(),
                "matches_oracle": bool(same),
                "sample": f"the 64 instances' igemm_s8s8 at M={M} as one task each over all threads"})
    return res


# ---------------------------------------------------------------------------
# config 5: R-SWA decode attention
# ---------------------------------------------------------------------------

def bench_rswa(args, ctx):
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import RingCache

    import ctypes as C

    from franken_ocr_amd import _abi

    B, G, NH, D, W = 8, 1024, 10, 128, 128
    copies = args.copies
    caches = []
    rng = np.random.default_rng(7)
    ring_lens = [int(x) for x in rng.integers(0, 129, B)]
    host = []  # per stream: ref K, ref V, ring K, ring V (head-major), ring_len
    for s in range(B):
        host.append((synth.f32_normal(synth.seed_of(2000 + s), NH * G * D),
                     synth.f32_normal(synth.seed_of(2100 + s), NH * G * D),
                     synth.f32_normal(synth.seed_of(2300 + s), NH * W * D),
                     synth.f32_normal(synth.seed_of(2400 + s), NH * W * D), ring_lens[s]))
    ring_pos = [rl % W if rl < W else int(rng.integers(0, W)) for rl in ring_lens]
    for c in range(copies):
        cache = RingCache(B, G, ctx)
        for s in range(B):
            rk, rv, gk, gv, rl = host[s]
            cache.record_prefill(s, ctx.to_device(rk), ctx.to_device(rv), G)
            reg = cache.regions(s)
            for key, arr in (("ring_k", gk), ("ring_v", gv)):
                _abi.call("focr_hip_h2d", ctx.handle, C.c_void_p(reg[key]), arr.ctypes.data_as(C.c_void_p),
                          arr.nbytes)
            cache.set_state(s, rl, ring_pos[s])
        caches.append(cache)
    q_host = synth.f32_normal(synth.seed_of(2200), B * NH * D).reshape(B, NH * D)
    q = ctx.to_device(q_host)
    out = ctx.empty((B, NH * D), np.float32)

    def step(i):
        caches[i % copies].decode_attention(q, out)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    g_ms = kernel_us(prof, "rswa_chunk") * 1e-3
    caches[0].decode_attention(q, out)
    gpu_out = out.numpy()
    keys = sum(G + r for r in ring_lens)
    nbytes = 2 * NH * keys * D * 4 + 2 * B * NH * D * 4
    achieved = nbytes / (g_ms * 1e-3) / 1e9
    return {
        "metric": "R-SWA decode attention steps/s (B=8, G=1024, 10x128), 1 GPU",
        "value": round(args.steps / el, 1), "unit": "steps/s", "ms_per_step": round(el / args.steps * 1e3, 5),
        "dtype": "f32", "config": {"workload": "rswa", "streams": B, "ref_rows": G, "ring_lens": ring_lens,
                                   "cache_copies_rotated": copies},
        "roofline": {"bound": "hbm", "kernel": "rswa_chunk", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for("rswa_chunk", "rswa"), "traffic_note": TRAFFIC_NOTE,
                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(g_ms * 1e3, 3), **launch_stats(prof, "rswa_chunk")},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": (host, q_host, gpu_out, G),
    }


def cpu_rswa(args, inputs):
    """decode_attention_scalar (rswa.rs:894-939) per stream, one thread,
    the 8 streams one after another (rswa.rs:1359-1366), on the same caches
    and queries as the GPU step (the oracle's restatement, oracle/)."""
    from oracle import pyoracle

    host, q, gpu_out, G = inputs
    L, P = pyoracle.lib(), pyoracle.p
    B, NH, D, W = len(host), 10, 128, 128
    out = np.zeros((B, NH * D), np.float32)
    qs = [np.ascontiguousarray(q[s]) for s in range(B)]

    def call():
        for s, (rk, rv, gk, gv, rl) in enumerate(host):
            st = L.oracle_decode_attention(P(rk), P(rv), G, G, P(gk), P(gv), rl, P(qs[s]), P(out[s]))
            assert st == 0

    res = cpu_stats(call, 1, "steps/s", args.cpu_seconds)
    err = float(np.max(np.abs(gpu_out - out) / np.maximum(np.abs(out), np.abs(out).max() * 1e-2)))
    res.update({"cores": 1, "kind": "port", "gpu_max_rel_err": err,
                "sample": f"decode attention steps over {B} streams (ref {G} rows + ring), the streams one after "
                          f"another, one thread; gpu_max_rel_err: the GPU step's output against this one"})
    return res


# ---------------------------------------------------------------------------
# chunked prefill attention (decoder.rs:1282-1340) on the f32 matrix cores
# ---------------------------------------------------------------------------

MFMA_F32_PEAK_TFLOPS = 157.3  # dense fp32 MFMA, MI355X


def attn_flops(seq: int, heads: int = 10, head_dim: int = 128) -> float:
    # query t attends t + 1 keys: 2 * head_dim flops for its score and 2 *
    # head_dim for its share of P.V, per key and head
    return 4.0 * head_dim * heads * seq * (seq + 1) / 2


def bench_prefill_attn(args, ctx):
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import RingCache, prefill_chunk_bounds

    NH, D = 10, 128
    seq, chunk = args.tokens, args.chunk
    log(f"prefill_attn: seq={seq}, chunk={chunk} (one layer's chunked prefill into an R-SWA stream)")
    q, k, v = (synth.f32_normal(synth.seed_of(3000 + i), seq * NH * D).reshape(seq, NH * D) for i in range(3))
    dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
    bounds = prefill_chunk_bounds(seq, chunk)
    cache = RingCache(1, seq, ctx)
    out = ctx.empty((seq, NH * D), np.float32)
    views = [(c0, dq.view_rows(c0, c1), dk.view_rows(c0, c1), dv.view_rows(c0, c1), out.view_rows(c0, c1))
             for c0, c1 in bounds]

    def step(i):
        for c0, qc, kc, vc, oc in views:
            cache.prefill_chunk(0, qc, kc, vc, c0, oc)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    a_us = kernel_us(prof, "attn_prefill")  # per chunk call (attention + key-range merge)
    flops = attn_flops(seq, NH, D)
    achieved = flops / (a_us * 1e-6 * len(bounds)) / 1e12
    return {
        "metric": f"chunked prefill attention tokens/s (one layer, {seq} tokens in chunks of {chunk}, 10x128, f32), 1 GPU",
        "value": round(seq * args.steps / el, 1), "unit": "tokens/s", "ms_per_step": round(el / args.steps * 1e3, 5),
        "dtype": "f32",
        "config": {"workload": "prefill_attn", "seq": seq, "chunk": chunk, "heads": NH, "head_dim": D,
                   "chunks": len(bounds)},
        "roofline": {"bound": "mfma", "kernel": "attn_prefill", "achieved": round(achieved, 2),
                     "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / MFMA_F32_PEAK_TFLOPS, 4),
                     "traffic": traffic_for("attn_prefill", f"prefill_attn_{seq}"), "algorithmic_flops_per_step": flops,
                     "avg_launch_us": round(a_us, 3), "launches_per_step": len(bounds), **launch_stats(prof, "attn_prefill")},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": (q, k, v, chunk),
    }


def cpu_prefill_attn(args, inputs):
    from oracle import pyoracle

    q, k, v, chunk = inputs
    seq = q.shape[0]
    L, P = pyoracle.lib(), pyoracle.p
    qc = [(c0, c1, np.ascontiguousarray(q[c0:c1]), np.zeros((c1 - c0, q.shape[1]), np.float32))
          for c0, c1 in [(c0, min(c0 + chunk, seq)) for c0 in range(0, seq, chunk)]]
    kc, vc = np.ascontiguousarray(k), np.ascontiguousarray(v)

    def call():
        for c0, c1, qq, oo in qc:
            L.oracle_chunk_prefill_attention_f32(P(qq), c1 - c0, P(kc), P(vc), c1, 10, 128, c0, P(oo))

    res = cpu_stats(call, seq, "tokens/s", args.cpu_seconds, min_iters=2)
    res.update({"cores": 1, "kind": "port",
                "sample": f"whole chunked prefills of {seq} tokens (chunks of {chunk}); the f32 restatement of "
                          f"decoder.rs:1282-1340 in the reference's described order, one thread (the reference's "
                          f"ft-kernel-cpu sdpa is not in the reference tree)"})
    return res


# ---------------------------------------------------------------------------
# config 4: int4 chunked-prefill MoE expert GEMMs (matrix cores)
# ---------------------------------------------------------------------------

MFMA_INT8_PEAK_TOPS = 5000.0  # dense int8, MI355X


def make_i4_layer(seed: int, group: int = 32):
    from franken_ocr_amd import synth

    wg = synth.bytes_uniform(synth.seed_of(seed), E * I * H // 2)
    wu = synth.bytes_uniform(synth.seed_of(seed + 1), E * I * H // 2)
    wd = synth.bytes_uniform(synth.seed_of(seed + 2), E * H * I // 2)
    sg = synth.f32_uniform(synth.seed_of(seed + 3), E * I * (H // group), 1e-3, 2e-2)
    su = synth.f32_uniform(synth.seed_of(seed + 4), E * I * (H // group), 1e-3, 2e-2)
    sd = synth.f32_uniform(synth.seed_of(seed + 5), E * H * (I // group), 1e-3, 2e-2)
    return wg, sg, wu, su, wd, sd


def h5_views(ctx, layers, dx, di, dg, dout, idx, T, prof, ms, steps, gu_name, dn_name, per_expert_bytes):
    """Three views of the prefill MoE's int8 MFMA utilisation (ops /
    time / 5.0 POPS): cold (rotating layer copies, the measured step), warm
    (one layer, MALL-resident) and the compute-bound bucket (every expert at
    M_e >= 195, where ops/byte ~ 3.2 M_e: token t routes to hot[(t + j) % 8],
    j < top_k, so each of the 8 most-hit experts gets T * top_k / 8 rows;
    rotating copies). Returns (views, warm ms, warm / bucket per-kernel us)."""
    pairs = T * K
    gu_ops, dn_ops = 2.0 * pairs * 2 * I * H, 2.0 * pairs * H * I
    nw = max(steps // 2, 10)
    el_w, prof_w, kernels_w, _ = timed(ctx, lambda i: layers[0].prefill(dx, di, dg, dout, check_idx=False), nw)
    counts = np.bincount(idx.ravel(), minlength=E)
    hot = np.sort(np.argsort(-counts, kind="stable")[:8]).astype(np.uint32)
    bidx = np.ascontiguousarray(np.stack([hot[(np.arange(T) + j) % 8] for j in range(K)], axis=1))
    dbi = ctx.to_device(bidx)
    el_b, prof_b, kernels_b, _ = timed(ctx, lambda i: layers[i % len(layers)].prefill(dx, dbi, dg, dout,
                                                                                  check_idx=False), nw)
    ms_w, ms_b = el_w / nw * 1e3, el_b / nw * 1e3

    def frac(ops, us):
        return round(ops / (us * 1e-6) / 1e12 / MFMA_INT8_PEAK_TOPS, 4)

    ku = kernel_us
    views = {
        "cold_layer": frac(gu_ops + dn_ops, ms * 1e3), "warm_layer": frac(gu_ops + dn_ops, ms_w * 1e3),
        "cold_gate_up": frac(gu_ops, ku(prof, gu_name)), "warm_gate_up": frac(gu_ops, ku(prof_w, gu_name)),
        "cold_down": frac(dn_ops, ku(prof, dn_name)), "warm_down": frac(dn_ops, ku(prof_w, dn_name)),
        "bucket": {"experts": 8, "rows_per_expert": pairs // 8, "layer": frac(gu_ops + dn_ops, ms_b * 1e3),
                   "gate_up": frac(gu_ops, ku(prof_b, gu_name)), "down": frac(dn_ops, ku(prof_b, dn_name)),
                   "weight_bytes_per_step": 8 * per_expert_bytes},
    }
    return views, ms_w, kernels_w, kernels_b


def i4_mfma_ceiling(counts, achieved_tops: float) -> dict:
    """The fraction of the int8 MFMA peak the int4 grouped GEMM can reach.
    int4.rs:304-343 scales each 32-wide K group's i32 partial separately:
    acc += s[n, g] * (f32)acc_g, two VALU instructions (convert, FMA) per
    output element and group. One v_mfma_i32_32x32x32_i8 is one group of a
    32 x 32 tile: 32 cycles of the SIMD's matrix core, while its 16 elements
    per lane cost 32 VALU instructions of 4 cycles each (wave64 on 16 lanes;
    packed FP32 is not used), so the formulation is VALU-bound at 32 / 128 =
    0.25 of the MFMA peak. The row tiles (64 rows of one expert, computed as
    one or two 32-row MFMA tiles) cost their padded rows: ceiling = 0.25 x
    rows routed / rows computed."""
    computed = 0
    for c in counts:
        for t in range((int(c) + 63) // 64):
            nr = min(64, int(c) - 64 * t)
            computed += 32 if nr <= 32 else 64
    useful = int(counts.sum())
    ceil = 0.25 * useful / max(computed, 1)
    frac = achieved_tops / MFMA_INT8_PEAK_TOPS
    return {"frac": round(ceil, 4), "valu_bound_frac": 0.25, "valu_per_mfma_floor": 32, "rows_routed": useful,
            "rows_computed": computed, "achieved_of_ceiling": round(frac / ceil, 4)}


def bench_prefill_i4(args, ctx):
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import MoeLayerI4

    T, group = args.tokens, 32
    log(f"moe_prefill_i4: M={T} tokens, top-{K}, Zipf(1.1) routing, group {group}, {args.copies} layer copies")
    host = make_i4_layer(300, group)
    layers = [MoeLayerI4(H, I, E, group, *host, ctx=ctx) for _ in range(args.copies)]
    x = synth.f32_normal(synth.seed_of(350), T * H).reshape(T, H)
    idx, gates = synth.zipf_routing(synth.seed_of(360), T, E, K)
    dx, di, dg = ctx.to_device(x), ctx.to_device(idx), ctx.to_device(gates)
    dout = ctx.empty((T, H), np.float32)

    def step(i):
        layers[i % len(layers)].prefill(dx, di, dg, dout, check_idx=False)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    pairs = T * K
    gu_ops = 2.0 * pairs * 2 * I * H
    dn_ops = 2.0 * pairs * H * I
    gu_us, dn_us = kernel_us(prof, "i4_gate_up"), kernel_us(prof, "i4_down")
    gu_tops = gu_ops / (gu_us * 1e-6) / 1e12
    layer_tops = (gu_ops + dn_ops) / (ms * 1e-3) / 1e12
    counts = np.bincount(idx.ravel(), minlength=E)
    per_expert_bytes = 2 * I * H // 2 + H * I // 2 + 4 * (2 * I * (H // group) + H * (I // group))
    wbytes = int((counts > 0).sum()) * per_expert_bytes
    views, ms_w, kernels_w, kernels_b = (None, float("nan"), {}, {}) if args.no_views else h5_views(
        ctx, layers, dx, di, dg, dout, idx, T, prof, ms, args.steps, "i4_gate_up", "i4_down", per_expert_bytes)
    log(f"per-kernel avg us {kernels}; warm {kernels_w}; bucket {kernels_b}")
    return {
        "metric": "int4 chunked-prefill MoE (M=512, top-6, Zipf routing) tokens/s + int8 MFMA utilisation, 1 GPU",
        "value": round(T * args.steps / el, 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "dtype": "int4xint8",
        "config": {"workload": "moe_prefill_i4", "tokens": T, "hidden": H, "inter": I, "experts": E, "top_k": K,
                   "group": group, "routing": "zipf(1.1) without replacement", "layer_copies_rotated": args.copies,
                   "tokens_per_expert_max": int(counts.max()), "experts_hit": int((counts > 0).sum())},
        "roofline": {"bound": "mfma", "kernel": "i4_gate_up", "achieved": round(gu_tops, 2),
                     "peak": MFMA_INT8_PEAK_TOPS, "unit": "TOP/s", "frac": round(gu_tops / MFMA_INT8_PEAK_TOPS, 4),
                     "traffic": traffic_for("i4_gate_up", f"moe_prefill_i4_m{T}"),
                     "algorithmic_ops_per_launch": gu_ops, "avg_launch_us": round(gu_us, 3), **launch_stats(prof, "i4_gate_up"),
                     "mfma_ceiling": i4_mfma_ceiling(counts, gu_tops)},
        "layer_mfma": {"achieved_tops": round(layer_tops, 2), "frac": round(layer_tops / MFMA_INT8_PEAK_TOPS, 4),
                       "ops_per_step": gu_ops + dn_ops, "weight_bytes_per_step": wbytes,
                       "hbm_gbs": round(wbytes / (ms * 1e-3) / 1e9, 1),
                       "warm_ms_per_step": round(ms_w, 5)},
        # int8 MFMA utilisation three ways (ops / time / 5.0 POPS): cold, warm, the compute-bound bucket
        "mfma_utilisation": views,
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "kernel_avg_us_warm": kernels_w,
        "kernel_avg_us_bucket": kernels_b,
        "_cpu_inputs": (x, idx, gates, host),
    }


def cpu_prefill_i4(args, inputs):
    """The reference's two x86 int4 paths (int4.rs:454-460: no x86 int4 MAC
    kernel): s4s8_packed_kernel_scalar and igemm_s4s8 (AVX2 nibble unpack,
    then the per-group loop), both built -O3 by LLVM for the baseline x86-64
    ISA as rustc's release profile builds them (oracle/cpu_int4.c), run in
    moe_block's structure (experts one after another, each expert's members
    as one GEMM call). Both are timed on the first 64 tokens; the faster is
    then timed on the whole M = 512 layer and reported."""
    from oracle import pyoracle

    x, idx, gates, host = inputs
    wg, sg, wu, su, wd, sd = host
    L, P = pyoracle.lib(), pyoracle.p
    T = x.shape[0]
    idx, gates = np.ascontiguousarray(idx), np.ascontiguousarray(gates)
    out = np.zeros(T * H, np.float32)

    def run(kind, t):
        st = L.cpu_moe_prefill_i4(kind, P(np.ascontiguousarray(x[:t])), t, H, I, E, K, P(idx), P(gates), 32, P(wg),
                                  P(sg), P(wu), P(su), P(wd), P(sd), P(out))
        assert st == 0

    sample_t = min(64, T)
    names = ("s4s8_packed_kernel_scalar", "igemm_s4s8 (avx2 unpack + per-group loop)")
    probe = {}
    for kind, name in enumerate(names):
        t0 = time.perf_counter()
        run(kind, sample_t)
        probe[name] = round(sample_t / (time.perf_counter() - t0), 2)
    kind = max(range(len(names)), key=lambda k_: probe[names[k_]])
    res = cpu_stats(lambda: run(kind, T), T, "tokens/s", args.cpu_seconds, min_iters=2)
    n_check = min(16, T)
    st, want, _, _ = pyoracle.moe_prefill_i4(x[:n_check], idx[:n_check], gates[:n_check], 32, *host, E, I)
    same = st == 0 and np.array_equal(out.reshape(T, H)[:n_check], want)
    res.update({"cores": 1, "kind": "port", "tier": names[kind],
                "paths_probed_tokens_per_s": probe, "matches_oracle": bool(same),
                "sample": f"whole M={T} int4 MoE layers with the faster path (both probed on {sample_t} tokens); "
                          f"one thread, experts one after another; matches_oracle on the first {n_check} rows"})
    return res


# ---------------------------------------------------------------------------
# prefill on int8 weights (int8 matrix cores): the dense linear and the MoE block
# ---------------------------------------------------------------------------

_INT_MM_CHILD = """
import sys, torch
M, N, K, steps = map(int, sys.argv[1:5])
a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda")
b = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda").t()  # [K, N], K contiguous
for _ in range(3):
    torch._int_mm(a, b)
torch.cuda.synchronize()
e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
e0.record()
for _ in range(steps):
    torch._int_mm(a, b)
e1.record()
torch.cuda.synchronize()
print(e0.elapsed_time(e1) * 1e3 / steps)
"""


def library_int_mm_us(M: int, N: int, K: int, steps: int) -> float:
    """The platform library's int8 GEMM at the same shape, as a reference
    point: torch._int_mm (hipBLASLt; int8 x int8 -> int32, no scales), timed
    with torch's events. It runs in a child process: torch ships its own HIP
    runtime, which finds no device in a process where this library's runtime
    already holds it. Not the product path."""
    import subprocess

    r = subprocess.run([sys.executable, "-c", _INT_MM_CHILD, str(M), str(N), str(K), str(steps)],
                       capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        raise RuntimeError(f"library int8 GEMM child failed ({r.returncode}): {r.stderr[-500:]}")
    return float(r.stdout.strip().splitlines()[-1])


def bench_linear_i8(args, ctx):
    """nn::linear_int8_dynamic at the dense layer-0 MLP gate shape (N = 6848,
    K = 1280) over M prefill rows: dynamic-rule quantize + int8 MFMA GEMM."""
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import QInt8, linear_i8_dynamic

    M, N, Kd = args.tokens, 6848, H
    log(f"linear_i8: M={M} N={N} K={Kd}, {args.copies} weight copies")
    w = synth.int8_uniform(synth.seed_of(700), N * Kd)
    ws = synth.f32_uniform(synth.seed_of(701), N, 1e-3, 2e-2)
    qs = [QInt8(w, ws, N, Kd, ctx) for _ in range(args.copies)]
    x = synth.f32_normal(synth.seed_of(702), M * Kd).reshape(M, Kd)
    dx, dy = ctx.to_device(x), ctx.empty((M, N), np.float32)

    def step(i):
        linear_i8_dynamic(qs[i % len(qs)], dx, dy)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    ops = 2.0 * M * N * Kd
    g_us = kernel_us(prof, "linear_i8")
    tops = ops / (g_us * 1e-6) / 1e12
    log(f"per-kernel avg us {kernels}")
    lib = None
    if args.library_ref:
        lib_us = library_int_mm_us(M, N, Kd, args.steps)
        lib = {"impl": "torch._int_mm (hipBLASLt), int8 x int8 -> int32", "avg_launch_us": round(lib_us, 3),
               "frac": round(ops / (lib_us * 1e-6) / 1e12 / MFMA_INT8_PEAK_TOPS, 4)}
        log(f"library int8 GEMM at the same shape: {lib}")
    return {
        "metric": "prefill int8 linear (linear_int8_dynamic) rows/s + int8 MFMA utilisation, 1 GPU",
        "value": round(M * args.steps / el, 1), "unit": "rows/s", "ms_per_step": round(ms, 5), "dtype": "int8",
        "config": {"workload": "linear_i8", "rows": M, "n": N, "k": Kd, "weight_copies_rotated": args.copies},
        "roofline": {"bound": "mfma", "kernel": "linear_i8", "achieved": round(tops, 2),
                     "peak": MFMA_INT8_PEAK_TOPS, "unit": "TOP/s", "frac": round(tops / MFMA_INT8_PEAK_TOPS, 4),
                     "traffic": traffic_for("linear_i8", f"linear_i8_m{M}"),
                     "algorithmic_ops_per_launch": ops, "avg_launch_us": round(g_us, 3), **launch_stats(prof, "linear_i8")},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        **({"library_ref": lib} if lib else {}),
        "_cpu_inputs": (x, w, ws),
    }


def cpu_linear_i8(args, inputs):
    """nn::linear_int8_dynamic (nn.rs:151-173) on the best int8 tier: the
    dynamic-rule row quantize, then the i32 products in 64-output-row blocks
    over all host threads and the dequant (oracle/cpu_tier.c; ft-kernel-cpu's
    own kernel is not in the reference tree). Timed on 512-row slices."""
    from oracle import pyoracle

    x, w, ws = inputs
    L, P = pyoracle.lib(), pyoracle.p
    tier = L.cpu_detect_tier()
    N, Kd = ws.shape[0], x.shape[1]
    rows = min(512, x.shape[0])
    xs = np.ascontiguousarray(x[:rows])
    y = np.zeros((rows, N), np.float32)
    res = cpu_stats(lambda: L.cpu_linear_i8_dynamic(tier, P(xs), rows, Kd, P(w), P(ws), N, P(y)), rows, "rows/s",
                    args.cpu_seconds)
    st, want, _, _ = pyoracle.linear_i8_dynamic(xs[:8], w, ws, N)
    res.update({"cores": int(L.cpu_threads()), "kind": "port", "tier": L.cpu_tier_feature(tier).decode(),
                "matches_oracle": bool(st == 0 and np.array_equal(y[:8], want)),
                "sample": f"linear_int8_dynamic over {rows}-row slices of the {x.shape[0]}-row input, "
                          f"{N}x{Kd} weights; matches_oracle on the first 8 rows"})
    return res


def bench_prefill_i8(args, ctx):
    """moe_block_i8 over M prefill rows with Zipf(1.1) top-6 routing (config
    4's routing) on the int8 MoE layer the decode path uses."""
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import MoeLayer

    T = args.tokens
    log(f"moe_prefill_i8: M={T} tokens, top-{K}, Zipf(1.1) routing, {args.copies} layer copies")
    base = make_moe_host(100)
    layers = [MoeLayer(H, I, E, K, *base, ctx=ctx) for _ in range(args.copies)]
    x = synth.f32_normal(synth.seed_of(350), T * H).reshape(T, H)
    idx, gates = synth.zipf_routing(synth.seed_of(360), T, E, K)
    dx, di, dg = ctx.to_device(x), ctx.to_device(idx), ctx.to_device(gates)
    dout = ctx.empty((T, H), np.float32)

    def step(i):
        layers[i % len(layers)].prefill(dx, di, dg, dout, check_idx=False)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    pairs = T * K
    gu_ops = 2.0 * pairs * 2 * I * H
    dn_ops = 2.0 * pairs * H * I
    gu_us = kernel_us(prof, "i8_gate_up")
    gu_tops = gu_ops / (gu_us * 1e-6) / 1e12
    layer_tops = (gu_ops + dn_ops) / (ms * 1e-3) / 1e12
    counts = np.bincount(idx.ravel(), minlength=E)
    per_expert_bytes = 3 * I * H + 4 * (2 * I + H)
    wbytes = int((counts > 0).sum()) * per_expert_bytes
    views, ms_w, kernels_w, kernels_b = (None, float("nan"), {}, {}) if args.no_views else h5_views(
        ctx, layers, dx, di, dg, dout, idx, T, prof, ms, args.steps, "i8_gate_up", "i8_down", per_expert_bytes)
    log(f"per-kernel avg us {kernels}; warm {kernels_w}; bucket {kernels_b}")
    return {
        "metric": "int8 chunked-prefill MoE (M=512, top-6, Zipf routing) tokens/s + int8 MFMA utilisation, 1 GPU",
        "value": round(T * args.steps / el, 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "dtype": "int8",
        "config": {"workload": "moe_prefill_i8", "tokens": T, "hidden": H, "inter": I, "experts": E, "top_k": K,
                   "routing": "zipf(1.1) without replacement", "layer_copies_rotated": args.copies,
                   "tokens_per_expert_max": int(counts.max()), "experts_hit": int((counts > 0).sum())},
        "roofline": {"bound": "mfma", "kernel": "i8_gate_up", "achieved": round(gu_tops, 2),
                     "peak": MFMA_INT8_PEAK_TOPS, "unit": "TOP/s", "frac": round(gu_tops / MFMA_INT8_PEAK_TOPS, 4),
                     "traffic": traffic_for("i8_gate_up", f"moe_prefill_i8_m{T}"),
                     "algorithmic_ops_per_launch": gu_ops, "avg_launch_us": round(gu_us, 3), **launch_stats(prof, "i8_gate_up")},
        "layer_mfma": {"achieved_tops": round(layer_tops, 2), "frac": round(layer_tops / MFMA_INT8_PEAK_TOPS, 4),
                       "ops_per_step": gu_ops + dn_ops, "weight_bytes_per_step": wbytes,
                       "hbm_gbs": round(wbytes / (ms * 1e-3) / 1e9, 1),
                       "warm_ms_per_step": round(ms_w, 5)},
        # int8 MFMA utilisation three ways (ops / time / 5.0 POPS): cold, warm, the compute-bound bucket
        "mfma_utilisation": views,
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "kernel_avg_us_warm": kernels_w,
        "kernel_avg_us_bucket": kernels_b,
        "_cpu_inputs": None,
    }


# ---------------------------------------------------------------------------
# one decoder layer's decode step (MoE layer + shared expert, R-SWA attention)
# ---------------------------------------------------------------------------

def bench_decode_layer(args, ctx):
    """decode_step_with_cache_i8 for one MoE layer over B streams (each with a
    1024-token reference block and a ring filled by the warm-up steps):
    RMSNorm, qkv GEMV, RoPE, ring write + R-SWA, o_proj, residual + RMSNorm,
    MoE (route_default + the 1792-wide shared expert), residual. Layer copies
    (each with its own weights and caches) rotate so weights come from HBM."""
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import DecoderLayer, MoeLayer, QInt8, RingCache

    B, G, D, SI = args.tokens, 1024, 1280, 1792
    log(f"decode_layer: {B} streams, ref {G} tokens, {args.copies} layer copies")
    base = make_moe_host(100)
    sh = [synth.int8_uniform(synth.seed_of(800), SI * H), synth.f32_uniform(synth.seed_of(801), SI, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(802), SI * H), synth.f32_uniform(synth.seed_of(803), SI, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(804), H * SI), synth.f32_uniform(synth.seed_of(805), H, 1e-3, 2e-2)]
    wqkv = synth.int8_uniform(synth.seed_of(806), 3 * D * H)
    sqkv = synth.f32_uniform(synth.seed_of(807), 3 * D, 1e-3, 2e-2)
    wo = synth.int8_uniform(synth.seed_of(808), H * D)
    so = synth.f32_uniform(synth.seed_of(809), H, 1e-3, 2e-2)
    ln1 = synth.f32_uniform(synth.seed_of(810), H, 0.5, 1.5)
    ln2 = synth.f32_uniform(synth.seed_of(811), H, 0.5, 1.5)
    kv_host = [synth.f32_normal(synth.seed_of(820 + i), 10 * G * 128) for i in range(2)]
    kv = [ctx.to_device(a) for a in kv_host]
    layers, caches = [], []
    for c in range(args.copies):
        router = synth.f32_normal(synth.seed_of(1000 + c), E * H, 0.0, 0.02).reshape(E, H)
        moe = MoeLayer(H, I, E, K, router, *base[1:], ctx=ctx)
        moe.set_shared(SI, *sh)
        layers.append(DecoderLayer(H, ln1, ln2, QInt8(wqkv, sqkv, 3 * D, H, ctx), QInt8(wo, so, H, D, ctx), moe=moe,
                                   ctx=ctx))
        cache = RingCache(B, G, ctx=ctx)
        for s in range(B):
            cache.record_prefill(s, kv[0], kv[1], G)
        caches.append(cache)
    x_host = synth.f32_normal(synth.seed_of(830), B * H).reshape(B, H)
    x = ctx.to_device(x_host)
    idx = [ctx.empty((B, K), np.uint32) for _ in layers]
    pos = np.full(B, G, np.uint32)
    n = len(layers)

    def step(i):
        j = i % n
        layers[j].step(caches[j], pos + i // n, x, idx[j], check_route=False)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    # distinct experts of each copy's last step (every copy has run by now)
    U = [len(np.unique(b.numpy())) for b in idx[:min(n, args.warmup + 2 * args.steps)]]
    ring = min(128, (args.warmup + 2 * args.steps) // n)  # about where the rings are during the timed passes
    keys = G + ring
    mean_u = float(np.mean(U))
    attn_bytes = B * 2 * 10 * keys * 128 * 4
    w_bytes = (3 * D * H + 3 * D * 4) + (H * D + H * 4) + mean_u * (3 * I * H + 2 * I * 4 + H * 4) + \
        (3 * SI * H + 2 * SI * 4 + H * 4) + E * H * 4
    layer_bytes = w_bytes + attn_bytes + 2 * B * H * 4
    gbs = layer_bytes / (ms * 1e-3) / 1e9
    log(f"U per copy {U}; per-kernel avg us {kernels}")
    return {
        "metric": "decoder-layer decode step tokens/s + achieved HBM GB/s (% of 8 TB/s peak), 1 GPU",
        "value": round(B * args.steps / el, 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "dtype": "int8",
        "config": {"workload": "decode_layer", "streams": B, "ref_tokens": G, "ring_tokens_approx": ring,
                   "hidden": H, "heads": 10, "head_dim": 128, "experts": E, "top_k": K, "inter": I,
                   "shared_inter": SI, "layer_copies_rotated": n, "distinct_experts_mean": mean_u},
        "roofline": {"bound": "hbm", "kernel": "layer (all kernels)", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_step": int(layer_bytes), "avg_step_us": round(ms * 1e3, 3)},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": dict(x=x_host, kv=kv_host, G=G, base=base, sh=sh, wqkv=wqkv, sqkv=sqkv, wo=wo, so=so, ln1=ln1, ln2=ln2, SI=SI),
    }


def cpu_decode_layer(args, inputs):
    """One layer of batched_decode_step_i8_streams (decoder.rs:2812-2933) on
    the host: M = B GEMVs on the best int8 tier over all threads, RoPE, ring
    write and R-SWA decode attention per stream (single thread, streams one
    after another), the MoE (top-6 + shared expert as concurrent serial
    tasks, tokens one after another) — oracle/cpu_tier.c
    cpu_decoder_layer_step, the same weights as layer copy 0 and 1024-token
    reference blocks."""
    import ctypes as C

    from franken_ocr_amd import synth
    from oracle import pyoracle

    d = inputs
    L, P = pyoracle.lib(), pyoracle.p
    tier = L.cpu_detect_tier()
    x0, G = d["x"], d["G"]
    B = x0.shape[0]
    _, wg, sg, wu, su, wd, sd = d["base"]
    router = synth.f32_normal(synth.seed_of(1000), E * H, 0.0, 0.02).reshape(E, H)
    rings = [pyoracle.Ring(G) for _ in range(B)]
    for r in rings:
        r.record_prefill(d["kv"][0], d["kv"][1], G)

    def ptrs(name):
        return (C.c_void_p * B)(*[getattr(r, name).ctypes.data for r in rings])

    refk, refv, ringk, ringv = ptrs("ref_k"), ptrs("ref_v"), ptrs("ring_k"), ptrs("ring_v")
    plen = np.full(B, G, np.uint32)
    rlen = np.zeros(B, np.uint32)
    rpos = np.zeros(B, np.uint32)
    x = np.array(x0, np.float32)
    sh = [P(a) for a in d["sh"]]
    step = [0]

    def call():
        x[:] = x0
        pos = np.full(B, G + step[0], np.uint32)
        step[0] += 1
        st = L.cpu_decoder_layer_step(tier, P(x), B, P(pos), refk, refv, G, P(plen), ringk, ringv, P(rlen), P(rpos),
                                      P(d["ln1"]), P(d["ln2"]), 1e-6, 10000.0, P(d["wqkv"]), P(d["sqkv"]),
                                      P(d["wo"]), P(d["so"]), P(router), E, K, I, P(wg), P(sg), P(wu), P(su), P(wd),
                                      P(sd), *sh, d["SI"])
        assert st == 0

    res = cpu_stats(call, B, "tokens/s", args.cpu_seconds)
    res.update({"cores": int(L.cpu_threads()), "kind": "port", "tier": L.cpu_tier_feature(tier).decode(),
                "sample": f"decoder-layer decode steps over {B} streams (1024-token reference blocks, rings "
                          f"filling); parity of this composition with the oracle's: tests/test_cpu_baseline.py"})
    return res


# ---------------------------------------------------------------------------
# one decoder layer over a chunked prefill (the MoE layer + shared expert)
# ---------------------------------------------------------------------------

def bench_prefill_layer(args, ctx):
    """One MoE decoder layer of prefill_with_cache_i8_chunked (decoder.rs:
    2461-2486) over a `tokens`-token sequence in chunks of `chunk`, each chunk
    one focr_hip_decoder_layer_prefill call: RMSNorm, the fused qkv int8 GEMM,
    RoPE, the chunk's K / V into the stream's reference block and its causal
    attention, o_proj, residual + RMSNorm, route_default, the 64 routed
    experts (top-6) and the 1792-wide shared expert on the matrix cores,
    residual. Every step restores the layer input with one device copy (the
    layer updates its rows in place), inside the timed region. Layer copies
    rotate so weights come from HBM."""
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import DecoderLayer, MoeLayer, QInt8, RingCache, prefill_chunk_bounds

    seq, chunk, D, SI = args.tokens, args.chunk, 1280, 1792
    log(f"prefill_layer: seq={seq}, chunk={chunk}, {args.copies} layer copies")
    base = make_moe_host(100)
    sh = [synth.int8_uniform(synth.seed_of(800), SI * H), synth.f32_uniform(synth.seed_of(801), SI, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(802), SI * H), synth.f32_uniform(synth.seed_of(803), SI, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(804), H * SI), synth.f32_uniform(synth.seed_of(805), H, 1e-3, 2e-2)]
    wqkv = synth.int8_uniform(synth.seed_of(806), 3 * D * H)
    sqkv = synth.f32_uniform(synth.seed_of(807), 3 * D, 1e-3, 2e-2)
    wo = synth.int8_uniform(synth.seed_of(808), H * D)
    so = synth.f32_uniform(synth.seed_of(809), H, 1e-3, 2e-2)
    ln1 = synth.f32_uniform(synth.seed_of(810), H, 0.5, 1.5)
    ln2 = synth.f32_uniform(synth.seed_of(811), H, 0.5, 1.5)
    layers, keep = [], []
    routers = []
    for c in range(args.copies):
        router = synth.f32_normal(synth.seed_of(1000 + c), E * H, 0.0, 0.02).reshape(E, H)
        routers.append(router)
        moe = MoeLayer(H, I, E, K, router, *base[1:], ctx=ctx)
        moe.set_shared(SI, *sh)
        qkv, o = QInt8(wqkv, sqkv, 3 * D, H, ctx), QInt8(wo, so, H, D, ctx)
        keep += [moe, qkv, o]
        layers.append(DecoderLayer(H, ln1, ln2, qkv, o, moe=moe, ctx=ctx))
    caches = [RingCache(1, seq, ctx=ctx) for _ in layers]
    x_host = synth.f32_normal(synth.seed_of(830), seq * H).reshape(seq, H)
    x0 = ctx.to_device(x_host)
    x = ctx.empty((seq, H), np.float32)
    idx = ctx.empty((seq, K), np.uint32)
    bounds = prefill_chunk_bounds(seq, chunk)
    views = [(c0, x.view_rows(c0, c1), idx.view_rows(c0, c1)) for c0, c1 in bounds]
    n = len(layers)

    def step(i):
        j = i % n
        x.copy_from_device(x0)
        for c0, xc, ic in views:
            layers[j].prefill(caches[j], 0, xc, c0, ic, check_route=False)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    # layer copy 0 once more for the CPU leg's comparison
    step(0)
    gpu_out = x.numpy()
    counts = np.bincount(idx.numpy().ravel(), minlength=E)
    # algorithmic work per step: int8 products (2 ops per multiply-add) and
    # the attention's f32 flops
    ops = {"linear_i8": 2.0 * seq * (3 * D * H + H * D),
           "i8_gate_up": 2.0 * seq * K * 2 * I * H, "i8_down": 2.0 * seq * K * H * I,
           "i8_shared": 2.0 * seq * 3 * SI * H}
    flops = {"attn_prefill": attn_flops(seq), "moe_route": 2.0 * seq * E * H}
    peak = {k: MFMA_INT8_PEAK_TOPS for k in ops}
    peak.update({k: MFMA_F32_PEAK_TFLOPS for k in flops})
    work = {**ops, **flops}
    n_stat = max(args.steps, STAT_STEPS)  # steps of timed()'s per-kernel pass
    per_step = {k: (prof[k]["ms"] / n_stat if k in prof else float("nan")) for k in work}
    ideal_ms = sum(work[k] / (peak[k] * 1e12) * 1e3 for k in work)
    int8_ops = sum(ops.values())
    util = {
        "int8_ops_per_step": int8_ops, "f32_flops_per_step": sum(flops.values()),
        "ideal_ms_at_peak": round(ideal_ms, 5),
        # the fraction of the step a machine at MI355X's dense peaks would need
        # for the same products (int8 at 5.0 POP/s, f32 at 157.3 TFLOP/s)
        "frac_of_step": round(ideal_ms / ms, 4),
        "int8_tops_over_step": round(int8_ops / (ms * 1e-3) / 1e12, 2),
        "per_kernel": {k: {"ms_per_step": round(per_step[k], 5),
                           "achieved": round(work[k] / (per_step[k] * 1e-3) / 1e12, 2),
                           "unit": "TOP/s" if k in ops else "TFLOP/s",
                           "frac": round(work[k] / (per_step[k] * 1e-3) / 1e12 / peak[k], 4)}
                       for k in work if per_step[k] == per_step[k]},
    }
    top = max((k for k in ops if k in prof), key=lambda k: per_step[k])
    launches = max(prof[top]["count"] // n_stat, 1)
    t_us = kernel_us(prof, top)
    ach = work[top] / launches / (t_us * 1e-6) / 1e12
    log(f"per-kernel avg us {kernels}")
    return {
        "metric": f"chunked-prefill decoder layer tokens/s (one MoE layer, {seq} tokens in chunks of {chunk}) + "
                  f"MFMA utilisation, 1 GPU",
        "value": round(seq * args.steps / el, 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "dtype": "int8",
        "config": {"workload": "prefill_layer", "seq": seq, "chunk": chunk, "chunks": len(bounds), "hidden": H,
                   "heads": 10, "head_dim": 128, "experts": E, "top_k": K, "inter": I, "shared_inter": SI,
                   "layer_copies_rotated": n, "experts_hit": int((counts > 0).sum()),
                   "tokens_per_expert_max": int(counts.max())},
        "roofline": {"bound": "mfma", "kernel": top, "achieved": round(ach, 2), "peak": MFMA_INT8_PEAK_TOPS,
                     "unit": "TOP/s", "frac": round(ach / MFMA_INT8_PEAK_TOPS, 4),
                     "traffic": traffic_for(top, f"prefill_layer_{seq}_c{chunk}"),
                     "algorithmic_ops_per_launch": work[top] / launches, "avg_launch_us": round(t_us, 3),
                     **launch_stats(prof, top)},
        "mfma_utilisation": util,
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": dict(x=x_host, gpu_out=gpu_out, chunk=chunk, base=base, sh=sh, wqkv=wqkv, sqkv=sqkv, wo=wo,
                            so=so, ln1=ln1, ln2=ln2, router=routers[0], SI=SI),
    }


def cpu_prefill_layer(args, inputs):
    """The same layer over the same sequence on the host: linear_int8_dynamic
    (nn.rs:151-173) on the best int8 tier over all threads for qkv, o_proj,
    every expert's gate / up / down and the shared expert's, moe_block_i8's
    gather / scatter (decoder.rs:2142-2181) in numpy, RMSNorm / RoPE /
    route_default from the oracle's C, and the chunk's causal attention by
    the f32 restatement of decoder.rs:1282-1340 on one thread."""
    from oracle import pyoracle as O

    d = inputs
    L, P = O.lib(), O.p
    tier = L.cpu_detect_tier()
    x0, chunk, SI = d["x"], d["chunk"], d["SI"]
    seq, Dm = x0.shape[0], 1280
    _, wg, sg, wu, su, wd, sd = d["base"]
    swg, ssg, swu, ssu, swd, ssd = d["sh"]
    router = d["router"]

    def lin(a, w, ws, n):
        a = np.ascontiguousarray(a, np.float32)
        y = np.empty((a.shape[0], n), np.float32)
        L.cpu_linear_i8_dynamic(tier, P(a), a.shape[0], a.shape[1], P(w), P(ws), n, P(y))
        return y

    def silu_mul(g, u):
        with np.errstate(over="ignore"):  # exp(-g) overflows to inf for g < -88: silu -> -0
            return (g / (1.0 + np.exp(-g)) * u).astype(np.float32)

    def layer():
        x = np.array(x0, np.float32)
        kall = np.zeros((seq, Dm), np.float32)
        vall = np.zeros((seq, Dm), np.float32)
        for c0 in range(0, seq, chunk):
            c1 = min(seq, c0 + chunk)
            xc = x[c0:c1]
            qkv = lin(O.rms_norm(xc, d["ln1"]), d["wqkv"], d["sqkv"], 3 * Dm)
            q = np.stack([O.rope(qkv[r, :Dm], c0 + r) for r in range(c1 - c0)])
            kall[c0:c1] = np.stack([O.rope(qkv[r, Dm:2 * Dm], c0 + r) for r in range(c1 - c0)])
            vall[c0:c1] = qkv[:, 2 * Dm:]
            cx = np.zeros((c1 - c0, Dm), np.float32)
            L.oracle_chunk_prefill_attention_f32(P(q), c1 - c0, P(kall), P(vall), c1, 10, 128, c0, P(cx))
            h = (xc + lin(cx, d["wo"], d["so"], H)).astype(np.float32)
            n2 = O.rms_norm(h, d["ln2"])
            st, idx, gates, _ = O.route(n2, router, E, K, norm_topk=False, routed_scale=1.0)
            assert st == 0
            mlp = np.zeros_like(h)
            for e in np.unique(idx):
                rows, slots = np.nonzero(idx == e)
                sub = n2[rows]
                a = silu_mul(lin(sub, wg[e * I * H:(e + 1) * I * H], sg[e * I:(e + 1) * I], I),
                             lin(sub, wu[e * I * H:(e + 1) * I * H], su[e * I:(e + 1) * I], I))
                y = lin(a, wd[e * H * I:(e + 1) * H * I], sd[e * H:(e + 1) * H], H)
                np.add.at(mlp, rows, gates[rows, slots][:, None] * y)
            a = silu_mul(lin(n2, swg, ssg, SI), lin(n2, swu, ssu, SI))
            mlp += lin(a, swd, ssd, H)
            x[c0:c1] = h + mlp
        return x

    out = [None]

    def call():
        out[0] = layer()

    res = cpu_stats(call, seq, "tokens/s", args.cpu_seconds, min_iters=2)
    got, want = d["gpu_out"], out[0]
    rr = (np.abs(got.astype(np.float64) - want) /
          np.maximum(np.abs(want), np.abs(want).max(axis=1, keepdims=True) * 1e-2)).max(axis=1)
    res.update({"cores": int(L.cpu_threads()), "kind": "port", "tier": L.cpu_tier_feature(tier).decode(),
                "gpu_rows_within_1e-3": round(float((rr <= 1e-3).mean()), 4),
                "sample": f"whole layer passes over {seq} tokens in chunks of {chunk} (int8 products over all "
                          f"threads, the attention on one); gpu_rows_within_1e-3 compares the GPU's output rows"})
    return res


def bench_decode_step(args, ctx):
    """One decode token for B streams through the whole decoder in one call
    (focr_hip_decoder_step): 12 layers (decoder.rs:2542-2627 per layer; layer
    0 the 6848-wide dense MLP, layers 1-11 MoE with the 1792-wide shared
    expert), the final RMSNorm and the 129280-row LM head + argmax
    (decoder.rs:2275-2296; sampler.rs:168-186).
    Each stream has a 1024-token reference block; every layer has its own
    weights and cache. The step's input row stands in for the token-embedding
    lookup (the embedding table is outside this path)."""
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import Decoder, DecoderLayer, MoeLayer, QInt8, RingCache

    B, G, D, SI, ID, V, NL = args.tokens, 1024, 1280, 1792, 6848, 129280, 12
    log(f"decode_step: {B} streams, {NL} layers, ref {G} tokens")
    base = make_moe_host(100)
    sh = [synth.int8_uniform(synth.seed_of(800), SI * H), synth.f32_uniform(synth.seed_of(801), SI, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(802), SI * H), synth.f32_uniform(synth.seed_of(803), SI, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(804), H * SI), synth.f32_uniform(synth.seed_of(805), H, 1e-3, 2e-2)]
    wqkv = synth.int8_uniform(synth.seed_of(806), 3 * D * H)
    sqkv = synth.f32_uniform(synth.seed_of(807), 3 * D, 1e-3, 2e-2)
    wo = synth.int8_uniform(synth.seed_of(808), H * D)
    so = synth.f32_uniform(synth.seed_of(809), H, 1e-3, 2e-2)
    ln = [synth.f32_uniform(synth.seed_of(810 + i), H, 0.5, 1.5) for i in range(3)]
    kv = [ctx.to_device(synth.f32_normal(synth.seed_of(820 + i), 10 * G * 128)) for i in range(2)]
    dense = [synth.int8_uniform(synth.seed_of(840), ID * H), synth.f32_uniform(synth.seed_of(841), ID, 1e-3, 2e-2),
             synth.int8_uniform(synth.seed_of(842), ID * H), synth.f32_uniform(synth.seed_of(843), ID, 1e-3, 2e-2),
             synth.int8_uniform(synth.seed_of(844), H * ID), synth.f32_uniform(synth.seed_of(845), H, 1e-3, 2e-2)]
    layers, caches = [], []
    for l in range(NL):
        qkv, o = QInt8(wqkv, sqkv, 3 * D, H, ctx), QInt8(wo, so, H, D, ctx)
        if l == 0:
            mlp = dict(dense=(QInt8(dense[0], dense[1], ID, H, ctx), QInt8(dense[2], dense[3], ID, H, ctx),
                              QInt8(dense[4], dense[5], H, ID, ctx)))
        else:
            router = synth.f32_normal(synth.seed_of(1000 + l), E * H, 0.0, 0.02).reshape(E, H)
            moe = MoeLayer(H, I, E, K, router, *base[1:], ctx=ctx)
            moe.set_shared(SI, *sh)
            mlp = dict(moe=moe)
        layers.append(DecoderLayer(H, ln[0], ln[1], qkv, o, ctx=ctx, **mlp))
        cache = RingCache(B, G, ctx=ctx)
        for st in range(B):
            cache.record_prefill(st, kv[0], kv[1], G)
        caches.append(cache)
    lm = QInt8(synth.int8_uniform(synth.seed_of(850), V * H), synth.f32_uniform(synth.seed_of(851), V, 1e-3, 2e-2), V,
               H, ctx)
    dec = Decoder(layers, ln[2], lm, ctx=ctx)
    x0 = ctx.to_device(synth.f32_normal(synth.seed_of(830), B * H).reshape(B, H))
    x = ctx.empty((B, H), np.float32)
    tok = ctx.empty((B,), np.uint32)
    pos = np.full(B, G, np.uint32)
    ridx = ctx.empty((NL, B, K), np.uint32)

    def step(i):
        x.copy_from_device(x0)  # stands in for the embedding lookup of the previous token
        dec.step(caches, pos + i, x, tok, route_idx=ridx)  # one call: 12 layers, final norm, LM head, argmax

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    U = [len(np.unique(ridx.numpy()[l])) for l in range(1, NL)]
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    keys = G + min(128, args.warmup + args.steps)  # the rings' fill during the timed pass
    attn = B * 2 * 10 * keys * 128 * 4
    proj = (3 * D * H + 3 * D * 4) + (H * D + H * 4)
    moe_b = sum(u * (3 * I * H + 2 * I * 4 + H * 4) for u in U) + \
        (NL - 1) * ((3 * SI * H + 2 * SI * 4 + H * 4) + E * H * 4)
    dense_b = 3 * ID * H + 2 * ID * 4 + H * 4
    step_bytes = NL * (proj + attn) + moe_b + dense_b + (V * H + V * 4)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"distinct experts per MoE layer {U}; per-kernel avg us {kernels}")
    return {
        "metric": "full decode step (12 layers + LM head) tokens/s, 1 GPU",
        "value": round(B * args.steps / el, 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "dtype": "int8",
        "config": {"workload": "decode_step", "streams": B, "layers": NL, "ref_tokens": G, "hidden": H,
                   "experts": E, "top_k": K, "vocab": V, "dense_inter": ID, "shared_inter": SI},
        "roofline": {"bound": "hbm", "kernel": "the whole step", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_step": int(step_bytes), "avg_step_us": round(ms * 1e3, 3)},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": None,
    }


def bench_prefill(args, ctx):
    """The whole prefill of one stream in one call (focr_hip_decoder_prefill:
    prefill_with_cache_i8_chunked, decoder.rs:2428-2520): a `tokens`-token
    sequence in chunks of `chunk` (0: the monolithic schedule) through 12
    layers (layer 0 the 6848-wide dense MLP, layers 1-11 MoE with the
    1792-wide shared expert, every layer its own weights and cache), then the
    final RMSNorm + LM head + argmax of the last row (the first generated
    token). Every step restores the input embeddings with one device copy,
    inside the timed region."""
    from franken_ocr_amd import synth
    from franken_ocr_amd.engine import Decoder, DecoderLayer, MoeLayer, QInt8, RingCache, prefill_chunk_bounds

    seq, chunk, D, SI, ID, V, NL = args.tokens, args.chunk, 1280, 1792, 6848, 129280, 12
    log(f"prefill: seq={seq}, chunk={chunk or 'monolithic'}, {NL} layers")
    base = make_moe_host(100)
    sh = [synth.int8_uniform(synth.seed_of(800), SI * H), synth.f32_uniform(synth.seed_of(801), SI, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(802), SI * H), synth.f32_uniform(synth.seed_of(803), SI, 1e-3, 2e-2),
          synth.int8_uniform(synth.seed_of(804), H * SI), synth.f32_uniform(synth.seed_of(805), H, 1e-3, 2e-2)]
    wqkv = synth.int8_uniform(synth.seed_of(806), 3 * D * H)
    sqkv = synth.f32_uniform(synth.seed_of(807), 3 * D, 1e-3, 2e-2)
    wo = synth.int8_uniform(synth.seed_of(808), H * D)
    so = synth.f32_uniform(synth.seed_of(809), H, 1e-3, 2e-2)
    ln = [synth.f32_uniform(synth.seed_of(810 + i), H, 0.5, 1.5) for i in range(3)]
    dense = [synth.int8_uniform(synth.seed_of(840), ID * H), synth.f32_uniform(synth.seed_of(841), ID, 1e-3, 2e-2),
             synth.int8_uniform(synth.seed_of(842), ID * H), synth.f32_uniform(synth.seed_of(843), ID, 1e-3, 2e-2),
             synth.int8_uniform(synth.seed_of(844), H * ID), synth.f32_uniform(synth.seed_of(845), H, 1e-3, 2e-2)]
    layers, caches = [], []
    for l in range(NL):
        qkv, o = QInt8(wqkv, sqkv, 3 * D, H, ctx), QInt8(wo, so, H, D, ctx)
        if l == 0:
            mlp = dict(dense=(QInt8(dense[0], dense[1], ID, H, ctx), QInt8(dense[2], dense[3], ID, H, ctx),
                              QInt8(dense[4], dense[5], H, ID, ctx)))
        else:
            router = synth.f32_normal(synth.seed_of(1000 + l), E * H, 0.0, 0.02).reshape(E, H)
            moe = MoeLayer(H, I, E, K, router, *base[1:], ctx=ctx)
            moe.set_shared(SI, *sh)
            mlp = dict(moe=moe)
        layers.append(DecoderLayer(H, ln[0], ln[1], qkv, o, ctx=ctx, **mlp))
        caches.append(RingCache(1, seq, ctx=ctx))
    lm = QInt8(synth.int8_uniform(synth.seed_of(850), V * H), synth.f32_uniform(synth.seed_of(851), V, 1e-3, 2e-2), V,
               H, ctx)
    dec = Decoder(layers, ln[2], lm, ctx=ctx)
    x0 = ctx.to_device(synth.f32_normal(synth.seed_of(830), seq * H).reshape(seq, H))
    x = ctx.empty((seq, H), np.float32)
    tok = ctx.empty((1,), np.uint32)

    def step(i):
        x.copy_from_device(x0)  # the input embeddings (the lookup is outside this path)
        dec.prefill(caches, 0, x, seq, chunk=chunk, token=tok)  # one call: every chunk through 12 layers + LM head

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    el, prof, kernels, sstats = timed(ctx, step, args.steps)
    ms = el / args.steps * 1e3
    nb = len(prefill_chunk_bounds(seq, chunk or seq))
    # algorithmic work per step: int8 products (2 ops per multiply-add) and
    # the attention's f32 flops
    int8_ops = 2.0 * seq * (NL * (3 * D * H + H * D) + (NL - 1) * (K * 3 * I * H + 3 * SI * H) + 3 * ID * H) + \
        2.0 * V * H
    f32_flops = NL * attn_flops(seq) + (NL - 1) * 2.0 * seq * E * H
    ideal_ms = (int8_ops / (MFMA_INT8_PEAK_TOPS * 1e12) + f32_flops / (MFMA_F32_PEAK_TFLOPS * 1e12)) * 1e3
    weights = NL * (3 * D * H + H * D) + (NL - 1) * (E * 3 * I * H + 3 * SI * H) + 3 * ID * H + V * H
    log(f"per-kernel avg us {kernels}")
    return {
        "metric": f"whole prefill tokens/s (12 layers, {seq} tokens, "
                  f"{'one chunk' if not chunk or chunk >= seq else f'chunks of {chunk}'}, + first token), 1 GPU",
        "value": round(seq * args.steps / el, 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "dtype": "int8",
        "config": {"workload": "prefill", "seq": seq, "chunk": chunk, "chunks": nb, "layers": NL, "hidden": H,
                   "experts": E, "top_k": K, "inter": I, "shared_inter": SI, "dense_inter": ID, "vocab": V},
        "roofline": {"bound": "mfma", "kernel": "the whole prefill", "achieved": round(int8_ops / (ms * 1e-3) / 1e12, 2),
                     "peak": MFMA_INT8_PEAK_TOPS, "unit": "TOP/s",
                     "frac": round(int8_ops / (ms * 1e-3) / 1e12 / MFMA_INT8_PEAK_TOPS, 4), "traffic": None,
                     "avg_step_us": round(ms * 1e3, 3)},
        "mfma_utilisation": {"int8_ops_per_step": int8_ops, "f32_flops_per_step": f32_flops,
                             "ideal_ms_at_peak": round(ideal_ms, 5), "frac_of_step": round(ideal_ms / ms, 4),
                             "weight_bytes_per_chunk": int(weights),
                             "weight_gbs_over_step": round(weights * nb / (ms * 1e-3) / 1e9, 1)},
        "kernel_avg_us": kernels,
        "step_us": sstats,
        "_cpu_inputs": None,
    }


# ---------------------------------------------------------------------------
# calibration: a plain device-to-device copy of known size (the reference
# point for the FETCH_SIZE / WRITE_SIZE counters)
# ---------------------------------------------------------------------------

COPY_BYTES = 512 << 20


def bench_copy(args, ctx):
    src = ctx.empty((COPY_BYTES,), np.uint8)
    dst = ctx.empty((COPY_BYTES,), np.uint8)

    def step(i):
        dst.copy_from_device(src)

    for i in range(args.warmup):
        step(i)
    ctx.device_synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    ctx.device_synchronize()
    el = time.perf_counter() - t0
    gbs = 2 * COPY_BYTES * args.steps / el / 1e9
    return {
        "metric": "device-to-device copy GB/s (read + write), 1 GPU",
        "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(el / args.steps * 1e3, 5), "dtype": "u8",
        "config": {"workload": "copy", "bytes": COPY_BYTES},
        "roofline": {"bound": "hbm", "kernel": "copyBuffer", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "_cpu_inputs": None,
    }


WORKLOADS = {
    "moe_decode": (bench_moe, cpu_moe),
    "lm_head": (bench_lm_head, cpu_lm_head),
    "lm_head_sample": (lambda args, ctx: bench_lm_head(args, ctx, sampler=True), None),
    "igemm": (bench_igemm, cpu_igemm),
    "igemm_batched": (bench_igemm_batched, cpu_igemm_batched),
    "rswa": (bench_rswa, cpu_rswa),
    "copy": (bench_copy, None),
    "moe_prefill_i4": (bench_prefill_i4, cpu_prefill_i4),
    "moe_prefill_i8": (bench_prefill_i8, None),
    "linear_i8": (bench_linear_i8, cpu_linear_i8),
    "decode_layer": (bench_decode_layer, cpu_decode_layer),
    "decode_step": (bench_decode_step, None),
    "prefill_attn": (bench_prefill_attn, cpu_prefill_attn),
    "prefill_layer": (bench_prefill_layer, cpu_prefill_layer),
    "prefill": (bench_prefill, None),
}


# Secondary configurations measured after the headline in the default run and
# reported under "extra" (key, workload, tokens, copies, steps, warmup): the
# other configs and the prefill paths, each timed the same way as its
# own --workload run, with fewer steps.
EXTRAS = [
    ("cfg1_igemm_m16", "igemm", 16, 64, 200, 20),
    ("cfg1_igemm_batched64_m16", "igemm_batched", 16, 1, 50, 5),
    ("cfg2_lm_head_m1", "lm_head", 1, 3, 50, 5),
    ("cfg2_lm_head_m8", "lm_head", 8, 3, 50, 5),
    ("cfg3_moe_decode_t1", "moe_decode", 1, 8, 100, 10),
    ("cfg3_moe_decode_t32", "moe_decode", 32, 8, 100, 10),
    ("cfg4_moe_prefill_i4_m512", "moe_prefill_i4", 512, 3, 20, 3),
    ("cfg5_rswa_b8", "rswa", 8, 4, 100, 10),
    ("prefill_attn_1024", "prefill_attn", 1024, 1, 20, 3),
    ("linear_i8_m8192", "linear_i8", 8192, 3, 20, 3),
    ("decode_layer_b8", "decode_layer", 8, 6, 50, 5),
    ("prefill_layer_1024", "prefill_layer", 1024, 2, 10, 2),
    # the same 1024 tokens as one chunk: HBM holds the whole prompt's rows, and
    # the routed experts are read once instead of once per 256-row chunk
    ("prefill_layer_1024_c1024", "prefill_layer", 1024, 2, 10, 2, {"chunk": 1024}),
    # the whole prefill of a 1024-token prompt, 12 layers + the first token, in one call
    ("prefill_1024", "prefill", 1024, 1, 10, 2),
    ("prefill_1024_c1024", "prefill", 1024, 1, 10, 2, {"chunk": 1024}),
]
_EXTRA_KEYS = ("layer_roofline", "mfma_utilisation", "layer_mfma", "kernel_avg_us", "step_us")


def run_extras(ctx, base_args) -> dict:
    """Each secondary configuration timed like its own --workload run, then
    its CPU baseline on the host (base_args.extra_cpu_seconds each, unless
    --no-cpu)."""
    import gc

    out = {}
    for key, wl, tokens, copies, steps, warmup, *over in EXTRAS:
        if wl not in WORKLOADS:
            continue
        a = argparse.Namespace(**vars(base_args))
        a.workload, a.tokens, a.copies, a.steps, a.warmup = wl, tokens, copies, steps, warmup
        for k, v in (over[0] if over else {}).items():
            setattr(a, k, v)
        a.cpu_seconds = base_args.extra_cpu_seconds
        log(f"extra {key}")
        run, cpu = WORKLOADS[wl]
        res = run(a, ctx)
        cpu_inputs = res.pop("_cpu_inputs", None)
        rl = res.get("roofline") or {}
        ent = {"metric": res["metric"], "value": res["value"], "unit": res["unit"],
               "ms_per_step": res["ms_per_step"], "steps": steps, "config": res["config"],
               "roofline": {k: rl.get(k) for k in ("bound", "kernel", "achieved", "peak", "unit", "frac", "traffic",
                                                   "avg_launch_us", "p50_launch_us", "p90_launch_us")}}
        for k in _EXTRA_KEYS:
            if k in res:
                ent[k] = res[k]
        if cpu is not None and not base_args.no_cpu and cpu_inputs is not None:
            log(f"extra {key}: cpu baseline")
            ent["cpu_baseline"] = cpu(a, cpu_inputs)
            ent["cpu_baseline"].update(host_cpu())
        else:
            ent["cpu_baseline"] = None
        out[key] = ent
        del res, cpu_inputs
        gc.collect()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="moe_decode", choices=sorted(WORKLOADS))
    ap.add_argument("--tokens", type=int, default=None, help="T (moe), M (lm_head/igemm)")
    ap.add_argument("--copies", type=int, default=None, help="distinct weight copies rotated (defeats MALL)")
    ap.add_argument("--chunk", type=int, default=256, help="prefill chunk (prefill_attn; DEFAULT_PREFILL_CHUNK)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="CPU baseline sample of the headline workload (seconds of timed calls)")
    ap.add_argument("--extra-cpu-seconds", type=float, default=4.0,
                    help="CPU baseline sample of each secondary configuration")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--stat-steps", type=int, default=STAT_STEPS,
                    help="steps of the per-kernel statistics pass (at least --steps)")
    ap.add_argument("--stat-groups", type=int, default=STAT_GROUPS,
                    help="samples of the step statistics (each the mean of 10 steps); small values for counter runs")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the secondary configurations the default (moe_decode) run reports under 'extra'")
    ap.add_argument("--library-ref", action="store_true",
                    help="linear_i8: also time the platform library's int8 GEMM (torch._int_mm) at the same shape")
    ap.add_argument("--no-views", action="store_true",
                    help="prefill MoE workloads: skip the warm and bucket re-runs (profile the cold step alone)")
    args = ap.parse_args()
    set_stat_sizes(args.stat_steps, args.stat_groups)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path has no multi-GPU code); run with --gpus 1",
              file=sys.stderr)
        return 2
    defaults = {"moe_decode": (8, 8), "lm_head": (1, 3), "lm_head_sample": (8, 3), "igemm": (1, 64), "rswa": (8, 4),
                "igemm_batched": (1, 1),
                "copy": (1, 1),
                "moe_prefill_i4": (512, 3), "moe_prefill_i8": (512, 2), "linear_i8": (2048, 3),
                "decode_layer": (8, 6), "decode_step": (8, 1), "prefill_attn": (1024, 1),
                "prefill_layer": (1024, 2), "prefill": (1024, 1)}
    dt, dc = defaults[args.workload]
    args.tokens = args.tokens or dt
    args.copies = args.copies or dc

    from franken_ocr_amd.device import Context

    ctx = Context(0)
    log(f"device {ctx.info()}")
    run, cpu = WORKLOADS[args.workload]
    res = run(args, ctx)
    cpu_inputs = res.pop("_cpu_inputs")
    line = {
        "metric": res.pop("metric"),
        "value": res.pop("value"),
        "unit": res.pop("unit"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res.pop("dtype"),
        "data": "synthetic (seeded splitmix64; int8 weights uniform [-127,127], scales U(1e-3,2e-2), "
                "activations N(0,1)); no checkpoint",
        "config": res.pop("config"),
    }
    line.update(res)
    if cpu is not None and not args.no_cpu and cpu_inputs is not None:
        log("cpu baseline (reference x86 int8 tier restated in C) ...")
        line["cpu_baseline"] = cpu(args, cpu_inputs)
        line["cpu_baseline"].update(host_cpu())
    else:
        line["cpu_baseline"] = None
    if args.workload == "moe_decode" and args.tokens == 8 and not args.no_extras:
        line["extra"] = run_extras(ctx, args)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
