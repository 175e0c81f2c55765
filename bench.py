#!/usr/bin/env python3
"""Benchmark of the quantized KV-cache hot path on one MI355X.

Headline (BASELINE.json metric, config 3): all 12 full-attention layers of a
Qwen3-Next-80B-A3B-shaped model, batch 1, Q4K cache holding 131072 tokens per layer.
One step = per layer, quantize-append one token and attend over 131073 keys
(pkv_append_attend), 12 dependent per-layer launches on one stream. Inputs are seeded
synthetic N(0,1) tensors already resident in HBM when the timed region starts.

Prints one JSON line. `value` is microseconds per 12-layer decode step (lower is
better); `roofline` prices the dominant kernel against MI355X's 8 TB/s HBM peak;
`cpu_baseline` times the CPU oracle's faithful restatement of the reference path
(dequantize-all + repeat_kv + SDPA, qwen3_next.rs:2470-2605) on the host cores.

The default run also measures the other BASELINE configs after the headline, in the
same process, and attaches them to the headline line as `other_configs` (value, unit,
roofline; their CPU baselines are left to their own `--config N` runs):
1 Q8_0 decode over 4097 keys, 2 a 512-token Q4K prefill chunk over 16896 keys, 4
PrefixCache restore of 12 full + 36 linear layers plus a 1024-token suffix, 5 a
16-sequence batched decode step over 12 layers. `--headline-only` skips them.

`--config N` measures one workload instead (one JSON line each; `--config all` prints
every config's line, 6 and 7 included).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4K decode-attn µs/step @128k ctx, 12 layers; achieved HBM GB/s & % of peak"
HBM_PEAK_GBS = 8000.0
FP16_DENSE_TFLOPS = 2500.0
Q4K_ROW = 144
Q8_ROW = 272
# HBM bytes per launch of each config's roofline kernel(s), from the two calibrated
# rocprofv3 --pmc runs (FETCH_SIZE x2.0, WRITE_SIZE x1.0) summarised in profiles/; the
# profiling step cannot run inside bench.py itself. Refreshed with the profiles.
MEASURED_TRAFFIC = {
    3: (85_000_000, "profiles/q4k_decode_config3.md: the decode launch with its in-launch "
                    "combine, per layer"),
    1: (11_130_572, "profiles/q8_decode_config1.md: decode + combine"),
    2: (170_260_000, "profiles/q4k_prefill_config2.md: prefill kernel + split merge"),
    "2q8": (136_320_102, "profiles/q8_prefill_config2.md: prefill kernel + split merge"),
    4: (1_064_255_795, "profiles/prefix_restore_config4.md: copy_segments_kernel read + "
                       "written"),
    5: (415_070_000, "profiles/q4k_batched_decode_config5.md: decode + combine per layer"),
    6: (73_730_000, "profiles/deltanet_step_config6.md: per launch at batch 16"),
}


def traffic(config):
    t = MEASURED_TRAFFIC.get(config)
    return None if t is None else t[0]


def layer_bytes(keys: int, row: int = Q4K_ROW) -> int:
    """Algorithmic HBM bytes of one layer's decode step: the K and V rows of every key
    (2 KV heads x `row` B each), q in and out (16 x 256 f32 each), the new token's f32
    k/v read and its 4 packed rows written."""
    return keys * 2 * 2 * row + 2 * 16 * 256 * 4 + 2 * 2 * 256 * 4 + 4 * row


def cpu_model() -> str:
    try:
        return [l for l in open("/proc/cpuinfo") if l.startswith("model name")][0].split(":")[1].strip()
    except Exception:
        return "unknown"


def append_roofline(kernel, bound, tokens, heads, us, row=None):
    """Roofline entry of a quantize-append launch: f32 K and V in, packed rows out
    (head_dim 256: 1024 B in and `row` B out per row and tensor; Q4K 144 B, Q8_0 272 B)."""
    nbytes = 2 * heads * tokens * (256 * 4 + (Q4K_ROW if row is None else row))
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"kernel": kernel, "bound": bound, "bytes_per_launch": nbytes,
            "avg_launch_us": round(us, 2), "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}


WARM_S = 0.25  # --warm-seconds: the warm-up also lasts at least this long
WARM_RUN = {"calls": 0}  # warm-up calls made by the last event_time (reported in lines)


def device_status_check():
    """After every timed region: the library's device status word (a fused decode step's
    bounded waits that gave up, pkv_device_status) must be clear, else the timed steps did
    not produce valid results and the run fails instead of printing a number."""
    from paramecia_amd import _lib
    L = _lib.lib()
    if L.pkv_device_status() != 0:
        raise RuntimeError("device status set after a timed region: " +
                           L.pkv_last_error().decode())


def event_time(torch, fn, steps, warmup):
    """Milliseconds per call of fn: HIP events around `steps` calls after the warm-up.
    The warm-up is at least `warmup` calls and lasts at least WARM_S seconds of wall time
    (the GPU's clocks ramp up under sustained work; a short warm-up leaves the first
    timed steps at lower clocks). Nothing of the timed calls changes."""
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < WARM_S:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    WARM_RUN["calls"] = n
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    device_status_check()
    return a.elapsed_time(b) / steps


NO_GRAPH = False  # --no-graph: every "graph" time is an eager one (profiler passes)


def graph_time(torch, fn, steps, warmup, reps=1):
    """Milliseconds per call of fn, run from a HIP graph: fn is captured `reps` times in a
    row into one graph (after an eager warm-up on the capture stream, which sizes every
    workspace), the graph is replayed, and the time of a replay is divided by `reps`.
    With reps > 1 the graph launch is shared by several steps, as it is in a serving
    loop whose graph holds the whole forward pass; every captured step does all of its
    work. With --no-graph the calls are timed eagerly instead."""
    if NO_GRAPH:
        return event_time(torch, fn, steps, warmup)
    # Two graphs of the same steps, replayed in turn: HIP submits a replay of a graph
    # only once that graph's previous replay has finished, so with a single graph the GPU
    # idles for a submission (about 10 us here) before every replay; with two, the next
    # replay is always queued behind the running one, as in a serving loop.
    graphs = [torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
        torch.cuda.synchronize()
        for g in graphs:
            with torch.cuda.graph(g, stream=side):
                for _ in range(reps):
                    fn()
    torch.cuda.current_stream().wait_stream(side)
    turn = [0]

    def replay():
        graphs[turn[0] & 1].replay()
        turn[0] += 1

    replays = max(1, steps // reps)  # steps timed: replays * reps (== steps when reps | steps)
    return event_time(torch, replay, replays, max(1, warmup // reps)) / reps


# ------------------------------------------------------------------ config 3 (headline)
def run_config3(args):
    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    dev = torch.device("cuda:0")
    L, S = args.layers, args.cached
    cap = S + 1
    Q = pk.KvCacheQuantization.Q4K

    # ---- setup: fill every layer's cache with S seeded tokens (quantize-append kernel)
    caches = []
    kbuf = torch.empty((1, W.NUM_KV_HEADS, S, W.HEAD_DIM), dtype=torch.float32, device=dev)
    vbuf = torch.empty_like(kbuf)
    fill_s = 0.0
    for l in range(L):
        c = pk.PreallocatedQuantizedKvCache(1, W.NUM_KV_HEADS, cap, W.HEAD_DIM, Q)
        pk.fill_normal(kbuf, W.SEED, W.stream_id(3, W.T_PREFILL_K, l))
        pk.fill_normal(vbuf, W.SEED, W.stream_id(3, W.T_PREFILL_V, l))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        c.append_quantized(kbuf, vbuf)
        torch.cuda.synchronize()
        fill_s += time.perf_counter() - t0
        caches.append(c)
    # the append alone, warm: the last layer's fill again at offset 0 (the same rows, so
    # the cache is unchanged), HIP events around 5 calls
    fill_ev_ms = event_time(torch, lambda: caches[-1].append_quantized(kbuf, vbuf, offset=0), 5, 2)
    del kbuf, vbuf
    q = torch.empty((L, 1, 1, W.NUM_HEADS, W.HEAD_DIM), dtype=torch.float32, device=dev)
    kn = torch.empty((L, 1, W.NUM_KV_HEADS, 1, W.HEAD_DIM), dtype=torch.float32, device=dev)
    vn = torch.empty_like(kn)
    for l in range(L):
        pk.fill_normal(q[l], W.SEED, W.stream_id(3, W.T_Q, l))
        pk.fill_normal(kn[l], W.SEED, W.stream_id(3, W.T_NEW_K, l))
        pk.fill_normal(vn[l], W.SEED, W.stream_id(3, W.T_NEW_V, l))
    outs = [torch.empty_like(q[l]) for l in range(L)]
    preps = make_preps(torch, pk, W, L, cap) if args.prep else None
    torch.cuda.synchronize()

    def step_plain(events=None):
        for l in range(L):
            if events is not None:
                events[l][0].record()
            # offset = S rewinds the previous step's token: identical work every step
            outs[l] = caches[l].append_attend(kn[l], vn[l], q[l], W.SCALE, offset=S)
            if events is not None:
                events[l][1].record()

    def step_prep(events=None):
        # q, k, v as projection outputs ([b, l, h, d]; for one token the new k / v rows
        # have the same memory layout): q_norm, k_norm and rope run inside the step
        for l in range(L):
            if events is not None:
                events[l][0].record()
            outs[l] = caches[l].append_attend_prep(q[l], kn[l].view(1, 1, W.NUM_KV_HEADS, W.HEAD_DIM),
                                                   vn[l].view(1, 1, W.NUM_KV_HEADS, W.HEAD_DIM),
                                                   preps[l], W.SCALE, offset=S)
            if events is not None:
                events[l][1].record()

    step = step_prep if args.prep else step_plain

    # eager: 12 ctypes launches per step from Python (host overhead included)
    eager_ms = event_time(torch, step, args.steps, args.warmup)
    # HIP graph of args.graph_reps 12-layer steps (default ten), replayed (the
    # serving-loop form, whose graph holds the whole forward pass: a replay's submission
    # gap is shared by ten steps), and a graph of a single step for reference
    reps = args.graph_reps if args.graph_reps > 0 else 10
    ms = graph_time(torch, step, args.steps, args.warmup, reps)
    warm_calls = WARM_RUN["calls"]
    ms_1 = graph_time(torch, step, args.steps, args.warmup, 1) if reps > 1 else ms

    # Per-launch duration of a layer's kernels (decode + combine): the layer's share of
    # the graph-timed step, ms / L, which also holds the gaps between launches and agrees
    # with rocprofv3's kernel durations. Also reported: each layer bracketed by its own
    # event pair while a sleep kernel keeps the GPU busy as the host enqueues (the event
    # records then add about 3 us per layer).
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(L)] for _ in range(args.steps)]
    sleep = getattr(torch.cuda, "_sleep", None)
    for s_ in range(args.steps):
        if sleep is not None:
            sleep(20_000_000)
        step(ev[s_])
    torch.cuda.synchronize()
    bracketed_ms = sum(a.elapsed_time(b) for row in ev for a, b in row) / (args.steps * L)
    device_status_check()
    graph_ms = ms
    # the step time: the faster of the two launch forms (both do every step's full work);
    # the other is reported beside it
    from_graph = graph_ms <= eager_ms
    ms = graph_ms if from_graph else eager_ms
    per_launch_ms = ms / L

    keys = S + 1
    step_bytes = L * layer_bytes(keys)
    achieved = layer_bytes(keys) / (per_launch_ms * 1e-3) / 1e9
    workload = ("config3: 12 Qwen3-Next full-attention layers, batch 1, Q4K KV cache "
                f"with {S} cached tokens; step = per layer quantize-append 1 token + "
                f"attend over {keys} keys (16 q heads, 2 kv heads, head_dim 256)")
    if args.prep:
        workload += ("; inputs are the q/k/v projection outputs: q_norm, k_norm and the "
                     "64-dim rope (theta 1e7) run inside the step (pkv_append_attend_prep)")
    result = {
        "metric": METRIC,
        "value": round(ms * 1000.0, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_calls_run": warm_calls,
        "warm_seconds": WARM_S,
        "ms_per_step": round(ms, 4),
        "value_from": "graph replay" if from_graph else "eager launches",
        "eager_us_per_step": round(eager_ms * 1000.0, 2),
        "graph_us_per_step": round(graph_ms * 1000.0, 2),
        "graph_steps_per_replay": reps,
        "one_step_graph_us_per_step": round(ms_1 * 1000.0, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Philox N(0,1), bit-identical to the CPU oracle's generator)",
        "config": {
            "workload": workload,
            "layers": L, "cached_tokens": S, "keys": keys, "kv_quant": "Q4K",
            "num_heads": 16, "num_kv_heads": 2, "head_dim": 256, "batch": 1,
            "qk_prep": bool(args.prep),
        },
        "step_hbm_gbs": round(step_bytes / (ms * 1e-3) / 1e9, 1),
        "step_pct_of_peak": round(100.0 * step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
        "roofline": {
            "kernel": ("pkv_append_attend_prep (one layer: one decode launch that prepares q "
                       "and the new K row, quantizes the new rows and merges its partials in "
                       "its combiner workgroups)") if args.prep else
                      ("pkv_append_attend (one layer: one decode launch that quantizes the "
                       "new rows and merges its split-K partials in its combiner workgroups)"),
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "bytes_per_launch": layer_bytes(keys),
            "avg_launch_us": round(per_launch_ms * 1000.0, 2),
            "avg_launch_source": "the step time (value) / layers (HIP events around the steps)",
            "event_bracketed_launch_us": round(bracketed_ms * 1000.0, 2),
            "traffic": traffic(3),
            "traffic_source": MEASURED_TRAFFIC[3][1],
        },
        "append_tokens_per_s": round(L * S / fill_s, 1),
        "append_roofline": append_roofline(
            f"q4k_append_kernel<1> ({S}-token layer, one lane per sub-block fit)", "valu", S,
            W.NUM_KV_HEADS, fill_ev_ms * 1000.0),
    }
    if args.prep:
        result["unprepared_us_per_step"] = round(
            graph_time(torch, step_plain, args.steps, args.warmup, reps) * 1000.0, 2)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_decode(
            caches[0], kn[0], vn[0], q[0], S, args.cpu_threads, 3, 4, W.N_FULL,
            single_keys=min(S, 16384))
    return result


def make_preps(torch, pk, W, layers, max_pos):
    """Per-layer q_norm / k_norm alphas (seeded, around 1 as trained RMSNorm weights are)
    and one rope shared by every layer, as the model loads them."""
    rope = pk.RotaryEmbedding(W.N_ROT, max_pos, W.ROPE_THETA)
    preps = []
    for l in range(layers):
        qa = torch.empty(W.HEAD_DIM, dtype=torch.float32, device="cuda")
        ka = torch.empty_like(qa)
        pk.fill_normal(qa, W.SEED, W.stream_id(6, W.T_Q, l), 0.1)
        pk.fill_normal(ka, W.SEED, W.stream_id(6, W.T_NEW_K, l), 0.1)
        preps.append(pk.QkPrep(qa + 1.0, ka + 1.0, W.RMS_EPS, rope))
    return preps


CPU_RUNS = 5  # timed runs per CPU-baseline leg; the median is reported


def cpu_threads(threads: int) -> int:
    """Host threads of the multi-threaded CPU leg: --cpu-threads, else every core the
    process sees, capped at the 16 cores a one-GPU box grants a job."""
    return threads if threads > 0 else min(os.cpu_count() or 1, 16)


def median(xs):
    ys = sorted(xs)
    return ys[len(ys) // 2] if len(ys) % 2 else 0.5 * (ys[len(ys) // 2 - 1] + ys[len(ys) // 2])


def oracle_cache_from(cache, quant, S, rows):
    """An oracle cache (capacity rows + 1) holding the first `rows` rows of a GPU cache's
    packed bytes."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    from paramecia_amd import workloads as W

    c = orc.Cache(quant, 1, W.NUM_KV_HEADS, W.HEAD_DIM, rows + 1)
    cache.truncate(S)
    kb, vb = cache.raw_bytes()
    c.load_bytes(kb.cpu().numpy(), vb.cpu().numpy(), rows)
    return c


def cpu_baseline_decode(cache, kn, vn, q, S, threads, config, quant, layers, single_keys=None):
    """The oracle's faithful restatement of the reference CPU path (CPU quantize of the new
    token, dequantize the whole cache, permute, repeat_kv, transposed-K copy, matmul,
    clamp, softmax, matmul) for one layer's decode step, extrapolated to `layers` layers.
    Two legs, each the median of CPU_RUNS timed runs: all cores (cpu_threads) over the
    full cache, and one thread over the first `single_keys` cached keys (the whole cache
    when None), scaled by the key count (every step of the path is linear in it)."""
    from paramecia_amd import workloads as W

    nthreads = cpu_threads(threads)
    knp, vnp, qnp = kn.cpu().numpy(), vn.cpu().numpy(), q.cpu().numpy()

    def once(c, rows, th):
        t0 = time.perf_counter()
        assert c.append_at(knp, vnp, rows) == 0
        c.attend(qnp, W.SCALE, rows, True, mode="faithful", threads=th)
        return time.perf_counter() - t0

    c = oracle_cache_from(cache, quant, S, S)
    multi = [once(c, S, nthreads) for _ in range(CPU_RUNS)]
    rows1 = S if single_keys is None else min(S, single_keys)
    c1 = c if rows1 == S else oracle_cache_from(cache, quant, S, rows1)
    single = [once(c1, rows1, 1) for _ in range(CPU_RUNS)]
    scale1 = (S + 1) / (rows1 + 1)
    del c, c1
    return {
        "value": round(median(multi) * layers * 1e6, 1), "unit": "us/step", "cores": nthreads,
        "kind": "port",
        "sample": f"config {config}: one decode step (append 1 token + attend {S + 1} keys) of "
                  f"1 of {layers} layers, median of {CPU_RUNS} runs, times {layers}; "
                  f"{nthreads} OpenMP threads (the cores this process sees, at most 16) on "
                  f"{cpu_model()}",
        "runs_s": [round(x, 4) for x in multi],
        "single_thread": {
            "value": round(median(single) * scale1 * layers * 1e6, 1), "unit": "us/step",
            "cores": 1,
            "sample": f"one thread, one decode step over the first {rows1 + 1} keys, median of "
                      f"{CPU_RUNS} runs, times {scale1:.4g} (key count) and {layers} (layers)",
            "runs_s": [round(x, 4) for x in single]},
    }


def cpu_baseline_prefill(cache, kc, vc, qc, k1, v1, q1, S, C, threads, quant=4):
    """Config 2's step on the oracle's faithful CPU path: quantize-append the C-token chunk,
    causal attention of its C queries over S + C keys, then one decode step (append 1
    token, attend S + C + 1 keys). The chunk attention is timed on two samples of its last
    query rows and extrapolated linearly in the keys the rows see (t = a + b * keys: the
    per-call dequantize and copies are a, the products b); the append and the decode step
    are timed whole. Legs: all cores (cpu_threads) and one thread, medians of CPU_RUNS."""
    from paramecia_amd import workloads as W

    nthreads = cpu_threads(threads)
    kcn, vcn, qcn = kc.cpu().numpy(), vc.cpu().numpy(), qc.cpu().numpy()
    k1n, v1n, q1n = k1.cpu().numpy(), v1.cpu().numpy(), q1.cpu().numpy()
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    c = orc.Cache(quant, 1, W.NUM_KV_HEADS, W.HEAD_DIM, S + C + 1)
    cache.truncate(S)
    kb, vb = cache.raw_bytes()
    c.load_bytes(kb.cpu().numpy(), vb.cpu().numpy(), S)
    keys = lambda i0, i1: sum(S + i + 1 for i in range(i0, i1))  # keys seen by rows [i0, i1)

    def leg(th, na, nb):
        ta, tb, tr = [], [], []
        for _ in range(CPU_RUNS):
            t0 = time.perf_counter()
            assert c.append_at(kcn, vcn, S) == 0
            t1 = time.perf_counter()
            assert c.append_at(k1n, v1n, S + C) == 0
            c.attend(q1n, W.SCALE, S + C, True, mode="faithful", threads=th)
            t2 = time.perf_counter()
            tr.append((t1 - t0) + (t2 - t1))
            for n, out in ((na, ta), (nb, tb)):
                t0 = time.perf_counter()
                c.attend(qcn[:, C - n:], W.SCALE, S + C - n, True, mode="faithful", threads=th)
                out.append(time.perf_counter() - t0)
        a_t, b_t = median(ta), median(tb)
        slope = (b_t - a_t) / (keys(C - nb, C) - keys(C - na, C))
        attn = a_t + slope * (keys(0, C) - keys(C - na, C))
        return median(tr) + attn, (na, nb, a_t, b_t)

    multi, sm = leg(nthreads, 8, 64)
    single, s1 = leg(1, 2, 8)
    desc = lambda th, s_: (f"{th} thread(s): append {C} tokens and one decode step timed whole; "
                           f"chunk attention timed on its last {s_[0]} and {s_[1]} query rows "
                           f"({s_[2]:.3f} s, {s_[3]:.3f} s) and extrapolated linearly in keys "
                           f"seen to all {C}; medians of {CPU_RUNS} runs")
    return {"value": round(multi * 1e6, 1), "unit": "us/step", "cores": nthreads, "kind": "port",
            "sample": f"config 2 on {cpu_model()}: " + desc(nthreads, sm),
            "single_thread": {"value": round(single * 1e6, 1), "unit": "us/step", "cores": 1,
                              "sample": desc(1, s1)}}


def copy_ceiling(torch, mib=1024, steps=10):
    """Measured device-to-device copy rate on this GPU: torch copy_ between two 1 GiB
    buffers (a runtime blit), read + written bytes over the HIP-event time. The practical
    ceiling an HBM-bound kernel is compared with, beside the 8 TB/s data-sheet peak."""
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    ms = event_time(torch, lambda: dst.copy_(src), steps, 3)
    del src, dst
    torch.cuda.empty_cache()
    gbs = 2 * n / (ms * 1e-3) / 1e9
    return {"gbs": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_copy": 2 * n,
            "method": f"torch copy_ of {mib} MiB device to device, {steps} copies after 3, "
                      "(read + write bytes) / HIP-event time"}


def calib_copy(torch, mib):
    """torch.neg of `mib` MiB into a second buffer, 3 times: a plain copy (read N, write
    N bytes) whose rocprofv3 FETCH_SIZE / WRITE_SIZE readings scale the counters to bytes."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def add_copy_ceiling(torch, r):
    """Attach the copy ceiling to a result line, and the roofline's fraction of it."""
    cc = copy_ceiling(torch)
    r["copy_ceiling"] = cc
    rf = r.get("roofline")
    if rf and rf.get("unit") == "GB/s":
        rf["frac_of_copy_ceiling"] = round(rf["achieved"] / cc["gbs"], 4)
    return r


def base_result(config, metric, value, unit, hib, ms, args, workload, extra):
    r = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
         "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": hib,
         "scaling": "weak", "vs_baseline": None, "dtype": "f32",
         "data": "synthetic (seeded Philox N(0,1))",
         "config": {"workload": workload, "index": config}}
    r.update(extra)
    return r


# ------------------------------------------------------------------ config 1
def run_config1(args):
    """Q8_0, one layer, 4096 cached tokens: append one token and attend 4097 keys."""
    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    S = 4096
    c = pk.PreallocatedQuantizedKvCache(1, 2, S + 1, 256, pk.KvCacheQuantization.Q8_0)
    kb = torch.empty((1, 2, S, 256), device="cuda")
    vb = torch.empty_like(kb)
    pk.fill_normal(kb, W.SEED, W.stream_id(1, W.T_PREFILL_K))
    pk.fill_normal(vb, W.SEED, W.stream_id(1, W.T_PREFILL_V))
    c.append_quantized(kb, vb)
    del kb, vb
    q = torch.empty((1, 1, 16, 256), device="cuda")
    kn = torch.empty((1, 2, 1, 256), device="cuda")
    vn = torch.empty_like(kn)
    pk.fill_normal(q, W.SEED, W.stream_id(1, W.T_Q))
    pk.fill_normal(kn, W.SEED, W.stream_id(1, W.T_NEW_K))
    pk.fill_normal(vn, W.SEED, W.stream_id(1, W.T_NEW_V))
    step = lambda: c.append_attend(kn, vn, q, W.SCALE, offset=S)
    reps = args.graph_reps if args.graph_reps > 0 else 20
    # A step is ~8 us: at least 10 replays of 20 steps are timed (200 steps, 1.6 ms of
    # GPU time), so that one replay's submission gap is not what a short --steps measures
    sub = argparse.Namespace(**vars(args))
    sub.steps = max(args.steps, 10 * reps)
    ms = graph_time(torch, step, sub.steps, args.warmup, reps)
    ms_1 = graph_time(torch, step, sub.steps, args.warmup, 1)
    args = sub
    nbytes = layer_bytes(S + 1, Q8_ROW)
    gbs = nbytes / (ms * 1e-3) / 1e9
    r = base_result(1, "Q8_0 decode-attn µs/step @4097 keys, 1 layer", round(ms * 1000, 2),
                    "us/step", False, ms, args,
                    "config1: Q8_0 cache with 4096 tokens; step = quantize-append 1 token + "
                    "attend 4097 keys (16 q heads, 2 kv heads, head_dim 256)",
                    {"graph_steps_per_replay": reps,
                     "one_step_graph_us_per_step": round(ms_1 * 1000, 2),
                     "roofline": {"kernel": "pkv_append_attend (Q8_0)", "bound": "hbm",
                                  "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": nbytes,
                                  "traffic": traffic(1)}})
    if not args.no_cpu_baseline:
        r["cpu_baseline"] = cpu_baseline_decode(c, kn, vn, q, S, args.cpu_threads, 1, 3, 1)
    return r


# ------------------------------------------------------------------ config 2
def run_config2(args):
    """Q4K (or Q8_0 with --quant q8_0), capacity 32768, 16384 cached: append a 512-token
    chunk and run its causal attention over 16896 keys (q_offset 16384), as
    FullAttention::forward does for a prefill chunk."""
    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    S, C, cap = 16384, 512, 32768
    q8 = args.quant == "q8_0"
    qname = "Q8_0" if q8 else "Q4K"
    quant = pk.KvCacheQuantization.Q8_0 if q8 else pk.KvCacheQuantization.Q4K
    c = pk.PreallocatedQuantizedKvCache(1, 2, cap, 256, quant)
    kb = torch.empty((1, 2, S, 256), device="cuda")
    vb = torch.empty_like(kb)
    pk.fill_normal(kb, W.SEED, W.stream_id(2, W.T_PREFILL_K))
    pk.fill_normal(vb, W.SEED, W.stream_id(2, W.T_PREFILL_V))
    c.append_quantized(kb, vb)
    del kb, vb
    kc = torch.empty((1, 2, C, 256), device="cuda")
    vc = torch.empty_like(kc)
    qc = torch.empty((1, C, 16, 256), device="cuda")
    pk.fill_normal(kc, W.SEED, W.stream_id(2, W.T_CHUNK_K))
    pk.fill_normal(vc, W.SEED, W.stream_id(2, W.T_CHUNK_V))
    pk.fill_normal(qc, W.SEED, W.stream_id(2, W.T_CHUNK_Q))

    q1 = torch.empty((1, 1, 16, 256), device="cuda")
    k1 = torch.empty((1, 2, 1, 256), device="cuda")
    v1 = torch.empty_like(k1)
    pk.fill_normal(q1, W.SEED, W.stream_id(2, W.T_Q))
    pk.fill_normal(k1, W.SEED, W.stream_id(2, W.T_NEW_K))
    pk.fill_normal(v1, W.SEED, W.stream_id(2, W.T_NEW_V))

    def step_plain():
        c.append_quantized(kc, vc, offset=S)
        c.attend(qc, W.SCALE, S, causal=True)
        return c.append_attend(k1, v1, q1, W.SCALE, offset=S + C)

    if args.prep:
        prep = make_preps(torch, pk, W, 1, cap)[0]
        # projection-output layout [b, l, h, d] of the same values
        kcp = kc.transpose(1, 2).contiguous()
        vcp = vc.transpose(1, 2).contiguous()

        def step():
            qp = c.append_prep(qc, kcp, vcp, prep, offset=S)
            c.attend(qp, W.SCALE, S, causal=True)
            return c.append_attend_prep(q1, k1.view(1, 1, 2, 256), v1.view(1, 1, 2, 256), prep,
                                        W.SCALE, offset=S + C)
    else:
        step = step_plain

    reps = args.graph_reps if args.graph_reps > 0 else 1
    ms = graph_time(torch, step, args.steps, args.warmup, reps)
    ms_1 = graph_time(torch, step, args.steps, args.warmup, 1)
    # the prefill attention alone (the MFMA kernel's roofline)
    ms_attn = graph_time(torch, lambda: c.attend(qc, W.SCALE, S, causal=True), args.steps,
                         args.warmup, reps)
    flops = 16 * (C * S + C * (C + 1) // 2) * 256 * 2 * 2
    tf = flops / (ms_attn * 1e-3) / 1e12
    workload = (f"config2: {qname} cache with 16384 tokens; step = quantize-append a 512-token "
                "chunk + causal attention of its 512 queries over 16896 keys + one decode "
                "step (append 1 token, attend 16897 keys)")
    extra = {}
    if args.prep:
        workload += ("; inputs are the q/k/v projection outputs: q_norm, k_norm and the "
                     "64-dim rope run inside the appends (pkv_append_prep, "
                     "pkv_append_attend_prep)")
        extra["unprepared_us_per_step"] = round(
            graph_time(torch, step_plain, args.steps, args.warmup, reps) * 1000, 2)
        extra["prep_append_chunk_us"] = round(graph_time(
            torch, lambda: c.append_prep(qc, kcp, vcp, prep, offset=S), args.steps,
            args.warmup, reps) * 1000, 2)
    # 20 appends per graph replay: the 7 µs kernel, not the graph launch
    app_ms = graph_time(torch, lambda: c.append_quantized(kc, vc, offset=S), args.steps,
                        args.warmup, 20)
    extra["append_chunk_us"] = round(app_ms * 1000, 2)
    extra["append_roofline"] = append_roofline(
        (f"q8_0_append_kernel ({C}-token chunk)" if q8 else
         f"q4k_append_kernel<4> ({C}-token chunk, four lanes per sub-block fit)"), "latency", C,
        2, app_ms * 1000, row=272 if q8 else Q4K_ROW)
    if not args.no_cpu_baseline:
        extra["cpu_baseline"] = cpu_baseline_prefill(c, kc, vc, qc, k1, v1, q1, S, C,
                                                     args.cpu_threads, int(quant))
    return base_result(2, f"{qname} prefill chunk + decode µs (512-token append, 512 x 16896 "
                       "causal attention, 1-token decode over 16897 keys)",
                       round(ms * 1000, 2), "us/step", False, ms, args, workload,
                       {**extra, "graph_steps_per_replay": reps,
                        "one_step_graph_us_per_step": round(ms_1 * 1000, 2),
                        "prefill_attention_us": round(ms_attn * 1000, 2),
                        "roofline": {"kernel": "pkv_attend prefill chunk (%s + "
                                     "prefill_merge_kernel)" % ("q8_prefill_kernel" if q8 else
                                                                "q4k_prefill_kernel"),
                                     "bound": "mfma", "achieved": round(tf, 2),
                                     "peak": FP16_DENSE_TFLOPS, "unit": "TFLOP/s",
                                     "frac": round(tf / FP16_DENSE_TFLOPS, 5), "flops": flops,
                                     "traffic": traffic("2q8" if q8 else 2)}})


# ------------------------------------------------------------------ config 4
def run_config4(args):
    """PrefixCache restore: 12 full-attention layers x 65536 Q4K tokens and 36 Gated-
    DeltaNet states in one batched copy, then a 1024-token suffix appended per layer."""
    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    S, SUF, cap = 65536, 1024, 131072
    m = pk.ModelKvState(W.N_LAYERS, W.FULL_INTERVAL, W.NUM_HEADS, W.NUM_KV_HEADS, W.HEAD_DIM, cap)
    kb = torch.empty((1, 2, S, 256), device="cuda")
    vb = torch.empty_like(kb)
    for i, l in enumerate(m.layers):
        if isinstance(l, pk.FullAttentionKv):
            pk.fill_normal(kb, W.SEED, W.stream_id(4, W.T_PREFILL_K, i))
            pk.fill_normal(vb, W.SEED, W.stream_id(4, W.T_PREFILL_V, i))
            l._ensure(1).append_quantized(kb, vb)
        else:
            ssm = torch.empty((1, W.DN_HEADS, W.DN_DK, W.DN_DV), device="cuda")
            conv = torch.empty((1, W.DN_CONV_DIM, W.DN_CONV_K - 1), device="cuda")
            gate = torch.empty((1, W.DN_HEADS), device="cuda")
            pk.fill_normal(ssm, W.SEED, W.stream_id(4, W.T_SSM, i), 0.02)
            pk.fill_normal(conv, W.SEED, W.stream_id(4, W.T_CONV, i))
            pk.fill_normal(gate, W.SEED, W.stream_id(4, W.T_GATE, i))
            l.recurrent_state = pk.RecurrentState(ssm, conv, gate)
    del kb, vb
    prefix = m.save_prefix_cache(list(range(S)))
    ks = torch.empty((1, 2, SUF, 256), device="cuda")
    vs = torch.empty_like(ks)
    pk.fill_normal(ks, W.SEED, W.stream_id(4, W.T_SUFFIX_K))
    pk.fill_normal(vs, W.SEED, W.stream_id(4, W.T_SUFFIX_V))
    full = m.full_layers()

    def restore():
        m.restore_prefix_cache(prefix)

    def step():
        restore()
        for l in full:
            l.quantized_cache.append_quantized(ks, vs, offset=S)

    # from HIP graphs, as a serving loop would replay them: the segment table travels in
    # the kernel's arguments, so a restore is one kernel launch; the eager times (host
    # work of building the per-layer targets from Python included) are reported beside
    ms_restore_eager = event_time(torch, restore, args.steps, args.warmup)
    ms_eager = event_time(torch, step, args.steps, args.warmup)
    ms_restore = graph_time(torch, restore, args.steps, args.warmup)
    ms = graph_time(torch, step, args.steps, args.warmup)

    def suffix():
        for l in full:
            l.quantized_cache.append_quantized(ks, vs, offset=S)
    ms_suffix = graph_time(torch, suffix, args.steps, args.warmup)
    full_bytes = len(full) * S * 2 * 2 * Q4K_ROW
    lin_bytes = (W.N_LAYERS - len(full)) * 4 * (W.DN_HEADS * W.DN_DK * W.DN_DV +
                                                W.DN_CONV_DIM * (W.DN_CONV_K - 1) + W.DN_HEADS)
    moved = 2 * (full_bytes + lin_bytes)  # read + write
    gbs = moved / (ms_restore * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_restore(full[0].quantized_cache, ks, vs, S, SUF, len(full))
    r = base_result(4, "PrefixCache restore GB/s (12 x 65536-token Q4K layers + 36 DeltaNet "
                          "states) and restore + 1024-token suffix µs",
                       round(gbs, 1), "GB/s", True, ms, args,
                       "config4: restore_prefix_cache of 12 full layers (65536 Q4K tokens each) "
                       "and 36 linear layers in one batched copy; then append a 1024-token "
                       "suffix to every full layer",
                       {"restore_us": round(ms_restore * 1000, 2),
                        "restore_plus_suffix_us": round(ms * 1000, 2),
                        "eager_restore_us": round(ms_restore_eager * 1000, 2),
                        "eager_restore_plus_suffix_us": round(ms_eager * 1000, 2),
                        "restored_bytes": full_bytes + lin_bytes,
                        "suffix_appends_us": round(ms_suffix * 1000, 2),
                        "append_roofline": append_roofline(
                            f"q4k_append_kernel<2> ({SUF}-token suffix, one layer; two lanes "
                            "per sub-block fit)", "latency", SUF, 2,
                            ms_suffix * 1000 / len(full)),
                        "roofline": {"kernel": "copy_segments (restore)", "bound": "hbm",
                                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                                     "bytes_per_launch": moved, "traffic": traffic(4),
                                     "traffic_source": MEASURED_TRAFFIC[4][1]}})
    if cpu is not None:
        r["cpu_baseline"] = cpu
    return r


def cpu_baseline_restore(cache, ks, vs, S, SUF, layers):
    """Config 4 on the oracle's restatement of the reference's CPU restore path
    (qwen3_next.rs:2819-2884): a saved quantized layer is f32 (save_kv_state dequantizes,
    :2780-2815), and restore_kv_state clears the cache, re-quantizes every saved row through
    append and dequantizes the whole cache once more (the discarded get_kv, :2843-2847);
    then the suffix's 1024 tokens are quantized and appended. The 36 DeltaNet states are
    restored by reference (Arc clones of contiguous tensors, :4106-4132): no work. The
    oracle's codecs are single-threaded. Timed: the restore over the first `sample` saved
    tokens (scaled by S / sample: every part is linear in the rows) plus the whole suffix
    append, for one layer, median of CPU_RUNS runs, times `layers`."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    from paramecia_amd import workloads as W

    sample = min(S, 16384)
    c = oracle_cache_from(cache, 4, S, sample)
    kd, vd = c.get_kv()  # the saved f32 K / V (save_kv_state)
    kd, vd = np.ascontiguousarray(kd), np.ascontiguousarray(vd)
    ksn, vsn = ks.cpu().numpy(), vs.cpu().numpy()
    r = orc.Cache(4, 1, W.NUM_KV_HEADS, W.HEAD_DIM, sample + SUF)
    t_rest, t_suf = [], []
    for _ in range(CPU_RUNS):
        t0 = time.perf_counter()
        r.clear()
        assert r.append(kd, vd) == 0
        r.get_kv()
        t1 = time.perf_counter()
        assert r.append(ksn, vsn) == 0
        t2 = time.perf_counter()
        t_rest.append(t1 - t0)
        t_suf.append(t2 - t1)
    per_layer = median(t_rest) * S / sample + median(t_suf)
    return {"value": round(per_layer * layers * 1e6, 1), "unit": "us per restore + suffix",
            "cores": 1, "kind": "port",
            "sample": f"config 4: one layer's re-quantizing restore over the first {sample} of "
                      f"{S} saved tokens (scaled by {S / sample:g}) plus its {SUF}-token suffix "
                      f"append, median of {CPU_RUNS} runs, times {layers} layers; DeltaNet "
                      f"states restore by reference (no work); single-threaded oracle codecs "
                      f"on {cpu_model()}",
            "restore_runs_s": [round(x, 4) for x in t_rest],
            "suffix_runs_s": [round(x, 4) for x in t_suf]}


# ------------------------------------------------------------------ config 5
def run_config5(args):
    """16 independent sequences (cached lengths seeded in [1024, 65536], 5 outlier
    channels x20 in K and V), 12 layers: one decode step appends a token to and attends
    over every sequence of every layer."""
    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    lens = W.c5_lengths()
    chans = W.c5_channels()
    L, N = W.N_FULL, W.C5_SEQS
    if args.paged:
        return run_config5_paged(args, lens, chans)
    caches = [[None] * N for _ in range(L)]
    for l in range(L):
        for i, S in enumerate(lens):
            c = pk.PreallocatedQuantizedKvCache(1, 2, S + 1, 256, pk.KvCacheQuantization.Q4K)
            kb = torch.empty((1, 2, S, 256), device="cuda")
            vb = torch.empty_like(kb)
            pk.fill_normal(kb, W.SEED, W.stream_id(5, W.T_PREFILL_K, l, i))
            pk.fill_normal(vb, W.SEED, W.stream_id(5, W.T_PREFILL_V, l, i))
            pk.scale_channels(kb, chans, W.C5_OUTLIER_SCALE)
            pk.scale_channels(vb, chans, W.C5_OUTLIER_SCALE)
            c.append_quantized(kb, vb)
            caches[l][i] = c
            del kb, vb
    q = torch.empty((L, N, 16, 256), device="cuda")
    kn = torch.empty((L, N, 2, 256), device="cuda")
    vn = torch.empty_like(kn)
    for l in range(L):
        pk.fill_normal(q[l], W.SEED, W.stream_id(5, W.T_Q, l))
        pk.fill_normal(kn[l], W.SEED, W.stream_id(5, W.T_NEW_K, l))
        pk.fill_normal(vn[l], W.SEED, W.stream_id(5, W.T_NEW_V, l))
        pk.scale_channels(kn[l], chans, W.C5_OUTLIER_SCALE)
        pk.scale_channels(vn[l], chans, W.C5_OUTLIER_SCALE)

    def step():
        for l in range(L):
            for i, S in enumerate(lens):
                caches[l][i].truncate(S)  # rewind the previous step's token
            pk.append_attend_batched(caches[l], kn[l], vn[l], q[l], W.SCALE)

    reps = args.graph_reps if args.graph_reps > 0 else 1
    ms = graph_time(torch, step, args.steps, args.warmup, reps)
    nbytes = L * sum(layer_bytes(S + 1) for S in lens)
    gbs = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_batched(caches[0], kn[0], vn[0], q[0], lens, args.cpu_threads, L)
    r = base_result(5, "batched decode µs/step (16 sequences, 12 layers, Q4K)",
                       round(ms * 1000, 2), "us/step", False, ms, args,
                       "config5: 16 batch-1 Q4K caches per layer (seeded lengths 1024-65536, "
                       "5 outlier channels x20), 12 layers; step = append 1 token + attend, "
                       "every sequence of every layer",
                       {"sequence_lengths": lens, "graph_steps_per_replay": reps,
                        "roofline": {"kernel": "pkv_append_attend_batched", "bound": "hbm",
                                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                                     "bytes_per_step": nbytes,
                                     "traffic_per_layer": traffic(5)}})
    if cpu is not None:
        r["cpu_baseline"] = cpu
    return r


def cpu_baseline_batched(caches, kn, vn, q, lens, threads, layers):
    """Config 5 on the oracle's faithful CPU path (each sequence's decode step as
    cpu_baseline_decode times it: the reference serves one sequence at a time). Timed on
    the shortest, a middle and the longest sequence of layer 0 (all cores; median of
    CPU_RUNS runs each), fitted as t = a + b * keys and summed over the 16 sequences and
    the layers; the one-thread leg times the shortest sequence and scales by the keys."""
    from paramecia_amd import workloads as W

    nthreads = cpu_threads(threads)
    order = sorted(range(len(lens)), key=lambda i: lens[i])
    picks = [order[0], order[len(order) // 2], order[-1]]
    xs, ts = [], []
    single = None
    for i in picks:
        S = lens[i]
        c = oracle_cache_from(caches[i], 4, S, S)
        knp = kn[i:i + 1].unsqueeze(2).cpu().numpy()
        vnp = vn[i:i + 1].unsqueeze(2).cpu().numpy()
        qnp = q[i:i + 1].unsqueeze(1).cpu().numpy()

        def once(th):
            t0 = time.perf_counter()
            assert c.append_at(knp, vnp, S) == 0
            c.attend(qnp, W.SCALE, S, True, mode="faithful", threads=th)
            return time.perf_counter() - t0

        xs.append(S + 1)
        ts.append(median([once(nthreads) for _ in range(CPU_RUNS)]))
        if i == order[0]:
            single = (S + 1, median([once(1) for _ in range(CPU_RUNS)]))
        del c
    b = (ts[-1] - ts[0]) / max(1, xs[-1] - xs[0])
    a = max(0.0, ts[0] - b * xs[0])
    keys = [S + 1 for S in lens]
    per_layer = sum(a + b * k for k in keys)
    return {"value": round(per_layer * layers * 1e6, 1), "unit": "us/step", "cores": nthreads,
            "kind": "port",
            "sample": f"config 5: decode steps of the sequences with {xs[0]}, {xs[1]} and {xs[2]} "
                      f"keys of layer 0, each the median of {CPU_RUNS} runs on {nthreads} OpenMP "
                      f"threads, fitted t = a + b keys (a {a * 1e3:.3g} ms, b {b * 1e9:.4g} ns) "
                      f"and summed over the 16 sequences and {layers} layers; {cpu_model()}",
            "sample_s": [round(x, 4) for x in ts],
            "single_thread": {
                "value": round(single[1] * sum(keys) / single[0] * layers * 1e6, 1),
                "unit": "us/step", "cores": 1,
                "sample": f"one thread, the {single[0]}-key sequence's step, median of {CPU_RUNS} "
                          f"runs, scaled by the step's {sum(keys)} keys per layer and {layers} "
                          f"layers"}}


def run_config5_paged(args, lens, chans):
    """Config 5's workload on paged caches: per layer one page pool (--paged tokens per
    page) holding the 16 sequences; a step is one fused call per layer
    (pkv_seq_append_decode_batched: one decode launch over all the sequences' pages that
    also quantizes their new tokens, then the combine), timed from a HIP graph and
    eagerly. The unfused form (one batched append launch, then pkv_seq_decode_batched) is
    timed eagerly beside it."""
    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    L, N, P = W.N_FULL, W.C5_SEQS, args.paged
    pools, seqs = [], []
    for l in range(L):
        pool = pk.PagedKvPool(2, 256, P, sum(-(-(S + 1) // P) for S in lens) + N,
                              pk.KvCacheQuantization.Q4K)
        row = []
        for i, S in enumerate(lens):
            sq = pool.sequence()
            kb = torch.empty((1, 2, S, 256), device="cuda")
            vb = torch.empty_like(kb)
            pk.fill_normal(kb, W.SEED, W.stream_id(5, W.T_PREFILL_K, l, i))
            pk.fill_normal(vb, W.SEED, W.stream_id(5, W.T_PREFILL_V, l, i))
            pk.scale_channels(kb, chans, W.C5_OUTLIER_SCALE)
            pk.scale_channels(vb, chans, W.C5_OUTLIER_SCALE)
            sq.append_quantized(kb, vb)
            row.append(sq)
            del kb, vb
        pools.append(pool)
        seqs.append(row)
    q = torch.empty((L, N, 16, 256), device="cuda")
    kn = torch.empty((L, N, 2, 1, 256), device="cuda")
    vn = torch.empty_like(kn)
    for l in range(L):
        pk.fill_normal(q[l], W.SEED, W.stream_id(5, W.T_Q, l))
        pk.fill_normal(kn[l], W.SEED, W.stream_id(5, W.T_NEW_K, l))
        pk.fill_normal(vn[l], W.SEED, W.stream_id(5, W.T_NEW_V, l))
        pk.scale_channels(kn[l], chans, W.C5_OUTLIER_SCALE)
        pk.scale_channels(vn[l], chans, W.C5_OUTLIER_SCALE)
    outs = [None] * L

    def step():
        for l in range(L):
            for i, S in enumerate(lens):
                seqs[l][i].truncate(S)  # rewind the previous step's token
            outs[l] = pools[l].append_decode_batched(seqs[l], kn[l], vn[l], q[l], W.SCALE)

    def step_unfused():
        for l in range(L):
            for i, S in enumerate(lens):
                seqs[l][i].truncate(S)
            pools[l].append_batched(seqs[l], kn[l], vn[l])
            outs[l] = pools[l].decode_batched(seqs[l], q[l], W.SCALE)

    # Q4K pools keep their page lists on the device, so a step whose sequences gain no
    # page is captured in a HIP graph like the contiguous caches' step; eager beside it
    eager_ms = event_time(torch, step, args.steps, args.warmup)
    ms = graph_time(torch, step, args.steps, args.warmup, 1)
    ms_unfused = event_time(torch, step_unfused, args.steps, args.warmup)
    nbytes = L * sum(layer_bytes(S + 1) for S in lens)
    gbs = nbytes / (ms * 1e-3) / 1e9
    pages = sum(-(-(S + 1) // P) for S in lens)
    return base_result(5, "batched decode µs/step (16 sequences, 12 layers, Q4K, paged caches)",
                       round(ms * 1000, 2), "us/step", False, ms, args,
                       f"config5 on paged caches: one pool per layer, {P}-token pages "
                       f"({pages} pages per layer), the 16 sequences of config 5; step = one "
                       "fused append + decode call per layer (HIP graph)",
                       {"sequence_lengths": lens, "page_tokens": P, "pages_per_layer": pages,
                        "eager_us_per_step": round(eager_ms * 1000, 2),
                        "unfused_us_per_step": round(ms_unfused * 1000, 2),
                        "roofline": {"kernel": "pkv_seq_append_decode_batched",
                                     "bound": "hbm", "achieved": round(gbs, 1),
                                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                                     "bytes_per_step": nbytes, "traffic": None}})


# ------------------------------------------------------------------ config 6
def run_config6(args):
    """The other 36 layers of the decode step: one Gated-DeltaNet autoregressive step per
    linear-attention layer (pkv_deltanet_step; qwen3_next.rs:3392-3470), Qwen3-Next shape
    (32 value heads, 128 x 128 f32 state), batch --dn-batch. Not a BASELINE config: the
    row after the KV-cache path (the recurrent state that PrefixCache also restores)."""
    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    B, L, H, D = args.dn_batch, W.N_LINEAR, W.DN_HEADS, W.DN_DK
    layers = []
    for l in range(L):
        lin = pk.LinearAttentionState(scale=D ** -0.5, eps=W.RMS_EPS)
        ssm = torch.empty((B, H, D, D), device="cuda")
        pk.fill_normal(ssm, W.SEED, W.stream_id(6, W.T_SSM, l), 0.02)
        conv = torch.zeros((B, W.DN_CONV_DIM, W.DN_CONV_K - 1), device="cuda")
        lin.recurrent_state = pk.RecurrentState(ssm, conv, torch.zeros((B, H), device="cuda"))
        layers.append(lin)
    ins = []
    for l in range(L):
        t = {}
        for name, code, shape in (("q", W.T_DN_Q, (B, 1, H, D)), ("k", W.T_DN_K, (B, 1, H, D)),
                                  ("v", W.T_DN_V, (B, 1, H, D)), ("g", W.T_DN_GATE, (B, 1, H)),
                                  ("b", W.T_DN_BETA, (B, 1, H))):
            t[name] = torch.empty(shape, device="cuda")
            pk.fill_normal(t[name], W.SEED, W.stream_id(6, code, l))
        t["g"] = -t["g"].abs() * 0.1  # log decay < 0
        ins.append(t)
    outs = [None] * L

    def step():
        for l in range(L):
            t = ins[l]
            outs[l] = layers[l].delta_net_autoregressive(t["q"], t["k"], t["v"], t["g"], t["b"])

    ms_eager = event_time(torch, step, args.steps, args.warmup)
    ms = graph_time(torch, step, args.steps, args.warmup)
    # the kernel's share of the graph step: every layer has its own state, so the 36
    # launches stream 36 distinct states (one layer relaunched alone would find its
    # state in the 256 MB last-level cache)
    per_layer = B * H * (2 * D * D * 4 + 3 * D * 4 + 2 * 4 + 4 + D * 4)  # state r+w, q k v, g b, offset, out
    gbs = per_layer * L / (ms * 1e-3) / 1e9
    gbs_one, ms_one = gbs, ms / L
    r = base_result(6, "Gated-DeltaNet decode step µs (36 linear-attention layers, one token)",
                    round(ms * 1000, 2), "us/step", False, ms, args,
                    f"config6: 36 Gated-DeltaNet layers, batch {B}, 32 value heads, 128 x 128 "
                    "f32 state updated in place per layer (l2norm q/k, decay, delta rule, "
                    "output)",
                    {"eager_us_per_step": round(ms_eager * 1000, 2),
                     "step_hbm_gbs": round(gbs, 1),
                     "roofline": {"kernel": "deltanet_step_kernel (one layer, its share of "
                                            "the graph-replayed step)", "bound": "hbm",
                                  "achieved": round(gbs_one, 1), "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(gbs_one / HBM_PEAK_GBS, 4),
                                  "bytes_per_launch": per_layer,
                                  "avg_launch_us": round(ms_one * 1000, 3),
                                  "traffic": traffic(6) if B == 16 else None}})
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import numpy as np
        import oracle as orc
        t = ins[0]
        npy = lambda x: np.ascontiguousarray(x.cpu().numpy()[:, 0])  # drop the token axis
        S = layers[0].recurrent_state.ssm_state.cpu().numpy().copy()
        go = layers[0].recurrent_state.gate_cumsum_offset.cpu().numpy().copy()
        args_np = [npy(t[n]) for n in ("q", "k", "v", "g", "b")]
        t0 = time.perf_counter()
        orc.deltanet_step(*args_np, S, go, D ** -0.5, W.RMS_EPS)
        dt = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": round(dt * L * 1e6, 1), "unit": "us/step", "cores": 1,
                             "kind": "port",
                             "sample": f"config 6: 1 of {L} layers, one step timed once and "
                                       f"multiplied by {L}; scalar oracle on {cpu_model()}"}
    return r


# ------------------------------------------------------------------ config 7
def run_config7(args):
    """The step after the attention in the 12 full-attention layers: sigmoid gate and the
    wo projection (pkv_gated_oproj; qwen3_next.rs:2657-2680), 4096 -> 2048 (the
    Qwen3-Next-80B hidden size), batch --op-batch tokens, weight type --op-wtype. From 8
    tokens on the library runs the batched MFMA form (pkv_oproj_mfma.hip), below it the
    per-token GEMV. Not a BASELINE config."""
    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    B, L = args.op_batch, W.N_FULL
    IN, OUT = W.NUM_HEADS * W.HEAD_DIM, W.HIDDEN
    wt = W.W_TYPES[args.op_wtype]
    blk, nbytes = W.W_BLOCK[wt]
    nsb = IN // 256
    ws, xs, gs = [], [], []
    for l in range(L):
        if wt == 12:
            # the layer's wo, drawn N(0, 0.02) and quantized to GGUF Q4K rows by the
            # library's own quantize-on-append kernel (one superblock per cache row)
            w = torch.empty((1, 1, OUT * nsb, 256), device="cuda")
            pk.fill_normal(w, W.SEED, W.stream_id(7, W.T_WO, l), 0.02)
            c = pk.PreallocatedQuantizedKvCache(1, 1, OUT * nsb, 256, pk.KvCacheQuantization.Q4K)
            c.append_quantized(w, w)
            kb, _ = c.raw_bytes()
            ws.append(kb.clone())
            del c, w, kb
        else:
            # random valid blocks of the type (no quantizer for it on the path)
            ws.append(torch.from_numpy(W.kquant_rows(wt, OUT, IN, W.SEED + 101 * l)).cuda())
        x = torch.empty((B, 1, IN), device="cuda")
        g = torch.empty((B, 1, IN), device="cuda")
        pk.fill_normal(x, W.SEED, W.stream_id(7, W.T_Q, l))
        pk.fill_normal(g, W.SEED, W.stream_id(7, W.T_GATE, l))
        xs.append(x)
        gs.append(g)
    outs = [None] * L

    def step():
        for l in range(L):
            outs[l] = pk.gated_o_proj(xs[l], gs[l], ws[l], OUT, w_type=wt)

    step()  # grow the library's workspace before any capture
    ms_eager = event_time(torch, step, args.steps, args.warmup)
    ms = graph_time(torch, step, args.steps, args.warmup)
    wbytes = OUT * (IN // blk) * nbytes
    per_layer = wbytes + B * (2 * IN * 4 + OUT * 4)  # weights, attn + gate in, out
    gbs = per_layer * L / (ms * 1e-3) / 1e9
    batched = B >= 8 and wt != 8
    name = args.op_wtype.upper()
    extra = {"eager_us_per_step": round(ms_eager * 1000, 2), "w_type": name,
             "form": "batched MFMA" if batched else "per-token GEMV"}
    if batched:
        flops = 2.0 * B * OUT * IN  # algorithmic: one multiply-add per weight and token
        tfs = flops * L / (ms * 1e-3) / 1e12
        extra["roofline"] = {"kernel": "oproj_xprep + oproj_mfma (+ reduce) per layer, its share "
                                       "of the graph-replayed step", "bound": "mfma",
                             "achieved": round(tfs, 1), "peak": 2500.0, "unit": "TFLOP/s",
                             "frac": round(tfs / 2500.0, 4), "flops_per_launch": flops,
                             "avg_launch_us": round(ms * 1000 / L, 3), "traffic": None,
                             "hbm_bytes_per_launch": per_layer,
                             "hbm_GBps": round(gbs, 1)}
    else:
        extra["roofline"] = {"kernel": f"oproj GEMV ({name}; one layer, its share of the "
                                       "graph-replayed step)", "bound": "hbm",
                             "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": per_layer,
                             "avg_launch_us": round(ms * 1000 / L, 3), "traffic": None}
    r = base_result(7, f"gated o_proj µs/step (12 full-attention layers, {name} wo 4096 -> 2048)",
                    round(ms * 1000, 2), "us/step", False, ms, args,
                    f"config7: sigmoid(gate) * attention output, then the {name} wo projection "
                    f"(4096 -> 2048), 12 layers, {B} token(s)", extra)
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        nb = min(B, 4)  # the scalar oracle takes ~0.1 s per token and layer
        x0, g0 = xs[0][:nb, 0].cpu().numpy().copy(), gs[0][:nb, 0].cpu().numpy().copy()
        w0 = ws[0].cpu().numpy()
        t0 = time.perf_counter()
        orc.gated_oproj(x0, g0, w0, wt, OUT)
        dt = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": round(dt * L * B / nb * 1e6, 1), "unit": "us/step",
                             "cores": 1, "kind": "port",
                             "sample": f"config 7: {nb} of {B} tokens of 1 of {L} layers "
                                       f"(dequantize every wo row per token, then the dot "
                                       f"products) timed once and scaled by {B / nb:g} x {L}; "
                                       f"scalar oracle on {cpu_model()}"}
    return r


COMPANIONS = ("1", "2", "4", "5")  # BASELINE configs measured beside the headline


def companion_configs(torch, args, runners):
    """Configs 1, 2, 4 and 5 measured after the headline in the same run (no CPU
    baselines), summarised for the headline line. A config that fails records its error
    instead, so that the headline line is still printed."""
    sub = argparse.Namespace(**vars(args))
    sub.no_cpu_baseline = True
    sub.paged = 0
    out = {}
    for cfg in COMPANIONS:
        try:
            r = runners[cfg](sub)
            c = {k: r[k] for k in ("metric", "value", "unit", "ms_per_step", "steps")}
            c["workload"] = r["config"]["workload"]
            rf = r.get("roofline")
            if rf:
                c["roofline"] = {k: rf[k] for k in ("kernel", "bound", "achieved", "peak",
                                                     "unit", "frac") if k in rf}
            out[cfg] = c
        except Exception as e:  # reported in the line, not raised
            out[cfg] = {"error": f"{type(e).__name__}: {e}"}
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="3",
                    help="1, 2, 3 (headline, default), 4, 5, 6 (Gated-DeltaNet step), "
                         "7 (gated o_proj) or all")
    ap.add_argument("--dn-batch", type=int, default=1, help="config 6: sequences per step")
    ap.add_argument("--op-batch", type=int, default=1, help="config 7: tokens per step")
    ap.add_argument("--op-wtype", default="q4k", choices=["q4k", "q5k", "q6k", "q8_0"],
                    help="config 7: GGUF type of wo")
    ap.add_argument("--cached", type=int, default=131072, help="config 3: cached tokens")
    ap.add_argument("--quant", default="q4k", choices=["q4k", "q8_0"],
                    help="config 2: cache quantization")
    ap.add_argument("--paged", type=int, default=0,
                    help="config 5: run the workload on paged caches with this many tokens "
                         "per page (a power of two)")
    ap.add_argument("--layers", type=int, default=12, help="config 3: layers")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph-reps", type=int, default=0,
                    help="steps captured per HIP graph replay (0: per-config default)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--prep", action="store_true",
                    help="configs 2 and 3: start from the q/k/v projection outputs, so q_norm, "
                         "k_norm and rope run inside the step (the fused preparation)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the timed runs, launch a plain elementwise copy of this many "
                         "MiB (read N, write N) 3 times: the reference kernel that scales "
                         "rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes")
    ap.add_argument("--no-graph", action="store_true",
                    help="time every step eagerly, capturing no HIP graph (for rocprofv3 "
                         "counter passes, which do not support graph capture here)")
    ap.add_argument("--no-copy-ceiling", action="store_true",
                    help="skip the device-to-device copy ceiling measured after each config")
    ap.add_argument("--warm-seconds", type=float, default=0.25,
                    help="each timed run's warm-up lasts at least this long (and at least "
                         "--warmup calls): the GPU clocks ramp up under sustained work")
    ap.add_argument("--headline-only", action="store_true",
                    help="default run: measure config 3 only, without configs 1, 2, 4 and 5")
    args = ap.parse_args()
    global NO_GRAPH, WARM_S
    NO_GRAPH = args.no_graph
    WARM_S = max(0.0, args.warm_seconds)
    if args.gpus != 1:
        print("bench.py measures the single-GPU path only: every GPU box in this build has "
              "one MI355X, and the KV-cache path needs no collectives (see DESIGN.md for how "
              "it would shard). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    torch.cuda.set_device(torch.device("cuda:0"))
    runners = {"1": run_config1, "2": run_config2, "3": run_config3, "4": run_config4,
               "5": run_config5, "6": run_config6, "7": run_config7}
    which = list(runners) if args.config == "all" else [args.config]
    for cfg in which:
        if cfg not in runners:
            print(f"unknown config {cfg}", file=sys.stderr)
            return 2
        r = runners[cfg](args)
        torch.cuda.empty_cache()
        if args.calib_copy_mib > 0:
            calib_copy(torch, args.calib_copy_mib)
        if not args.no_copy_ceiling:
            add_copy_ceiling(torch, r)
        if cfg == "3" and args.config == "3" and not args.headline_only:
            r["other_configs"] = companion_configs(torch, args, runners)
        print(json.dumps(r), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
