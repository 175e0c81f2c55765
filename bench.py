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
Q4K_ROW = 144


def layer_bytes(keys: int) -> int:
    """Algorithmic HBM bytes of one layer's decode step: the K and V rows of every key
    (2 KV heads x 144 B each), q in and out (16 x 256 f32 each), the new token's f32
    k/v read and its 4 packed rows written."""
    return keys * 2 * 2 * Q4K_ROW + 2 * 16 * 256 * 4 + 2 * 2 * 256 * 4 + 4 * Q4K_ROW


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cached", type=int, default=131072)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the timed runs, launch a plain elementwise copy of this many MiB "
                         "(read N, write N) 3 times: the reference kernel that scales rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures the single-GPU path only: every GPU box in this build has "
              "one MI355X, and the KV-cache path needs no collectives (see DESIGN.md for how "
              "it would shard). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    import paramecia_amd as pk
    from paramecia_amd import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
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
    del kbuf, vbuf
    q = torch.empty((L, 1, 1, W.NUM_HEADS, W.HEAD_DIM), dtype=torch.float32, device=dev)
    kn = torch.empty((L, 1, W.NUM_KV_HEADS, 1, W.HEAD_DIM), dtype=torch.float32, device=dev)
    vn = torch.empty_like(kn)
    for l in range(L):
        pk.fill_normal(q[l], W.SEED, W.stream_id(3, W.T_Q, l))
        pk.fill_normal(kn[l], W.SEED, W.stream_id(3, W.T_NEW_K, l))
        pk.fill_normal(vn[l], W.SEED, W.stream_id(3, W.T_NEW_V, l))
    outs = [torch.empty_like(q[l]) for l in range(L)]
    torch.cuda.synchronize()

    def step(events=None):
        for l in range(L):
            if events is not None:
                events[l][0].record()
            # offset = S rewinds the previous step's token: identical work every step
            outs[l] = caches[l].append_attend(kn[l], vn[l], q[l], W.SCALE, offset=S)
            if events is not None:
                events[l][1].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    # eager: 12 ctypes launches per step from Python (host overhead included)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(end) / args.steps

    # HIP graph of one 12-layer step, replayed (the serving-loop form)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm the workspace on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps

    # per-launch duration of the layer kernel(s): the GPU is kept busy by a sleep kernel
    # while the host enqueues, so each event pair brackets device time only
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(L)] for _ in range(args.steps)]
    sleep = getattr(torch.cuda, "_sleep", None)
    for s_ in range(args.steps):
        if sleep is not None:
            sleep(20_000_000)
        step(ev[s_])
    torch.cuda.synchronize()
    per_launch_ms = sum(a.elapsed_time(b) for row in ev for a, b in row) / (args.steps * L)

    keys = S + 1
    step_bytes = L * layer_bytes(keys)
    achieved = layer_bytes(keys) / (per_launch_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(ms * 1000.0, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "eager_us_per_step": round(eager_ms * 1000.0, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Philox N(0,1), bit-identical to the CPU oracle's generator)",
        "config": {
            "workload": "config3: 12 Qwen3-Next full-attention layers, batch 1, Q4K KV cache "
                        f"with {S} cached tokens; step = per layer quantize-append 1 token + "
                        f"attend over {keys} keys (16 q heads, 2 kv heads, head_dim 256)",
            "layers": L, "cached_tokens": S, "keys": keys, "kv_quant": "Q4K",
            "num_heads": 16, "num_kv_heads": 2, "head_dim": 256, "batch": 1,
        },
        "step_hbm_gbs": round(step_bytes / (ms * 1e-3) / 1e9, 1),
        "step_pct_of_peak": round(100.0 * step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
        "roofline": {
            "kernel": "pkv_append_attend (one layer: append + dequant-fused attention)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "bytes_per_launch": layer_bytes(keys),
            "avg_launch_us": round(per_launch_ms * 1000.0, 2),
            "traffic": None,
        },
        "append_tokens_per_s": round(L * S / fill_s, 1),
    }

    if args.calib_copy_mib > 0:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(caches[0], kn[0], vn[0], q[0], S, args.cpu_threads)
    print(json.dumps(result), flush=True)
    return 0


def cpu_baseline(cache, kn, vn, q, S, threads):
    """The oracle's faithful restatement of the reference CPU path (CPU quantize of the new
    token, dequantize the whole cache, permute, repeat_kv, transposed-K copy, matmul,
    clamp, softmax, matmul) on one layer, extrapolated to the 12-layer step."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    from paramecia_amd import workloads as W

    nthreads = threads if threads > 0 else (os.cpu_count() or 1)
    c = orc.Cache(orc.Q4K, 1, W.NUM_KV_HEADS, W.HEAD_DIM, S + 1)
    cache.truncate(S)
    kb, vb = cache.raw_bytes()
    c.load_bytes(kb.cpu().numpy(), vb.cpu().numpy(), S)
    knp, vnp, qnp = kn.cpu().numpy(), vn.cpu().numpy(), q.cpu().numpy()
    t0 = time.perf_counter()
    assert c.append_at(knp, vnp, S) == 0
    c.attend(qnp, W.SCALE, S, True, mode="faithful", threads=nthreads)
    dt = time.perf_counter() - t0
    try:
        model = [l for l in open("/proc/cpuinfo") if l.startswith("model name")][0].split(":")[1].strip()
    except Exception:
        model = "unknown"
    return {
        "value": round(dt * W.N_FULL * 1e6, 1), "unit": "us/step", "cores": nthreads,
        "kind": "port",
        "sample": f"1 of 12 layers, one decode step (append 1 token + attend {S + 1} keys) "
                  f"timed once and multiplied by 12; {nthreads} OpenMP threads on {model}",
    }


if __name__ == "__main__":
    sys.exit(main())
