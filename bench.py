#!/usr/bin/env python3
"""Decoder KV-cache step benchmark on one MI355X.

Workload: the longform streaming decoder -- 26 layers, an 8192-slot sliding
ring that is full and wrapping (every step evicts the oldest position), F16 KV,
32 query / 8 KV heads x 128, one stream.  One step = one token = for every
layer, append the token's K/V row (f32 -> f16) at pos % 8192 and run the
single-query GQA attention over all 8192 retained positions, through the
vkv_decoder_step C entry point: one decode kernel (append fused in its
prologue, split-K attention over slot chunks) plus a small kernel merging the
chunk partials.  Inputs (Q, K, V for every timed step) are generated on the
device before timing.

Prints one JSON line: tokens/s, the roofline of the decode step (algorithmic
bytes / average step time from HIP events on the launch stream, bracketing
both kernels of the step, so it understates the decode kernel alone), and the CPU
baseline (the oracle's threaded restatement of ggml's CPU flash-attention
step, timed on a bounded sample on this host).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "voxtral.cpp_amd"))
sys.path.insert(0, ROOT)

LAYERS, CAP, KVH, HD, QH = 26, 8192, 8, 128, 32
KV_DIM, Q_DIM = KVH * HD, QH * HD
SEED = 20261201
HBM_PEAK_GBPS = 8000.0


def algorithmic_bytes_per_step(n_valid, elem_bytes):
    """K+V read of the window, new K/V f32 read, appended row write, Q read,
    output write -- per layer, times the layer count."""
    per_layer = (n_valid * 2 * KV_DIM * elem_bytes + 2 * KV_DIM * 4 + 2 * KV_DIM * elem_bytes +
                 Q_DIM * 4 + Q_DIM * 4)
    return LAYERS * per_layer


def gpu_leg(steps, warmup):
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    cache = vkv.Cache(n_streams=1, n_layers=LAYERS, capacity=CAP, n_kv_heads=KVH, head_dim=HD,
                      n_q_heads=QH, dtype=vkv.F16)
    ring = vkv.new_ring(CAP)
    # fill the ring: positions [0, 8192) through the planned append path
    plan = vkv.decoder_plan(ring, 0, CAP)
    k0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    v0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    vkv.synth_rows(k0.data_ptr(), KV_DIM, SEED, vkv.TAG_K, nl=LAYERS, p0=0, np_=CAP, hip_stream=sp)
    vkv.synth_rows(v0.data_ptr(), KV_DIM, SEED, vkv.TAG_V, nl=LAYERS, p0=0, np_=CAP, hip_stream=sp)
    cache.append(0, 0, LAYERS, vkv.plan_segs(plan.write_seg, plan.write_nseg), k0.data_ptr(),
                 v0.data_ptr(), hip_stream=sp)
    vkv.decoder_commit(ring, plan)
    del k0, v0
    # resident per-step inputs, [step][layer][...]
    T = warmup + steps
    q = torch.empty(T, LAYERS, Q_DIM, device="cuda")
    k = torch.empty(T, LAYERS, KV_DIM, device="cuda")
    v = torch.empty(T, LAYERS, KV_DIM, device="cuda")
    for t, tag, n in ((q, vkv.TAG_Q, Q_DIM), (k, vkv.TAG_K, KV_DIM), (v, vkv.TAG_V, KV_DIM)):
        vkv.synth_rows(t.data_ptr(), n, SEED, tag, nl=LAYERS, l_stride=1, p0=CAP, np_=T,
                       p_stride=LAYERS, hip_stream=sp)
    out = torch.empty(T, LAYERS, Q_DIM, device="cuda")
    rings = (vkv.Ring * 1)(ring)
    scale = 1.0 / (HD ** 0.5)
    pos = CAP

    def step(i):
        nonlocal pos
        cache.decoder_step(0, rings, [pos], 0, LAYERS, q[i].data_ptr(), k[i].data_ptr(),
                           v[i].data_ptr(), out[i].data_ptr(), scale, hip_stream=sp)
        pos += 1

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(st)
    for i in range(steps):
        ev[2 * i].record(st)
        step(warmup + i)
        ev[2 * i + 1].record(st)
    t_end.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_start.elapsed_time(t_end)
    kern_ms = [ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(steps)]
    ring_after = rings[0]
    assert ring_after.used == CAP and ring_after.next_absolute_position == CAP + T
    assert bool(torch.isfinite(out).all())
    cache.close()
    return total_ms, kern_ms, wall


def cpu_leg(target_seconds):
    """The oracle's threaded ggml-CPU restatement of the same step (append +
    attention over 8192 positions, 26 layers) on a bounded number of tokens."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle

    threads = min(os.cpu_count() or 1, 16)
    rb = oracle.row_bytes(oracle.F16, KV_DIM)
    layer_bytes = rb * CAP
    kimg = np.empty(LAYERS * layer_bytes, np.uint8)
    vimg = np.empty(LAYERS * layer_bytes, np.uint8)

    def fill(job):
        img, tag, l = job
        img[l * layer_bytes:(l + 1) * layer_bytes] = oracle.expected_layer(
            oracle.F16, CAP, CAP, KV_DIM, CAP, SEED, tag, 0, l)

    with ThreadPoolExecutor(threads) as pool:
        list(pool.map(fill, [(img, tag, l) for img, tag in ((kimg, oracle.TAG_K), (vimg, oracle.TAG_V))
                             for l in range(LAYERS)]))
    scale = 1.0 / (HD ** 0.5)
    secs, n = 0.0, 0
    while n < 1 or (secs < target_seconds and n < 64):
        pos = CAP + n
        qs = np.stack([oracle.synth_row(SEED, oracle.TAG_Q, 0, l, pos, Q_DIM) for l in range(LAYERS)])
        ks = np.stack([oracle.synth_row(SEED, oracle.TAG_K, 0, l, pos, KV_DIM) for l in range(LAYERS)])
        vs = np.stack([oracle.synth_row(SEED, oracle.TAG_V, 0, l, pos, KV_DIM) for l in range(LAYERS)])
        dt, _ = oracle.decode_step_mimic_mt(oracle.F16, kimg, vimg, layer_bytes, rb, LAYERS, CAP, qs,
                                            QH, KVH, HD, scale, threads, ks, vs, pos % CAP)
        secs += dt
        n += 1
    return {"value": n / secs, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} decode steps (26 layers, 8192-position window, f16 KV) of the oracle's "
                      f"restatement of ggml's CPU flash-attention step, {threads} threads, "
                      f"{secs:.1f} s"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB 20 times (scales rocprof "
                         "FETCH_SIZE/WRITE_SIZE counters to bytes)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 20}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures the single-GPU KV step; --gpus {args.gpus} is not supported "
              "(this path has no multi-GPU leg)", file=sys.stderr)
        sys.exit(2)

    traffic = None
    pmc = os.path.join(ROOT, "profiles", "decode_f16_26x8192_pmc.json")
    if os.path.exists(pmc):
        # HBM bytes per decode launch from the committed rocprofv3 FETCH_SIZE /
        # WRITE_SIZE runs of this same workload (scaled by a plain-copy calibration)
        with open(pmc) as f:
            traffic = json.load(f).get("traffic_bytes_per_launch")

    total_ms, kern_ms, wall = gpu_leg(args.steps, args.warmup)
    ms_per_step = total_ms / args.steps
    kern_avg = sum(kern_ms) / len(kern_ms)
    bytes_step = algorithmic_bytes_per_step(CAP, 2)
    achieved = bytes_step / (kern_avg * 1e-3) / 1e9
    res = {
        "metric": "decode attn+KV-append tokens/s and achieved HBM GB/s (% of peak) at 8192 window",
        "value": round(args.steps / (total_ms * 1e-3), 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded integer Irwin-Hall N(0,1) Q/K/V, generated on device)",
        "config": {"workload": "decoder KV step: 26 layers, 8192-slot ring full and wrapping, "
                               "f16 KV, 32 q / 8 kv heads x 128, 1 stream, append + 1-query "
                               "attention per layer",
                   "layers": LAYERS, "window": CAP, "kv_heads": KVH, "q_heads": QH,
                   "head_dim": HD, "streams": 1},
        "hbm_gbps": round(bytes_step / (ms_per_step * 1e-3) / 1e9, 1),
        "pct_hbm_peak": round(100 * bytes_step / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": round(traffic) if traffic else None,
                     "kernel": "k_decode<FmtF16,4,fused append> + k_combine (one step)",
                     "bytes_per_launch": bytes_step,
                     "avg_launch_ms": round(kern_avg, 5)},
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_leg(args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
