#!/usr/bin/env python3
"""Throughput of the DINOv3 ViT-S+/16 forward pass on one MI355X.

A step is one resident hipGraph replay of the full 12-block forward over one
batch of synthetic images already in HBM (the scope of the reference's
ForwardTimings, engine.rs:272): float32 NCHW pixels in, float32
[batch, 201, 384] tokens out. The headline workload is BASELINE.json's
config 3 (batch 64 at 224x224); batch 32 (config 2) is reported beside it.
Weights are the seeded BASELINE random init; inputs are seeded N(0, 1).

Prints one JSON line with the metric, the roofline of the dominant kernel
(device time from HIP events on the model's stream) and the float64 CPU
oracle timed on this host as a baseline.
"""
import argparse
import json
import os
import re
import statistics
import subprocess
import sys
import tempfile
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dinov3-loom_amd"))

METRIC = "images/sec ViT-S+/16 224² at batch 32/64 on 1 MI355X; % MFMA roofline"
PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA
PEAK_GBS = 8000.0  # MI355X HBM3E
GFLOP_PER_IMAGE = 12.2415  # 224x224 forward, algorithmic


def kernel_work(name, b, T, G):
    """Algorithmic (flops, bytes) of one launch."""
    r, P, H = b * T, G * G, 384
    f16, f32 = 2, 4
    if name == "patch_embed":
        return 2 * b * P * 768 * H, b * 3 * (16 * G) ** 2 * f32 + H * 768 * f16 + r * H * f16
    if name == "layernorm":
        return 0, 2 * r * H * f16
    if name == "layernorm_f32":
        return 0, r * H * (f16 + f32)
    if name == "qkv_rope":
        return 2 * r * H * 3 * H, r * H * f16 + 3 * H * H * f16 + 3 * r * H * f16
    if name == "attention":
        return 4 * b * 6 * T * T * 64, 4 * r * H * f16
    if name == "resid_384":
        return 2 * r * H * H, r * H * f16 + H * H * f16 + 2 * r * H * f16
    if name == "resid_1536":
        return 2 * r * 1536 * H, r * 1536 * f16 + 1536 * H * f16 + 2 * r * H * f16
    if name == "swiglu":
        return 2 * r * H * 3072, r * H * f16 + 3072 * H * f16 + r * 1536 * f16
    if name == "splitk":
        return 2 * r * 1536 * H, r * 1536 * f16 + 1536 * H * f16 + 4 * r * H * f32
    if name == "splitk_reduce":
        return 0, 4 * r * H * f32 + 2 * r * H * f16
    raise KeyError(name)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "forward_b64_traffic.md")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` at batch 64, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated there), or None."""
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"traffic\[" + re.escape(kernel) + r"\] = (\d+) bytes/launch", text)
    return int(m.group(1)) if m else None


def timed_replays(model, b, steps):
    model.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.replay(b)
    model.synchronize()
    return (time.perf_counter() - t0) / steps


def trial_time(model, b, stage, passes=2, warmup=3, steps=30):
    """Seconds per replay of one plan for the short trials that pick the
    image grouping: the best of `passes` runs of `steps` replays, each
    after `warmup` replays (a single run of a few replays picked a plan 5 %
    slower now and then)."""
    stage()
    best = float("inf")
    for _ in range(passes):
        for _ in range(warmup):
            model.replay(b)
        best = min(best, timed_replays(model, b, steps))
    return best


def replay_distribution(model, b, samples):
    """Host-clock times of synchronised replays, the reference's
    ForwardTimings scope and statistics (engine.rs:130-190): median =
    t[n/2], p95 = t[ceil(0.95 n) - 1] of the sorted samples, in seconds."""
    t = []
    for _ in range(samples):
        model.synchronize()
        t0 = time.perf_counter()
        model.replay(b)
        model.synchronize()
        t.append(time.perf_counter() - t0)
    t.sort()
    return t[len(t) // 2], t[-(-95 * len(t) // 100) - 1]


def sync_stats(model, b, samples):
    med, p95 = replay_distribution(model, b, samples)
    return {"median_ms": round(med * 1e3, 4), "p95_ms": round(p95 * 1e3, 4), "samples": samples,
            "images_per_s_at_median": round(b / med, 1),
            "what": "the reference's ForwardTimings statistic (engine.rs:130-190): host clock around each replay "
                    "with a synchronisation before and after; median t[n/2] and p95 t[ceil(0.95 n) - 1]"}


def read_sclk_mhz():
    """Current shader clock from rocm-smi (None where it is unavailable)."""
    try:
        out = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    m = re.search(r"sclk clock level: \d+: \((\d+)Mhz\)", out)
    return int(m.group(1)) if m else None


def sustained(model, b, seconds=4.0, chunk=40):
    """Throughput over several seconds of back-to-back replays (synchronised
    every `chunk` replays) with the shader clock sampled meanwhile: the GPU
    lowers its clock under sustained MFMA load, so this rate sits below the
    short timed region's."""
    clocks, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            v = read_sclk_mhz()
            if v is None:
                return
            clocks.append(v)
            stop.wait(0.1)

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(chunk):
            model.replay(b)
        model.synchronize()
        n += chunk
    dt = time.perf_counter() - t0
    stop.set()
    th.join()
    settled = clocks[len(clocks) // 4:] or clocks
    return {"value": round(n * b / dt, 1), "seconds": round(dt, 2),
            "sclk_mhz": ({"median": int(statistics.median(settled)), "min": min(settled), "max": max(settled),
                          "samples": len(clocks)} if clocks else None),
            "what": "back-to-back replays for several seconds, shader clock from rocm-smi (first quarter of the "
                    "samples dropped while it settles)"}


def ceilings(full=False):
    """Machine ceilings from dhx_probe (one wave per SIMD, 32x32x16 f16 MFMAs;
    the measurement library libdinov3_probe.so, not the forward's): the MFMA
    loop alone on random and on zero operands, and with full=True the vector
    work and the load rates that still leave the MFMAs unslowed."""
    from dinov3_hrx.ceilings import probe
    out = {"mfma_random": probe("mfma_random"), "mfma_zeros": probe("mfma_zeros")}
    if full:
        out["valu_fma_per_mfma"] = {n: probe("valu", n) for n in (0, 2, 4, 6, 8)}
        out["exp2_per_mfma"] = {n: probe("exp2", n) for n in (1, 2)}
        out["accumulator_chains"] = {n: probe("chains", n) for n in (1, 2, 4, 8)}
        for where in ("l1", "l2", "hbm"):
            rows = {n: probe(f"loads_{where}", n) for n in (0, 2, 3, 4, 6)}
            for n, r in rows.items():  # per-CU load rate: 4 waves x n KB per 8-MFMA iteration
                r["cu_bytes_per_clk"] = round(4 * n * 1024 / r["cycles_per_8_mfma"], 1)
            out[f"loads_{where}_per_8_mfma"] = rows
    for v in out.values():
        for r in (v.values() if "tflops" not in v else [v]):
            for k in ("cycles_per_8_mfma", "tflops", "clock_ghz"):
                r[k] = round(r[k], 3 if k == "clock_ghz" else 1)
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(path, seconds):
    """The float64 C oracle on this host: one thread (the `cpu_baseline`
    object, like the reference's single-threaded oracle) and, beside it, all
    usable cores (OpenMP over rows and heads), each for about `seconds`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import dinov3_hrx as d
    import oracle

    w = oracle.Weights.from_file(path)
    px = d.random_pixels(1, 64)

    def run(threads, budget):
        oracle.set_threads(threads)
        n, t0 = 0, time.perf_counter()
        while n < 64:
            oracle.forward(w, px[n], 14)
            n += 1
            if time.perf_counter() - t0 >= budget:
                break
        return n, time.perf_counter() - t0

    n, dt = run(1, seconds)
    usable = len(os.sched_getaffinity(0))
    cores = min(16, usable)
    nm, dtm = run(cores, seconds / 3)
    return {"value": round(n / dt, 4), "unit": "images/s", "cores": 1, "kind": "port", "cpu": cpu_model(),
            "sample": f"{n} image(s) of the b=64 workload at 224x224 through the float64 C oracle "
                      f"(oracle/dinov3_oracle.c), 1 thread, {dt:.1f} s",
            "all_cores": {"value": round(nm / dtm, 4), "cores": cores, "nproc": os.cpu_count(),
                          "usable_cpus": usable,
                          "sample": f"{nm} image(s), {cores} threads (min(16, usable CPUs)), {dtm:.1f} s"}}


def library_gemms(batch, iters=20, reps=30):
    """Vendor-library (torch.matmul -> hipBLASLt) f16 GEMMs at the forward's four shapes, for
    comparison with the fused kernels (which also do LayerNorm folding, RoPE, SwiGLU or the
    residual update in their epilogues). Each GEMM is captured `iters` times into one CUDA graph
    (so host launch overhead does not count, as for the fused kernels' graph replays) and the
    graph replayed `reps` times; the median replay over `iters` is the time per GEMM. Only the
    time is used, not the products. Prints a markdown table; not the metric."""
    import torch
    rows = batch * 201
    print(f"| GEMM (M = {rows}) | N | K | library us | library TFLOP/s |")
    print("|---|---|---|---|---|")
    for name, n, k in [("gate/up", 3072, 384), ("qkv", 1152, 384), ("down", 384, 1536), ("o-proj", 384, 384)]:
        a = torch.randn(rows, k, device="cuda", dtype=torch.float16)
        w = torch.randn(n, k, device="cuda", dtype=torch.float16)
        for _ in range(10):
            torch.nn.functional.linear(a, w)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(iters):
                torch.nn.functional.linear(a, w)
        times = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            graph.replay()
            torch.cuda.synchronize()
            times.append((time.perf_counter() - t0) * 1e6 / iters)
        us = statistics.median(times)
        print(f"| {name} | {n} | {k} | {us:.2f} | {2 * rows * n * k / us / 1e6:.0f} |", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--image-size", type=int, default=224,
                    help="224: the headline (batch 64) with batch 32, batch 1, end-to-end and 512x512 legs beside it; "
                         "512: BASELINE.json config 5 alone (use --batch 8), for profiling that workload")
    ap.add_argument("--sync-samples", type=int, default=100,
                    help="synchronised replays for the median / p95 (at least 10)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the batch-32, batch-1, end-to-end and 512x512 measurements (for profiling runs)")
    ap.add_argument("--branches", type=int, default=0,
                    help="image groups run as concurrent graph branches (0: pick 1-4 by a short trial)")
    ap.add_argument("--down-proj", choices=("auto", "resid", "splitk"), default="auto",
                    help="down-projection variant (auto: pick by a short trial)")
    ap.add_argument("--unfused-layernorm", action="store_true",
                    help="run the plan with separate f16 LayerNorm kernels (the reference's) instead of LayerNorm "
                         "folded into the QKV and gate/up GEMMs (for profiling those kernels)")
    ap.add_argument("--library-gemms", action="store_true",
                    help="only time the vendor library's GEMMs at the forward's shapes (a reference table)")
    ap.add_argument("--ceilings", action="store_true",
                    help="only run the machine-ceiling probes (MFMA issue, power-limited clock, co-issued vector "
                         "work, load rates) and print them as one JSON line")
    args = ap.parse_args()
    if args.library_gemms:
        library_gemms(args.batch)
        return
    if args.ceilings:
        print(json.dumps(ceilings(full=True)))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the forward would shard by image, "
              "with no exchange between GPUs). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import dinov3_hrx as d

    b, S = args.batch, args.image_size
    G = S // 16
    T = G * G + 5
    full = S == 224 and not args.no_legs  # the headline run with its side legs
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "weights.safetensors")
        d.write_random_weights(path, seed=0, preset=0)
        model = d.DINOv3.load(path, d.Options(device=0, max_batch=max(b, 32) if full else b, image_size=S))
        px = d.random_pixels(1, b, S)
        if args.unfused_layernorm:
            model.set_layernorm_fusion(0)

        # Pick the down-projection variant (the reference uses the residual
        # GEMM for b > 1, split-K at b = 1) and the number of image groups run
        # side by side by a short trial: every grouping gives the same bits,
        # the two variants agree to f16 rounding.
        trial = {}
        for mode in {"auto": (0, 1), "resid": (0,), "splitk": (1,)}[args.down_proj]:
            for nb in ([args.branches] if args.branches else range(1, max(1, min(4, b // 4)) + 1)):
                model.set_splitk(mode)
                model.set_branches(nb)
                trial[(mode, nb)] = trial_time(model, b, lambda: model.stage(px))
        mode, branches = min(trial, key=trial.get)
        print(json.dumps({"trial_images_per_s": {f"{'splitk' if k[0] else 'resid'}/{k[1]}": round(b / v, 1)
                                                 for k, v in trial.items()}}), file=sys.stderr)
        model.set_splitk(mode)
        model.set_branches(branches)
        model.stage(px)
        for _ in range(args.warmup):
            model.replay(b)
        sec = timed_replays(model, b, args.steps)
        value = b / sec
        sync = sync_stats(model, b, max(10, args.sync_samples))
        steady = sustained(model, b) if full else None

        if full:
            sec32, sync32, branches32, sec1, p95_1, mode1, e2e_rate = side_legs(d, model, px, b, branches, mode, args)

        # Per-launch device time (HIP events on the model's stream), each
        # kernel alone over the whole batch: the single-group plan.
        model.set_branches(1)
        model.stage(px)
        table = kernel_table(model.launch_timings(b, iters=20), b, T, G)
        dom = table[0]
        flops, nbytes = kernel_work(dom["kernel"], b, T, G)
        ridge = PEAK_TFLOPS * 1e12 / (PEAK_GBS * 1e9)
        if flops and flops / nbytes >= ridge:
            roof = {"kernel": dom["kernel"], "bound": "mfma", "achieved": dom["tflops"], "peak": PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(dom["tflops"] / PEAK_TFLOPS, 4)}
        else:
            roof = {"kernel": dom["kernel"], "bound": "hbm", "achieved": dom["gbs"], "peak": PEAK_GBS,
                    "unit": "GB/s", "frac": round(dom["gbs"] / PEAK_GBS, 4)}
        roof["traffic"] = measured_traffic(dom["kernel"]) if (b == 64 and S == 224) else None
        ceiling = ceilings() if full else None
        if ceiling:
            # The MFMA loop alone on random operands, on this GPU and its power
            # budget: what the published peak shrinks to once the clock drops.
            ceil_random = ceiling["mfma_random"]
            if roof["bound"] == "mfma":
                roof["attainable"] = {"peak": ceil_random["tflops"], "clock_ghz": ceil_random["clock_ghz"],
                                      "frac": round(dom["tflops"] / ceil_random["tflops"], 4),
                                      "what": "MFMA-only loop on random f16 operands, one wave per SIMD (dhx_probe)"}
        roof["algorithmic_bytes"] = nbytes
        roof["avg_us"] = dom["avg_us"]
        model.close()

        if full:
            # Config 5 beside it: 512x512 (1029 tokens), batch 8, the same weights.
            hr = d.DINOv3.load(path, d.Options(device=0, max_batch=8, image_size=512))
            pxh = d.random_pixels(2, 8, 512)
            trial_hr = {}
            for nb in ([args.branches] if args.branches else [1, 2]):
                hr.set_branches(nb)
                hr.stage(pxh)
                trial_hr[nb] = timed_replays(hr, 8, 5)
            branches_hr = min(trial_hr, key=trial_hr.get)
            hr.set_branches(branches_hr)
            hr.stage(pxh)
            for _ in range(5):
                hr.replay(8)
            sec_hr = timed_replays(hr, 8, max(10, args.steps // 4))
            hr.close()

        cpu = None if (args.no_cpu or not full) else cpu_baseline(path, args.cpu_seconds)

    for row in table:
        print(json.dumps(row), file=sys.stderr)
    gflop_image = GFLOP_PER_IMAGE if S == 224 else sum(kernel_work(k, 1, T, G)[0] * n for k, n in
                                                   (("patch_embed", 1), ("qkv_rope", 12), ("attention", 12),
                                                    ("resid_384", 12), ("swiglu", 12), ("resid_1536", 12))) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "images/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": f"DINOv3 ViT-S+/16 forward, {S}x{S}, batch {b}, resident hipGraph replay "
                               f"(BASELINE.json config {3 if S == 224 else 5})", "batch": b, "image_size": S, "tokens": T,
                   "down_proj": "splitk" if mode == 1 else "resid", "branches": branches,
                   "layernorm": "separate kernels" if args.unfused_layernorm else "folded into the GEMMs",
                   "weights": "seeded random init (BASELINE)"},
        "mfma_frac_forward": round(value * gflop_image / 1e3 / PEAK_TFLOPS, 4),
        "value_scope": f"back-to-back replays: batch / (host time of {args.steps} replays queued without waiting, "
                       f"one synchronisation before and after / {args.steps}), after {args.warmup} warmup replays; "
                       "sync_replay is the reference's per-replay statistic",
        "sync_replay": sync,
    }
    if full:
        line.update({
            "batch32": {"value": round(32 / sec32, 1), "ms_per_step": round(sec32 * 1e3, 4), "branches": branches32,
                        "sync_replay": sync32},
            "batch1": {"value": round(1 / sec1, 1), "ms_per_step": round(sec1 * 1e3, 4),
                       "p95_ms": round(p95_1 * 1e3, 4), "down_proj": "splitk" if mode1 == 1 else "resid",
                       "what": "median synchronised graph-replay latency of one image (the reference's b = 1 case)"},
            "highres_512_b8": {"value": round(8 / sec_hr, 1), "unit": "images/s",
                               "ms_per_step": round(sec_hr * 1e3, 4), "branches": branches_hr,
                               "what": "BASELINE.json config 5: 512x512, 1029 tokens, batch 8"},
            "sustained": steady,
            "end_to_end": {"value": round(e2e_rate[4], 1), "unit": "images/s",
                           "value_16_chunks": round(e2e_rate[16], 1),
                           "b1_ms": round(e2e_rate["b1"][0] * 1e3, 4), "b1_p95_ms": round(e2e_rate["b1"][1] * 1e3, 4),
                           "b4_ms": round(e2e_rate["b4"][0] * 1e3, 4), "b4_p95_ms": round(e2e_rate["b4"][1] * 1e3, 4),
                           "what": f"forward() of {4 * b} (and {16 * b}) images from host memory to host memory "
                                   f"(PCIe and host copies included, chunks of {b} pipelined); b1/b4: median and "
                                   f"p95 latency of forward() of 1 and 4 images, host to host; not the metric"},
        })
    line.update({"roofline": roof, "cpu_baseline": cpu, "ceilings": ceiling, "kernels": table})
    print(json.dumps(line))


def kernel_table(launches, b, T, G):
    """Per-kernel rows (launch count, average and total device time, achieved
    TFLOP/s and GB/s at algorithmic work) from one plan's launch timings,
    largest total first."""
    kernels = {}
    for i, (name, ms) in enumerate(launches):
        name = {"patch_embed_stats": "patch_embed", "qkv_rope_ln": "qkv_rope", "resid_stats": "resid",
                "swiglu_ln": "swiglu", "splitk_reduce_stats": "splitk_reduce"}.get(name, name)
        if name == "resid":
            # the down projection (k = 1536) follows the SwiGLU GEMM; the o-projection (k = 384) follows attention
            name = "resid_1536" if launches[i - 1][0].startswith("swiglu") else "resid_384"
        k = kernels.setdefault(name, {"count": 0, "ms": 0.0})
        k["count"] += 1
        k["ms"] += ms
    table = []
    for name, k in kernels.items():
        flops, nbytes = kernel_work(name, b, T, G)
        avg = k["ms"] / k["count"]
        tf = flops / (avg * 1e-3) / 1e12
        gbs = nbytes / (avg * 1e-3) / 1e9
        table.append({"kernel": name, "launches": k["count"], "avg_us": round(avg * 1e3, 2),
                      "total_us": round(k["ms"] * 1e3, 1), "tflops": round(tf, 1), "gbs": round(gbs, 1),
                      "mfma_frac": round(tf / PEAK_TFLOPS, 4), "hbm_frac": round(gbs / PEAK_GBS, 4)})
    table.sort(key=lambda r: -r["total_us"])
    return table


def side_legs(d, model, px, b, branches, mode, args):
    """The headline run's side measurements on the same resident model:
    batch 32 (config 2), batch 1 (the reference's own case) and forward()
    end to end through host memory."""
    # Batch 32 (config 2) on the same resident model, with its own short
    # trial of the image grouping.
    px32 = px[:32] if b >= 32 else d.random_pixels(1, 32)
    trial32 = {}
    for nb in ([args.branches] if args.branches else [1, 2, 3, 4]):
        model.set_branches(nb)
        trial32[nb] = trial_time(model, 32, lambda: model.stage(px32))
    branches32 = min(trial32, key=trial32.get)
    model.set_branches(branches32)
    model.stage(px32)
    for _ in range(args.warmup):
        model.replay(32)
    sec32 = timed_replays(model, 32, args.steps)
    sync32 = sync_stats(model, 32, max(10, args.sync_samples))
    model.set_branches(branches)

    # Batch 1 (the reference's own benchmark case: graph-replay latency of
    # one image), with the down-projection variant picked by its own short
    # trial (the reference takes split-K there, lib.rs:218-225).
    trial1 = {}
    for variant in (0, 1):
        model.set_splitk(variant)
        model.stage(px[:1])  # records this variant's batch-1 graph
        for _ in range(args.warmup):
            model.replay(1)
        trial1[variant] = replay_distribution(model, 1, 20)[0]
    mode1 = min(trial1, key=trial1.get)
    model.set_splitk(mode1)
    model.stage(px[:1])
    sec1, p95_1 = replay_distribution(model, 1, max(10, args.sync_samples))
    model.set_splitk(mode)

    # End to end through the host API (PCIe-inclusive; never `value`):
    # forward() of 4 and of 16 chunks of b images from host memory to host
    # memory (each call returning a new array, as the API does), with the
    # pipelined uploads and readbacks; 16 chunks show the pipeline's steady
    # state, 4 the weight of its first and last chunk.
    e2e_rate = {}
    for chunks in (4, 16):
        big = np.concatenate([px] * chunks)
        model.forward(big)
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            model.forward(big)
            times.append(time.perf_counter() - t0)
        e2e_rate[chunks] = len(big) / sorted(times)[1]
        del big
    # The reference's own warm end-to-end figure: forward() of 1 and of 4
    # images, host to host, median and p95 over repeated calls.
    for n in (1, 4):
        model.forward(px[:n])
        lat = []
        for _ in range(max(20, args.sync_samples // 2)):
            t0 = time.perf_counter()
            model.forward(px[:n])
            lat.append(time.perf_counter() - t0)
        lat.sort()
        e2e_rate[f"b{n}"] = (statistics.median(lat), lat[min(len(lat) - 1, int(0.95 * len(lat)))])
    return sec32, sync32, branches32, sec1, p95_1, mode1, e2e_rate


if __name__ == "__main__":
    main()
