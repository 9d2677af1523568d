"""Benchmark of the KV-reuse hot path on one MI355X.

Default workload (the headline metric): Llama-3-8B KV
shape -- 32 layers of a [2, 65536, 16, 8, 128] bf16 paged cache (128 GiB),
8 cached chunks x 1024 tokens staged in the store's record layout (per chunk,
per layer in sorted name order, [K|V][pages][16,8,128]), K stored at positions
0..1023 and re-rotated to the concatenated offsets 0..8191 (delta 1024*c,
rope_theta 500000) while being scattered into the cache through a seeded
random block table. One step = one CacheCopier.scatter_pages_rerotate call
(256 jobs). The return path (gather of the whole request into a contiguous
[L, 2, T, H, D] staging buffer) is timed as well and reported beside it.

  python bench.py [--steps K] [--warmup W] [--no-cpu]

Prints one JSON line. `value` = reused KV tokens/s of the whole call (wall
clock around K back-to-back steps, inputs resident in HBM); `roofline` uses
the fused kernel's own duration, measured with HIP events on its launch
stream; `cpu_baseline` times the CPU oracle (a single-threaded numpy/torch
restatement) on a time-bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0

CFG2 = dict(layers=32, kv_heads=8, head_dim=128, block_size=16, num_blocks=65536,
            chunks=8, chunk_tokens=1024, rope_theta=500000.0, dtype="bf16")


def layer_names(n):
    # the reference orders layers lexicographically (configs/engine.py:25-27)
    return sorted(f"model.layers.{i}.self_attn.attn" for i in range(n))


def build_workload(cfg, device, num_blocks=None, layers=None, seed=0):
    """Synthetic config-2 inputs: paged cache, staging records, block table."""
    L = layers if layers is not None else cfg["layers"]
    NB = num_blocks if num_blocks is not None else cfg["num_blocks"]
    H, D, PS = cfg["kv_heads"], cfg["head_dim"], cfg["block_size"]
    C, CT = cfg["chunks"], cfg["chunk_tokens"]
    T = C * CT
    n_pages = T // PS
    g = torch.Generator().manual_seed(seed)
    ids = (torch.randperm(NB - 1, generator=g)[:n_pages] + 1).to(torch.int32)
    names = layer_names(L)
    cache = [torch.empty(2, NB, PS, H, D, dtype=torch.bfloat16, device=device) for _ in range(L)]
    span = PS * H * D * 2
    job_bytes = 2 * (CT // PS) * span
    gd = torch.Generator(device=device).manual_seed(seed + 1) if device.type == "cuda" else \
        torch.Generator().manual_seed(seed + 1)
    staging = torch.randn(C * L * job_bytes // 2, generator=gd, device=device,
                          dtype=torch.bfloat16).view(torch.uint8)
    jobs = dict(names=[], offsets=[], sizes=[], flat=[], ioff=[0], deltas=[], ntok=[])
    off = 0
    for c in range(C):
        bids = ids[c * (CT // PS):(c + 1) * (CT // PS)].tolist()
        for name in names:
            jobs["names"].append(name)
            jobs["offsets"].append(off)
            jobs["sizes"].append(job_bytes)
            jobs["flat"].extend(bids)
            jobs["ioff"].append(len(jobs["flat"]))
            jobs["deltas"].append(c * CT)      # new ptr[0] - saved_pos
            jobs["ntok"].append(CT)
            off += job_bytes
    inv = (1.0 / (cfg["rope_theta"] ** (torch.arange(0, D, 2, dtype=torch.float32) / D))).float()
    return dict(L=L, NB=NB, T=T, names=names, cache=cache, staging=staging, jobs=jobs, ids=ids,
                inv_freq=inv, span=span)


def algorithmic_bytes(cfg, T=None, L=None):
    L = L or cfg["layers"]
    T = T or cfg["chunks"] * cfg["chunk_tokens"]
    return T * L * 2 * (2 * cfg["kv_heads"] * cfg["head_dim"] * 2)


def time_steps(step, steps, warmup, stream):
    """W untimed warm-up steps, then two timed passes of `steps` steps each:
    pass 1 (the measurement) brackets the K steps with device synchronisation
    and HIP events on `stream`; pass 2 times every kernel launch of the library
    with its own HIP events on the launch stream (kernel duration for the
    roofline), kept out of pass 1 so that the per-launch events cannot slow the
    measured steps."""
    from daric_amd import cache_ops
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        step()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = start.elapsed_time(stop) / steps
    cache_ops.timing_enable(True)
    cache_ops.timing_read()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kern_ms, launches = cache_ops.timing_read()
    cache_ops.timing_enable(False)
    return dict(step_ms=step_ms, wall_s=wall, kern_ms=kern_ms / max(launches, 1),
                launches_per_step=launches / max(steps, 1))


def run_gpu(cfg, steps, warmup):
    from daric_amd import cache_ops
    dev = torch.device("cuda:0")
    w = build_workload(cfg, dev)
    cp = cache_ops.CacheCopier()
    for name, t in zip(w["names"], w["cache"]):
        cp.register_layer(name, t, False)
    cp.register_store(w["staging"])
    j = w["jobs"]
    idx = torch.tensor(j["flat"], dtype=torch.int32, device=dev)
    inv = w["inv_freq"].to(dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        cp.scatter_pages_rerotate(j["names"], j["offsets"], j["sizes"], idx, j["ioff"], j["deltas"],
                                  j["ntok"], inv, cfg["head_dim"], True, stream.cuda_stream)

    fused = time_steps(step, steps, warmup, stream)

    # return path: gather the whole request into [L, 2, T, H, D]
    T, L = w["T"], w["L"]
    out = torch.empty(L * 2 * T * cfg["kv_heads"] * cfg["head_dim"] * 2, dtype=torch.uint8, device=dev)
    gcp = cache_ops.CacheCopier()
    for name, t in zip(w["names"], w["cache"]):
        gcp.register_layer(name, t, False)
    gcp.register_store(out)
    per_layer = 2 * T * cfg["kv_heads"] * cfg["head_dim"] * 2
    gids = w["ids"].to(dev)
    g_off = [i * per_layer for i in range(L)]
    g_sizes = [per_layer] * L
    g_flat = torch.cat([gids] * L)
    g_ioff = [i * gids.numel() for i in range(L + 1)]

    def gstep():
        gcp.gather_pages(w["names"], g_off, g_sizes, g_flat, g_ioff, stream.cuda_stream)

    gather = time_steps(gstep, steps, warmup, stream)
    return dict(step_ms=fused["step_ms"], wall_s=fused["wall_s"], kern_ms=fused["kern_ms"],
                g_step_ms=gather["step_ms"], g_kern_ms=gather["kern_ms"], T=T, L=L)


def run_cpu_baseline(cfg, budget_s=12.0):
    """The CPU oracle's fused scatter + re-rotate over the whole workload (all
    layers, 256 jobs) with a reduced 1024-block pool (same bytes moved): one
    warm-up run, then repeated runs until `budget_s` has elapsed (at most 5);
    the median run time gives tokens/s."""
    from oracle.copy import OracleCopier
    torch.set_num_threads(1)
    w = build_workload(cfg, torch.device("cpu"), num_blocks=1024)
    j = w["jobs"]
    inv = w["inv_freq"].numpy()
    oc = OracleCopier()
    for name, t in zip(w["names"], w["cache"]):
        oc.register_layer(name, t, False)
    oc.register_store(w["staging"])
    idx = torch.tensor(j["flat"], dtype=torch.int32)

    def run():
        oc.scatter_pages_rerotate(j["names"], j["offsets"], j["sizes"], idx, j["ioff"], j["deltas"],
                                  j["ntok"], inv, cfg["head_dim"], True)

    run()
    times = []
    while len(times) < 5 and sum(times) < budget_s:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    T = w["T"]
    return dict(value=T / med, unit="reused KV tokens/s", cores=1, kind="port",
                sample=f"whole workload (32 layers x 8 chunks x 1024 tokens, 1024-block pool) through "
                       f"the CPU oracle oracle/copy.py scatter_pages_rerotate, one thread, median of "
                       f"{len(times)} runs ({med:.2f} s each) after one warm-up",
                GBps=algorithmic_bytes(cfg) / med / 1e9)


def run_copy_calibration(steps, nbytes=1 << 30):
    """A plain contiguous device copy of `nbytes` (reads nbytes, writes nbytes),
    run `steps` times: the kernel whose rocprofv3 FETCH_SIZE / WRITE_SIZE
    readings calibrate those counters against a known byte count."""
    dev = torch.device("cuda:0")
    src = torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(7)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def read_traffic():
    """HBM bytes per launch of the fused kernel from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration)."""
    p = os.path.join(ROOT, "profiles", "pmc_scatter_rerotate_llama3_8b.md")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1].strip()))
            except ValueError:
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (torch copy_) `steps` times, the "
                         "known-size reference that scales rocprofv3 FETCH_SIZE/WRITE_SIZE")
    a = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the KV-reuse hot path is per-GPU work with no "
              "cross-GPU exchange (see DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    cfg = CFG2
    r = run_gpu(cfg, a.steps, a.warmup)
    if a.calib_copy:
        run_copy_calibration(a.steps)
    nbytes = algorithmic_bytes(cfg)
    tok_s = r["T"] / (r["step_ms"] / 1e3)
    achieved = nbytes / (r["kern_ms"] / 1e3) / 1e9
    g_achieved = nbytes / (r["g_kern_ms"] / 1e3) / 1e9
    cpu = None if a.no_cpu else run_cpu_baseline(cfg, a.cpu_budget)
    line = {
        "metric": "reused KV tokens/sec (re-rotate+scatter) at Llama-3-8B shape; HBM GB/s",
        "value": tok_s,
        "unit": "reused KV tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": r["step_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V, seeded random block table)",
        "config": {"workload": "BASELINE config 2: Llama-3-8B KV re-rotate+scatter, 8x1024-token "
                               "chunks to offsets 0..8191, 65536-block paged cache",
                   **{k: v for k, v in cfg.items()}, "jobs_per_step": r["L"] * cfg["chunks"]},
        "GBps": nbytes / (r["step_ms"] / 1e3) / 1e9,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBPS, "traffic": read_traffic(),
                     "kernel": "scatter_rotate_lane_kernel<bf16,neox>", "kernel_ms": r["kern_ms"],
                     "algorithmic_bytes": nbytes},
        "gather": {"ms_per_step": r["g_step_ms"], "kernel_ms": r["g_kern_ms"],
                   "GBps": g_achieved, "frac": g_achieved / PEAK_HBM_GBPS,
                   "tokens_per_s": r["T"] / (r["g_step_ms"] / 1e3)},
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample", "GBps")},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
