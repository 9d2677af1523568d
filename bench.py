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
stream; `cpu_baseline` times the CPU oracle's C restatement (OpenMP, up to 16
host threads) on a time-bounded sample of the same workload.
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
    dt = torch.float16 if cfg.get("dtype") == "fp16" else torch.bfloat16
    cache = [torch.empty(2, NB, PS, H, D, dtype=dt, device=device) for _ in range(L)]
    span = PS * H * D * 2
    job_bytes = 2 * (CT // PS) * span
    gd = torch.Generator(device=device).manual_seed(seed + 1) if device.type == "cuda" else \
        torch.Generator().manual_seed(seed + 1)
    staging = torch.randn(C * L * job_bytes // 2, generator=gd, device=device, dtype=dt).view(torch.uint8)
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


def algorithmic_bytes(cfg, T=None, L=None, e=2):
    L = L or cfg["layers"]
    T = T or cfg["chunks"] * cfg["chunk_tokens"]
    return T * L * 2 * (2 * cfg["kv_heads"] * cfg["head_dim"] * e)


def kernel_ms_per_step(step, steps, stream):
    """Summed kernel time of one step (all of its launches), from the
    kernel-timing pass of time_steps."""
    r = time_steps(step, steps, 1, stream)
    return r["kern_ms"] * r["launches_per_step"]


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

    # the same 256 jobs as a plain scatter_pages (no rotation): the copy rate of
    # this exact access pattern on this box, the ceiling the fused kernel meets
    def pstep():
        cp.scatter_pages(j["names"], j["offsets"], j["sizes"], idx, j["ioff"], stream.cuda_stream)

    plain = time_steps(pstep, steps, warmup, stream)

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

    # the worker-side form: in-place re-rotation of the same 8 chunks in all
    # 32 layers (rerotate_pages, the Adapter's call; K rotated part only)
    CT = cfg["chunk_tokens"]
    pages = CT // cfg["block_size"]
    segs = [(c * pages, 0, CT, c * CT) for c in range(cfg["chunks"]) if c > 0]
    bt_all = w["ids"].to(dev)

    def rstep():
        cache_ops.rerotate_pages(w["cache"], False, bt_all, segs, inv, cfg["head_dim"], True,
                                 stream=stream.cuda_stream)

    inplace = time_steps(rstep, steps, warmup, stream)
    inplace_bytes = sum(s[2] for s in segs) * L * cfg["kv_heads"] * cfg["head_dim"] * 2 * 2

    # the same call on consecutive pages (blocks 1..512): the kernel's rate
    # without the block table's random page addresses
    bt_seq = torch.arange(1, bt_all.numel() + 1, dtype=torch.int32, device=dev)
    inplace_seq = time_steps(lambda: cache_ops.rerotate_pages(w["cache"], False, bt_seq, segs, inv,
                                                              cfg["head_dim"], True, stream=stream.cuda_stream),
                             steps, 1, stream)
    return dict(step_ms=fused["step_ms"], wall_s=fused["wall_s"], kern_ms=fused["kern_ms"],
                p_kern_ms=plain["kern_ms"],
                g_step_ms=gather["step_ms"], g_kern_ms=gather["kern_ms"], T=T, L=L,
                r_step_ms=inplace["step_ms"], r_kern_ms=inplace["kern_ms"], r_bytes=inplace_bytes,
                r_seq_kern_ms=inplace_seq["kern_ms"], r_tokens=sum(s[2] for s in segs))


# ---------------------------------------------------------------------------
# Other BASELINE configurations, measured beside the headline (one GPU each).

CFG3 = dict(layers=32, kv_heads=8, head_dim=128, block_size=16, requests=32, chunks=6,
            chunk_tokens=512, k_frac=0.15, noise_scale=0.1, t_df=3, dtype="bf16")
CFG4 = dict(layers=32, kv_heads=8, head_dim=128, block_size=16, tokens=65536, num_blocks=8192,
            dtype="bf16")
CFG5 = dict(layers=80, kv_heads=8, head_dim=128, block_size=16, chunks=16, chunk_tokens=2048,
            num_blocks=4 * 2048 + 1, rope_theta=500000.0, k_frac=0.10, dtype="e4m3")


def _gbps(nbytes, ms):
    return nbytes / (ms / 1e3) / 1e9


def _student_t(shape, df, gen, device):
    """Student-t samples as N / sqrt(chi2_df / df), chi2 from df squared normals."""
    z = torch.randn(shape, generator=gen, device=device)
    chi = torch.zeros(shape, device=device)
    for _ in range(df):
        chi += torch.randn(shape, generator=gen, device=device) ** 2
    return z / torch.sqrt(chi / df)


def config3_inputs(dev, seed=0):
    """BASELINE config 3's inputs: 32 requests x 6 chunks x 512 tokens = 98304
    tokens, Llama-3-8B KV shape, bf16. Chunk pages come from a seeded
    permutation of the block pool and each request's chunk order is shuffled by
    seed. Recomputed K = cached K + 0.1 * StudentT(3); recomputed V ~ N(0,1);
    k = 77 of 512 per chunk."""
    c = CFG3
    L, H, D, PS = c["layers"], c["kv_heads"], c["head_dim"], c["block_size"]
    n_chunk = c["requests"] * c["chunks"]
    T = n_chunk * c["chunk_tokens"]
    pages_per_chunk = c["chunk_tokens"] // PS
    NB = T // PS + 1024
    g = torch.Generator().manual_seed(seed)
    ids = (torch.randperm(NB - 1, generator=g)[: T // PS] + 1).to(torch.int32)
    # per request, the stored chunks are visited in a shuffled order
    order = []
    for r in range(c["requests"]):
        perm = torch.randperm(c["chunks"], generator=g).tolist()
        order += [r * c["chunks"] + p for p in perm]
    bt = torch.cat([ids[o * pages_per_chunk:(o + 1) * pages_per_chunk] for o in order]).to(dev)
    k = max(1, int(round(c["k_frac"] * c["chunk_tokens"])))
    chunks = [(i * pages_per_chunk, i * c["chunk_tokens"], c["chunk_tokens"], k) for i in range(n_chunk)]
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    layers = [torch.randn(2, NB, PS, H, D, generator=gd, device=dev, dtype=torch.bfloat16) for _ in range(L)]
    k_new = torch.empty(L, T, H, D, dtype=torch.bfloat16, device=dev)
    slot_blk = bt.long().repeat_interleave(PS)
    slot_in = torch.arange(T, device=dev) % PS
    for l in range(L):
        base = layers[l][0][slot_blk, slot_in].float()
        k_new[l] = (base + c["noise_scale"] * _student_t(base.shape, c["t_df"], gd, dev)).to(torch.bfloat16)
    v_new = torch.randn(L, T, H, D, generator=gd, device=dev, dtype=torch.bfloat16)
    return dict(L=L, H=H, D=D, PS=PS, NB=NB, T=T, n_chunk=n_chunk, k=k, layers=layers, bt=bt,
                chunks=chunks, k_new=k_new, v_new=v_new)


def run_config3(steps, warmup, seed=0):
    """Batched selective recompute (config3_inputs). One
    step = select_merge: the deviation keys, the top-k (k = 77 of 512) and the
    merge of the selected K/V rows (the deviation kernel, then one workgroup
    per (layer, chunk) for top-k and merge). The same work as three calls
    (kv_deviation, topk_per_chunk, merge_rows) and as one launch is timed
    beside it."""
    from daric_amd import cache_ops
    dev = torch.device("cuda:0")
    w = config3_inputs(dev, seed)
    L, H, D, T, k, n_chunk = w["L"], w["H"], w["D"], w["T"], w["k"], w["n_chunk"]
    layers, bt, chunks, k_new, v_new = w["layers"], w["bt"], w["chunks"], w["k_new"], w["v_new"]
    keys = torch.empty(L, T, dtype=torch.float32, device=dev)
    sel = torch.empty(L, n_chunk, k, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream

    def dev_step():
        cache_ops.kv_deviation(layers, False, bt, k_new, chunks, keys=keys, stream=st)

    def topk_step():
        cache_ops.topk_per_chunk(keys, chunks, kmax=k, out=sel, stream=st)

    def merge_step():
        cache_ops.merge_rows(layers, False, bt, k_new, v_new, chunks, sel, stream=st)

    def three_calls():
        dev_step()
        topk_step()
        merge_step()

    def step():
        # the library's selection call: the deviation kernel, then one
        # workgroup per (layer, chunk) for the chunk's top-k and merge
        cache_ops.select_merge(layers, False, bt, k_new, v_new, chunks, kmax=k, keys=keys, sel_idx=sel, stream=st)

    def one_pass():
        cache_ops.select_merge(layers, False, bt, k_new, v_new, chunks, kmax=k, keys=keys, sel_idx=sel, stream=st,
                               one_pass=True)

    whole = time_steps(step, steps, warmup, stream)
    # the three forms alternately, three rounds each: medians
    forms = {"select_merge": [], "three_calls": [], "one_pass": []}
    for _ in range(3):
        for name, f in (("select_merge", step), ("three_calls", three_calls), ("one_pass", one_pass)):
            forms[name].append(time_steps(f, steps, 1, stream)["step_ms"])
    forms = {n: sorted(v)[1] for n, v in forms.items()}
    parts = {n: kernel_ms_per_step(f, steps, stream)
             for n, f in (("deviation", dev_step), ("topk", topk_step), ("merge", merge_step),
                          ("topk_merge_fused", lambda: cache_ops.select_merge(
                              layers, False, bt, k_new, v_new, chunks, kmax=k, keys=keys, sel_idx=sel, stream=st,
                              keys_ready=True)))}
    # The merge's address pattern in isolation: the same kernel moving the
    # same rows' worth of bytes, but with each chunk's first k tokens selected
    # and chunks laid on consecutive blocks, so both the recomputed rows read
    # and the cache rows written are sequential at the same 2 KiB granularity.
    PS = w["PS"]
    ppc = w["chunks"][0][2] // PS
    seq_bt = torch.arange(1, n_chunk * ppc + 1, dtype=torch.int32, device=dev)
    seq_sel = torch.arange(k, dtype=torch.int32, device=dev).repeat(L, n_chunk, 1).contiguous()
    seq_ms = time_steps(lambda: cache_ops.merge_rows(layers, False, seq_bt, k_new, v_new, chunks, seq_sel,
                                                     stream=st), steps, 1, stream)["kern_ms"]
    # and the library's page scatter moving the same byte count from a
    # contiguous staging buffer onto random pages of the same cache layers:
    # the same access pattern with 32 KiB page spans for 2 KiB rows
    span = PS * H * D * 2
    npg = (n_chunk * k * (2 * H * D * 2)) // (2 * span)            # pages per layer
    staging = torch.empty(L * npg * 2 * span, dtype=torch.uint8, device=dev)
    cp = cache_ops.CacheCopier()
    names = [f"merge_ref.{i}" for i in range(L)]
    for n, t in zip(names, layers):
        cp.register_layer(n, t, False)
    cp.register_store(staging)
    gen = torch.Generator().manual_seed(seed + 7)
    NB = layers[0].shape[1]
    page_ids = torch.cat([torch.randperm(NB - 1, generator=gen)[:npg] + 1 for _ in range(L)]).to(torch.int32).to(dev)
    sc_offs = [i * npg * 2 * span for i in range(L)]
    sc_ioff = [i * npg for i in range(L + 1)]
    sc_ms = time_steps(lambda: cp.scatter_pages(names, sc_offs, [npg * 2 * span] * L, page_ids, sc_ioff, st),
                       steps, 1, stream)["kern_ms"]
    sc_bytes = 2 * L * npg * 2 * span
    del cp, staging
    e = 2
    dev_bytes = T * L * (2 * H * D * e) + T * L * 4
    topk_bytes = T * L * 4 + n_chunk * L * k * 4
    merge_bytes = n_chunk * k * L * 2 * (2 * H * D * e)
    total = dev_bytes + topk_bytes + merge_bytes
    out = dict(workload="BASELINE config 3: batched selective recompute, 32 req x 6 chunks x 512 "
                        "tokens, Llama-3-8B KV shape bf16, top-15% (k=77) per chunk",
               tokens=T, k=k, ms_per_step=whole["step_ms"], tokens_per_s=T / (whole["step_ms"] / 1e3),
               algorithmic_bytes=total, GBps=_gbps(total, whole["step_ms"]),
               frac=_gbps(total, whole["step_ms"]) / PEAK_HBM_GBPS,
               step_forms=dict(
                   ms=forms, note="the same selection, same process, alternating (median of 3): select_merge "
                                  "(deviation kernel, then one workgroup per (layer, chunk) for top-k and "
                                  "merge; the step above), three_calls (kv_deviation, topk_per_chunk, "
                                  "merge_rows), one_pass (one launch: each workgroup also computes its "
                                  "chunk's keys)"),
               kernels={"deviation": dict(ms=parts["deviation"], bytes=dev_bytes,
                                          GBps=_gbps(dev_bytes, parts["deviation"])),
                        "topk": dict(ms=parts["topk"], bytes=topk_bytes),
                        "topk_merge_fused": dict(ms=parts["topk_merge_fused"], bytes=topk_bytes + merge_bytes,
                                                 GBps=_gbps(topk_bytes + merge_bytes, parts["topk_merge_fused"])),
                        "merge": dict(ms=parts["merge"], bytes=merge_bytes,
                                      GBps=_gbps(merge_bytes, parts["merge"]),
                                      frac=_gbps(merge_bytes, parts["merge"]) / PEAK_HBM_GBPS,
                                      sequential_rows=dict(
                                          ms=seq_ms, GBps=_gbps(merge_bytes, seq_ms),
                                          note="the same merge_rows kernel and byte count with every "
                                               "chunk's first k tokens on consecutive blocks: sequential "
                                               "2 KiB rows on both sides"),
                                      page_scatter=dict(
                                          ms=sc_ms, bytes=sc_bytes, GBps=_gbps(sc_bytes, sc_ms),
                                          merge_frac_of_it=_gbps(merge_bytes, parts["merge"]) / _gbps(sc_bytes, sc_ms),
                                          note="scatter_pages of about the same byte count from a contiguous "
                                               "staging buffer onto random 32 KiB page spans of the same cache "
                                               "layers, same process"))})
    del w, layers, k_new, v_new, keys, sel
    torch.cuda.empty_cache()
    return out


def run_placement(steps, warmup, seed=0):
    """The headline fused call on two config-2 caches held at once (the same
    seeded contents and block table, allocated one after the other), timed
    alternately: how much the cache's place in memory moves the kernel.
    Opt-in (--extra place): the two caches take 258 GiB."""
    from daric_amd import cache_ops
    dev = torch.device("cuda:0")
    cfg = CFG2
    stream = torch.cuda.current_stream(dev)
    calls = []
    for _ in range(2):
        w = build_workload(cfg, dev, seed=seed)
        cp = cache_ops.CacheCopier()
        for name, t in zip(w["names"], w["cache"]):
            cp.register_layer(name, t, False)
        cp.register_store(w["staging"])
        j = w["jobs"]
        idx = torch.tensor(j["flat"], dtype=torch.int32, device=dev)
        inv = w["inv_freq"].to(dev)
        calls.append((w, cp, idx, inv, j))

    def step_of(c):
        w, cp, idx, inv, j = c
        return lambda: cp.scatter_pages_rerotate(j["names"], j["offsets"], j["sizes"], idx, j["ioff"],
                                                 j["deltas"], j["ntok"], inv, cfg["head_dim"], True,
                                                 stream.cuda_stream)
    times = [[], []]
    for _ in range(3):
        for k in (0, 1):
            times[k].append(time_steps(step_of(calls[k]), steps, warmup, stream)["kern_ms"])
    nbytes = algorithmic_bytes(cfg)
    out = {f"cache_{k}": dict(kernel_ms=times[k], GBps=[_gbps(nbytes, t) for t in times[k]],
                              cache_address=hex(calls[k][0]["cache"][0].data_ptr()))
           for k in (0, 1)}
    out["note"] = ("the headline fused call on two caches allocated one after the other and held at "
                   "once, timed alternately three times each")
    del calls
    torch.cuda.empty_cache()
    return out


LAYOUTS = (  # (blocks per layer, layer stride in bytes)
    (8192, 512 << 20),
    (8192, 4 << 30),
    (32768, 2 << 30),
    (32768, 4 << 30),
    (65536, 4 << 30),
)


def run_layout(steps, warmup, seed=0):
    """The headline's 256 jobs (same staging, 512 seeded random pages per
    layer) on 32 layer caches carved from one 132 GiB allocation at the
    layer strides of LAYOUTS, fused call and plain scatter timed alternately,
    three rounds each (kernel-time medians): how the layers' spacing in memory
    sets the rate. Opt-in (--extra layout)."""
    from daric_amd import cache_ops
    dev = torch.device("cuda:0")
    cfg = CFG2
    H, D, PS = cfg["kv_heads"], cfg["head_dim"], cfg["block_size"]
    span = PS * H * D * 2
    w = build_workload(cfg, dev, num_blocks=1024, seed=seed)
    del w["cache"]
    torch.cuda.empty_cache()
    L, C, CT = w["L"], cfg["chunks"], cfg["chunk_tokens"]
    pages_per_chunk = CT // PS
    need = max((L - 1) * stride + 2 * nb * span for nb, stride in LAYOUTS)
    big = torch.empty(need, dtype=torch.uint8, device=dev)
    j = w["jobs"]
    inv = w["inv_freq"].to(dev)
    stream = torch.cuda.current_stream(dev)
    g = torch.Generator().manual_seed(seed)
    runs = []
    for nb, stride in LAYOUTS:
        cp = cache_ops.CacheCopier()
        for l, name in enumerate(w["names"]):
            o = l * stride
            cp.register_layer(name, big[o:o + 2 * nb * span].view(torch.bfloat16).view(2, nb, PS, H, D), False)
        cp.register_store(w["staging"])
        pages = (torch.randperm(nb - 1, generator=g)[: C * pages_per_chunk] + 1).tolist()
        # job order as build_workload's: chunk-major, then the layers
        flat = [p for c in range(C) for _ in range(L) for p in pages[c * pages_per_chunk:(c + 1) * pages_per_chunk]]
        idx = torch.tensor(flat, dtype=torch.int32, device=dev)
        fused = (lambda cp=cp, idx=idx: cp.scatter_pages_rerotate(
            j["names"], j["offsets"], j["sizes"], idx, j["ioff"], j["deltas"], j["ntok"], inv, D, True,
            stream.cuda_stream))
        plain = (lambda cp=cp, idx=idx: cp.scatter_pages(j["names"], j["offsets"], j["sizes"], idx, j["ioff"],
                                                          stream.cuda_stream))
        runs.append((nb, stride, fused, plain))
    times = {(nb, stride): ([], []) for nb, stride, _, _ in runs}
    for _ in range(3):
        for nb, stride, fused, plain in runs:
            times[(nb, stride)][0].append(time_steps(fused, steps, warmup, stream)["kern_ms"])
            times[(nb, stride)][1].append(time_steps(plain, steps, warmup, stream)["kern_ms"])
    nbytes = algorithmic_bytes(cfg)
    out = []
    for nb, stride in LAYOUTS:
        f, p = (float(np.median(x)) for x in times[(nb, stride)])
        out.append(dict(blocks_per_layer=nb, layer_stride_GiB=stride / (1 << 30), fused_kernel_ms=f,
                        fused_GBps=_gbps(nbytes, f), plain_kernel_ms=p, plain_GBps=_gbps(nbytes, p)))
    del big, runs
    torch.cuda.empty_cache()
    return dict(layouts=out, note="headline jobs on 32 layer caches carved from one allocation at the "
                                  "given layer stride (same staging, seeded random pages); fused call "
                                  "and plain scatter alternating, median of 3 rounds")


def run_config2_hnd(steps, warmup, seed=0):
    """Config 2's return path on a head-major cache: the request's 8 x 1024
    tokens in 32 layers of a [2, 65536, 16, 8, 128] bf16 cache stored HND
    ([2, NB, H, PS, D] in memory), gathered token-major into [L, 2, T, H, D]
    (gather_tokens: the LDS-transpose kernel) and scattered back
    (scatter_tokens). gather_pages of the same pages -- the reference's
    physical-span staging, no transpose -- is timed beside them. The cache is
    left uninitialised: the kernels copy bytes, whatever their values."""
    from daric_amd import cache_ops
    c = CFG2
    dev = torch.device("cuda:0")
    L, H, D, PS, NB = c["layers"], c["kv_heads"], c["head_dim"], c["block_size"], c["num_blocks"]
    T = c["chunks"] * c["chunk_tokens"]
    n_pages = T // PS
    g = torch.Generator().manual_seed(seed)
    ids = (torch.randperm(NB - 1, generator=g)[:n_pages] + 1).to(torch.int32)
    names = layer_names(L)
    cache = [torch.empty(2, NB, H, PS, D, device=dev, dtype=torch.bfloat16).permute(0, 1, 3, 2, 4)
             for _ in range(L)]
    per_layer = 2 * T * H * D * 2
    staging = torch.empty(L * per_layer, dtype=torch.uint8, device=dev)
    cp = cache_ops.CacheCopier()
    for n, t in zip(names, cache):
        cp.register_layer(n, t, False)
    cp.register_store(staging)
    flat = torch.cat([ids] * L).to(dev)
    offs = [i * per_layer for i in range(L)]
    sizes = [per_layer] * L
    ioff = [i * n_pages for i in range(L + 1)]
    stream = torch.cuda.current_stream(dev)
    out = {"workload": "config 2 return path on an HND cache ([2, 65536, H=8, PS=16, D=128] bf16 in memory), "
                       "32 layers x 8192 tokens to token-major [L, 2, T, H, D] and back",
           "tokens": T}
    nbytes = 2 * L * per_layer
    for key, fn in (("gather_tokens", cp.gather_tokens), ("scatter_tokens", cp.scatter_tokens),
                    ("gather_pages_physical_span", cp.gather_pages)):
        r = time_steps(lambda fn=fn: fn(names, offs, sizes, flat, ioff, stream.cuda_stream),
                       steps, warmup, stream)
        out[key] = {"ms": r["step_ms"], "kernel_ms": r["kern_ms"], "GBps": _gbps(nbytes, r["kern_ms"]),
                    "frac": _gbps(nbytes, r["kern_ms"]) / PEAK_HBM_GBPS}
    out["algorithmic_bytes"] = nbytes
    del cache, staging
    torch.cuda.empty_cache()
    return out


def config4_inputs(dev, seed=0):
    """BASELINE config 4's inputs: 65536 tokens (4096 pages) of a Llama-3-8B bf16
    cache ([2, 8192, 16, 8, 128] per layer, 32 layers, N(0,1)) chosen by a
    seeded random block table (the null block excluded)."""
    c = CFG4
    L, H, D, PS, NB = c["layers"], c["kv_heads"], c["head_dim"], c["block_size"], c["num_blocks"]
    T = c["tokens"]
    n_pages = T // PS
    g = torch.Generator().manual_seed(seed)
    ids = (torch.randperm(NB - 1, generator=g)[:n_pages] + 1).to(torch.int32)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    cache = [torch.randn(2, NB, PS, H, D, generator=gd, device=dev, dtype=torch.bfloat16) for _ in range(L)]
    return dict(L=L, H=H, D=D, PS=PS, NB=NB, T=T, n_pages=n_pages, ids=ids, names=layer_names(L),
                cache=cache)


def kvio_plan(w, meta_tokens=1024):
    """The store/load pipeline's records over config4_inputs: 64 metas of 1024
    tokens, each record = the 32 layers' page spans + the 4096-byte header."""
    from daric_amd.kv_io import POSITION_SIZE
    meta_pages = meta_tokens // w["PS"]
    ids = w["ids"]
    blocks = [(ids[m * meta_pages:(m + 1) * meta_pages].tolist(),) for m in range(w["n_pages"] // meta_pages)]
    bpb = [2 * w["PS"] * w["H"] * w["D"] * 2] * w["L"]
    rec = w["L"] * bpb[0] * meta_pages + POSITION_SIZE
    return dict(blocks=blocks, bpb=bpb, rec=rec, offsets=[m * rec for m in range(len(blocks))])


def run_config4(steps, warmup, seed=0):
    """KV offload/load: 65536 tokens (4096 pages) of a
    Llama-3-8B bf16 cache with a seeded random block table. Store: gather the
    pages into a device staging buffer (one call, 32 jobs), then one
    hipMemcpyAsync per layer record into pinned host memory on a side stream.
    Load: the reverse (H2D, then scatter). Device-side and host-link rates are
    reported separately."""
    from daric_amd import cache_ops
    dev = torch.device("cuda:0")
    w = config4_inputs(dev, seed)
    L, H, D, PS, T, n_pages = w["L"], w["H"], w["D"], w["PS"], w["T"], w["n_pages"]
    ids, names, cache = w["ids"], w["names"], w["cache"]
    per_layer = 2 * n_pages * PS * H * D * 2
    staging = torch.empty(L * per_layer, dtype=torch.uint8, device=dev)
    host = torch.empty(L * per_layer, dtype=torch.uint8, pin_memory=True)
    cp = cache_ops.CacheCopier()
    for n, t in zip(names, cache):
        cp.register_layer(n, t, False)
    cp.register_store(staging)
    flat = torch.cat([ids] * L).to(dev)
    offs = [i * per_layer for i in range(L)]
    sizes = [per_layer] * L
    ioff = [i * n_pages for i in range(L + 1)]
    stream = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(device=dev)

    gather = time_steps(lambda: cp.gather_pages(names, offs, sizes, flat, ioff, stream.cuda_stream),
                        steps, warmup, stream)
    scatter = time_steps(lambda: cp.scatter_pages(names, offs, sizes, flat, ioff, stream.cuda_stream),
                         steps, warmup, stream)

    def host_copy(d2h):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        side.wait_stream(stream)
        ev0.record(side)
        if d2h:
            cache_ops.batched_memcpy_d2h(staging, host, offs, offs, sizes, side.cuda_stream)
        else:
            cache_ops.batched_memcpy_h2d(host, staging, offs, offs, sizes, side.cuda_stream)
        ev1.record(side)
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1)

    # one untimed copy each way first, then the median of n_host timed copies
    host_copy(True)
    host_copy(False)
    n_host = max(1, min(steps, 3))
    d2h_runs = [host_copy(True) for _ in range(n_host)]
    h2d_runs = [host_copy(False) for _ in range(n_host)]
    d2h_ms = float(np.median(d2h_runs))
    h2d_ms = float(np.median(h2d_runs))
    dev_bytes = 2 * L * per_layer
    link_bytes = L * per_layer
    # the store/load pipeline: 64 records of 1024 tokens, gather/scatter overlapped with host DMA
    from daric_amd.kv_io import KVIOContext
    del staging
    cp = None
    torch.cuda.empty_cache()
    plan = kvio_plan(w)
    blocks, bpb, rec, rec_offs = plan["blocks"], plan["bpb"], plan["rec"], plan["offsets"]
    host_rec = torch.empty(len(blocks) * rec, dtype=torch.uint8, pin_memory=True)
    io = KVIOContext(names, [0] * L, bpb, [False] * L, dict(zip(names, cache)), host_rec,
                     staging_bytes=512 << 20)

    def timed(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    # every 1024-token record was saved at positions 0..1023; the fused load
    # moves meta m to 1024 m (the request's concatenated offsets)
    saved = [0] * len(blocks)
    timed(lambda: io.store(rec_offs, blocks, saved))
    store_ms = float(np.median([timed(lambda: io.store(rec_offs, blocks, saved)) for _ in range(n_host)]))
    load_ms = float(np.median([timed(lambda: io.load(rec_offs, blocks)) for _ in range(n_host)]))
    inv = (1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))).to(dev)
    rot = ([1024 * m for m in range(len(blocks))], [1024] * len(blocks), inv, D, True)
    timed(lambda: io.load(rec_offs, blocks, rerotate=rot))
    fused_ms = float(np.median([timed(lambda: io.load(rec_offs, blocks, rerotate=rot)) for _ in range(n_host)]))

    def kernel_ms(fn):
        """Average duration of the library's kernels launched by fn (dispatch events)."""
        torch.cuda.synchronize()
        cache_ops.timing_enable(True)
        cache_ops.timing_read()
        fn()
        torch.cuda.synchronize()
        ms, n = cache_ops.timing_read()
        cache_ops.timing_enable(False)
        return ms / max(n, 1), n

    k_plain, n_plain = kernel_ms(lambda: io.load(rec_offs, blocks))
    k_fused, n_fused = kernel_ms(lambda: io.load(rec_offs, blocks, rerotate=rot))
    # the same fused calls with no host DMA running beside them: one staging
    # half (4 records) re-scattered from device memory, as many times
    from daric_amd.kv_io import build_copy_plan
    flat, _, ioff, jn, jsz = build_copy_plan(names, [0] * L, bpb, [0] * 4, blocks[:4])
    stg = np.cumsum([0] + jsz[:-1]).astype(np.int64).tolist()
    idx4 = torch.from_numpy(flat).to(dev)
    dl4 = [1024 * m for m in range(1, 5) for _ in range(L)]

    def quiet():
        for _ in range(n_fused):
            io.read_copier.scatter_pages_rerotate(jn, stg, jsz, idx4, ioff, dl4, [1024] * len(jn), inv, D,
                                                  True, stream.cuda_stream)

    k_quiet, _ = kernel_ms(quiet)
    del io, host_rec
    out = dict(workload="BASELINE config 4: KV offload/load of 65536 tokens (4096 random pages), "
                        "Llama-3-8B KV shape bf16",
               tokens=T,
               gather=dict(ms=gather["step_ms"], kernel_ms=gather["kern_ms"],
                           GBps=_gbps(dev_bytes, gather["kern_ms"]),
                           frac=_gbps(dev_bytes, gather["kern_ms"]) / PEAK_HBM_GBPS),
               scatter=dict(ms=scatter["step_ms"], kernel_ms=scatter["kern_ms"],
                            GBps=_gbps(dev_bytes, scatter["kern_ms"]),
                            frac=_gbps(dev_bytes, scatter["kern_ms"]) / PEAK_HBM_GBPS),
               device_algorithmic_bytes=dev_bytes,
               d2h=dict(ms=d2h_ms, GBps=_gbps(link_bytes, d2h_ms), runs_ms=[round(x, 3) for x in d2h_runs]),
               h2d=dict(ms=h2d_ms, GBps=_gbps(link_bytes, h2d_ms), runs_ms=[round(x, 3) for x in h2d_runs]),
               host_link_bytes=link_bytes,
               store_pipeline=dict(ms=store_ms, GBps=_gbps(link_bytes, store_ms),
                                   tokens_per_s=T / (store_ms / 1e3)),
               load_pipeline=dict(ms=load_ms, GBps=_gbps(link_bytes, load_ms),
                                  tokens_per_s=T / (load_ms / 1e3),
                                  scatter_kernel_ms=k_plain, scatter_launches=n_plain),
               load_pipeline_fused=dict(ms=fused_ms, GBps=_gbps(link_bytes, fused_ms),
                                        tokens_per_s=T / (fused_ms / 1e3),
                                        fused_kernel_ms=k_fused, fused_launches=n_fused,
                                        fused_kernel_ms_without_dma=k_quiet,
                                        note="KVIOContext.load(rerotate=...): each batch of 4 records "
                                             "(128 jobs) scattered and re-rotated by 1024 m positions in "
                                             "one scatter_pages_rerotate while the next batch's H2D runs; "
                                             "fused_kernel_ms_without_dma: the same 128-job call alone"),
               note="host link: pinned torch memory, one hipMemcpyAsync per layer record on a side "
                    "stream; pipelines: KVIOContext store/load of 64 records of 1024 tokens through "
                    "two 512 MiB staging halves (wall clock, host-synchronised)")
    del w, cache, host
    torch.cuda.empty_cache()
    return out


def config5_inputs(dev, seed=0):
    """BASELINE config 5's inputs: fp8 KV cache at Llama-3-70B per-layer KV
    shape, 80 layers x [2, 8193, 16, 8, 128] e4m3 (zeroed) with per-(layer,
    head) fp32 K and V scales (amax / 448); 16 chunks x 2048 tokens staged in
    the store's record layout as e4m3 codes of N(0,1) values at those scales;
    the fused call's jobs (chunk c moves by 2048 c). Selection inputs: k = 205
    of 2048 per chunk, recomputed K and V rows in bf16."""
    c = CFG5
    L, H, D, PS, NB = c["layers"], c["kv_heads"], c["head_dim"], c["block_size"], c["num_blocks"]
    C, CT = c["chunks"], c["chunk_tokens"]
    T = C * CT
    g = torch.Generator().manual_seed(seed)
    ids = (torch.randperm(NB - 1, generator=g)[: T // PS] + 1).to(torch.int32)
    names = layer_names(L)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    cache = [torch.zeros(2, NB, PS, H, D, dtype=torch.uint8, device=dev) for _ in range(L)]
    k_scales = (torch.rand(L, H, generator=gd, device=dev) * 2.0 + 3.0) / 448.0   # amax ~ 3..5 sigma
    span = PS * H * D
    job_bytes = 2 * (CT // PS) * span
    staging = torch.empty(C * L * job_bytes, dtype=torch.uint8, device=dev)
    piece = 1 << 28
    for o in range(0, staging.numel(), piece):
        n = min(piece, staging.numel() - o)
        vals = torch.randn(n, generator=gd, device=dev) / 0.01      # codes of N(0,1) / (~4/448)
        staging[o:o + n] = vals.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    del vals
    jobs = dict(names=[], offsets=[], sizes=[], flat=[], ioff=[0], deltas=[], ntok=[])
    off = 0
    for ci in range(C):
        bids = ids[ci * (CT // PS):(ci + 1) * (CT // PS)].tolist()
        for n in names:
            jobs["names"].append(n)
            jobs["offsets"].append(off)
            jobs["sizes"].append(job_bytes)
            jobs["flat"].extend(bids)
            jobs["ioff"].append(len(jobs["flat"]))
            jobs["deltas"].append(ci * CT)
            jobs["ntok"].append(CT)
            off += job_bytes
    idx = torch.tensor(jobs["flat"], dtype=torch.int32, device=dev)
    inv = (1.0 / (c["rope_theta"] ** (torch.arange(0, D, 2, dtype=torch.float32) / D))).to(dev)
    k = max(1, int(round(c["k_frac"] * CT)))
    v_scales = (torch.rand(L, H, generator=gd, device=dev) * 2.0 + 3.0) / 448.0
    k_new = torch.randn(L, T, H, D, generator=gd, device=dev, dtype=torch.bfloat16)
    v_new = torch.randn(L, T, H, D, generator=gd, device=dev, dtype=torch.bfloat16)
    chunks = [(ci * (CT // PS), ci * CT, CT, k) for ci in range(C)]
    return dict(L=L, H=H, D=D, PS=PS, NB=NB, C=C, CT=CT, T=T, ids=ids, names=names, cache=cache,
                k_scales=k_scales, v_scales=v_scales, staging=staging, jobs=jobs, idx=idx, inv=inv,
                job_bytes=job_bytes, k=k, bt=ids.to(dev), chunks=chunks, k_new=k_new, v_new=v_new)


def run_config5(steps, warmup, seed=0):
    """fp8 KV cache at Llama-3-70B per-layer KV shape (
    config5_inputs): one step = scatter_pages_rerotate (dequant -> rotate to
    offsets 0..32767 -> saturating RTNE requant -> scatter, 1280 jobs). The
    selection at 10% per chunk (k = 205) on the fp8 cache -- deviation, top-k
    and the quantising merge of the selected bf16 K/V rows -- is timed as a
    second figure."""
    from daric_amd import cache_ops
    dev = torch.device("cuda:0")
    w = config5_inputs(dev, seed)
    L, H, D, C, T, k = w["L"], w["H"], w["D"], w["C"], w["T"], w["k"]
    cache, k_scales, v_scales, j = w["cache"], w["k_scales"], w["v_scales"], w["jobs"]
    cp = cache_ops.CacheCopier()
    for l, (n, t) in enumerate(zip(w["names"], cache)):
        cp.register_layer(n, t, False)
        cp.register_k_scale(n, k_scales[l].contiguous())
    cp.register_store(w["staging"])
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    fused = time_steps(lambda: cp.scatter_pages_rerotate(j["names"], j["offsets"], j["sizes"], w["idx"],
                                                         j["ioff"], j["deltas"], j["ntok"], w["inv"], D,
                                                         True, st), steps, warmup, stream)
    fused_bytes = T * L * 2 * (2 * H * D * 1)
    # the same 1280 jobs as a plain scatter_pages (no rotation): this access
    # pattern's copy rate on this box
    pattern = time_steps(lambda: cp.scatter_pages(j["names"], j["offsets"], j["sizes"], w["idx"], j["ioff"], st),
                         steps, 1, stream)
    # the worker's form on the fp8 cache, the reference's own fp8 rotation
    # (adapter.py:370-373, in place on the e4m3 view): rerotate_pages of chunks
    # 1..15 in all 80 layers (chunk 0 does not move); K codes read and written
    CT, PS = w["CT"], w["PS"]
    segs = [(ci * (CT // PS), 0, CT, ci * CT) for ci in range(1, C)]
    inplace = time_steps(lambda: cache_ops.rerotate_pages(cache, False, w["bt"], segs, w["inv"], D, True,
                                                          stream=st), steps, 1, stream)
    inplace_bytes = (C - 1) * CT * L * 2 * H * D * 1
    # selection on the fp8 cache: recomputed K (bf16) vs the dequantised cached
    # K, top-10%, then the selected bf16 K/V rows quantised into the cache
    bt, chunks, k_new, v_new = w["bt"], w["chunks"], w["k_new"], w["v_new"]
    keys = torch.empty(L, T, dtype=torch.float32, device=dev)
    sel = torch.empty(L, C, k, dtype=torch.int32, device=dev)

    def dev_step():
        cache_ops.kv_deviation(cache, False, bt, k_new, chunks, keys=keys, stream=st, k_scales=k_scales)

    def topk_step():
        cache_ops.topk_per_chunk(keys, chunks, kmax=k, out=sel, stream=st)

    def merge_step():
        cache_ops.merge_rows(cache, False, bt, k_new, v_new, chunks, sel, stream=st, k_scales=k_scales,
                             v_scales=v_scales)

    def three_calls():
        dev_step()
        topk_step()
        merge_step()

    def sel_step():
        cache_ops.select_merge(cache, False, bt, k_new, v_new, chunks, kmax=k, keys=keys, sel_idx=sel, stream=st,
                               k_scales=k_scales, v_scales=v_scales)

    def one_pass():
        cache_ops.select_merge(cache, False, bt, k_new, v_new, chunks, kmax=k, keys=keys, sel_idx=sel, stream=st,
                               k_scales=k_scales, v_scales=v_scales, one_pass=True)

    selection = time_steps(sel_step, steps, warmup, stream)
    forms = {"select_merge": [], "three_calls": [], "one_pass": []}
    for _ in range(3):
        for name, f in (("select_merge", sel_step), ("three_calls", three_calls), ("one_pass", one_pass)):
            forms[name].append(time_steps(f, steps, 1, stream)["step_ms"])
    forms = {n: sorted(v)[1] for n, v in forms.items()}
    parts = {n: kernel_ms_per_step(f, steps, stream)
             for n, f in (("deviation", dev_step), ("topk", topk_step), ("merge", merge_step),
                          ("topk_merge_fused", lambda: cache_ops.select_merge(
                              cache, False, bt, k_new, v_new, chunks, kmax=k, keys=keys, sel_idx=sel, stream=st,
                              k_scales=k_scales, v_scales=v_scales, keys_ready=True)))}
    dev_bytes = T * L * H * D * (2 + 1) + T * L * 4
    topk_bytes = T * L * 4 + C * L * k * 4
    merge_bytes = C * k * L * 2 * (H * D * (2 + 1))      # bf16 rows read, e4m3 codes written
    sel_bytes = dev_bytes + topk_bytes + merge_bytes
    out = dict(workload="BASELINE config 5: fp8 e4m3 KV at Llama-3-70B per-layer shape, 80 layers, "
                        "16 chunks x 2048 tokens, dequant->rotate->requant+scatter to offsets 0..32767",
               tokens=T, ms_per_step=fused["step_ms"], tokens_per_s=T / (fused["step_ms"] / 1e3),
               kernel_ms=fused["kern_ms"], algorithmic_bytes=fused_bytes,
               GBps=_gbps(fused_bytes, fused["kern_ms"]),
               frac=_gbps(fused_bytes, fused["kern_ms"]) / PEAK_HBM_GBPS,
               pattern_copy=dict(kernel="copy_pages_kernel<16,scatter> on the same 1280 jobs, no rotation",
                                 kernel_ms=pattern["kern_ms"], GBps=_gbps(fused_bytes, pattern["kern_ms"]),
                                 fused_frac_of_it=pattern["kern_ms"] / fused["kern_ms"]),
               rerotate_inplace=dict(ms_per_step=inplace["step_ms"], kernel_ms=inplace["kern_ms"],
                                     algorithmic_bytes=inplace_bytes,
                                     GBps=_gbps(inplace_bytes, inplace["kern_ms"]),
                                     frac=_gbps(inplace_bytes, inplace["kern_ms"]) / PEAK_HBM_GBPS,
                                     tokens_per_s=(C - 1) * CT / (inplace["step_ms"] / 1e3),
                                     note="rerotate_pages of chunks 1..15 in all 80 layers of the e4m3 "
                                          "cache (in place, the Adapter's call): K codes read and written"),
               selection=dict(k=k, ms_per_step=selection["step_ms"], algorithmic_bytes=sel_bytes,
                              GBps=_gbps(sel_bytes, selection["step_ms"]),
                              step_forms=dict(ms=forms, note="as for config 3: select_merge (the step above), "
                                                             "three_calls, one_pass; alternating, median of 3"),
                              kernels={"deviation": dict(ms=parts["deviation"], bytes=dev_bytes,
                                                         GBps=_gbps(dev_bytes, parts["deviation"])),
                                       "topk": dict(ms=parts["topk"], bytes=topk_bytes),
                                       "topk_merge": dict(ms=parts["topk_merge_fused"],
                                                          bytes=topk_bytes + merge_bytes,
                                                          GBps=_gbps(topk_bytes + merge_bytes,
                                                                     parts["topk_merge_fused"]),
                                                          note="select_merge with the keys given: at 205 "
                                                               "rows per chunk it runs the top-k and "
                                                               "merge kernels, not the fused one"),
                                       "merge_quantising": dict(ms=parts["merge"], bytes=merge_bytes,
                                                                GBps=_gbps(merge_bytes, parts["merge"]))}))
    del w, cache, cp, k_new, v_new, keys, sel
    torch.cuda.empty_cache()
    return out


CFG1 = dict(layers=16, kv_heads=8, head_dim=64, block_size=16, num_blocks=1024, chunks=4, chunk_tokens=512,
            rope_theta=500000.0, dtype="fp16")


def host_cpu() -> dict:
    """The host's CPU: model name, the cores this process may run on, and the
    threads the baseline uses (at most 16, one GPU's share of an MI355X box)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(cpu_model=model, cores_available=avail, threads=max(1, min(16, avail)),
                thread_cap="16: one GPU's share of the box's cores")


def cpu_threads() -> int:
    return host_cpu()["threads"]


def _time_cpu(run, budget_s, min_runs=5, max_runs=20):
    """One warm-up, then at least min_runs timed runs (more while the budget
    lasts, at most max_runs); returns (median seconds, runs)."""
    run()
    times = []
    while len(times) < max_runs and (len(times) < min_runs or sum(times) < budget_s):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def run_cpu_baseline(cfg, budget_s=12.0):
    """The CPU oracle's fused scatter + re-rotate, timed on this host: the C
    restatement (oracle/c/oracle_copy.c) on host_cpu()["threads"] OpenMP
    threads, or the numpy oracle on one thread when the C library has not been
    built. Two workloads: the headline's (config 2: all 32 layers, 256 jobs,
    with a reduced 1024-block pool -- the same bytes move) and BASELINE
    config 1 at its real size (16 layers of [2, 1024, 16, 8, 64] fp16, 4
    chunks of 512 tokens moved to 0, 512, 1024, 1536). Median of at least 5
    runs after one warm-up each."""
    from oracle import native
    from oracle.copy import OracleCopier
    cpu = host_cpu()
    threads = cpu["threads"]
    if native.available():
        make = lambda: native.NativeOracleCopier(threads)
        what = f"the C restatement oracle/c/oracle_copy.c on {threads} OpenMP threads"
    else:
        torch.set_num_threads(1)
        threads = 1
        make = OracleCopier
        what = "the numpy oracle oracle/copy.py on one thread"

    def timed(c, pool, budget):
        oc = make()
        w = build_workload(c, torch.device("cpu"), num_blocks=pool)
        j = w["jobs"]
        inv = w["inv_freq"].numpy()
        for name, t in zip(w["names"], w["cache"]):
            oc.register_layer(name, t, False)
        oc.register_store(w["staging"])
        idx = torch.tensor(j["flat"], dtype=torch.int32)
        med, n = _time_cpu(lambda: oc.scatter_pages_rerotate(j["names"], j["offsets"], j["sizes"], idx,
                                                             j["ioff"], j["deltas"], j["ntok"], inv,
                                                             c["head_dim"], True), budget)
        return w["T"], med, n

    T, med, n = timed(cfg, 1024, budget_s)
    T1, med1, n1 = timed(CFG1, CFG1["num_blocks"], budget_s / 4)
    return dict(value=T / med, unit="reused KV tokens/s", cores=threads, kind="port",
                sample=f"whole config-2 workload (32 layers x 8 chunks x 1024 tokens, 1024-block pool) "
                       f"through scatter_pages_rerotate of {what}, median of {n} runs ({med:.3f} s each) "
                       f"after one warm-up",
                GBps=algorithmic_bytes(cfg) / med / 1e9,
                cores_available=cpu["cores_available"], thread_cap=cpu["thread_cap"],
                cpu_model=cpu["cpu_model"], torch_version=torch.__version__,
                config1=dict(value=T1 / med1, unit="reused KV tokens/s",
                             GBps=algorithmic_bytes(CFG1, e=2) / med1 / 1e9, seconds=med1, runs=n1,
                             workload="BASELINE config 1 at its real size: 16 layers x [2, 1024, 16, 8, 64] "
                                      "fp16, 4 x 512 tokens scattered and moved to 0/512/1024/1536"))


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
    ap.add_argument("--extra", default="2h,3,4,5",
                    help="other BASELINE configs to measure after the headline (comma list of 2h, 3, 4, "
                         "5, or 'none'; 'place' adds the cache-placement check, 258 GiB; 'layout' the "
                         "layer-stride check, 129 GiB)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (torch copy_) `steps` times, the "
                         "known-size reference that scales rocprofv3 FETCH_SIZE/WRITE_SIZE")
    a = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the KV-reuse hot path is per-GPU work with no "
              "cross-GPU exchange; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    cfg = CFG2
    r = run_gpu(cfg, a.steps, a.warmup)
    if a.calib_copy:
        run_copy_calibration(a.steps)
    nbytes = algorithmic_bytes(cfg)
    tok_s = r["T"] / (r["step_ms"] / 1e3)
    achieved = nbytes / (r["kern_ms"] / 1e3) / 1e9
    g_achieved = nbytes / (r["g_kern_ms"] / 1e3) / 1e9
    torch.cuda.empty_cache()
    extra = {}
    runners = {"2h": run_config2_hnd, "3": run_config3, "4": run_config4, "5": run_config5,
               "place": run_placement, "layout": run_layout}
    for cname in [x.strip() for x in a.extra.split(",") if x.strip() and x.strip() != "none"]:
        key = {"place": "placement", "layout": "layer_layout"}.get(cname, f"config{cname}")
        # a secondary configuration that raises (out of memory on a shared
        # box, say) is recorded as such; the headline line is still printed
        try:
            extra[key] = runners[cname](max(3, a.steps // 2), max(1, a.warmup))
        except (RuntimeError, ValueError, MemoryError) as e:
            extra[key] = {"error": f"{type(e).__name__}: {e}"}
            print(f"bench: {key} failed: {e}", file=sys.stderr, flush=True)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
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
                     "algorithmic_bytes": nbytes,
                     "pattern_copy": {"kernel": "copy_pages_kernel<16,scatter> on the same jobs, no rotation",
                                      "kernel_ms": r["p_kern_ms"], "GBps": _gbps(nbytes, r["p_kern_ms"]),
                                      "fused_frac_of_it": achieved / _gbps(nbytes, r["p_kern_ms"])}},
        "gather": {"ms_per_step": r["g_step_ms"], "kernel_ms": r["g_kern_ms"],
                   "GBps": g_achieved, "frac": g_achieved / PEAK_HBM_GBPS,
                   "tokens_per_s": r["T"] / (r["g_step_ms"] / 1e3)},
        "rerotate_inplace": {"ms_per_step": r["r_step_ms"], "kernel_ms": r["r_kern_ms"],
                             "algorithmic_bytes": r["r_bytes"],
                             "GBps": _gbps(r["r_bytes"], r["r_kern_ms"]),
                             "frac": _gbps(r["r_bytes"], r["r_kern_ms"]) / PEAK_HBM_GBPS,
                             "tokens_per_s": r["r_tokens"] / (r["r_step_ms"] / 1e3),
                             "sequential_pages": {"kernel_ms": r["r_seq_kern_ms"],
                                                  "GBps": _gbps(r["r_bytes"], r["r_seq_kern_ms"]),
                                                  "note": "the same call with the pages on blocks 1..512"},
                             "note": "rerotate_pages of chunks 1..7 (chunk 0 does not move) in all "
                                     "layers: K rotated elements read and written"},
        "extra": extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
