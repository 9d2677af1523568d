"""The allocation-free fused scatter + re-rotation
(daric_copier_scatter_pages_rerotate_noalloc), called through the C ABI,
against the existing entry point (daric_copier_scatter_pages_rerotate) on
the same inputs: bit-exact, on calls in a row whose job lists shrink (the
static scratch array keeps the previous call's descriptors), with two launch
groups staged in one call, and with a job list small enough to travel in the
kernel arguments. Device memory stays unallocated across the calls, and the
library's own counters show that no call touches the descriptor ring (whose
slots are pinned host and device allocations), the first call included.
Calls on two streams in a row, with different job lists, are ordered on the
shared scratch array by the library and stay bit-exact."""
import ctypes

import numpy as np
import pytest
import torch

from daric_amd import _lib, cache_ops
from tests.gpu_util import same_bytes

pytestmark = pytest.mark.gpu

NB, PS, H = 96, 16, 8


def make_layers(dev, dims, gen):
    return [torch.randn(2, NB, PS, H, d, generator=gen).to(torch.bfloat16).to(dev) for d in dims]


def plan(n_layers, chunks, span_of, rng):
    """Jobs of gpu_kv_io._build_copy_plan order: for each chunk, for each layer."""
    names, offsets, sizes, flat, ioff, deltas, ntok = [], [], [], [], [0], [], []
    off = 0
    for pages in chunks:
        d = int(rng.integers(-3000, 3000))
        n = int(rng.integers(1, len(pages) * PS + 1))
        for l in range(n_layers):
            names.append(f"model.layers.{l}.self_attn.attn")
            offsets.append(off)
            sz = 2 * len(pages) * span_of(l)
            sizes.append(sz)
            flat.extend(pages)
            ioff.append(len(flat))
            deltas.append(d)
            ntok.append(n)
            off += sz
    return names, offsets, sizes, flat, ioff, deltas, ntok, off


def call(lib, fn, copier, names, offsets, sizes, idx, ioff, deltas, ntok, rope, stream):
    off, sz, io = _lib.I64(offsets), _lib.I64(sizes), _lib.I64(ioff)
    dl, nt = _lib.I64(deltas), _lib.I64(ntok)
    ix = _lib.desc(idx)
    return fn(copier._h, _lib.str_array(names), len(names), off.ptr, off.n, sz.ptr, sz.n,
              ctypes.byref(ix), io.ptr, io.n, dl.ptr, nt.ptr, ctypes.byref(rope), ctypes.c_uint64(stream))


def counters(lib):
    up, al, wt = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    assert lib.daric_debug_counters(ctypes.byref(up), ctypes.byref(al), ctypes.byref(wt)) == 0
    return up.value, al.value, wt.value


def test_noalloc_matches_fused_entry_point(dev):
    lib = _lib.load()
    gen = torch.Generator().manual_seed(7)
    rng = np.random.default_rng(7)
    dims = [128] * 4 + [64] * 4                       # two row geometries: two launch groups
    base = make_layers(dev, dims, gen)
    span_of = lambda l: PS * H * dims[l] * 2       # bytes of one page's K (or V) half
    inv = (1.0 / (500000.0 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))).to(dev)
    rope = _lib.DaricRope()
    rope.inv_freq = inv.data_ptr()
    rope.rotary_dim = 64
    rope.is_neox = 1

    copiers, outs = [], []
    for _ in range(2):
        c = cache_ops.CacheCopier()
        layers = [t.clone() for t in base]
        for l, t in enumerate(layers):
            c.register_layer(f"model.layers.{l}.self_attn.attn", t, False)
        copiers.append(c)
        outs.append(layers)

    perm = (rng.permutation(NB - 1) + 1).tolist()
    # Per launch group (4 layers each): 12 chunks x 4 = 48 jobs (3840
    # descriptor bytes, over the 2816-byte inline limit: staged), then
    # 9 x 4 = 36 jobs (2880 bytes, staged, smaller), then 2 x 4 = 8 jobs
    # (640 bytes, inline). Chunks never share a page.
    calls = [[perm[3 * i: 3 * i + 3] for i in range(12)],
             [perm[40 + 2 * i: 42 + 2 * i] for i in range(9)],
             [perm[60:63], [perm[63]]]]
    side = torch.cuda.Stream()
    for k, chunks in enumerate(calls):
        names, offsets, sizes, flat, ioff, deltas, ntok, total = plan(len(dims), chunks, span_of, rng)
        staging = torch.randint(-128, 127, (total,), dtype=torch.int8, generator=gen).view(torch.uint8).to(dev)
        idx = torch.tensor(flat, dtype=torch.int32, device=dev)
        for c in copiers:
            c.register_store(staging)
        torch.cuda.synchronize()
        st = call(lib, lib.daric_copier_scatter_pages_rerotate, copiers[0], names, offsets, sizes, idx,
                  ioff, deltas, ntok, rope, torch.cuda.current_stream().cuda_stream)
        assert st == 0, lib.daric_last_error()
        torch.cuda.synchronize()
        # The first call also sets up the side stream in the HIP runtime (its
        # first launch there took 2 MiB of device memory on MI355X); the later
        # calls must take none: the ring's device half alone would be 16 MiB.
        free_before = torch.cuda.mem_get_info()[0]
        ring_before = counters(lib)[:2]
        st = call(lib, lib.daric_copier_scatter_pages_rerotate_noalloc, copiers[1], names, offsets, sizes,
                  idx, ioff, deltas, ntok, rope, side.cuda_stream)
        assert st == 0, lib.daric_last_error()
        assert counters(lib)[:2] == ring_before, f"call {k} used the descriptor ring"
        torch.cuda.synchronize()
        if k > 0:
            assert torch.cuda.mem_get_info()[0] == free_before, f"call {k} took device memory"
        for l in range(len(dims)):
            assert same_bytes(outs[1][l], outs[0][l]), f"call {k} layer {l}"
    # both paths really rotated something
    assert not same_bytes(outs[0][0], base[0])


def test_noalloc_calls_on_two_streams_are_ordered(dev):
    """Two calls in a row on different streams, each staging its own job list
    in the same region of the scratch array, then a third back on the first
    stream: the second call's stash waits for the first call's kernel (and
    the third for the second's), so every call rotates with its own
    descriptors. Each result is bit-exact against the regular entry point."""
    lib = _lib.load()
    gen = torch.Generator().manual_seed(11)
    rng = np.random.default_rng(11)
    dims = [128] * 8
    span_of = lambda l: PS * H * dims[l] * 2
    inv = (1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).to(dev)
    rope = _lib.DaricRope()
    rope.inv_freq = inv.data_ptr()
    rope.rotary_dim = 128
    rope.is_neox = 1
    perm = (rng.permutation(NB - 1) + 1).tolist()
    # 10 x 8 = 80 jobs (6400 descriptor bytes, staged), 6 x 8 = 48 (staged), 8 x 8 = 64 (staged)
    job_lists = [[perm[4 * i: 4 * i + 4] for i in range(10)],
                 [perm[40 + 3 * i: 43 + 3 * i] for i in range(6)],
                 [perm[60 + 2 * i: 62 + 2 * i] for i in range(8)]]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    which = [0, 1, 0]
    cases = []
    for chunks in job_lists:
        names, offsets, sizes, flat, ioff, deltas, ntok, total = plan(len(dims), chunks, span_of, rng)
        staging = torch.randint(-128, 127, (total,), dtype=torch.int8, generator=gen).view(torch.uint8).to(dev)
        idx = torch.tensor(flat, dtype=torch.int32, device=dev)
        base = make_layers(dev, dims, gen)
        pair = []
        for _ in range(2):
            c = cache_ops.CacheCopier()
            layers = [t.clone() for t in base]
            for l, t in enumerate(layers):
                c.register_layer(f"model.layers.{l}.self_attn.attn", t, False)
            c.register_store(staging)
            pair.append((c, layers))
        cases.append((pair, (names, offsets, sizes, idx, ioff, deltas, ntok), base))
    torch.cuda.synchronize()
    for pair, args, _ in cases:
        assert call(lib, lib.daric_copier_scatter_pages_rerotate, pair[0][0], *args, rope,
                    torch.cuda.current_stream().cuda_stream) == 0, lib.daric_last_error()
    torch.cuda.synchronize()
    waits = []
    for (pair, args, _), s in zip(cases, which):
        assert call(lib, lib.daric_copier_scatter_pages_rerotate_noalloc, pair[1][0], *args, rope,
                    streams[s].cuda_stream) == 0, lib.daric_last_error()
        waits.append(counters(lib)[2])
    torch.cuda.synchronize()
    # the second and third calls change stream: each waits for the call before
    # (the first waits too if an earlier test's last call used another stream)
    assert [b - a for a, b in zip(waits, waits[1:])] == [1, 1], waits
    for k, (pair, _, base) in enumerate(cases):
        for l in range(len(dims)):
            assert same_bytes(pair[1][1][l], pair[0][1][l]), f"call {k} layer {l}"
        assert not same_bytes(pair[0][1][0], base[0])


def test_noalloc_call_captured_in_a_graph_replays_exactly(dev):
    """A fused call whose 48 jobs (3840 descriptor bytes) are too many for the
    kernel arguments, which the regular entry point would stage in its
    descriptor ring and so refuse under capture, recorded in a HIP graph
    through the allocation-free entry point. Each replay restages its own
    descriptors: between replays an eager call with another job list
    overwrites the scratch array, the target layers are cleared, and every
    replay still writes what the regular entry point writes eagerly. Neither
    the capture nor the replays touch the descriptor ring."""
    lib = _lib.load()
    gen = torch.Generator().manual_seed(23)
    rng = np.random.default_rng(23)
    dims = [128] * 4
    span_of = lambda l: PS * H * dims[l] * 2
    inv = (1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).to(dev)
    rope = _lib.DaricRope()
    rope.inv_freq = inv.data_ptr()
    rope.rotary_dim = 128
    rope.is_neox = 1
    perm = (rng.permutation(NB - 1) + 1).tolist()
    # the captured call: 12 chunks x 4 layers = 48 jobs; the eager call between
    # replays: 10 x 4 = 40 jobs on other pages of other layers
    job_lists = [[perm[3 * i: 3 * i + 3] for i in range(12)],
                 [perm[40 + 2 * i: 42 + 2 * i] for i in range(10)]]
    cases = []
    for chunks in job_lists:
        names, offsets, sizes, flat, ioff, deltas, ntok, total = plan(len(dims), chunks, span_of, rng)
        staging = torch.randint(-128, 127, (total,), dtype=torch.int8, generator=gen).view(torch.uint8).to(dev)
        idx = torch.tensor(flat, dtype=torch.int32, device=dev)
        base = make_layers(dev, dims, gen)
        pair = []
        for _ in range(2):
            c = cache_ops.CacheCopier()
            layers = [t.clone() for t in base]
            for l, t in enumerate(layers):
                c.register_layer(f"model.layers.{l}.self_attn.attn", t, False)
            c.register_store(staging)
            pair.append((c, layers))
        cases.append((pair, (names, offsets, sizes, idx, ioff, deltas, ntok), staging))
    for t in cases[0][0][0][1]:     # the captured call's replays start from cleared layers
        t.zero_()
    torch.cuda.synchronize()
    # what each call writes, by the regular entry point, eagerly
    for pair, args, _ in cases:
        assert call(lib, lib.daric_copier_scatter_pages_rerotate, pair[0][0], *args, rope,
                    torch.cuda.current_stream().cuda_stream) == 0, lib.daric_last_error()
    torch.cuda.synchronize()
    (cap_pair, cap_args, _), (other_pair, other_args, _) = cases
    cap_copier, cap_layers = cap_pair[1]
    # warm-up outside the capture (sets up the scratch array's per-GPU state)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    assert call(lib, lib.daric_copier_scatter_pages_rerotate_noalloc, cap_copier, *cap_args, rope,
                side.cuda_stream) == 0, lib.daric_last_error()
    torch.cuda.synchronize()
    for t in cap_layers:
        t.zero_()
    torch.cuda.synchronize()
    ring_before = counters(lib)[:2]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert call(lib, lib.daric_copier_scatter_pages_rerotate_noalloc, cap_copier, *cap_args, rope,
                    torch.cuda.current_stream().cuda_stream) == 0, lib.daric_last_error()
    torch.cuda.synchronize()
    assert all(int(t.count_nonzero()) == 0 for t in cap_layers), "capturing ran the call"
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for l in range(len(dims)):
            assert same_bytes(cap_layers[l], cap_pair[0][1][l]), f"replay {rep} layer {l}"
        # another job list through the same scratch array, eagerly
        other_copier, other_layers = other_pair[1]
        assert call(lib, lib.daric_copier_scatter_pages_rerotate_noalloc, other_copier, *other_args, rope,
                    side.cuda_stream) == 0, lib.daric_last_error()
        torch.cuda.synchronize()
        for l in range(len(dims)):
            assert same_bytes(other_layers[l], other_pair[0][1][l]), f"eager call after replay {rep} layer {l}"
        for t in cap_layers:
            t.zero_()
        _ = float(torch.randn(4096, device=dev).abs().sum())   # eager work between replays
        torch.cuda.synchronize()
    assert counters(lib)[:2] == ring_before, "the captured call or its replays used the descriptor ring"
