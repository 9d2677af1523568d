"""Repeat runs give bit-identical output. No kernel on the path uses atomics
whose order reaches the result or a reduction whose order depends on
scheduling, so every kernel family is run twice from the same inputs: once with
plain launches on the current stream, once with per-launch timing events
(the dispatch-event launch path) on a side stream while a third stream copies
unrelated memory. The rotating kernels are held only to a tolerance against
the float64 oracle elsewhere; here they must repeat themselves exactly."""
import numpy as np
import pytest
import torch

from daric_amd import cache_ops

pytestmark = pytest.mark.gpu

L, NB, PS, H, D = 4, 512, 16, 8, 128
C, CT = 4, 256


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def _twice(dev, reset, run, snapshot):
    """snapshot() after run() on the current stream, then after run() on a
    side stream with kernel timing on and a concurrent copy elsewhere."""
    reset()
    run(torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    first = snapshot()
    reset()
    side, busy = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    a = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    side.wait_stream(torch.cuda.current_stream(dev))
    busy.wait_stream(torch.cuda.current_stream(dev))
    cache_ops.timing_enable(True)
    try:
        with torch.cuda.stream(busy):
            for _ in range(4):
                b.copy_(a)
        run(side.cuda_stream)
        torch.cuda.synchronize()
    finally:
        cache_ops.timing_enable(False)
        cache_ops.timing_read()
    second = snapshot()
    assert len(first) == len(second)
    for x, y in zip(first, second):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
    return first


def _workload(dev, dtype):
    g = torch.Generator().manual_seed(11)
    ids = (torch.randperm(NB - 1, generator=g)[: C * CT // PS] + 1).to(torch.int32)
    es = torch.empty(0, dtype=dtype).element_size()
    base = [torch.randint(0, 120, (2, NB, PS, H, D * es), generator=g, dtype=torch.uint8).view(dtype)
            if dtype == torch.uint8 else torch.randn(2, NB, PS, H, D, generator=g).to(dtype)
            for _ in range(L)]
    span = PS * H * D * es
    job = 2 * (CT // PS) * span
    staging = torch.randint(0, 120, (C * L * job,), generator=g, dtype=torch.uint8)
    if dtype != torch.uint8:
        staging = torch.randn(C * L * job // es, generator=g).to(dtype).view(torch.uint8)
    names, offs, sizes, flat, ioff, deltas, ntok = [], [], [], [], [0], [], []
    for c in range(C):
        bids = ids[c * (CT // PS):(c + 1) * (CT // PS)].tolist()
        for l in range(L):
            names.append(f"layer.{l}")
            offs.append(len(offs) * job)
            sizes.append(job)
            flat.extend(bids)
            ioff.append(len(flat))
            deltas.append(c * CT + 3)
            ntok.append(CT - 5)
    inv = (1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))).to(dev)
    return dict(ids=ids, base=[t.to(dev) for t in base], staging=staging.to(dev), names=names,
                offs=offs, sizes=sizes, idx=torch.tensor(flat, dtype=torch.int32, device=dev), ioff=ioff,
                deltas=deltas, ntok=ntok, inv=inv)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.uint8])
def test_fused_and_inplace_rotation_repeat_exactly(dev, dtype):
    w = _workload(dev, dtype)
    layers = [t.clone() for t in w["base"]]
    cp = cache_ops.CacheCopier()
    for l, t in enumerate(layers):
        cp.register_layer(f"layer.{l}", t, False)
        if dtype == torch.uint8:
            cp.register_k_scale(f"layer.{l}", (0.5 + 0.1 * torch.arange(H, dtype=torch.float32)).to(dev))
    cp.register_store(w["staging"])

    def reset():
        for t, b in zip(layers, w["base"]):
            t.copy_(b)

    def fused(st):
        cp.scatter_pages_rerotate(w["names"], w["offs"], w["sizes"], w["idx"], w["ioff"], w["deltas"],
                                  w["ntok"], w["inv"], D, True, st)

    got = _twice(dev, reset, fused, lambda: [t.clone() for t in layers])
    assert not torch.equal(got[0].view(torch.uint8), w["base"][0].view(torch.uint8))

    bt = w["ids"].to(dev)
    segs = [(c * (CT // PS), 2, CT - 7, 1000 * c - 4096) for c in range(C)]

    def inplace(st):
        cache_ops.rerotate_pages(layers, False, bt, segs, w["inv"], D, True, stream=st)

    got = _twice(dev, reset, inplace, lambda: [t.clone() for t in layers])
    assert not torch.equal(got[-1].view(torch.uint8), w["base"][-1].view(torch.uint8))


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.uint8])
def test_selection_repeats_exactly(dev, cache_dtype):
    w = _workload(dev, cache_dtype)
    layers = [t.clone() for t in w["base"]]
    bt = w["ids"].to(dev)
    T = C * CT
    g = torch.Generator(device=dev).manual_seed(5)
    k_new = torch.randn(L, T, H, D, generator=g, device=dev).to(torch.bfloat16)
    v_new = torch.randn(L, T, H, D, generator=g, device=dev).to(torch.bfloat16)
    chunks = [(c * (CT // PS), c * CT, CT, 38) for c in range(C)]
    fp8 = cache_dtype == torch.uint8
    ks = (0.02 + 0.01 * torch.rand(L, H, generator=g, device=dev)) if fp8 else None
    vs = (0.02 + 0.01 * torch.rand(L, H, generator=g, device=dev)) if fp8 else None
    if not fp8:
        k_new, v_new = k_new.to(cache_dtype), v_new.to(cache_dtype)
    out = {}

    def reset():
        for t, b in zip(layers, w["base"]):
            t.copy_(b)

    def select(st):
        keys = torch.empty(L, T, dtype=torch.float32, device=dev)
        sel = torch.empty(L, C, 38, dtype=torch.int32, device=dev)
        cache_ops.kv_deviation(layers, False, bt, k_new, chunks, keys=keys, stream=st, k_scales=ks)
        cache_ops.topk_per_chunk(keys, chunks, kmax=38, out=sel, stream=st)
        cache_ops.merge_rows(layers, False, bt, k_new, v_new, chunks, sel, stream=st,
                             k_scales=ks, v_scales=vs)
        out["keys"], out["sel"] = keys, sel

    got = _twice(dev, reset, select,
                 lambda: [out["keys"].clone(), out["sel"].clone()] + [t.clone() for t in layers])
    assert not torch.equal(got[2].view(torch.uint8), w["base"][0].view(torch.uint8))
    assert int((out["sel"] >= 0).sum()) == L * C * 38
    assert np.isfinite(out["keys"].cpu().numpy()).all()
