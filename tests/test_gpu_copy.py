"""GPU parity of CacheCopier.gather_pages / scatter_pages and batched memcpy
against the CPU oracle: bit-exact on every layout, dtype and alignment path
(16-, 4- and 1-byte accesses), with the null block and out-of-range ids."""
import numpy as np
import pytest
import torch

from daric_amd import cache_ops
from oracle.copy import OracleCopier
from tests.gpu_util import make_layer, same_bytes, to_dev

pytestmark = pytest.mark.gpu


def job_plan(n_layers, chunks, per_page_span, prefix, base=0, pad=0):
    """Store layout of gpu_kv_io._build_copy_plan: for each chunk, for each layer."""
    names, offsets, sizes, flat, ioff = [], [], [], [], [0]
    off = base
    for bids in chunks:
        for l in range(n_layers):
            names.append(f"model.layers.{l}.self_attn.attn")
            offsets.append(off)
            sz = prefix * len(bids) * per_page_span
            sizes.append(sz)
            flat.extend(bids)
            ioff.append(len(flat))
            off += sz + pad
    return names, offsets, sizes, flat, ioff, off


@pytest.mark.parametrize("layout,dtype", [
    ("nhd", torch.bfloat16), ("hnd", torch.float16), ("pf", torch.bfloat16),
    ("packed", torch.float16), ("mla", torch.bfloat16), ("nhd", torch.uint8),
])
@pytest.mark.parametrize("pad", [0, 4, 1])
def test_gather_scatter_parity(dev, layout, dtype, pad):
    g = torch.Generator().manual_seed(11)
    nb, ps, h, d, L = 40, 16, 4, 64, 3
    layers = [make_layer(layout, nb, ps, h, d, dtype, g, kind="bytes") for _ in range(L)]
    pf = layers[0][1]
    shp = layers[0][0]
    from oracle.layout import page_copy_shape
    s = page_copy_shape(tuple(shp.shape), tuple(shp.stride()), shp.element_size(), pf)
    perm = np.random.default_rng(3).permutation(np.arange(1, nb)).tolist()
    # distinct pages per layer (duplicates would race), the null block and an
    # out-of-range id (both skipped by kernel and oracle)
    chunks = [perm[:5], [0, perm[5], perm[6], nb + 5], [perm[7]]]
    names, offsets, sizes, flat, ioff, total = job_plan(L, chunks, s.suffix_size, s.prefix_size,
                                                        base=pad, pad=pad)
    idx = torch.tensor(flat, dtype=torch.int32)

    oc = OracleCopier()
    gc = cache_ops.CacheCopier()
    dl = []
    for l, (t, _) in enumerate(layers):
        oc.register_layer(f"model.layers.{l}.self_attn.attn", t, pf)
        td = to_dev(t, dev)
        dl.append(td)
        gc.register_layer(f"model.layers.{l}.self_attn.attn", td, pf)
    store_cpu = torch.full((total + 64,), 0x5A, dtype=torch.uint8)
    store_dev = store_cpu.to(dev)
    oc.register_store(store_cpu)
    gc.register_store(store_dev)

    oc.gather_pages(names, offsets, sizes, idx, ioff)
    gc.gather_pages(names, offsets, sizes, idx.to(dev), ioff)
    torch.cuda.synchronize()
    assert same_bytes(store_dev, store_cpu)

    # scatter into fresh layers from a random store
    g2 = torch.Generator().manual_seed(12)
    new_store = torch.randint(0, 256, store_cpu.shape, dtype=torch.uint8, generator=g2)
    store_cpu.copy_(new_store)
    store_dev.copy_(new_store.to(dev))
    oc.scatter_pages(names, offsets, sizes, idx, ioff)
    gc.scatter_pages(names, offsets, sizes, idx.to(dev), ioff)
    torch.cuda.synchronize()
    for (t, _), td in zip(layers, dl):
        assert same_bytes(td, t)


def test_large_pages_multi_round(dev):
    # page span of 96 KiB: several rounds of the 32 KiB-per-workgroup loop
    g = torch.Generator().manual_seed(5)
    t, pf = make_layer("nhd", 6, 32, 12, 128, torch.bfloat16, g, kind="bytes")
    s_span = 32 * 12 * 128 * 2
    idx = torch.tensor([5, 2, 4], dtype=torch.int32)
    oc, gc = OracleCopier(), cache_ops.CacheCopier()
    td = to_dev(t, dev)
    oc.register_layer("x", t, pf)
    gc.register_layer("x", td, pf)
    n = 2 * 3 * s_span
    sc, sd = torch.zeros(n, dtype=torch.uint8), torch.zeros(n, dtype=torch.uint8, device=dev)
    oc.register_store(sc)
    gc.register_store(sd)
    oc.gather_pages(["x"], [0], [n], idx, [0, 3])
    gc.gather_pages(["x"], [0], [n], idx.to(dev), [0, 3])
    torch.cuda.synchronize()
    assert same_bytes(sd, sc)


@pytest.mark.parametrize("n_sel", [32, 33, 35, 40])
def test_gather_xcd_runs_with_tail(dev, n_sel):
    # 32 KiB page spans in 4 parts of 8 KiB: 8 * n_sel units in the largest
    # job. Units are dealt to the XCDs in runs of 32 up to the largest multiple
    # of 256; the tail (0, 8, 24 or 64 units) keeps its place. The second job is
    # shorter, a null page and an out-of-range page sit in both regions.
    g = torch.Generator().manual_seed(21 + n_sel)
    nb = 64
    t, pf = make_layer("nhd", nb, 16, 8, 128, torch.bfloat16, g, kind="bytes")
    u, _ = make_layer("nhd", nb, 16, 8, 128, torch.bfloat16, g, kind="bytes")
    span = 16 * 8 * 128 * 2
    sel = [int(x) for x in np.random.default_rng(n_sel).permutation(np.arange(1, nb))[:n_sel]]
    sel[2], sel[-3] = 0, nb + 7
    sel2 = sel[: n_sel - 9]
    oc, gc = OracleCopier(), cache_ops.CacheCopier()
    for name, x in (("x", t), ("y", u)):
        oc.register_layer(name, x, pf)
        gc.register_layer(name, to_dev(x, dev), pf)
    n1, n2 = 2 * len(sel) * span, 2 * len(sel2) * span
    store = torch.randint(0, 256, (n1 + n2,), dtype=torch.uint8, generator=g)
    oc.register_store(store.clone())
    sd = store.to(dev)
    gc.register_store(sd)
    idx = torch.tensor(sel + sel2, dtype=torch.int32)
    args = (["x", "y"], [0, n1], [n1, n2])
    oc.gather_pages(*args, idx, [0, len(sel), len(sel) + len(sel2)])
    gc.gather_pages(*args, idx.to(dev), [0, len(sel), len(sel) + len(sel2)])
    torch.cuda.synchronize()
    assert same_bytes(sd, oc.store)


def test_errors_surface_as_runtime_error(dev):
    gc = cache_ops.CacheCopier()
    t = torch.zeros(2, 4, 16, 2, 8, dtype=torch.bfloat16, device=dev)
    gc.register_layer("a", t, False)
    idx = torch.tensor([1], dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="store buffer not registered"):
        gc.gather_pages(["a"], [0], [512], idx, [0, 1])
    gc.register_store(torch.zeros(1024, dtype=torch.uint8, device=dev))
    with pytest.raises(RuntimeError, match="byte_size mismatch at job 0"):
        gc.gather_pages(["a"], [0], [511], idx, [0, 1])
    with pytest.raises(RuntimeError, match="layer not registered: b"):
        gc.scatter_pages(["b"], [0], [512], idx, [0, 1])
    with pytest.raises(RuntimeError, match="kvcache tensor must be on GPU"):
        gc.register_layer("c", torch.zeros(2, 2), False)
    gc.gather_pages([], [], [], idx, [0])


def test_explicit_stream_and_default_stream(dev):
    t = torch.randn(2, 8, 16, 2, 8, device=dev).to(torch.bfloat16)
    gc = cache_ops.CacheCopier()
    gc.register_layer("a", t, False)
    st = torch.zeros(2 * 2 * 512, dtype=torch.uint8, device=dev)
    gc.register_store(st)
    idx = torch.tensor([3, 6], dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    gc.gather_pages(["a"], [0], [2048], idx, [0, 2], stream=s.cuda_stream)
    s.synchronize()
    want = t[:, [3, 6]].contiguous().view(torch.uint8).reshape(-1)
    assert torch.equal(st, want)
    st.zero_()
    gc.gather_pages(["a"], [0], [2048], idx, [0, 2])
    torch.cuda.synchronize()
    assert torch.equal(st, want)
    # stream 0 is torch's current stream, also inside a stream context
    assert cache_ops._resolve_stream(0, dev) == torch.cuda.current_stream().cuda_stream
    s2 = torch.cuda.Stream()
    with torch.cuda.stream(s2):
        assert cache_ops._resolve_stream(0, dev) == s2.cuda_stream
        assert cache_ops._resolve_stream(0, torch.device("cuda")) == s2.cuda_stream
        st.zero_()
        gc.gather_pages(["a"], [0], [2048], idx, [0, 2])
    s2.synchronize()
    assert torch.equal(st, want)


def test_batched_memcpy_roundtrip(dev):
    host = torch.empty(1 << 20, dtype=torch.uint8, pin_memory=True)
    host.copy_(torch.randint(0, 256, (1 << 20,), dtype=torch.uint8))
    stg = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    cache_ops.batched_memcpy_h2d(host, stg, [0, 4096, 500000], [100, 8192, 600000], [4000, 70000, 1234])
    torch.cuda.synchronize()
    s = stg.cpu()
    assert torch.equal(s[100:4100], host[0:4000])
    assert torch.equal(s[8192:78192], host[4096:74096])
    assert torch.equal(s[600000:601234], host[500000:501234])
    back = torch.zeros(1 << 20, dtype=torch.uint8, pin_memory=True)
    cache_ops.batched_memcpy_d2h(stg, back, [100, 8192], [0, 5000], [4000, 70000])
    torch.cuda.synchronize()
    assert torch.equal(back[0:4000], host[0:4000]) and torch.equal(back[5000:75000], host[4096:74096])
    with pytest.raises(RuntimeError, match="out of bounds"):
        cache_ops.batched_memcpy_d2h(stg, back, [1 << 20], [0], [1])
