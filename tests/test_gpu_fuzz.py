"""Randomised GPU parity: the HIP path against the CPU oracle on drawn layouts,
dtypes, pairings, page sizes, head counts, rotary dims, page lists (null and
out-of-range ids included), token counts and shifts.

hypothesis draws the cases deterministically (derandomize), so a failure
names a reproducible case. Pages are distinct within one call and layer:
concurrent workgroups writing one page would race, as the reference's kernels
would.
"""
import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from daric_amd import cache_ops
from oracle import fp8 as ofp8
from oracle import rope as orope
from oracle.copy import OracleCopier
from oracle.layout import page_copy_shape
from tests.gpu_util import assert_rotation_parity, make_layer, rotation_region, same_bytes, to_dev

pytestmark = pytest.mark.gpu

LAYOUTS = ["nhd", "hnd", "pf", "pf_hnd", "packed", "mla"]
DTYPES = [torch.bfloat16, torch.float16, torch.uint8]
FUZZ = settings(max_examples=60, deadline=None, derandomize=True, database=None,
                suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture,
                                       HealthCheck.data_too_large])


def _geometry(data, aligned_for_fused):
    layout = data.draw(st.sampled_from(LAYOUTS), label="layout")
    dtype = data.draw(st.sampled_from(DTYPES), label="dtype")
    neox = data.draw(st.booleans(), label="neox")
    ps = data.draw(st.sampled_from([1, 8, 16, 32]), label="page_size")
    h = data.draw(st.sampled_from([1, 2, 4, 8]), label="heads")
    fp8 = dtype == torch.uint8
    d = data.draw(st.sampled_from([32, 64, 128] if fp8 else [16, 32, 64, 128]), label="head_dim")
    width = h * d if layout == "mla" else d
    ve = 16 if fp8 else 8
    if aligned_for_fused:
        step = 2 * ve if neox else ve
    else:
        step = 2
    dims = list(range(step, width + 1, step))
    rotary_dim = data.draw(st.sampled_from(dims), label="rotary_dim")
    return layout, dtype, neox, ps, h, d, rotary_dim


def _chunks(data, nb, ps, max_chunks=4):
    """[(page ids, n_tokens, delta)]: page ids distinct across chunks except
    for null (0) and out-of-range ids, which every path skips."""
    perm = data.draw(st.permutations(list(range(1, nb))), label="pages")
    n = data.draw(st.integers(1, max_chunks), label="chunks")
    out, k = [], 0
    for _ in range(n):
        npg = data.draw(st.integers(1, 4), label="chunk pages")
        pages = []
        for _ in range(npg):
            kind = data.draw(st.sampled_from(["page"] * 6 + ["null", "oob"]), label="page kind")
            if kind == "null":
                pages.append(0)
            elif kind == "oob":
                pages.append(nb + 3)
            elif k < len(perm):
                pages.append(perm[k])
                k += 1
            else:
                pages.append(0)
        ntok = data.draw(st.integers(0, npg * ps + 3), label="n_tokens")
        delta = data.draw(st.one_of(st.just(0), st.integers(-40000, 40000)), label="delta")
        out.append((pages, ntok, delta))
    return out


def _store_values(nbytes, dtype, gen):
    if dtype == torch.uint8:
        return torch.from_numpy(ofp8.encode(torch.randn(nbytes, generator=gen).numpy()))
    e = torch.empty(0, dtype=dtype).element_size()
    return torch.randn(nbytes // e, generator=gen).to(dtype).view(torch.uint8)


@FUZZ
@given(data=st.data())
def test_fused_scatter_rerotate_fuzz(dev, data):
    _fused_case(dev, data, aligned_for_fused=True)


@FUZZ
@given(data=st.data())
def test_fused_call_on_layouts_the_fused_kernel_does_not_take_fuzz(dev, data):
    """Any even rotary dim (halves that are not 16-byte multiples) and store
    offsets aligned to 1, 2, 4 or 8 bytes: scatter_pages_rerotate scatters and
    then rotates in place, to the same bar against the oracle."""
    _fused_case(dev, data, aligned_for_fused=False)


def _fused_case(dev, data, aligned_for_fused):
    layout, dtype, neox, ps, h, d, R = _geometry(data, aligned_for_fused=aligned_for_fused)
    # element-aligned padding (any byte for fp8) keeps the staged values finite
    pads = [0, 1, 2, 4, 8] if dtype == torch.uint8 else [0, 2, 4, 8]
    pad = 0 if aligned_for_fused else data.draw(st.sampled_from(pads), label="store padding")
    nb = data.draw(st.integers(6, 40), label="num_blocks")
    L = data.draw(st.integers(1, 3), label="layers")
    seed = data.draw(st.integers(0, 2 ** 16), label="seed")
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g) for _ in range(L)]
    pf = layers[0][1]
    t0 = layers[0][0]
    shp = page_copy_shape(tuple(t0.shape), tuple(t0.stride()), t0.element_size(), pf)
    chunks = _chunks(data, nb, ps)
    names, offsets, sizes, flat, ioff, dl, nt = [], [], [], [], [0], [], []
    off = pad
    for pages, ntok, delta in chunks:
        for li in range(L):
            names.append(f"layer.{li}")
            offsets.append(off)
            sz = shp.prefix_size * len(pages) * shp.suffix_size
            sizes.append(sz)
            flat.extend(pages)
            ioff.append(len(flat))
            dl.append(delta)
            nt.append(ntok)
            off += sz + pad
    store = _store_values(off + 16, dtype, g)
    inv = orope.default_inv_freq(R, 500000.0)
    oc, gc = OracleCopier(), cache_ops.CacheCopier()
    dev_layers = []
    for li, (t, _) in enumerate(layers):
        oc.register_layer(f"layer.{li}", t, pf)
        td = to_dev(t, dev)
        dev_layers.append(td)
        gc.register_layer(f"layer.{li}", td, pf)
        if dtype == torch.uint8:
            sc = (0.5 + torch.rand(h if layout != "mla" else 1, generator=g)).float()
            oc.register_k_scale(f"layer.{li}", sc.numpy())
            gc.register_k_scale(f"layer.{li}", sc.to(dev))
    oc.register_store(store.clone())
    gc.register_store(store.to(dev))
    idx = torch.tensor(flat, dtype=torch.int32)
    oc.scatter_pages_rerotate(names, offsets, sizes, idx, ioff, dl, nt, inv, R, neox)
    gc.scatter_pages_rerotate(names, offsets, sizes, idx.to(dev), ioff, dl, nt,
                              torch.from_numpy(inv).to(dev), R, neox)
    torch.cuda.synchronize()
    kps = orope.k_view(layers[0][0], pf, R).shape[1]
    slots = []
    for pages, ntok, delta in chunks:
        if delta == 0:
            continue
        for j in range(min(ntok, len(pages) * kps)):
            p = pages[j // kps]
            if 0 < p < shp.num_pages:
                slots.append(p * kps + j % kps)
    for (t, _), td in zip(layers, dev_layers):
        mask, pn = rotation_region(t, pf, R, slots, neox)
        assert_rotation_parity(td, t, mask, pn)


@FUZZ
@given(data=st.data())
def test_inplace_rerotate_fuzz(dev, data):
    layout, dtype, neox, ps, h, d, R = _geometry(data, aligned_for_fused=False)
    nb = data.draw(st.integers(6, 40), label="num_blocks")
    L = data.draw(st.integers(1, 3), label="layers")
    seed = data.draw(st.integers(0, 2 ** 16), label="seed")
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g) for _ in range(L)]
    pf = layers[0][1]
    kps = orope.k_view(layers[0][0], pf, R).shape[1]
    # segments over one block table; each token's slot appears once
    perm = data.draw(st.permutations(list(range(0, nb))), label="blocks")
    n_seg = data.draw(st.integers(1, 4), label="segments")
    bt, segs, k = [], [], 0
    for _ in range(n_seg):
        npg = data.draw(st.integers(1, 3), label="segment pages")
        if k + npg > len(perm):
            break
        start = data.draw(st.integers(0, kps - 1), label="tok_start")
        n = data.draw(st.integers(0, npg * kps - start), label="n_tokens")
        delta = data.draw(st.one_of(st.just(0), st.integers(-40000, 40000)), label="delta")
        segs.append((len(bt), start, n, delta))
        bt.extend(perm[k:k + npg])
        k += npg
    bt = np.asarray(bt, dtype=np.int32)
    inv = orope.default_inv_freq(R, 500000.0)
    scales = None
    if dtype == torch.uint8:
        scales = (0.5 + torch.rand(L, h if layout != "mla" else 1, generator=g)).float()
    dev_layers = [to_dev(t, dev) for t, _ in layers]
    cpu_layers = [t for t, _ in layers]
    orope.rerotate_pages(cpu_layers, pf, bt, segs, inv, R, neox,
                         None if scales is None else scales.numpy())
    cache_ops.rerotate_pages(dev_layers, pf, torch.from_numpy(bt).to(dev), segs,
                             torch.from_numpy(inv).to(dev), R, neox,
                             None if scales is None else scales.to(dev))
    torch.cuda.synchronize()
    slots = []
    for o, ts, n, delta in segs:
        if delta != 0 and n > 0:
            slots += orope.segment_slots(bt, o, ts, n, kps)
    for t, td in zip(cpu_layers, dev_layers):
        mask, pn = rotation_region(t, pf, R, slots, neox)
        assert_rotation_parity(td, t, mask, pn)


@FUZZ
@given(data=st.data())
def test_gather_scatter_fuzz(dev, data):
    layout = data.draw(st.sampled_from(LAYOUTS), label="layout")
    dtype = data.draw(st.sampled_from(DTYPES + [torch.float32]), label="dtype")
    ps = data.draw(st.sampled_from([1, 3, 16]), label="page_size")
    h = data.draw(st.sampled_from([1, 2, 3, 8]), label="heads")
    d = data.draw(st.sampled_from([5, 16, 64]), label="head_dim")   # 5: the byte / word paths
    if layout == "packed" and dtype == torch.float32:
        dtype = torch.bfloat16
    nb = data.draw(st.integers(4, 30), label="num_blocks")
    L = data.draw(st.integers(1, 3), label="layers")
    seed = data.draw(st.integers(0, 2 ** 16), label="seed")
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g, kind="bytes") for _ in range(L)]
    pf = layers[0][1]
    t0 = layers[0][0]
    shp = page_copy_shape(tuple(t0.shape), tuple(t0.stride()), t0.element_size(), pf)
    chunks = _chunks(data, nb, ps)
    names, offsets, sizes, flat, ioff = [], [], [], [], [0]
    off = data.draw(st.sampled_from([0, 16, 4096]), label="store base")
    for pages, _, _ in chunks:
        for li in range(L):
            names.append(f"layer.{li}")
            offsets.append(off)
            sz = shp.prefix_size * len(pages) * shp.suffix_size
            sizes.append(sz)
            flat.extend(pages)
            ioff.append(len(flat))
            off += sz
    store = torch.randint(0, 256, (off + 32,), dtype=torch.uint8, generator=g)
    gather = data.draw(st.booleans(), label="gather")
    oc, gc = OracleCopier(), cache_ops.CacheCopier()
    dev_layers = []
    for li, (t, _) in enumerate(layers):
        oc.register_layer(f"layer.{li}", t, pf)
        td = to_dev(t, dev)
        dev_layers.append(td)
        gc.register_layer(f"layer.{li}", td, pf)
    oc.register_store(store.clone())
    gstore = store.to(dev)
    gc.register_store(gstore)
    idx = torch.tensor(flat, dtype=torch.int32)
    fn = "gather_pages" if gather else "scatter_pages"
    getattr(oc, fn)(names, offsets, sizes, idx, ioff)
    getattr(gc, fn)(names, offsets, sizes, idx.to(dev), ioff)
    torch.cuda.synchronize()
    assert torch.equal(gstore.cpu(), oc.store)
    for (t, _), td in zip(layers, dev_layers):
        assert same_bytes(td, t)


def _selection_case(data, dtype=None):
    """A drawn selection workload: layers of a drawn layout, chunks over a
    block table with null, out-of-range and negative ids, chunk starts inside
    their first page (tok_start) and k from 0 to past the chunk's length."""
    from oracle import select as osel
    layout = data.draw(st.sampled_from(LAYOUTS), label="layout")
    if dtype is None:
        dtype = data.draw(st.sampled_from(DTYPES), label="cache dtype")
    ps = data.draw(st.sampled_from([1, 8, 16]), label="page_size")
    h = data.draw(st.sampled_from([1, 2, 4, 8]), label="heads")
    d = data.draw(st.sampled_from([8, 16, 24, 64, 128]), label="head_dim")
    nb = data.draw(st.integers(4, 40), label="num_blocks")
    L = data.draw(st.integers(1, 3), label="layers")
    seed = data.draw(st.integers(0, 2 ** 16), label="seed")
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g) for _ in range(L)]
    pf = layers[0][1]
    kv = osel.k_rows_view(layers[0][0], pf)
    kps, H, D = kv.shape[1], kv.shape[2], kv.shape[3]
    perm = data.draw(st.permutations(list(range(0, nb))), label="blocks")
    n_chunks = data.draw(st.integers(1, 4), label="chunks")
    bt, chunks, row, k_used = [], [], 0, 0
    for _ in range(n_chunks):
        npg = data.draw(st.integers(1, 3), label="chunk pages")
        ids = []
        for _ in range(npg):
            kind = data.draw(st.sampled_from(["page"] * 5 + ["oob", "neg"]), label="block kind")
            if kind == "oob":
                ids.append(nb + 2)
            elif kind == "neg":
                ids.append(-1)
            elif k_used < len(perm):
                ids.append(perm[k_used])
                k_used += 1
            else:
                ids.append(nb + 2)
        ts = data.draw(st.integers(0, kps - 1), label="tok_start")
        n = data.draw(st.integers(0, npg * kps - ts), label="n_tokens")
        k = data.draw(st.integers(0, n + 2), label="k")
        chunks.append((len(bt), row, n, k, ts))
        bt.extend(ids)
        row += n
    T = max(row, 1)
    return dict(layers=[t for t, _ in layers], pf=pf, bt=np.asarray(bt, np.int32), chunks=chunks, T=T, L=L,
                H=H, D=D, dtype=dtype, g=g)


@FUZZ
@given(data=st.data())
def test_selection_fuzz(dev, data):
    from oracle import select as osel
    c = _selection_case(data)
    cpu, pf, bt, chunks, T, L, H, D, dtype, g = (c[k] for k in ("layers", "pf", "bt", "chunks", "T", "L", "H",
                                                                "D", "dtype", "g"))
    new_dtype = data.draw(st.sampled_from([torch.bfloat16, torch.float16]), label="k_new dtype")
    k_new = torch.randn(L, T, H, D, generator=g).to(new_dtype)
    scales = None
    if dtype == torch.uint8:
        scales = (0.25 + torch.rand(L, H, generator=g)).float()
    gpu = [to_dev(t, dev) for t in cpu]
    btd = torch.from_numpy(bt).to(dev)
    keys_o = osel.deviation(cpu, pf, bt, k_new, chunks, None if scales is None else scales.numpy())
    keys_g = cache_ops.kv_deviation(gpu, pf, btd, k_new.to(dev), chunks,
                                    k_scales=None if scales is None else scales.to(dev))
    torch.cuda.synchronize()
    kg = keys_g.cpu().numpy()
    assert np.array_equal(kg.view(np.uint32), keys_o.view(np.uint32)), \
        f"{int((kg.view(np.uint32) != keys_o.view(np.uint32)).sum())} keys differ"
    kmax = max(min(ch[3], ch[2]) for ch in chunks) + data.draw(st.integers(0, 3), label="kmax extra")
    sel_o = osel.topk_per_chunk(keys_o, chunks, kmax)
    sel_g = cache_ops.topk_per_chunk(keys_g, chunks, kmax=kmax)
    torch.cuda.synchronize()
    if kmax > 0:
        assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    # merge: recomputed rows in the cache's own element type, or (fp8 cache)
    # bf16/fp16 rows quantised with per-(layer, head) K and V scales
    quant = dtype == torch.uint8 and data.draw(st.booleans(), label="quantising merge")
    ks = vs = None
    if quant:
        km = (torch.randn(L, T, H, D, generator=g) * 4).to(new_dtype)
        vm = (torch.randn(L, T, H, D, generator=g) * 4).to(new_dtype)
        if data.draw(st.booleans(), label="special values"):
            # signed zeros, infinities, NaNs of both signs, subnormals and
            # saturating magnitudes at random places of the rows
            special = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), -float("nan"),
                                    1e-6, -3e-7, 6e4, -6e4]).to(new_dtype)
            for rows in (km, vm):
                flat = rows.view(-1)
                pos = torch.randint(0, flat.numel(), (max(1, flat.numel() // 50),), generator=g)
                flat[pos] = special[torch.randint(0, len(special), (len(pos),), generator=g)]
        ks = (0.002 + 0.02 * torch.rand(L, H, generator=g)).float()
        vs = (0.002 + 0.02 * torch.rand(L, H, generator=g)).float()
    elif dtype == torch.uint8:
        km = torch.from_numpy(ofp8.encode(torch.randn(L * T * H * D, generator=g).numpy())).view(L, T, H, D)
        vm = torch.from_numpy(ofp8.encode(torch.randn(L * T * H * D, generator=g).numpy())).view(L, T, H, D)
    else:
        km = torch.randn(L, T, H, D, generator=g).to(dtype)
        vm = torch.randn(L, T, H, D, generator=g).to(dtype)
    osel.merge_rows(cpu, pf, bt, km, vm, chunks, sel_o,
                    k_scales=None if ks is None else ks.numpy(), v_scales=None if vs is None else vs.numpy())
    cache_ops.merge_rows(gpu, pf, btd, km.to(dev), vm.to(dev), chunks, torch.from_numpy(sel_o).to(dev),
                         k_scales=None if ks is None else ks.to(dev), v_scales=None if vs is None else vs.to(dev))
    torch.cuda.synchronize()
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)


@FUZZ
@given(data=st.data())
def test_select_merge_fuzz(dev, data):
    """The whole selection in one call (select_merge: default, keys given, or
    one pass) on the drawn workloads: keys, indices and merged bytes
    bit-exact against the oracle's three steps. fp8 caches merge bf16/fp16
    rows quantised with the cache's K and V scales, which also dequantise
    the cached K for the keys."""
    from oracle import select as osel
    c = _selection_case(data)
    cpu, pf, bt, chunks, T, L, H, D, dtype, g = (c[k] for k in ("layers", "pf", "bt", "chunks", "T", "L", "H",
                                                                "D", "dtype", "g"))
    quant = dtype == torch.uint8
    row_dtype = data.draw(st.sampled_from([torch.bfloat16, torch.float16]), label="row dtype") if quant else dtype
    km = (torch.randn(L, T, H, D, generator=g) * (4 if quant else 1)).to(row_dtype)
    vm = (torch.randn(L, T, H, D, generator=g) * (4 if quant else 1)).to(row_dtype)
    ks = vs = None
    if quant:
        ks = (0.002 + 0.02 * torch.rand(L, H, generator=g)).float()
        vs = (0.002 + 0.02 * torch.rand(L, H, generator=g)).float()
    mode = data.draw(st.sampled_from(["default", "keys_ready", "one_pass"]), label="mode")
    kmax = max(min(ch[3], ch[2]) for ch in chunks) + data.draw(st.integers(0, 3), label="kmax extra")
    has_v = osel.v_view(cpu[0], pf) is not None
    keys_o = osel.deviation(cpu, pf, bt, km, chunks, None if ks is None else ks.numpy())
    sel_o = osel.topk_per_chunk(keys_o, chunks, kmax)
    gpu = [to_dev(t, dev) for t in cpu]
    btd = torch.from_numpy(bt).to(dev)
    keys = None
    if mode == "keys_ready":
        keys = cache_ops.kv_deviation(gpu, pf, btd, km.to(dev), chunks, k_scales=None if ks is None else ks.to(dev))
    if kmax == 0:
        return      # no index rows: select_merge only computes the keys (checked by the selection fuzz)
    osel.merge_rows(cpu, pf, bt, km, vm, chunks, sel_o,
                    k_scales=None if ks is None else ks.numpy(), v_scales=None if vs is None else vs.numpy())
    keys_g, sel_g = cache_ops.select_merge(gpu, pf, btd, km.to(dev), vm.to(dev) if has_v else None, chunks,
                                           kmax=kmax, keys=keys, keys_ready=mode == "keys_ready",
                                           one_pass=mode == "one_pass",
                                           k_scales=None if ks is None else ks.to(dev),
                                           v_scales=None if vs is None else vs.to(dev))
    torch.cuda.synchronize()
    kg = keys_g.cpu().numpy()
    assert np.array_equal(kg.view(np.uint32), keys_o.view(np.uint32))
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)


@FUZZ
@given(data=st.data())
def test_token_copies_fuzz(dev, data):
    layout = data.draw(st.sampled_from(LAYOUTS), label="layout")
    dtype = data.draw(st.sampled_from(DTYPES + [torch.float32]), label="dtype")
    ps = data.draw(st.sampled_from([1, 3, 16]), label="page_size")
    h = data.draw(st.sampled_from([1, 2, 3, 8]), label="heads")
    d = data.draw(st.sampled_from([5, 16, 64, 128]), label="head_dim")
    if layout == "packed" and dtype == torch.float32:
        dtype = torch.bfloat16
    nb = data.draw(st.integers(4, 30), label="num_blocks")
    L = data.draw(st.integers(1, 3), label="layers")
    seed = data.draw(st.integers(0, 2 ** 16), label="seed")
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g, kind="bytes") for _ in range(L)]
    pf = layers[0][1]
    n_kv = 1 if layout == "mla" else 2
    chunks = _chunks(data, nb, ps)
    names, offsets, sizes, flat, ioff = [], [], [], [], [0]
    off = data.draw(st.sampled_from([0, 16, 4096, 5]), label="store base")
    e = layers[0][0].element_size()
    for pages, _, _ in chunks:
        for li in range(L):
            names.append(f"layer.{li}")
            offsets.append(off)
            sz = n_kv * len(pages) * ps * h * d * e
            sizes.append(sz)
            flat.extend(pages)
            ioff.append(len(flat))
            off += sz
    store = torch.randint(0, 256, (off + 32,), dtype=torch.uint8, generator=g)
    gather = data.draw(st.booleans(), label="gather")
    oc, gc = OracleCopier(), cache_ops.CacheCopier()
    dev_layers = []
    for li, (t, _) in enumerate(layers):
        oc.register_layer(f"layer.{li}", t, pf)
        td = to_dev(t, dev)
        dev_layers.append(td)
        gc.register_layer(f"layer.{li}", td, pf)
    oc.register_store(store.clone())
    gstore = store.to(dev)
    gc.register_store(gstore)
    idx = torch.tensor(flat, dtype=torch.int32)
    fn = "gather_tokens" if gather else "scatter_tokens"
    getattr(oc, fn)(names, offsets, sizes, idx, ioff)
    getattr(gc, fn)(names, offsets, sizes, idx.to(dev), ioff)
    torch.cuda.synchronize()
    assert torch.equal(gstore.cpu(), oc.store)
    for (t, _), td in zip(layers, dev_layers):
        assert same_bytes(td, t)
