"""Parity at the BASELINE configurations' full sizes.

Configuration 1 (the reference's CPU-runnable case) runs end to end against
the CPU oracle at its real size: 16 layers x [2, 1024, 16, 8, 64] fp16, 4
cached chunks of 512 tokens whose K was rotated at positions 0..511, moved to
offsets 0, 512, 1024, 1536 while being scattered through a random block table;
then the return gather and the top-15% selection against a perturbed K.

Configurations 2 to 5 run at their full sizes on the bench's own inputs
(bench.py's builders) and are checked through size-independent properties
(gather after scatter, store then load) and, where the oracle finishes in
seconds, bit-exactly against it.
"""
import os
import sys

import numpy as np
import pytest
import torch

from daric_amd import cache_ops
from oracle import rope as orope
from oracle import select as osel
from oracle.copy import OracleCopier
from tests.gpu_util import assert_rotation_parity, rotation_region, same_bytes, to_dev

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
THETA = 500000.0


def test_config1_full_size(dev):
    L, H, D, PS, NB, C, CT = 16, 8, 64, 16, 1024, 4, 512
    g = torch.Generator().manual_seed(0)
    inv = orope.default_inv_freq(D, THETA)
    # raw K/V ~ N(0,1); K stored rotated to positions 0..511 (fp64 RoPE, then fp16)
    k_raw = torch.randn(C, L, CT, H, D, generator=g, dtype=torch.float64)
    v_raw = torch.randn(C, L, CT, H, D, generator=g, dtype=torch.float64)
    pos = np.arange(CT)
    ang = pos[:, None].astype(np.float64) * inv.astype(np.float64)[None, :]      # [CT, D/2]
    cs, sn = torch.from_numpy(np.cos(ang))[:, None, :], torch.from_numpy(np.sin(ang))[:, None, :]
    x1, x2 = k_raw[..., : D // 2], k_raw[..., D // 2:]
    k_stored = torch.cat([x1 * cs - x2 * sn, x2 * cs + x1 * sn], dim=-1).to(torch.float16)
    v_stored = v_raw.to(torch.float16)
    # staging records: per chunk, per layer in sorted name order, [K pages | V pages]
    names = sorted(f"model.layers.{i}.self_attn.attn" for i in range(L))
    pages = CT // PS
    ids = (torch.randperm(NB - 1, generator=g)[: C * pages] + 1).to(torch.int32)
    recs, jn, offs, sizes, flat, ioff, deltas, ntok = [], [], [], [], [], [0], [], []
    off = 0
    job_bytes = 2 * CT * H * D * 2
    for c in range(C):
        bids = ids[c * pages:(c + 1) * pages].tolist()
        for li, n in enumerate(names):
            recs.append(torch.stack([k_stored[c, li], v_stored[c, li]]).contiguous().view(torch.uint8).reshape(-1))
            jn.append(n); offs.append(off); sizes.append(job_bytes); flat.extend(bids)
            ioff.append(len(flat)); deltas.append(c * CT); ntok.append(CT)
            off += job_bytes
    staging = torch.cat(recs)
    layers = [torch.zeros(2, NB, PS, H, D, dtype=torch.float16) for _ in range(L)]
    oc, gc = OracleCopier(), cache_ops.CacheCopier()
    dev_layers = [to_dev(t, dev) for t in layers]
    for n, t, td in zip(names, layers, dev_layers):
        oc.register_layer(n, t, False)
        gc.register_layer(n, td, False)
    oc.register_store(staging.clone())
    gc.register_store(staging.to(dev))
    idx = torch.tensor(flat, dtype=torch.int32)
    oc.scatter_pages_rerotate(jn, offs, sizes, idx, ioff, deltas, ntok, inv, D, True)
    gc.scatter_pages_rerotate(jn, offs, sizes, idx.to(dev), ioff, deltas, ntok,
                              torch.from_numpy(inv).to(dev), D, True)
    torch.cuda.synchronize()
    slots = [int(b) * PS + j for c in range(1, C) for b in ids[c * pages:(c + 1) * pages].tolist()
             for j in range(PS)]
    for t, td in zip(layers, dev_layers):
        mask, pn = rotation_region(t, False, D, slots, True)
        assert_rotation_parity(td, t, mask, pn)
    # the moved K is RoPE of the raw K at its new position 512c + j (fp64), to fp16 accuracy
    for c in range(1, C):
        bids = ids[c * pages:(c + 1) * pages].long()
        for li in (0, L - 1):
            got = dev_layers[li][0][bids.to(dev)].reshape(CT, H, D).double().cpu()
            a2 = (pos + c * CT)[:, None].astype(np.float64) * inv.astype(np.float64)[None, :]
            c2, s2 = torch.from_numpy(np.cos(a2))[:, None, :], torch.from_numpy(np.sin(a2))[:, None, :]
            r1, r2 = k_raw[c, li][..., : D // 2], k_raw[c, li][..., D // 2:]
            want = torch.cat([r1 * c2 - r2 * s2, r2 * c2 + r1 * s2], dim=-1)
            assert float((got - want).abs().max()) < 8 * 2.0 ** -10 * float(want.abs().max())
    # return path: gather the request back; bytes equal the oracle's gather of
    # the same (device-rotated) cache contents
    oc2, gc2 = OracleCopier(), cache_ops.CacheCopier()
    for n, td in zip(names, dev_layers):
        oc2.register_layer(n, td.cpu(), False)
        gc2.register_layer(n, td, False)
    oc2.register_store(torch.zeros(off, dtype=torch.uint8))
    gc2.register_store(torch.zeros(off, dtype=torch.uint8, device=dev))
    oc2.gather_pages(jn, offs, sizes, idx, ioff)
    gc2.gather_pages(jn, offs, sizes, idx.to(dev), ioff)
    torch.cuda.synchronize()
    assert torch.equal(gc2._store.cpu(), oc2.store)
    # selection: top 15% per chunk by deviation from K + N(0, 0.05), on the
    # device-rotated cache contents (the oracle reads the same bytes)
    layers = [td.cpu() for td in dev_layers]
    bt = ids.numpy()
    chunks = [(c * pages, c * CT, CT, int(round(0.15 * CT))) for c in range(C)]
    k_new = torch.empty(L, C * CT, H, D, dtype=torch.float16)
    for li in range(L):
        kv = osel.k_rows_view(layers[li], False)
        for (bo, ro, n, _k) in chunks:
            blk, s = osel.chunk_slots(bt, bo, n, PS)
            base = kv[torch.as_tensor(blk), torch.as_tensor(s)].float()
            k_new[li, ro:ro + n] = (base + 0.05 * torch.randn(base.shape, generator=g)).to(torch.float16)
    keys_o = osel.deviation(layers, False, bt, k_new, chunks)
    keys_g = cache_ops.kv_deviation(dev_layers, False, torch.from_numpy(bt).to(dev), k_new.to(dev), chunks)
    sel_g = cache_ops.topk_per_chunk(keys_g, chunks)
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    assert np.array_equal(sel_g.cpu().numpy(), osel.topk_per_chunk(keys_o, chunks, 77))


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(torch.clamp(x.abs(), min=2.0 ** -126)))
    return torch.exp2(e - 7)


def _e4m3_quantum(x: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(torch.clamp(x.abs(), min=2.0 ** -6)))
    return torch.exp2(e - 3)


def _rotate64(k: torch.Tensor, delta: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    """NeoX rotation in float64 of k [J, T, H, D] by the float32 angles
    float32(delta[j]) * inv_freq[i]."""
    D = k.shape[-1]
    ang = (delta.to(torch.float32)[:, None] * inv[None, :]).double()       # fp32 product, as the kernel
    c, s = ang.cos()[:, None, None, :], ang.sin()[:, None, None, :]
    x1, x2 = k[..., : D // 2], k[..., D // 2:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def _bench():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import bench
    return bench


def test_config2_full_size_properties(dev):
    """Config 2 at full size: gathering the scattered, re-rotated pages back
    gives V and chunk 0 bit-exact, and every rotated K element of all 224
    moved jobs within 1 bf16 ulp of the float64 rotation of the staged value
    (plus the 2^-20 pair-norm allowance for float32 cancellation, which only
    results below 2^-10 of their pair's norm may use)."""
    bench = _bench()
    cfg = bench.CFG2
    w = bench.build_workload(cfg, dev)
    j = w["jobs"]
    H, D = cfg["kv_heads"], cfg["head_dim"]
    CT = cfg["chunk_tokens"]
    cp = cache_ops.CacheCopier()
    for n, t in zip(w["names"], w["cache"]):
        cp.register_layer(n, t, False)
    cp.register_store(w["staging"])
    idx = torch.tensor(j["flat"], dtype=torch.int32, device=dev)
    inv = w["inv_freq"].to(dev)
    cp.scatter_pages_rerotate(j["names"], j["offsets"], j["sizes"], idx, j["ioff"], j["deltas"],
                              j["ntok"], inv, D, True)
    back = torch.zeros_like(w["staging"])
    gp = cache_ops.CacheCopier()
    for n, t in zip(w["names"], w["cache"]):
        gp.register_layer(n, t, False)
    gp.register_store(back)
    gp.gather_pages(j["names"], j["offsets"], j["sizes"], idx, j["ioff"])
    torch.cuda.synchronize()
    n_jobs, per_job = len(j["offsets"]), j["sizes"][0]
    assert j["offsets"] == [i * per_job for i in range(n_jobs)]
    src = w["staging"].view(torch.bfloat16).view(n_jobs, 2, CT, H, D)
    got = back.view(torch.bfloat16).view(n_jobs, 2, CT, H, D)
    assert torch.equal(got[:, 1].view(torch.int16), src[:, 1].view(torch.int16)), "V bytes differ"
    deltas = torch.tensor(j["deltas"], device=dev)
    still = deltas == 0
    assert torch.equal(got[still, 0].view(torch.int16), src[still, 0].view(torch.int16)), "chunk 0 K differs"
    moved = (~still).nonzero().flatten()
    assert moved.numel() == 224
    worst, cancelling = 0.0, 0
    for part in moved.split(16):
        k_in, k_out = src[part, 0].double(), got[part, 0].double()
        want = _rotate64(k_in, deltas[part], inv)
        x1, x2 = k_in[..., : D // 2], k_in[..., D // 2:]
        norm = torch.sqrt(x1 ** 2 + x2 ** 2).repeat(1, 1, 1, 2)
        one_ulp = _bf16_ulp(torch.maximum(want.abs(), k_out.abs()))
        tol = one_ulp + 2.0 ** -20 * norm
        err = (k_out - want).abs()
        ratio = float((err / tol).max())
        assert ratio <= 1.0, f"jobs {part.tolist()[:3]}..: worst {ratio:.2f} x tolerance"
        worst = max(worst, ratio)
        # within 1 ulp with no allowance wherever the result is not a near
        # cancellation (at least 2^-10 of its pair's norm)
        plain = want.abs() >= 2.0 ** -10 * norm
        assert bool((err[plain] <= one_ulp[plain]).all()), f"jobs {part.tolist()[:3]}..: beyond 1 ulp"
        cancelling += int((~plain).sum())
    assert worst <= 1.0
    assert cancelling < moved.numel() * CT * H * D // 250


@pytest.mark.timeout(900)
def test_config2_inplace_full_size(dev):
    """The worker-side form at config 2's full size (the call bench.py times
    as rerotate_inplace): the staged pages scattered unrotated, then
    rerotate_pages moves chunks 1..7 in all 32 layers in place (the Adapter's
    call); gathered back, V and chunk 0 are bit-exact and every rotated K
    element is within the rotation bar of the fp64 rotation, with no allowance
    outside near-cancellations."""
    bench = _bench()
    cfg = bench.CFG2
    w = bench.build_workload(cfg, dev)
    j = w["jobs"]
    H, D, CT = cfg["kv_heads"], cfg["head_dim"], cfg["chunk_tokens"]
    cp = cache_ops.CacheCopier()
    for n, t in zip(w["names"], w["cache"]):
        cp.register_layer(n, t, False)
    cp.register_store(w["staging"])
    idx = torch.tensor(j["flat"], dtype=torch.int32, device=dev)
    inv = w["inv_freq"].to(dev)
    cp.scatter_pages(j["names"], j["offsets"], j["sizes"], idx, j["ioff"])
    pages = CT // cfg["block_size"]
    segs = [(c * pages, 0, CT, c * CT) for c in range(1, cfg["chunks"])]
    cache_ops.rerotate_pages(w["cache"], False, w["ids"].to(dev), segs, inv, D, True)
    back = torch.zeros_like(w["staging"])
    gp = cache_ops.CacheCopier()
    for n, t in zip(w["names"], w["cache"]):
        gp.register_layer(n, t, False)
    gp.register_store(back)
    gp.gather_pages(j["names"], j["offsets"], j["sizes"], idx, j["ioff"])
    torch.cuda.synchronize()
    n_jobs = len(j["offsets"])
    src = w["staging"].view(torch.bfloat16).view(n_jobs, 2, CT, H, D)
    got = back.view(torch.bfloat16).view(n_jobs, 2, CT, H, D)
    assert torch.equal(got[:, 1].view(torch.int16), src[:, 1].view(torch.int16)), "V bytes differ"
    deltas = torch.tensor(j["deltas"], device=dev)
    still = deltas == 0
    assert torch.equal(got[still, 0].view(torch.int16), src[still, 0].view(torch.int16)), "chunk 0 K differs"
    moved = (~still).nonzero().flatten()
    assert moved.numel() == 224
    for part in moved.split(16):
        k_in, k_out = src[part, 0].double(), got[part, 0].double()
        want = _rotate64(k_in, deltas[part], inv)
        x1, x2 = k_in[..., : D // 2], k_in[..., D // 2:]
        norm = torch.sqrt(x1 ** 2 + x2 ** 2).repeat(1, 1, 1, 2)
        one_ulp = _bf16_ulp(torch.maximum(want.abs(), k_out.abs()))
        err = (k_out - want).abs()
        assert bool((err <= one_ulp + 2.0 ** -20 * norm).all()), f"jobs {part.tolist()[:3]}.."
        plain = want.abs() >= 2.0 ** -10 * norm
        assert bool((err[plain] <= one_ulp[plain]).all()), f"jobs {part.tolist()[:3]}..: beyond 1 ulp"


@pytest.mark.timeout(900)
def test_config3_full_size(dev):
    """Config 3 at full size, on the bench's own inputs (bench.config3_inputs:
    32 layers x 98304 tokens in 192 shuffled chunks, k = 77): deviation keys
    and selected indices bit-exact against the oracle on every layer; merged
    cache bytes bit-exact on every layer."""
    bench = _bench()
    w = bench.config3_inputs(dev)
    L, k = w["L"], w["k"]
    layers, bt, chunks, k_new, v_new = w["layers"], w["bt"], w["chunks"], w["k_new"], w["v_new"]
    assert len(chunks) == 192 and w["T"] == 98304
    keys = cache_ops.kv_deviation(layers, False, bt, k_new, chunks)
    sel = cache_ops.topk_per_chunk(keys, chunks, kmax=k)
    torch.cuda.synchronize()
    bt_np = bt.cpu().numpy()
    keys_np, sel_np = keys.cpu().numpy(), sel.cpu().numpy()
    pre = {}
    for l in range(L):
        lc = layers[l].cpu()
        ko = osel.deviation([lc], False, bt_np, k_new[l:l + 1].cpu(), chunks)
        assert np.array_equal(keys_np[l:l + 1].view(np.uint32), ko.view(np.uint32)), f"keys of layer {l}"
        assert np.array_equal(sel_np[l:l + 1], osel.topk_per_chunk(ko, chunks, k)), f"indices of layer {l}"
        pre[l] = lc
    cache_ops.merge_rows(layers, False, bt, k_new, v_new, chunks, sel)
    torch.cuda.synchronize()
    for l in range(L):
        osel.merge_rows([pre[l]], False, bt_np, k_new[l:l + 1].cpu(), v_new[l:l + 1].cpu(), chunks,
                        sel_np[l:l + 1])
        assert torch.equal(layers[l].cpu().view(torch.int16), pre[l].view(torch.int16)), f"merge of layer {l}"
        del pre[l]


@pytest.mark.timeout(900)
def test_config2_hnd_token_copies_full_size(dev):
    """Config 2's return path on a head-major cache at full size (bench's
    config2h: 32 layers of [2, 65536, 16, 8, 128] bf16 stored HND, 128 GiB,
    8192 tokens on 512 random pages): gather_tokens writes exactly the
    token-major rows torch indexing reads from the same pages, and
    scatter_tokens of changed rows rewrites exactly those pages' K and V
    rows, every other page of the cache keeping its bytes (checked through a
    checksum of all pages)."""
    bench = _bench()
    c = bench.CFG2
    L, H, D, PS, NB = c["layers"], c["kv_heads"], c["head_dim"], c["block_size"], c["num_blocks"]
    T = c["chunks"] * c["chunk_tokens"]
    n_pages = T // PS
    g = torch.Generator().manual_seed(0)
    ids = (torch.randperm(NB - 1, generator=g)[:n_pages] + 1).to(torch.int32).to(dev)
    gd = torch.Generator(device=dev).manual_seed(1)
    cache = []
    for _ in range(L):
        t = torch.empty(2, NB, H, PS, D, device=dev, dtype=torch.int16)
        t.random_(generator=gd)
        cache.append(t.view(torch.bfloat16).permute(0, 1, 3, 2, 4))
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    per_layer = 2 * T * H * D * 2
    staging = torch.zeros(L * per_layer, dtype=torch.uint8, device=dev)
    cp = cache_ops.CacheCopier()
    for n, t in zip(names, cache):
        cp.register_layer(n, t, False)
    cp.register_store(staging)
    flat = ids.repeat(L)
    args = (names, [i * per_layer for i in range(L)], [per_layer] * L, flat,
            [i * n_pages for i in range(L + 1)])
    cp.gather_tokens(*args)
    torch.cuda.synchronize()
    rows = staging.view(L, 2, T, H, D * 2)
    for l in range(L):
        want = cache[l][:, ids.long()].reshape(2, T, H, D)           # [2, pages, PS, H, D] token-major
        assert torch.equal(rows[l].view(torch.int16).view(2, T, H, D), want.view(torch.int16)), f"layer {l}"
    # scatter changed rows back: exactly the listed pages change
    def page_sums():
        return torch.stack([t.view(torch.int16).sum(dim=(0, 2, 3, 4), dtype=torch.int64) for t in cache])
    before = page_sums()
    staging.view(torch.int16).bitwise_not_()
    cp.scatter_tokens(*args)
    torch.cuda.synchronize()
    for l in range(L):
        want = rows[l].view(torch.int16).view(2, T, H, D)
        got = cache[l][:, ids.long()].reshape(2, T, H, D).view(torch.int16)
        assert torch.equal(got, want), f"scatter, layer {l}"
    after = page_sums()
    listed = torch.zeros(NB, dtype=torch.bool, device=dev)
    listed[ids.long()] = True
    assert torch.equal(after[:, ~listed], before[:, ~listed]), "pages outside the list changed"


@pytest.mark.timeout(900)
@pytest.mark.parametrize("config", [3, 5])
def test_select_merge_full_size(dev, config):
    """select_merge, the selection step bench.py times (config 3: the
    deviation kernel, then each (layer, chunk)'s top-k and merge fused in one
    workgroup; config 5: the three kernels, its chunks' selected rows being
    too many for one workgroup), against the three separate calls on a copy
    of the same cache at full size: keys, indices and every merged cache byte
    identical. The three calls are held to the oracle on every layer by
    test_config3_full_size and test_config5_full_size."""
    bench = _bench()
    w = bench.config3_inputs(dev) if config == 3 else bench.config5_inputs(dev)
    layers = w["layers"] if config == 3 else w["cache"]
    L, k = w["L"], w["k"]
    bt, chunks, k_new, v_new = w["bt"], w["chunks"], w["k_new"], w["v_new"]
    ks, vs = (None, None) if config == 3 else (w["k_scales"], w["v_scales"])
    twin = [t.clone() for t in layers]
    keys3 = cache_ops.kv_deviation(twin, False, bt, k_new, chunks, k_scales=ks)
    sel3 = cache_ops.topk_per_chunk(keys3, chunks, kmax=k)
    cache_ops.merge_rows(twin, False, bt, k_new, v_new, chunks, sel3, k_scales=ks, v_scales=vs)
    keys, sel = cache_ops.select_merge(layers, False, bt, k_new, v_new, chunks, kmax=k, k_scales=ks, v_scales=vs)
    torch.cuda.synchronize()
    assert torch.equal(keys.view(torch.int32), keys3.view(torch.int32)), "keys differ"
    assert torch.equal(sel, sel3), "indices differ"
    for l in range(L):
        assert torch.equal(layers[l].view(torch.uint8), twin[l].view(torch.uint8)), f"merge of layer {l}"


@pytest.mark.timeout(900)
def test_config4_store_load_full_size(dev):
    """Config 4 at full size: KVIOContext stores the 65536 tokens (64 records
    of 1024 tokens, 32 layers) of bench.config4_inputs into pinned host
    records, then loads them into a zeroed cache. The records hold each
    layer's pages in the reference's [K|V][pages][span] layout with the int64
    saved position at the head of each 4096-byte header; the loaded pages are
    byte-identical, every other page stays zero, and load returns the saved
    positions. The fused re-rotating load of the same records moves record m
    by m * 1024 positions: V bit-exact, record 0 unchanged, every moved K
    element within the rotation bar of the fp64 rotation."""
    from daric_amd.kv_io import KVIOContext
    bench = _bench()
    w = bench.config4_inputs(dev)
    plan = bench.kvio_plan(w)
    names, cache, L = w["names"], w["cache"], w["L"]
    blocks, rec = plan["blocks"], plan["rec"]
    host = torch.empty(len(blocks) * rec, dtype=torch.uint8, pin_memory=True)
    io = KVIOContext(names, [0] * L, plan["bpb"], [False] * L, dict(zip(names, cache)), host,
                     staging_bytes=512 << 20)
    positions = [int(x) for x in np.random.default_rng(4).integers(-(1 << 40), 1 << 40, len(blocks))]
    io.store(plan["offsets"], blocks, positions)
    span = plan["bpb"][0] // 2
    for m in (0, len(blocks) - 1):
        ids_m = torch.tensor(blocks[m][0], device=dev).long()
        pos = plan["offsets"][m]
        for layer in cache:
            want = layer[:, ids_m].contiguous().view(torch.uint8).reshape(-1).cpu()
            assert torch.equal(host[pos:pos + want.numel()], want), f"record {m}"
            pos += want.numel()
        assert pos == plan["offsets"][m] + rec - 4096 and want.numel() == 2 * len(blocks[m][0]) * span
        assert int(host[pos:pos + 8].numpy().view(np.int64)[0]) == positions[m]
    del io
    cache2 = [torch.zeros_like(t) for t in cache]
    io2 = KVIOContext(names, [0] * L, plan["bpb"], [False] * L, dict(zip(names, cache2)), host,
                      staging_bytes=512 << 20)
    saved = io2.load(plan["offsets"], blocks)
    io2.done.synchronize()
    assert saved == positions
    ids = w["ids"].long().to(dev)
    untouched = torch.ones(w["NB"], dtype=torch.bool, device=dev)
    untouched[ids] = False
    for a, b in zip(cache, cache2):
        assert torch.equal(b[:, ids].view(torch.int16), a[:, ids].view(torch.int16))
        assert not bool(b[:, untouched].view(torch.int16).any())
    del io2, cache2
    # the fused re-rotating load (bench.py's load_pipeline_fused): record m's
    # 1024 tokens move from their saved position by m * 1024 (record 0 stays)
    cache3 = [torch.zeros_like(t) for t in cache]
    io3 = KVIOContext(names, [0] * L, plan["bpb"], [False] * L, dict(zip(names, cache3)), host,
                      staging_bytes=512 << 20)
    H, D = w["H"], w["D"]
    inv = (1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))).to(dev)
    M = len(blocks)
    new_pos = [positions[m] + m * 1024 for m in range(M)]
    assert io3.load(plan["offsets"], blocks, rerotate=(new_pos, [1024] * M, inv, D, True)) == positions
    io3.done.synchronize()
    deltas = torch.arange(M, device=dev) * 1024
    for a, b in zip(cache, cache3):
        assert torch.equal(b[1, ids].view(torch.int16), a[1, ids].view(torch.int16)), "V differs"
        assert not bool(b[:, untouched].view(torch.int16).any())
        k_in = a[0, ids].double().reshape(M, 1024, H, D)
        k_out = b[0, ids].double().reshape(M, 1024, H, D)
        assert torch.equal(k_out[0], k_in[0]), "record 0 moved"
        want = _rotate64(k_in, deltas, inv)
        x1, x2 = k_in[..., : D // 2], k_in[..., D // 2:]
        norm = torch.sqrt(x1 ** 2 + x2 ** 2).repeat(1, 1, 1, 2)
        err = (k_out - want).abs()
        assert bool((err <= _bf16_ulp(torch.maximum(want.abs(), k_out.abs())) + 2.0 ** -20 * norm).all())


@pytest.mark.timeout(900)
def test_config5_full_size(dev):
    """Config 5 at full size (bench.config5_inputs: 80 layers, 16 chunks x
    2048 tokens of e4m3 codes, chunk c moved by 2048 c): gathering the
    scattered, re-rotated pages back gives V codes and chunk 0 bit-exact, and
    every moved K code within 1 e4m3 quantum of the float64 rotation of the
    decoded staged code (saturated at 448), on every layer. Then the 10%
    selection with the quantising merge of bf16 rows: keys, indices and merged
    codes bit-exact against the oracle on every layer."""
    bench = _bench()
    w = bench.config5_inputs(dev)
    L, H, D, C, CT, k = w["L"], w["H"], w["D"], w["C"], w["CT"], w["k"]
    j = w["jobs"]
    cp = cache_ops.CacheCopier()
    for l, (n, t) in enumerate(zip(w["names"], w["cache"])):
        cp.register_layer(n, t, False)
        cp.register_k_scale(n, w["k_scales"][l].contiguous())
    cp.register_store(w["staging"])
    cp.scatter_pages_rerotate(j["names"], j["offsets"], j["sizes"], w["idx"], j["ioff"], j["deltas"],
                              j["ntok"], w["inv"], D, True)
    back = torch.zeros_like(w["staging"])
    gp = cache_ops.CacheCopier()
    for n, t in zip(w["names"], w["cache"]):
        gp.register_layer(n, t, False)
    gp.register_store(back)
    gp.gather_pages(j["names"], j["offsets"], j["sizes"], w["idx"], j["ioff"])
    torch.cuda.synchronize()
    n_jobs = len(j["offsets"])
    assert n_jobs == C * L and j["offsets"] == [i * w["job_bytes"] for i in range(n_jobs)]
    src = w["staging"].view(n_jobs, 2, CT, H, D)
    got = back.view(n_jobs, 2, CT, H, D)
    assert torch.equal(got[:, 1], src[:, 1]), "V codes differ"
    assert torch.equal(got[:L, 0], src[:L, 0]), "chunk 0 K codes differ"
    deltas = torch.tensor(j["deltas"], device=dev)
    for c in range(1, C):
        for part in torch.arange(c * L, (c + 1) * L, device=dev).split(20):
            k_in = src[part, 0].view(torch.float8_e4m3fn).float().double()
            k_out = got[part, 0].view(torch.float8_e4m3fn).float().double()
            want = _rotate64(k_in, deltas[part], w["inv"]).clamp(-448.0, 448.0)
            tol = _e4m3_quantum(torch.maximum(want.abs(), k_out.abs()))
            ratio = float(((k_out - want).abs() / tol).max())
            assert ratio <= 1.0, f"chunk {c}: worst {ratio:.2f} e4m3 quanta"
    del back, got
    # selection on the fp8 cache and the quantising merge
    bt, chunks, k_new, v_new = w["bt"], w["chunks"], w["k_new"], w["v_new"]
    keys = cache_ops.kv_deviation(w["cache"], False, bt, k_new, chunks, k_scales=w["k_scales"])
    sel = cache_ops.topk_per_chunk(keys, chunks, kmax=k)
    torch.cuda.synchronize()
    bt_np, keys_np, sel_np = bt.cpu().numpy(), keys.cpu().numpy(), sel.cpu().numpy()
    ks, vs = w["k_scales"].cpu().numpy(), w["v_scales"].cpu().numpy()
    pre = {}
    for l in range(L):
        pre[l] = w["cache"][l].cpu()
        ko = osel.deviation([pre[l]], False, bt_np, k_new[l:l + 1].cpu(), chunks, k_scales=ks[l:l + 1])
        assert np.array_equal(keys_np[l:l + 1].view(np.uint32), ko.view(np.uint32)), f"keys of layer {l}"
        assert np.array_equal(sel_np[l:l + 1], osel.topk_per_chunk(ko, chunks, k)), f"indices of layer {l}"
    cache_ops.merge_rows(w["cache"], False, bt, k_new, v_new, chunks, sel, k_scales=w["k_scales"],
                         v_scales=w["v_scales"])
    torch.cuda.synchronize()
    for l in range(L):
        osel.merge_rows([pre[l]], False, bt_np, k_new[l:l + 1].cpu(), v_new[l:l + 1].cpu(), chunks,
                        sel_np[l:l + 1], k_scales=ks[l:l + 1], v_scales=vs[l:l + 1])
        assert torch.equal(w["cache"][l].cpu(), pre[l]), f"merge of layer {l}"
        del pre[l]


@pytest.mark.timeout(900)
def test_config5_inplace_full_size(dev):
    """The worker-side fp8 form at config 5's full size (the call bench.py
    times as config5.rerotate_inplace, the reference's own fp8 rotation on the
    e4m3 view, adapter.py:370-373): the staged codes scattered unrotated, then
    rerotate_pages moves chunks 1..15 in all 80 layers in place; gathered
    back, V codes and chunk 0 are bit-exact and every moved K code is within 1
    e4m3 quantum of the float64 rotation of the decoded staged code (saturated
    at 448)."""
    bench = _bench()
    w = bench.config5_inputs(dev)
    L, H, D, C, CT, PS = w["L"], w["H"], w["D"], w["C"], w["CT"], w["PS"]
    j = w["jobs"]
    cp = cache_ops.CacheCopier()
    for n, t in zip(w["names"], w["cache"]):
        cp.register_layer(n, t, False)
    cp.register_store(w["staging"])
    cp.scatter_pages(j["names"], j["offsets"], j["sizes"], w["idx"], j["ioff"])
    segs = [(c * (CT // PS), 0, CT, c * CT) for c in range(1, C)]
    cache_ops.rerotate_pages(w["cache"], False, w["bt"], segs, w["inv"], D, True, k_scales=w["k_scales"])
    back = torch.zeros_like(w["staging"])
    gp = cache_ops.CacheCopier()
    for n, t in zip(w["names"], w["cache"]):
        gp.register_layer(n, t, False)
    gp.register_store(back)
    gp.gather_pages(j["names"], j["offsets"], j["sizes"], w["idx"], j["ioff"])
    torch.cuda.synchronize()
    n_jobs = len(j["offsets"])
    assert n_jobs == C * L and j["offsets"] == [i * w["job_bytes"] for i in range(n_jobs)]
    src = w["staging"].view(n_jobs, 2, CT, H, D)
    got = back.view(n_jobs, 2, CT, H, D)
    assert torch.equal(got[:, 1], src[:, 1]), "V codes differ"
    assert torch.equal(got[:L, 0], src[:L, 0]), "chunk 0 K codes differ"
    deltas = torch.tensor(j["deltas"], device=dev)
    for c in range(1, C):
        for part in torch.arange(c * L, (c + 1) * L, device=dev).split(20):
            k_in = src[part, 0].view(torch.float8_e4m3fn).float().double()
            k_out = got[part, 0].view(torch.float8_e4m3fn).float().double()
            want = _rotate64(k_in, deltas[part], w["inv"]).clamp(-448.0, 448.0)
            tol = _e4m3_quantum(torch.maximum(want.abs(), k_out.abs()))
            ratio = float(((k_out - want).abs() / tol).max())
            assert ratio <= 1.0, f"chunk {c}: worst {ratio:.2f} e4m3 quanta"
