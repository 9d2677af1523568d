"""Parity at the BASELINE configurations' full sizes.

Configuration 1 (the reference's CPU-runnable case) runs end to end against
the CPU oracle at its real size: 16 layers x [2, 1024, 16, 8, 64] fp16, 4
cached chunks of 512 tokens whose K was rotated at positions 0..511, moved to
offsets 0, 512, 1024, 1536 while being scattered through a random block table;
then the return gather and the top-15% selection against a perturbed K.

Configuration 2 (the headline, 32 layers x [2, 65536, 16, 8, 128] bf16 =
128 GiB) is checked through size-independent properties: gathering the
scattered, re-rotated pages back gives the staging bytes exactly where nothing
rotates (V, chunk 0 with shift 0) and, for K, an fp32 torch rotation of the
staging values within the 1-ulp bar.
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


def test_config2_full_size_properties(dev):
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import bench
    cfg = bench.CFG2
    w = bench.build_workload(cfg, dev)
    j = w["jobs"]
    L, T, H, D, PS = w["L"], w["T"], cfg["kv_heads"], cfg["head_dim"], cfg["block_size"]
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
    CT = cfg["chunk_tokens"]
    per_job = j["sizes"][0]
    half = per_job // 2
    worst = 0.0
    for i, (o, d) in enumerate(zip(j["offsets"], j["deltas"])):
        src = w["staging"][o:o + per_job]
        got = back[o:o + per_job]
        assert torch.equal(got[half:], src[half:]), f"V bytes differ at job {i}"
        if d == 0:
            assert torch.equal(got[:half], src[:half]), f"unshifted K differs at job {i}"
            continue
        if i % 37 != 1:          # K checked numerically on a spread subset of jobs
            continue
        k_in = src[:half].view(torch.bfloat16).view(CT, H, D).float()
        k_out = got[:half].view(torch.bfloat16).view(CT, H, D).float()
        ang = torch.tensor(float(d), dtype=torch.float32, device=dev) * inv        # fp32 angle
        c, s = torch.cos(ang.double()), torch.sin(ang.double())
        x1, x2 = k_in[..., : D // 2].double(), k_in[..., D // 2:].double()
        want = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)
        norm = torch.sqrt(x1 ** 2 + x2 ** 2).repeat(1, 1, 2)
        tol = _bf16_ulp(torch.maximum(want.abs(), k_out.double().abs())) + 2.0 ** -20 * norm
        err = (k_out.double() - want).abs()
        assert bool((err <= tol).all()), f"job {i}: worst {float((err / tol).max()):.2f} x tolerance"
        worst = max(worst, float((err / tol).max()))
    assert worst <= 1.0
