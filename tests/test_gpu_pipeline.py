"""A request's life through the path on the GPU, checked against what the
model would have computed, not against this build's own restatement:

1. three chunks' K/V are computed independently (K rotated at positions
   0..n-1 in fp64, stored bf16) in a source cache and stored to pinned host
   records (KVIOContext.store, saved position 0);
2. a new request loads them into its own blocks with the fused re-rotation
   to the positions its group boundaries give (KVIOContext.load with
   rerotate=, inv_freq from adapter.rotary_inv_freq): every K row must equal
   the fp64 RoPE of the raw K at the new position, to the bf16 rounding of
   the stored and the moved value; V and every other byte as stored;
3. the recompute policy's per-group counts (Adapter.plan_recompute_selection)
   select, by deviation from recomputed K (the fp64 RoPE at the new position
   plus noise), the rows select_merge merges: keys, indices and merged bytes
   bit-exact against the oracle's three steps.
"""
import numpy as np
import pytest
import torch

from daric_amd import adapter as ad
from daric_amd import cache_ops, kv_io
from oracle import select as osel
from tests.adapter_fakes import FakeRotary
from tests.gpu_util import INT_VIEW, same_bytes

pytestmark = pytest.mark.gpu

L, H, D, PS, NB = 3, 8, 128, 16, 96
CHUNK_PAGES = (6, 4, 8)          # 96, 64 and 128 tokens
PREFIX = 32                      # the request's first group (a system prompt), not loaded


def rope64(x, pos, inv):
    """NeoX RoPE of x [T, H, D] (float64) at positions pos [T]."""
    ang = pos[:, None].astype(np.float64) * inv.astype(np.float64)[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[..., : D // 2], x[..., D // 2:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def test_request_lifecycle(dev):
    rng = np.random.default_rng(0)
    rot = FakeRotary(D, max_pos=4096)
    inv = ad.rotary_inv_freq(rot).numpy()
    names = sorted(f"model.layers.{i}.self_attn.attn" for i in range(L))
    # 1. the chunks as computed on their own: raw K/V, K rotated at 0..n-1
    chunk_tok = [p * PS for p in CHUNK_PAGES]
    raw_k = [rng.standard_normal((L, n, H, D)) for n in chunk_tok]
    raw_v = [rng.standard_normal((L, n, H, D)) for n in chunk_tok]
    src = [torch.zeros(2, NB, PS, H, D, dtype=torch.bfloat16) for _ in range(L)]
    ids = rng.permutation(np.arange(1, NB))
    src_blocks, o = [], 0
    for c, n in enumerate(chunk_tok):
        blocks = ids[o:o + CHUNK_PAGES[c]].tolist()
        o += CHUNK_PAGES[c]
        src_blocks.append((blocks,))
        for li in range(L):
            k = torch.from_numpy(rope64(raw_k[c][li], np.arange(n), inv)).to(torch.bfloat16)
            v = torch.from_numpy(raw_v[c][li]).to(torch.bfloat16)
            src[li][0, blocks] = k.view(len(blocks), PS, H, D)
            src[li][1, blocks] = v.view(len(blocks), PS, H, D)
    src_dev = {n: t.to(dev) for n, t in zip(names, src)}
    bpb = [2 * PS * H * D * 2] * L
    host = torch.zeros(16 << 20, dtype=torch.uint8, pin_memory=True)
    store = kv_io.KVIOContext(names, [0] * L, bpb, [False] * L, src_dev, host, staging_bytes=4 << 20)
    offs, pos = [], 4096
    for b in src_blocks:
        offs.append(pos)
        pos += store.record_size(b) + 4096
    store.store(offs, src_blocks, [0, 0, 0])
    store.close()

    # 2. a new request: prefix group, then the three chunks, at new positions
    group_ptr = [0, PREFIX]
    for n in chunk_tok:
        group_ptr.append(group_ptr[-1] + n)
    req_pages = group_ptr[-1] // PS
    req_blocks = ids[o:o + req_pages].tolist()           # the request's own blocks (fresh ids)
    dst = {n: torch.zeros(2, NB, PS, H, D, dtype=torch.bfloat16, device=dev) for n in names}
    load = kv_io.KVIOContext(names, [0] * L, bpb, [False] * L, dst, host, staging_bytes=4 << 20)
    load_blocks, new_pos = [], []
    for c in range(3):
        first = group_ptr[c + 1] // PS
        load_blocks.append((req_blocks[first:first + CHUNK_PAGES[c]],))
        new_pos.append(group_ptr[c + 1])
    saved = load.load(offs, load_blocks, rerotate=(new_pos, chunk_tok, torch.from_numpy(inv).to(dev), D, True))
    load.done.synchronize()
    assert saved == [0, 0, 0]
    loaded = {n: t.cpu() for n, t in dst.items()}
    for c, n in enumerate(chunk_tok):
        blocks = load_blocks[c][0]
        for li, name in enumerate(names):
            got_k = loaded[name][0, blocks].reshape(n, H, D).double().numpy()
            want_k = rope64(raw_k[c][li], new_pos[c] + np.arange(n), inv)
            x1, x2 = want_k[..., : D // 2], want_k[..., D // 2:]
            pnorm = np.tile(np.sqrt(x1 ** 2 + x2 ** 2), (1, 1, 2))
            ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want_k), 2.0 ** -126))) - 7)
            err = np.abs(got_k - want_k)
            tol = ulp + 2.0 ** -8 * pnorm      # the moved value's rounding + the stored value's
            assert (err <= tol).all(), f"chunk {c} layer {li}: worst {float((err / tol).max()):.2f} x tolerance"
            want_v = torch.from_numpy(raw_v[c][li]).to(torch.bfloat16).view(len(blocks), PS, H, D)
            assert torch.equal(loaded[name][1, blocks].view(torch.int16), want_v.view(torch.int16))
    untouched = torch.ones(NB, dtype=torch.bool)
    untouched[[b for blocks in load_blocks for b in blocks[0]]] = False
    for t in loaded.values():
        assert not bool(t[:, untouched].view(torch.int16).any())

    # 3. recompute selection on the request, merged by select_merge
    topo = ad.CacheTopo(layers={n: ad.LayerCacheTopo(0, PS, bpb[0], False) for n in names}, groups=[names])
    adapter = ad.Adapter(ad.AdaptionConfig(rerotate=True, recompute=True, recompute_policy="daric",
                                           recompute_avg_num=24, function="linear", r=0.5), topo)
    bt, chunks, T = adapter.plan_recompute_selection([group_ptr], [(req_blocks,)])
    assert T == group_ptr[-1] and chunks[0, 3] == 0 and chunks[1:, 3].sum() > 0
    k_rec = torch.zeros(L, T, H, D, dtype=torch.bfloat16)
    for c, n in enumerate(chunk_tok):
        r0 = group_ptr[c + 1]
        for li in range(L):
            noisy = rope64(raw_k[c][li], new_pos[c] + np.arange(n), inv) + 0.05 * rng.standard_t(3, (n, H, D))
            k_rec[li, r0:r0 + n] = torch.from_numpy(noisy).to(torch.bfloat16)
    v_rec = torch.from_numpy(rng.standard_normal((L, T, H, D))).to(torch.bfloat16)
    cpu_layers = [loaded[n] for n in names]
    kmax = int(chunks[:, 3].max())
    keys_o = osel.deviation(cpu_layers, False, bt, k_rec, chunks)
    sel_o = osel.topk_per_chunk(keys_o, chunks, kmax)
    osel.merge_rows(cpu_layers, False, bt, k_rec, v_rec, chunks, sel_o)
    keys_g, sel_g = cache_ops.select_merge([dst[n] for n in names], False, torch.from_numpy(bt).to(dev),
                                           k_rec.to(dev), v_rec.to(dev), chunks)
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    for n, t in zip(names, cpu_layers):
        assert same_bytes(dst[n], t)
    load.close()
