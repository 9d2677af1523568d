"""GPU parity of the re-rotation entry points against the CPU oracle.

scatter_pages_rerotate (fused) and rerotate_pages (in place) on every
supported layout and dtype: bytes outside the rotated K elements bit-exact;
rotated bf16/fp16 elements within 1 ulp of the oracle's fp64 rotation (plus
an fp32 arithmetic allowance, see gpu_util.assert_rotation_parity); fp8
within 1 e4m3 quantum.
"""
import numpy as np
import pytest
import torch

from daric_amd import cache_ops
from oracle import rope as orope
from oracle.copy import OracleCopier
from oracle.layout import page_copy_shape
from tests.gpu_util import assert_rotation_parity, make_layer, rotation_region, same_bytes, to_dev

pytestmark = pytest.mark.gpu

THETA = 500000.0


def name(l):
    return f"model.layers.{l}.self_attn.attn"


def fused_case(dev, layout, dtype, neox, rotary_dim, nb=48, ps=16, h=4, d=64, L=2, seed=0,
               chunk_tokens=(37, 64, 16, 5), deltas=(1024, 30720, 0, -300)):
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g) for _ in range(L)]
    pf = layers[0][1]
    t0 = layers[0][0]
    s = page_copy_shape(tuple(t0.shape), tuple(t0.stride()), t0.element_size(), pf)
    perm = np.random.default_rng(seed).permutation(np.arange(1, nb)).tolist()
    chunks, k = [], 0
    for n in chunk_tokens:
        npages = -(-n // ps)
        chunks.append(perm[k:k + npages])
        k += npages
    names, offsets, sizes, flat, ioff, dl, nt = [], [], [], [], [0], [], []
    off = 0
    for c, bids in enumerate(chunks):
        for l in range(L):
            names.append(name(l))
            offsets.append(off)
            sz = s.prefix_size * len(bids) * s.suffix_size
            sizes.append(sz)
            flat.extend(bids)
            ioff.append(len(flat))
            dl.append(deltas[c])
            nt.append(chunk_tokens[c])
            off += sz
    inv = orope.default_inv_freq(rotary_dim, THETA)
    # staging: random values of the cache dtype (rotatable, no NaN)
    gs = torch.Generator().manual_seed(seed + 1)
    if dtype == torch.uint8:
        from oracle import fp8 as ofp8
        store = torch.from_numpy(ofp8.encode(torch.randn(off // 1, generator=gs).numpy()))
    else:
        e = torch.empty(0, dtype=dtype).element_size()
        store = torch.randn(off // e, generator=gs).to(dtype).view(torch.uint8)
    oc, gc = OracleCopier(), cache_ops.CacheCopier()
    dev_layers = []
    scales = {}
    for l, (t, _) in enumerate(layers):
        oc.register_layer(name(l), t, pf)
        td = to_dev(t, dev)
        dev_layers.append(td)
        gc.register_layer(name(l), td, pf)
        if dtype == torch.uint8:
            sc = (0.5 + torch.rand(h if layout != "mla" else 1, generator=gs)).float()
            scales[l] = sc
            oc.register_k_scale(name(l), sc.numpy())
            gc.register_k_scale(name(l), sc.to(dev))
    oc.register_store(store.clone())
    gc.register_store(store.to(dev))
    idx = torch.tensor(flat, dtype=torch.int32)
    oc.scatter_pages_rerotate(names, offsets, sizes, idx, ioff, dl, nt, inv, rotary_dim, neox)
    gc.scatter_pages_rerotate(names, offsets, sizes, idx.to(dev), ioff, dl, nt,
                              torch.from_numpy(inv).to(dev), rotary_dim, neox)
    torch.cuda.synchronize()
    worst = 0.0
    for l, ((t, _), td) in enumerate(zip(layers, dev_layers)):
        ps_ = orope.k_view(t, pf, rotary_dim).shape[1]
        slots = []
        for c, bids in enumerate(chunks):
            if deltas[c] == 0:
                continue
            for j in range(chunk_tokens[c]):
                slots.append(bids[j // ps_] * ps_ + j % ps_)
        mask, pn = rotation_region(t, pf, rotary_dim, slots, neox)
        worst = max(worst, assert_rotation_parity(td, t, mask, pn))
    return worst


@pytest.mark.parametrize("layout", ["nhd", "hnd", "pf", "pf_hnd", "packed", "mla"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_layouts(dev, layout, dtype):
    fused_case(dev, layout, dtype, True, 64)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rotary_dim", [64, 32, 16])
def test_fused_pairing_partial_rotary(dev, neox, rotary_dim):
    fused_case(dev, "nhd", torch.bfloat16, neox, rotary_dim, seed=2)


@pytest.mark.parametrize("layout", ["nhd", "pf", "packed", "mla"])
@pytest.mark.parametrize("neox", [True, False])
def test_fused_fp8(dev, layout, neox):
    # mla: 576-byte rows (36 units, not a divisor of the wavefront) take the
    # item-based kernel; the other layouts take the lane-exchange kernel
    d = {"packed": 64, "mla": 144}.get(layout, 128)
    fused_case(dev, layout, torch.uint8, neox, 64, d=d, seed=3)


def test_fused_llama3_8b_page_shape(dev):
    # H=8, D=128 bf16 pages of 32 KiB, as the benchmark shape (two 16 KiB parts per page)
    fused_case(dev, "nhd", torch.bfloat16, True, 128, nb=40, h=8, d=128, L=2, seed=4,
               chunk_tokens=(128, 64, 40), deltas=(1024, 7168, 3))


@pytest.mark.parametrize("layout,dtype,neox", [
    ("pf", torch.bfloat16, True),        # 64 KiB K+V spans: four 16 KiB parts, K in the first two
    ("pf_hnd", torch.bfloat16, False),   # head-major rows, four parts
    ("pf", torch.uint8, True),           # 32 KiB fp8 K+V spans: two parts
    ("hnd", torch.float16, True),        # 32 KiB head-major K pages: two parts
])
def test_fused_large_spans_in_parts(dev, layout, dtype, neox):
    fused_case(dev, layout, dtype, neox, 128, nb=40, h=8, d=128, L=2, seed=12,
               chunk_tokens=(128, 37, 40), deltas=(1024, -7168, 3))


@pytest.mark.parametrize("layout,dtype,neox,rotary_dim", [
    ("nhd", torch.bfloat16, True, 24),     # NeoX halves of 12 elements: not 16-byte multiples
    ("hnd", torch.float16, False, 20),     # GPT-J pairs over 40 bytes
    ("pf", torch.uint8, True, 48),         # fp8 halves of 24 bytes
])
def test_fused_call_on_unaligned_rotary_scatters_then_rotates(dev, layout, dtype, neox, rotary_dim):
    """Rotated halves that are not 16-byte multiples: the fused call scatters
    and then rotates in place, to the oracle's bar."""
    fused_case(dev, layout, dtype, neox, rotary_dim, seed=21)


def inplace_case(dev, layout, dtype, neox, rotary_dim, nb=40, ps=16, h=4, d=64, L=3, seed=0, plan=None):
    """plan(perm) -> (block table, segments), given a permutation of the
    block ids; by default two requests' block lists with segments as
    apply_rerotate_load/multi plan them."""
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g) for _ in range(L)]
    pf = layers[0][1]
    perm = np.random.default_rng(seed).permutation(np.arange(0, nb)).tolist()
    if plan is not None:
        bt, segs = plan(perm)
    else:
        metas = [(0, 40, 0, perm[0:3]), (40, 70, 0, perm[3:5]), (70, 70, 5, perm[5:6]),
                 (100, 133, 7, perm[6:9])]
        bt, segs = orope.load_segments(metas)
        bt2, segs2 = orope.multi_segments([[0, 10, 25, 40, 60, 64]], [perm[10:14]])
        segs += [(o + len(bt), a, b, c) for (o, a, b, c) in segs2]
        bt = np.concatenate([bt, bt2]).astype(np.int32)
    inv = orope.default_inv_freq(rotary_dim, THETA)
    scales = None
    if dtype == torch.uint8:
        scales = (0.5 + torch.rand(L, h if layout != "mla" else 1, generator=g)).float()
    dev_layers = [to_dev(t, dev) for t, _ in layers]
    cpu_layers = [t for t, _ in layers]
    orope.rerotate_pages(cpu_layers, pf, bt, segs, inv, rotary_dim, neox,
                         None if scales is None else scales.numpy())
    cache_ops.rerotate_pages(dev_layers, pf, torch.from_numpy(bt).to(dev), segs,
                             torch.from_numpy(inv).to(dev), rotary_dim, neox,
                             None if scales is None else scales.to(dev))
    torch.cuda.synchronize()
    slots = []
    ps_ = orope.k_view(cpu_layers[0], pf, rotary_dim).shape[1]
    for o, ts, n, delta in segs:
        if delta != 0 and n > 0:
            slots += orope.segment_slots(bt, o, ts, n, ps_)
    worst = 0.0
    for t, td in zip(cpu_layers, dev_layers):
        mask, pn = rotation_region(t, pf, rotary_dim, slots, neox)
        worst = max(worst, assert_rotation_parity(td, t, mask, pn))
    return worst


# Shifts of long-context models, both signs: 128K positions and past 1M. The
# first pair's fp32 angle, shift x inv_freq[0] = shift, reaches 10^6 radians,
# where only sincosf's argument reduction keeps cos and sin accurate.
LONG_SHIFTS = (131071, -131072, 1048575, -1000003)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.uint8])
def test_fused_long_context_shifts(dev, dtype):
    fused_case(dev, "nhd", dtype, True, 128, nb=40, h=4, d=128, L=2, seed=31,
               chunk_tokens=(37, 64, 16, 5), deltas=LONG_SHIFTS)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.uint8])
@pytest.mark.parametrize("neox", [True, False])
def test_inplace_long_context_shifts(dev, dtype, neox):
    def plan(perm):
        # (bt_offset, tok_start, n_tokens, delta); the segments' slots are distinct
        segs = [(0, 0, 40, LONG_SHIFTS[0]), (3, 5, 20, LONG_SHIFTS[1]), (5, 0, 30, LONG_SHIFTS[2]),
                (7, 2, 9, LONG_SHIFTS[3])]
        return np.asarray([b for b in perm if b != 0][:8], dtype=np.int32), segs
    inplace_case(dev, "nhd", dtype, neox, 128, nb=24, d=128, L=2, seed=33, plan=plan)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.uint8])
@pytest.mark.parametrize("neox,rotary_dim", [(True, 256), (False, 256), (True, 128)])
def test_head_dim_256(dev, dtype, neox, rotary_dim):
    # 256-wide heads (512-byte bf16 rows), whole and half rotary
    fused_case(dev, "nhd", dtype, neox, rotary_dim, h=2, d=256, seed=35)
    inplace_case(dev, "hnd", dtype, neox, rotary_dim, h=2, d=256, L=2, seed=36)


@pytest.mark.parametrize("layout", ["nhd", "hnd", "pf", "packed", "mla"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.uint8])
def test_inplace_layouts(dev, layout, dtype):
    inplace_case(dev, layout, dtype, True, 64, d=64 if dtype != torch.uint8 else 128)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.uint8])
@pytest.mark.parametrize("neox", [True, False])
def test_inplace_item_path_padded_rows(dev, dtype, neox):
    # head rows followed by padding are not dense in the page: the 16-byte
    # item kernel runs instead of the page-tile kernel
    inplace_case(dev, "nhd_pad", dtype, neox, 64, d=64 if dtype != torch.uint8 else 128, seed=8)


@pytest.mark.parametrize("layout", ["nhd", "hnd"])
def test_inplace_large_pages(dev, layout):
    # 64-token pages of 8 heads x 128: 8192 units per page, several rounds per lane
    inplace_case(dev, layout, torch.bfloat16, True, 128, nb=24, ps=64, h=8, d=128, L=2, seed=9)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rotary_dim", [64, 24, 10])
def test_inplace_pairing_and_element_path(dev, neox, rotary_dim):
    # rotary_dim 24 / 10 take the per-element kernel (pairs not 16-byte aligned)
    inplace_case(dev, "nhd", torch.bfloat16, neox, rotary_dim, seed=5)


@pytest.mark.parametrize("neox", [True, False])
def test_inplace_fp8_element_path(dev, neox):
    # rotary_dim 24 on fp8: pair halves of 12 bytes take the per-element kernel
    inplace_case(dev, "nhd", torch.uint8, neox, 24, d=128, seed=6)


def test_fp8_identity_rotation_is_exact(dev):
    # inv_freq = 0 gives cos = 1, sin = 0: dequant -> rotate -> requant must
    # return every finite code's value unchanged (scale 1 and a non-power-of-two
    # scale); -0 may come back as +0 (x1*1 - (-0) is +0 in IEEE arithmetic)
    codes = torch.tensor([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=torch.uint8)
    n = codes.numel()
    ps, h, d, nb = 16, 2, 64, 4
    layer = torch.zeros(2, nb, ps, h, d, dtype=torch.uint8)
    k = layer[0, 1].reshape(-1)
    k[: n * 8] = codes.repeat(8)
    for scale in (1.0, 0.3):
        ld = layer.to(dev)
        bt = torch.tensor([1], dtype=torch.int32, device=dev)
        cache_ops.rerotate_pages([ld], False, bt, [(0, 0, ps, 100)], torch.zeros(32, device=dev), 64, True,
                                 torch.full((1, h), scale, device=dev))
        torch.cuda.synchronize()
        got = ld.cpu()
        canon = lambda t: torch.where(t == 0x80, torch.zeros_like(t), t)  # noqa: E731
        diff = (canon(got) != canon(layer)).nonzero()
        pairs = [(int(layer[tuple(i)]), int(got[tuple(i)])) for i in diff[:12].tolist()]
        assert len(diff) == 0, f"scale {scale}: {len(diff)} codes changed, (in, out): {pairs}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_identity_rotation_is_exact_16bit(dev, dtype):
    # cos = 1, sin = 0: every element must come back bit-identical
    g = torch.Generator().manual_seed(9)
    layer = torch.randn(2, 4, 16, 2, 64, generator=g).to(dtype)
    ld = layer.to(dev)
    bt = torch.tensor([1, 2], dtype=torch.int32, device=dev)
    cache_ops.rerotate_pages([ld], False, bt, [(0, 0, 32, 100)], torch.zeros(32, device=dev), 64, True)
    torch.cuda.synchronize()
    got = ld.cpu()
    bad = (got.view(torch.int16) != layer.view(torch.int16)).nonzero()
    pairs = [(float(layer[tuple(i)]), float(got[tuple(i)])) for i in bad[:8].tolist()]
    assert len(bad) == 0, f"{len(bad)} elements changed, (in, out): {pairs}"
