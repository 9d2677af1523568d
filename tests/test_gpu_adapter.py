"""Adapter counterpart end to end on the GPU: apply_rerotate_load (all layers
and layerwise) and apply_rerotate_multi on fake metas and fake rotary
embeddings. The expected K rows are built the way the reference builds its
angles, from the rotary module's own cos_sin_cache (combined rows of
adapter.py:271-283 for loads, the shift's row of adapter.py:147-150, 176-181
for multi), in float64, and the slots the reference's planning
(adapter.py:118-295) names."""
import numpy as np
import pytest
import torch

from daric_amd import adapter as ad
from oracle import rope as orope
from tests import adapter_fakes as afakes
from tests.adapter_fakes import FakeMeta, FakeRotary
from tests.gpu_util import assert_rotation_parity, make_layer, rotation_region, to_dev

pytestmark = pytest.mark.gpu

MAX_POS = 2048


def build(dev, layout, dtype, neox, R=64, L=3, nb=48, seed=0, rot=None):
    g = torch.Generator().manual_seed(seed)
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    cpu = {}
    pf = False
    for n in names:
        t, pf = make_layer(layout, nb, 16, 4, 64, dtype, g)
        cpu[n] = t
    topo = ad.CacheTopo(layers={n: ad.LayerCacheTopo(0, 16, 1, pf) for n in names}, groups=[names])
    cfg = ad.AdaptionConfig(rerotate=True, recompute=True, recompute_policy="daric", recompute_avg_num=16)
    a = ad.Adapter(cfg, topo)
    a.register_kvcaches({n: to_dev(t, dev) for n, t in cpu.items()})
    if rot is None:
        rot = FakeRotary(R, is_neox_style=neox, max_pos=MAX_POS)
    for n in names:
        a.register_rotary_embed(n, rot)
    return a, names, cpu, pf, rot


def check(a, names, cpu, pf, rot, moves, layer_subset=None):
    """moves: (slots, cos, sin, largest |position| behind the angles)."""
    torch.cuda.synchronize()
    subset = names if layer_subset is None else layer_subset
    slots = []
    top = 1
    for sl, c, s, p in moves:
        for n in subset:
            orope.rotate_slots_cs(cpu[n], pf, sl, c, s, rot.rotary_dim, rot.is_neox_style)
        slots += list(sl)
        top = max(top, p)
    # the table's angles are float32 products p * inv_freq[i] (|inv_freq| <= 1),
    # rounded once per table row; the kernel's is one float32 product per shift
    angle_tol = 2.0 ** -22 * (3 * top + 4)
    for n in names:
        want = cpu[n]
        mask, pn = rotation_region(want, pf, rot.rotary_dim, slots if n in subset else [],
                                   rot.is_neox_style)
        assert_rotation_parity(a.kvcaches[n], want, mask, pn, angle_tol=angle_tol)


def load_moves(metas, table, ps):
    """(slots, cos, sin, top position) of apply_rerotate_load's metas."""
    out = []
    for m in metas:
        n = int(m.ptr[1] - m.ptr[0])
        if n <= 0 or int(m.saved_pos) == int(m.ptr[0]):
            continue
        j = np.arange(n)
        old, new = int(m.saved_pos) + j, int(m.ptr[0]) + j
        c, s = orope.table_cos_sin_load(table, old, new)
        out.append((orope.segment_slots(m.block_ids[0], 0, 0, n, ps), c, s, max(old.max(), new.max())))
    return out


def multi_moves(ptrs, blocks, table, ps):
    bt, segs = orope.multi_segments(ptrs, [b[0] for b in blocks])
    out = []
    for o, ts, n, d in segs:
        c, s = orope.table_cos_sin_multi(table, [d] * n)
        out.append((orope.segment_slots(bt, o, ts, n, ps), c, s, abs(d)))
    return out


def five_metas():
    perm = np.random.default_rng(1).permutation(np.arange(1, 48)).tolist()
    return [FakeMeta("a", [0, 40], 0, (perm[0:3],)), FakeMeta("b", [40, 70], 3, (perm[3:5],)),
            FakeMeta("c", [70, 70], 9, (perm[5:6],)), FakeMeta("d", [70, 103], 70, (perm[6:9],)),
            FakeMeta("e", [103, 160], 1000, (perm[9:13],))]


@pytest.mark.parametrize("layout,dtype,neox", [("nhd", torch.bfloat16, True),
                                               ("pf", torch.float16, False),
                                               ("packed", torch.bfloat16, True),
                                               ("nhd", torch.uint8, True),     # fp8 (e4m3) caches
                                               ("pf", torch.uint8, False)])
def test_apply_rerotate_load(dev, layout, dtype, neox):
    a, names, cpu, pf, rot = build(dev, layout, dtype, neox)
    metas = five_metas()
    a.apply_rerotate_load(metas)
    check(a, names, cpu, pf, rot, load_moves(metas, rot.cos_sin_cache, 16))


def test_apply_rerotate_load_layerwise(dev):
    a, names, cpu, pf, rot = build(dev, "nhd", torch.bfloat16, True)
    metas = [FakeMeta("a", [16, 50], 0, ([5, 9, 12],))]
    a.apply_rerotate_load(metas, layer_name=names[1])
    check(a, names, cpu, pf, rot, load_moves(metas, rot.cos_sin_cache, 16), layer_subset=[names[1]])


def test_apply_rerotate_multi(dev):
    a, names, cpu, pf, rot = build(dev, "nhd", torch.bfloat16, True)
    ptrs = [[0, 10, 25, 40, 60, 64], [100, 120, 130], [0, 16, 16, 47, 80]]
    blocks = [([3, 4, 5, 6],), ([7, 8],), ([9, 10, 11, 12, 13],)]
    a.apply_rerotate_multi(ptrs, blocks)
    check(a, names, cpu, pf, rot, multi_moves(ptrs, blocks, rot.cos_sin_cache, 16))


@pytest.mark.parametrize("table_dtype", [torch.float32, torch.bfloat16])
def test_yarn_form_table_with_its_own_scale(dev, table_dtype):
    """A YaRN-form module (frequencies from _compute_inv_freq(scaling_factor),
    table scaled by m = 1.25, bf16 or fp32 table): rows move by the table's
    angles and keep their norm."""
    rot = afakes.MScaleRotary(64, max_pos=MAX_POS, dtype=table_dtype)
    a, names, cpu, pf, rot = build(dev, "nhd", torch.bfloat16, True, rot=rot)
    metas = five_metas()
    a.apply_rerotate_load(metas)
    # the expected angles come from the fp32 form of the same table (a bf16
    # table's own rounding, 2^-9, would swamp the comparison)
    table = afakes.MScaleRotary(64, max_pos=MAX_POS).cos_sin_cache
    check(a, names, cpu, pf, rot, load_moves(metas, table, 16))


@pytest.mark.parametrize("cls", [afakes.ScaledPositionsRotary, afakes.OtherBaseRotary])
def test_tables_the_kernels_cannot_reproduce_are_refused(dev, cls):
    a, names, cpu, pf, rot = build(dev, "nhd", torch.bfloat16, True, rot=cls(64, max_pos=MAX_POS))
    with pytest.raises(ValueError, match=cls.__name__):
        a.apply_rerotate_load(five_metas())
    torch.cuda.synchronize()
    for n in names:
        assert torch.equal(a.kvcaches[n].cpu(), cpu[n])
