"""Adapter counterpart end to end on the GPU: apply_rerotate_load (all layers
and layerwise) and apply_rerotate_multi on fake metas and a fake rotary
embedding, against the oracle's rotation of the slots the reference's
planning (adapter.py:118-295) names."""
import numpy as np
import pytest
import torch

from daric_amd import adapter as ad
from oracle import rope as orope
from tests.adapter_fakes import FakeMeta, FakeRotary
from tests.gpu_util import assert_rotation_parity, make_layer, rotation_region, to_dev

pytestmark = pytest.mark.gpu


def build(dev, layout, dtype, neox, R=64, L=3, nb=48, seed=0):
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
    rot = FakeRotary(R, is_neox_style=neox)
    for n in names:
        a.register_rotary_embed(n, rot)
    return a, names, cpu, pf, rot


def check(a, names, cpu, pf, rot, bt, segs, layer_subset=None):
    inv = rot._compute_inv_freq(rot.base).numpy().astype(np.float32)
    subset = names if layer_subset is None else layer_subset
    orope.rerotate_pages([cpu[n] for n in subset], pf, bt, segs, inv, rot.rotary_dim, rot.is_neox_style)
    torch.cuda.synchronize()
    ps = orope.k_view(cpu[names[0]], pf, rot.rotary_dim).shape[1]
    slots = []
    for o, ts, n, d in segs:
        if d != 0 and n > 0:
            slots += orope.segment_slots(bt, o, ts, n, ps)
    for n in names:
        want = cpu[n]
        mask, pn = rotation_region(want, pf, rot.rotary_dim, slots if n in subset else [],
                                   rot.is_neox_style)
        assert_rotation_parity(a.kvcaches[n], want, mask, pn)


@pytest.mark.parametrize("layout,dtype,neox", [("nhd", torch.bfloat16, True),
                                               ("pf", torch.float16, False),
                                               ("packed", torch.bfloat16, True)])
def test_apply_rerotate_load(dev, layout, dtype, neox):
    a, names, cpu, pf, rot = build(dev, layout, dtype, neox)
    perm = np.random.default_rng(1).permutation(np.arange(1, 48)).tolist()
    metas = [FakeMeta("a", [0, 40], 0, (perm[0:3],)), FakeMeta("b", [40, 70], 3, (perm[3:5],)),
             FakeMeta("c", [70, 70], 9, (perm[5:6],)), FakeMeta("d", [70, 103], 70, (perm[6:9],)),
             FakeMeta("e", [103, 160], 1000, (perm[9:13],))]
    a.apply_rerotate_load(metas)
    bt, segs = orope.load_segments([(m.ptr[0], m.ptr[1], m.saved_pos, m.block_ids[0]) for m in metas])
    check(a, names, cpu, pf, rot, bt, segs)


def test_apply_rerotate_load_layerwise(dev):
    a, names, cpu, pf, rot = build(dev, "nhd", torch.bfloat16, True)
    metas = [FakeMeta("a", [16, 50], 0, ([5, 9, 12],))]
    a.apply_rerotate_load(metas, layer_name=names[1])
    bt, segs = orope.load_segments([(16, 50, 0, [5, 9, 12])])
    check(a, names, cpu, pf, rot, bt, segs, layer_subset=[names[1]])


def test_apply_rerotate_multi(dev):
    a, names, cpu, pf, rot = build(dev, "nhd", torch.bfloat16, True)
    ptrs = [[0, 10, 25, 40, 60, 64], [100, 120, 130], [0, 16, 16, 47, 80]]
    blocks = [([3, 4, 5, 6],), ([7, 8],), ([9, 10, 11, 12, 13],)]
    a.apply_rerotate_multi(ptrs, blocks)
    bt, segs = orope.multi_segments(ptrs, [b[0] for b in blocks])
    check(a, names, cpu, pf, rot, bt, segs)
