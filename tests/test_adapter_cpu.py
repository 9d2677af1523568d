"""Adapter counterpart, host side: segment planning against the oracle's
restatement of apply_rerotate_load/multi (reference adapter.py:118-295),
layer batching by group and geometry, the rerotate/recompute switches."""
import math

import numpy as np
import pytest
import torch

from daric_amd import adapter as ad
from daric_amd.policy import DARICPolicy
from oracle import rope as orope
from tests import adapter_fakes as afakes
from tests.adapter_fakes import FakeMeta, FakeRotary


def test_load_planning_matches_oracle():
    rng = np.random.default_rng(3)
    metas, raw = [], []
    pos = 0
    for i in range(12):
        n = int(rng.integers(0, 70))
        saved = int(rng.choice([pos, 0, 5, pos + 3]))
        blocks = rng.permutation(np.arange(1, 400))[: -(-n // 16) or 1].tolist()
        metas.append(FakeMeta(f"c{i}", [pos, pos + n], saved, (blocks, [b + 1000 for b in blocks])))
        raw.append((pos, pos + n, saved, blocks))
        pos += n
    bt, segs = ad.plan_load_segments(metas, 0)
    obt, osegs = orope.load_segments(raw)
    assert bt.tolist() == obt.tolist() and segs == osegs
    bt1, segs1 = ad.plan_load_segments(metas, 1)     # second KV-cache group: its own block lists
    assert bt1.tolist() == [b + 1000 for b in obt.tolist()] and segs1 == osegs


@pytest.mark.parametrize("form", ["list", "tuple", "numpy", "tensor", "nested", "mixed"])
def test_planning_takes_every_block_list_form(form):
    """Block lists as lists, tuples, numpy arrays, torch tensors, nested lists
    or a mix plan the same block table as plain lists."""
    lists = [[5, 9, 12], [3], [40, 41], [7, 8, 6, 2]]

    def as_form(i, b):
        f = form if form != "mixed" else ["list", "numpy", "tensor", "tuple"][i % 4]
        return {"list": list(b), "tuple": tuple(b), "numpy": np.asarray(b, dtype=np.int64),
                "tensor": torch.tensor(b, dtype=torch.int32), "nested": [[x] for x in b]}[f]

    metas = [FakeMeta(f"c{i}", [16 * i, 16 * i + 10], 3 + i, (as_form(i, b),)) for i, b in enumerate(lists)]
    ref = [FakeMeta(f"c{i}", [16 * i, 16 * i + 10], 3 + i, (b,)) for i, b in enumerate(lists)]
    bt, segs = ad.plan_load_segments(metas, 0)
    rbt, rsegs = ad.plan_load_segments(ref, 0)
    assert bt.dtype == np.int32 and bt.tolist() == rbt.tolist() == sum(lists, []) and segs == rsegs
    ptrs = [[0, 4, 9, 20, 30]] * len(lists)
    bt, segs = ad.plan_multi_segments(ptrs, [(as_form(i, b),) for i, b in enumerate(lists)], 0)
    rbt, rsegs = ad.plan_multi_segments(ptrs, [(b,) for b in lists], 0)
    assert bt.dtype == np.int32 and bt.tolist() == rbt.tolist() and segs == rsegs


def test_multi_planning_matches_oracle():
    ptrs = [[10, 20, 30, 45, 50], [0, 5, 9], [0, 16, 16, 40, 64, 80]]
    blocks = [([1, 2, 3, 4],), ([9],), ([5, 6, 7, 8, 11],)]
    bt, segs = ad.plan_multi_segments(ptrs, blocks, 0)
    obt, osegs = orope.multi_segments(ptrs, [b[0] for b in blocks])
    assert bt.tolist() == obt.tolist() and segs == osegs


class Recorder:
    def __init__(self):
        self.calls = []

    def __call__(self, layers, page_first, block_table, segments, inv_freq, rotary_dim,
                 is_neox_style=True, k_scales=None, stream=0):
        self.calls.append(dict(n_layers=len(layers), page_first=page_first,
                               bt=block_table.tolist(), segs=list(segments),
                               inv=inv_freq.tolist(), R=rotary_dim, neox=is_neox_style))


def make_adapter(rerotate=True, policy="daric"):
    names = [f"model.layers.{i}.self_attn.attn" for i in range(4)]
    topo = ad.CacheTopo(layers={n: ad.LayerCacheTopo(0 if i < 3 else 1, 16, 1, False)
                                for i, n in enumerate(names)},
                        groups=[names[:3], names[3:]])
    cfg = ad.AdaptionConfig(rerotate=rerotate, recompute=True, recompute_policy=policy,
                            recompute_avg_num=32, function="linear", r=0.5)
    a = ad.Adapter(cfg, topo)
    kv = {n: torch.zeros(2, 8, 16, 2, 32, dtype=torch.bfloat16) for n in names}
    kv[names[2]] = torch.zeros(2, 8, 16, 2, 64, dtype=torch.bfloat16)   # different geometry
    a.register_kvcaches(kv)
    rot = FakeRotary(32)
    for n in names:
        a.register_rotary_embed(n, rot)
    return a, names


def test_batching_by_group_and_geometry(monkeypatch):
    rec = Recorder()
    monkeypatch.setattr(ad.cache_ops, "rerotate_pages", rec)
    a, names = make_adapter()
    assert a.register_done()
    metas = [FakeMeta("a", [0, 20], 100, ([3, 4], [7, 8])), FakeMeta("b", [20, 30], 20, ([5], [9]))]
    a.apply_rerotate_load(metas)
    # group 0: two geometries -> two calls; group 1: one call; meta "b" is not moved
    assert sorted(c["n_layers"] for c in rec.calls) == [1, 1, 2]
    for c in rec.calls:
        assert c["segs"] == [(0, 0, 20, -100)]
        assert c["bt"] in ([3, 4], [7, 8])
        assert c["R"] == 32 and c["neox"] and not c["page_first"]
        np.testing.assert_allclose(c["inv"], FakeRotary(32)._compute_inv_freq(500000.0).numpy())
    rec.calls.clear()
    a.apply_rerotate_load(metas, layer_name=names[3])          # layerwise load
    assert len(rec.calls) == 1 and rec.calls[0]["bt"] == [7, 8]


def test_switches(monkeypatch):
    rec = Recorder()
    monkeypatch.setattr(ad.cache_ops, "rerotate_pages", rec)
    a, _ = make_adapter(rerotate=False, policy=None)
    a.apply_rerotate_load([FakeMeta("a", [0, 20], 100, ([3, 4], [7, 8]))])
    a.apply_rerotate_multi([[0, 10, 20, 30]], [([1, 2], [3, 4])])
    assert rec.calls == [] and a.get_recompute_length([0, 10, 20]) == []
    b, _ = make_adapter()
    ptr = [0, 256, 512, 768, 1024]
    assert b.get_recompute_length(ptr) == DARICPolicy(32, 0.5, "linear").get_recompute_ptrs(ptr)
    b.apply_rerotate_multi([[0, 10, 20]], [([1, 2], [3, 4])])   # two groups: nothing moves
    assert rec.calls == []


def test_inv_freq_source():
    r = FakeRotary(64)
    np.testing.assert_array_equal(ad._inv_freq(r).numpy(), r._compute_inv_freq(r.base).numpy())

    class Bare:
        rotary_dim, is_neox_style = 8, True
    with pytest.raises(ValueError, match="Bare: rotary embedding has no .* cos_sin_cache"):
        ad._inv_freq(Bare())


@pytest.mark.parametrize("max_pos,dtype", [(64, torch.float32), (131072, torch.float32),
                                           (131072, torch.bfloat16), (8192, torch.float16)])
def test_inv_freq_accepts_the_default_table(max_pos, dtype):
    r = FakeRotary(128, max_pos=max_pos, dtype=dtype)
    np.testing.assert_array_equal(ad._inv_freq(r).numpy(), r._compute_inv_freq(r.base).numpy())


@pytest.mark.parametrize("max_pos", [64, 8192, 131072])
def test_inv_freq_refuses_tables_of_scaled_positions_or_another_base(max_pos):
    """Tables the kernels' angle float32(d) * inv_freq cannot reproduce: the
    re-rotation raises ValueError naming the class instead of rotating by
    another angle."""
    with pytest.raises(ValueError, match="ScaledPositionsRotary: rotary cos_sin_cache is not"):
        ad._inv_freq(afakes.ScaledPositionsRotary(128, max_pos=max_pos))
    with pytest.raises(ValueError, match="OtherBaseRotary: rotary cos_sin_cache is not"):
        ad._inv_freq(afakes.OtherBaseRotary(128, max_pos=max_pos, dtype=torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_inv_freq_accepts_a_scaled_table_of_yarn_form(dtype):
    """m = cos_sin_cache[0, 0] = 1.25 is the table's own scale; the frequencies
    come from _compute_inv_freq(scaling_factor) (YaRN's signature) after
    _compute_inv_freq(base) fails the check."""
    r = afakes.MScaleRotary(64, max_pos=16384, dtype=dtype)
    np.testing.assert_array_equal(ad._inv_freq(r).numpy(), r._compute_inv_freq(r.scaling_factor).numpy())


def test_inv_freq_check_catches_small_frequency_errors():
    """A candidate off by one part in 10^5 drifts past the tolerance by the
    table's last positions and is passed over; one off by a whole turn (2*pi)
    is the same rotation at every integer position and is accepted."""
    r = FakeRotary(64, max_pos=131072)
    good = r._compute_inv_freq(r.base)
    r.inv_freq = good * (1 + 1e-5)
    np.testing.assert_array_equal(ad._inv_freq(r).numpy(), good.numpy())   # _compute_inv_freq(base)
    r.base = 400000.0                                                      # now no candidate fits
    with pytest.raises(ValueError, match=r"tried: inv_freq, _compute_inv_freq\(base\)"):
        ad._inv_freq(r)
    r3 = FakeRotary(64, max_pos=4096)
    r3.inv_freq = good + 2 * math.pi
    assert torch.equal(ad._inv_freq(r3), (good + 2 * math.pi).float())


def test_table_positions_cover_every_power_of_two():
    pos = ad._table_positions(131072)
    assert pos[:4] == [0, 1, 2, 3] and pos[-1] == 131071
    assert all((1 << k) in pos for k in range(17))
    assert ad._table_positions(1) == [0]


def test_rotation_refused_before_any_layer_moves(monkeypatch):
    rec = Recorder()
    monkeypatch.setattr(ad.cache_ops, "rerotate_pages", rec)
    a, names = make_adapter()
    a.rotary_embeds[names[3]] = afakes.OtherBaseRotary(32)
    metas = [FakeMeta("a", [0, 20], 100, ([3, 4], [7, 8]))]
    with pytest.raises(ValueError, match="OtherBaseRotary"):
        a.apply_rerotate_load(metas)
    assert rec.calls == []


def test_rotary_inv_freq_is_the_checked_vector():
    r = afakes.MScaleRotary(64, max_pos=4096)
    assert torch.equal(ad.rotary_inv_freq(r), ad._inv_freq(r))
    with pytest.raises(ValueError, match="OtherBaseRotary"):
        ad.rotary_inv_freq(afakes.OtherBaseRotary(64, max_pos=4096))
