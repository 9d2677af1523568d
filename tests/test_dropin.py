"""The drop-in boundary seen from the reference's own call sites (CPU only).

- `daric_amd.cache_ops` serves the signatures the reference's type stub
  declares (daric/cache_ops.pyi:6-53): parameter names, order, kinds,
  defaults and annotations, against tests/golden/cache_ops_pyi_signatures.json
  (written from the stub by tests/golden/make_pyi_signatures.py);
- the drop-in files (daric_amd/dropin/) installed as daric/cache_ops.py and
  daric/adaption/adapter.py in a stand-in `daric` package are imported the way
  the reference imports them (gpu_kv_io.py:9, adaption/__init__.py,
  cache_engine.py:12, 260);
- Adapter(config) takes the layer topology from
  daric.configs.ProcessLocalConfig.cache_topo, reads it at each use, and
  raises at construction when there is none;
- bad cache layouts raise ValueError with the reference's text
  (adapter.py:20-27, 336-368), before any layer is rotated.
"""
import inspect
import json
import os
import shutil
import subprocess
import sys
import types

import pytest
import torch

from daric_amd import adapter as ad
from daric_amd import cache_ops
from tests.adapter_fakes import FakeMeta, FakeRotary

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden", "cache_ops_pyi_signatures.json")
DROPIN = os.path.join(ROOT, "daric_amd", "dropin")


def signature_record(obj):
    sig = inspect.signature(obj)
    params = []
    for p in sig.parameters.values():
        has = p.default is not inspect.Parameter.empty
        params.append({
            "name": p.name,
            "kind": p.kind.name,
            "has_default": has,
            "default": p.default if has else None,
            "annotation": None if p.annotation is inspect.Parameter.empty else str(p.annotation),
        })
    ret = None if sig.return_annotation is inspect.Signature.empty else str(sig.return_annotation)
    return {"params": params, "returns": ret}


def resolve(module, dotted):
    obj = module
    for part in dotted.split("."):
        obj = getattr(obj, part)
    return obj


def test_signatures_match_reference_stub():
    golden = json.load(open(GOLDEN))["signatures"]
    assert set(golden) == {"CacheCopier.__init__", "CacheCopier.register_layer",
                           "CacheCopier.register_store", "CacheCopier.gather_pages",
                           "CacheCopier.scatter_pages", "batched_memcpy_d2h", "batched_memcpy_h2d"}
    for name, want in golden.items():
        got = signature_record(resolve(cache_ops, name))
        assert got == want, name


def test_dropin_modules_reexport_the_implementation():
    from daric_amd import host_runtime
    from daric_amd.dropin import adapter as dad
    from daric_amd.dropin import cache_ops as dco
    from daric_amd.dropin import gpu_runtime as dgr
    for name in ("CacheCopier", "batched_memcpy_d2h", "batched_memcpy_h2d", "rerotate_pages",
                 "kv_deviation", "topk_per_chunk", "merge_rows", "select_merge"):
        assert getattr(dco, name) is getattr(cache_ops, name)
    assert dad.Adapter is ad.Adapter
    # the names daric/utils/__init__.py:17 imports from gpu_runtime
    assert dgr.get_gpu_host_runtime is host_runtime.get_gpu_host_runtime
    assert dgr.HOST_MEMORY_ALREADY_REGISTERED == 712


STANDIN_CONFIGS = '''
from daric_amd.adapter import AdaptionConfig, CacheTopo, LayerCacheTopo


class ProcessLocalConfig:
    block_size: int
    cache_topo: CacheTopo
'''

IMPORT_SCRIPT = r'''
import json, sys
sys.path[:0] = [TREE, REPO]
from daric import cache_ops                       # gpu_kv_io.py:9 (package-relative there)
from daric.adaption import Adapter                # cache_engine.py:12
from daric.configs import AdaptionConfig, CacheTopo, LayerCacheTopo, ProcessLocalConfig
from daric.utils import get_gpu_host_runtime, HOST_MEMORY_ALREADY_REGISTERED   # gpu_kv_io.py:9-18
import daric_amd.adapter, daric_amd.cache_ops
names = ["model.layers.1.attn", "model.layers.0.attn", "model.layers.2.attn"]
ProcessLocalConfig.cache_topo = CacheTopo(
    layers={n: LayerCacheTopo(0, 16, 1, False) for n in names}, groups=[names])
cfg = AdaptionConfig(rerotate=True, recompute=True, recompute_policy="daric", recompute_avg_num=32)
a = Adapter(cfg)                                   # cache_engine.py:260
print(json.dumps({
    "copier": cache_ops.CacheCopier is daric_amd.cache_ops.CacheCopier,
    "memcpy": cache_ops.batched_memcpy_d2h is daric_amd.cache_ops.batched_memcpy_d2h,
    "adapter": Adapter is daric_amd.adapter.Adapter,
    "num_layers": a.num_layers,
    "topo": a.cache_topo is ProcessLocalConfig.cache_topo,
    "host_runtime": get_gpu_host_runtime().prefix,
    "already_registered": HOST_MEMORY_ALREADY_REGISTERED,
}))
'''


def test_dropin_files_import_like_the_reference(tmp_path):
    tree = tmp_path / "tree"
    pkg = tree / "daric"
    (pkg / "adaption").mkdir(parents=True)
    (pkg / "configs").mkdir()
    (pkg / "utils").mkdir()
    (pkg / "__init__.py").write_text("")
    shutil.copy(os.path.join(DROPIN, "cache_ops.py"), pkg / "cache_ops.py")
    shutil.copy(os.path.join(DROPIN, "gpu_runtime.py"), pkg / "utils" / "gpu_runtime.py")
    # the reference's utils/__init__.py:17 import
    (pkg / "utils" / "__init__.py").write_text(
        "from .gpu_runtime import get_gpu_host_runtime, HOST_MEMORY_ALREADY_REGISTERED\n")
    shutil.copy(os.path.join(DROPIN, "adapter.py"), pkg / "adaption" / "adapter.py")
    (pkg / "adaption" / "__init__.py").write_text("from .adapter import Adapter\n")
    (pkg / "configs" / "__init__.py").write_text(STANDIN_CONFIGS)
    script = f"TREE = {str(tree)!r}\nREPO = {ROOT!r}\n" + IMPORT_SCRIPT
    r = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out == {"copier": True, "memcpy": True, "adapter": True, "num_layers": 3, "topo": True,
                   "host_runtime": "hip", "already_registered": 712}


# ------------------------------------------------------------------ Adapter(config)
class Recorder:
    def __init__(self):
        self.calls = []

    def __call__(self, layers, page_first, block_table, segments, inv_freq, rotary_dim,
                 is_neox_style=True, k_scales=None, stream=0):
        self.calls.append(dict(n_layers=len(layers), page_first=page_first, segs=list(segments),
                               bt=block_table.tolist()))


@pytest.fixture
def process_local(monkeypatch):
    """A stand-in daric.configs whose ProcessLocalConfig carries cache_topo."""
    pkg = types.ModuleType("daric")
    pkg.__path__ = []
    configs = types.ModuleType("daric.configs")

    class ProcessLocalConfig:
        pass

    configs.ProcessLocalConfig = ProcessLocalConfig
    pkg.configs = configs
    monkeypatch.setitem(sys.modules, "daric", pkg)
    monkeypatch.setitem(sys.modules, "daric.configs", configs)
    return ProcessLocalConfig


def config(rerotate=True):
    return ad.AdaptionConfig(rerotate=rerotate, recompute=True, recompute_policy="daric",
                             recompute_avg_num=32, function="linear", r=0.5)


def topology(names, page_first=False):
    return ad.CacheTopo(layers={n: ad.LayerCacheTopo(0, 16, 1, page_first) for n in names},
                        groups=[list(names)])


def test_adapter_reads_process_local_topology(process_local, monkeypatch):
    names = [f"model.layers.{i}.self_attn.attn" for i in range(3)]
    process_local.cache_topo = topology(names)
    rec = Recorder()
    monkeypatch.setattr(ad.cache_ops, "rerotate_pages", rec)
    a = ad.Adapter(config())                      # as cache_engine.py:260 builds it
    assert a.num_layers == 3 and not a.register_done()
    a.register_kvcaches({n: torch.zeros(2, 8, 16, 2, 32, dtype=torch.bfloat16) for n in names})
    rot = FakeRotary(32)
    for n in names:
        a.register_rotary_embed(n, rot)
    assert a.register_done()
    metas = [FakeMeta("a", [0, 20], 100, ([3, 4],))]
    a.apply_rerotate_load(metas)
    assert len(rec.calls) == 1 and rec.calls[0]["n_layers"] == 3
    assert rec.calls[0]["segs"] == [(0, 0, 20, -100)] and not rec.calls[0]["page_first"]
    # finish_register_process_local_config (integration/vllm/utils.py:212-220) sets
    # page_first after the Adapter exists; the Adapter must see it
    for n in names:
        process_local.cache_topo.layers[n].page_first = True
    a.register_kvcaches({n: torch.zeros(8, 2, 16, 2, 32, dtype=torch.bfloat16) for n in names})
    rec.calls.clear()
    a.apply_rerotate_load(metas)
    assert len(rec.calls) == 1 and rec.calls[0]["page_first"]
    # a topology object replaced later is read too
    process_local.cache_topo = ad.CacheTopo(layers=dict(process_local.cache_topo.layers), groups=[])
    with pytest.raises(ValueError, match="not found in any group"):
        a.apply_rerotate_load(metas)


def test_adapter_without_topology_fails_at_construction(monkeypatch):
    monkeypatch.setitem(sys.modules, "daric.configs", None)      # not importable
    with pytest.raises(RuntimeError, match="cache_topo"):
        ad.Adapter(config())
    # an explicit topology needs no DARIC package
    assert ad.Adapter(config(), topology(["x"])).num_layers == 1


def test_adapter_with_unset_process_local_topology(process_local):
    with pytest.raises(RuntimeError, match="not set yet"):
        ad.Adapter(config())


# ------------------------------------------------------------------ ValueError cases
def adapter_with(kv: dict, page_first: bool, rotary_dim: int = 16):
    names = list(kv)
    a = ad.Adapter(config(), topology(names, page_first))
    a.register_kvcaches(kv)
    rot = FakeRotary(rotary_dim)
    for n in names:
        a.register_rotary_embed(n, rot)
    return a


LOAD = [FakeMeta("a", [0, 20], 100, ([3, 4],))]


@pytest.mark.parametrize("shape,stride,page_first,rd,why", [
    ((8, 2, 4, 32), None, False, 16, "page_first must be true"),
    ((8, 2, 4, 31), None, True, 16, "packed content dimension must be positive and even"),
    ((8, 2, 4, 32), (512, 256, 64, 2), True, 16, "packed content feature stride must equal 1"),
    ((8, 2, 4, 32), None, True, 18,
     "rotary_dim must be positive, even, and no greater than the packed K head dimension"),
])
def test_packed_layout_errors_are_value_errors(monkeypatch, shape, stride, page_first, rd, why):
    rec = Recorder()
    monkeypatch.setattr(ad.cache_ops, "rerotate_pages", rec)
    good = torch.zeros(8, 2, 4, 32, dtype=torch.bfloat16)
    if stride is None:
        bad = torch.zeros(shape, dtype=torch.bfloat16)
    else:
        bad = torch.zeros(8 * 512, dtype=torch.bfloat16).as_strided(shape, stride)
    a = adapter_with({"L0": good, "L1": bad}, page_first, rd)
    want = (f"Invalid 4D KV cache for rerotate: layer=L1, shape={shape}, stride={tuple(bad.stride())}, "
            f"dtype=torch.bfloat16, rotary_dim={rd}, constraint={why}")
    if why == "page_first must be true" or rd > 16:
        want = want.replace("layer=L1", "layer=L0").replace(f"stride={tuple(bad.stride())}",
                                                            f"stride={tuple(good.stride())}")
    with pytest.raises(ValueError) as ei:
        a.apply_rerotate_load(LOAD)
    assert str(ei.value) == want
    assert rec.calls == []            # nothing rotated before the failing layer


def test_packed_layout_error_literal():
    kv = torch.zeros(8, 2, 4, 32, dtype=torch.float16)
    with pytest.raises(ValueError) as ei:
        ad.check_rerotate_layout("model.layers.7.attn", kv, False, 16)
    assert str(ei.value) == ("Invalid 4D KV cache for rerotate: layer=model.layers.7.attn, "
                             "shape=(8, 2, 4, 32), stride=(256, 128, 32, 1), dtype=torch.float16, "
                             "rotary_dim=16, constraint=page_first must be true")


def test_unsupported_rank_is_value_error(monkeypatch):
    rec = Recorder()
    monkeypatch.setattr(ad.cache_ops, "rerotate_pages", rec)
    a = adapter_with({"L0": torch.zeros(8, 64, dtype=torch.bfloat16)}, True)
    with pytest.raises(ValueError) as ei:
        a.apply_rerotate_load(LOAD)
    assert str(ei.value) == "Unsupported KV cache rank for rerotate: 2"
    # nothing to rotate: the reference returns before looking at the layout
    a.apply_rerotate_load([FakeMeta("b", [0, 20], 0, ([3, 4],))])
    a.apply_rerotate_multi([[0, 10, 20]], [([1, 2],)])
    assert rec.calls == []


def test_good_layouts_pass():
    for kv, pf in ((torch.zeros(8, 2, 4, 32), True), (torch.zeros(2, 8, 4, 2, 16), False),
                   (torch.zeros(8, 2, 4, 2, 16), True), (torch.zeros(8, 4, 64), True)):
        ad.check_rerotate_layout("L", kv, pf, 16)
