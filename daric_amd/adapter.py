"""Counterpart of the reference's Adapter (daric/adaption/adapter.py:90-402)
on the gfx950 kernels: same methods, same arguments, same call sites
(daric/integration/vllm/worker.py:217, 230-231, 280, 321).

The reference launches one Triton program per (token, head) and one launch
per layer, after building per-token combined cos/sin tables with torch ops.
Here every re-rotation request becomes a list of same-shift segments
(bt_offset, tok_start, n_tokens, delta) over one concatenated block table,
and one rerotate_pages call covers every layer that shares a cache geometry
and rotary embedding; cos/sin are formed from the rotary inverse frequencies
in registers on the GPU. Those frequencies are checked once per rotary module
against its cos_sin_cache, the table the reference rotates with; a table
they do not reproduce raises ValueError instead of rotating by another angle.

Layer topology. The reference reads the process-global
ProcessLocalConfig.cache_topo (configs/engine.py:11-70, 73-161) at
construction and again at every rotation (adapter.py:94, 154, 241, 311), and
is built as Adapter(config.adaption_config) (cache_engine.py:260). Built that
way here, the adapter does the same: it imports daric.configs and reads
ProcessLocalConfig.cache_topo at each use, so the page_first flags that
finish_register_process_local_config sets after construction
(integration/vllm/utils.py:212-220) are seen. Outside DARIC, pass the
topology as `cache_topo` (any object with get_all_layer_names(),
get_group_idx(name) and layers[name].page_first); with neither, the
constructor raises.

Bad cache layouts raise ValueError with the reference's text
(adapter.py:20-27, 336-368), before any layer is touched.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from itertools import chain
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import cache_ops
from .policy import DARICPolicy, plan_selection

__all__ = ["AdaptionConfig", "LayerCacheTopo", "CacheTopo", "Adapter", "plan_load_segments",
           "plan_multi_segments", "check_rerotate_layout", "rotary_inv_freq"]


@dataclass
class AdaptionConfig:
    """configs/engine.py:164-171."""
    rerotate: bool
    recompute: bool
    recompute_policy: Optional[str]
    recompute_avg_num: int
    function: str = "linear"
    r: float = 0.1


@dataclass
class LayerCacheTopo:
    """configs/engine.py:11-17 (the fields the adapter reads)."""
    group_idx: int
    logical_block_size: int
    block_byte_size: int
    page_first: bool
    is_mamba: bool = False


@dataclass
class CacheTopo:
    """configs/engine.py:20-35: layers by name, KV-cache groups of layer names."""
    layers: dict = field(default_factory=dict)
    groups: list = field(default_factory=list)

    def get_all_layer_names(self) -> list:
        return sorted(self.layers.keys())

    def get_group_idx(self, layer_name: str) -> int:
        for g_idx, group in enumerate(self.groups):
            if layer_name in group:
                return g_idx
        raise ValueError(f"Layer {layer_name} not found in any group.")


def _block_ids(blocks) -> np.ndarray:
    """A block list (list, tuple, array or tensor of ids) as int32 numpy."""
    if isinstance(blocks, torch.Tensor):
        return blocks.detach().to("cpu", torch.int32).reshape(-1).numpy()
    return np.asarray(blocks, dtype=np.int32).reshape(-1)


def _concat(parts) -> np.ndarray:
    return np.concatenate(parts) if parts else np.zeros(0, dtype=np.int32)


def _id_lists(parts, total: int, plain: bool) -> np.ndarray:
    """Block lists concatenated as int32 (`total` ids). plain: every part is a
    list or tuple of ids, the metas' usual form, converted in one numpy call;
    other forms are converted one by one."""
    if plain:
        try:
            return np.fromiter(chain.from_iterable(parts), dtype=np.int32, count=total)
        except (TypeError, ValueError):     # nested lists: converted one by one below
            pass
    return _concat([_block_ids(p) for p in parts])


def plan_load_segments(metas, group_idx: int):
    """apply_rerotate_load's planning (adapter.py:208-265): metas with a
    non-empty chunk whose saved position differs from ptr[0] move every token
    by ptr[0] - saved_pos. Returns (block table int32, segments)."""
    parts: list = []
    segs = []
    off = 0
    plain = True
    for meta in metas:
        old_pos = int(meta.saved_pos)
        new_pos = int(meta.ptr[0])
        n = int(meta.ptr[1] - meta.ptr[0])
        if n <= 0 or old_pos == new_pos:
            continue
        blocks = meta.block_ids[group_idx]
        if type(blocks) not in (list, tuple):
            blocks = _block_ids(blocks)
            plain = False
        segs.append((off, 0, n, new_pos - old_pos))
        parts.append(blocks)
        off += len(blocks)
    return _id_lists(parts, off, plain), segs


def plan_multi_segments(group_ptrs, block_ids_list, group_idx: int):
    """apply_rerotate_multi's planning (adapter.py:127-171): in a request with
    more than two groups, groups 1..n-2 of non-zero length move by
    group_ptr[i] - group_ptr[0]; token offsets count from group_ptr[0] in the
    request's block list."""
    parts: list = []
    segs = []
    off = 0
    plain = True
    for req_idx, group_ptr in enumerate(group_ptrs):
        n_groups = len(group_ptr) - 1
        if n_groups <= 2:
            continue
        base = group_ptr[0]
        req_segs = []
        for i in range(1, n_groups - 1):
            glen = group_ptr[i + 1] - group_ptr[i]
            if glen > 0:
                req_segs.append((group_ptr[i] - base, glen, group_ptr[i] - base))
        if not req_segs:
            continue
        blocks = block_ids_list[req_idx][group_idx]
        if type(blocks) not in (list, tuple):
            blocks = _block_ids(blocks)
            plain = False
        segs.extend((off, t0, n, d) for t0, n, d in req_segs)
        parts.append(blocks)
        off += len(blocks)
    return _id_lists(parts, off, plain), segs


def _table_positions(max_pos: int) -> list:
    """Positions at which a rotary table is checked: 0..3, every power of two
    and 1.5 times it below max_pos, and max_pos - 1. An inverse frequency that
    differs from the table's by e (mod 2*pi) drifts by p*e at position p, so
    the first power of two at which the drift passes the tolerance, or the last
    position, shows it before it can wrap round."""
    pos = {0, 1, 2, 3, max_pos - 1}
    p = 4
    while p < max_pos:
        pos.update((p, p + p // 2))
        p *= 2
    return sorted(x for x in pos if 0 <= x < max_pos)


def _inv_freq_candidates(rotary):
    """Inverse-frequency vectors a vLLM rotary module can have built its table
    from: an `inv_freq` attribute; _compute_inv_freq(base) (the default and
    llama3-scaled embeddings); _compute_inv_freq(scaling_factor) (the YaRN
    family's signature)."""
    inv = getattr(rotary, "inv_freq", None)
    if inv is not None:
        yield "inv_freq", inv
    fn = getattr(rotary, "_compute_inv_freq", None)
    if fn is None:
        return
    for attr in ("base", "scaling_factor"):
        arg = getattr(rotary, attr, None)
        if arg is None:
            continue
        try:
            yield f"_compute_inv_freq({attr})", fn(arg)
        except Exception:       # a signature that does not take this argument
            continue


def _inv_freq(rotary) -> torch.Tensor:
    """fp32 inverse frequencies that reproduce the rotary module's own table,
    rotary.cos_sin_cache: the table the reference's rotation reads
    (adapter.py:177-181, 271-283). The table is vLLM's layout,
    [max_pos, rotary_dim] = m * cat(cos(p * inv_freq), sin(p * inv_freq)),
    with m = cos_sin_cache[0, 0] its own scale (1, or YaRN's mscale). A
    candidate (see _inv_freq_candidates) is taken when, at every position of
    _table_positions, cos_sin_cache[p] / m is within
    eps(table dtype) + 2^-22 * (1 + p * inv_freq[i]) of cos / sin of the float32
    angle float32(p) * inv_freq[i] (the second term allows for the rounding of
    the table's own angle). No candidate matching -- positions scaled by a
    factor, a base other than rotary.base, a table of another form -- raises
    ValueError naming the class, since rotating by another angle would
    silently move K rows to the wrong position.

    The scale m is not applied: the rotation by a shift d is the unit rotation
    by d * inv_freq, as K computed at the new position would carry it. (The
    reference's combined table carries m squared, adapter.py:280-281.)"""
    name = type(rotary).__name__
    R = int(rotary.rotary_dim)
    table = getattr(rotary, "cos_sin_cache", None)
    if not isinstance(table, torch.Tensor) or table.ndim < 2 or table.shape[0] < 1:
        raise ValueError(f"{name}: rotary embedding has no [max_pos, rotary_dim] cos_sin_cache tensor")
    table = table.detach().reshape(table.shape[0], -1)
    if table.shape[1] != R or not table.is_floating_point():
        raise ValueError(f"{name}: cos_sin_cache of shape {tuple(rotary.cos_sin_cache.shape)} and dtype "
                         f"{table.dtype} is not a [max_pos, rotary_dim={R}] table of cos and sin")
    pos = _table_positions(int(table.shape[0]))
    rows = table.index_select(0, torch.tensor(pos, device=table.device)).to("cpu", torch.float64)
    m = float(rows[0, 0])
    if not (math.isfinite(m) and m > 0.0):
        raise ValueError(f"{name}: cos_sin_cache[0, 0] = {m} is not a positive scale")
    rows = rows / m
    eps = torch.finfo(table.dtype).eps
    p32 = torch.tensor(pos, dtype=torch.float32)[:, None]
    tried = []
    for label, cand in _inv_freq_candidates(rotary):
        inv = torch.as_tensor(cand).detach().to("cpu", torch.float32).reshape(-1)
        tried.append(label)
        if inv.numel() != R // 2 or not bool(torch.isfinite(inv).all()):
            continue
        ang = (p32 * inv[None, :]).to(torch.float64)          # float32 product, as the kernels form it
        tol = eps + 2.0 ** -22 * (1.0 + ang.abs())
        want = torch.cat([ang.cos(), ang.sin()], dim=1)
        if bool(((rows - want).abs() <= torch.cat([tol, tol], dim=1)).all()):
            return inv.contiguous()
    raise ValueError(
        f"{name}: rotary cos_sin_cache is not cos/sin(p * inv_freq) for any inverse frequencies the "
        f"module exposes (tried: {', '.join(tried) or 'none'}); re-rotation supports tables of that form "
        f"only (default, llama3- and YaRN-scaled frequencies)")


def rotary_inv_freq(rotary) -> torch.Tensor:
    """The fp32 inverse frequencies of a rotary module, proven against its own
    cos_sin_cache (ValueError when none reproduces it): what a caller of the
    fused load (scatter_pages_rerotate, KVIOContext.load(rerotate=...))
    passes as inv_freq, so that it rotates as the Adapter does."""
    return _inv_freq(rotary)


def check_rerotate_layout(layer_name: str, kv: torch.Tensor, page_first: bool, rotary_dim: int) -> None:
    """The layouts the reference's rotation accepts (adapter.py:20-27 for the
    rank, 336-350 for packed 4-D caches); anything else raises ValueError with
    the reference's message."""
    if kv.ndim not in (3, 4, 5):
        raise ValueError(f"Unsupported KV cache rank for rerotate: {kv.ndim}")
    if kv.ndim != 4:
        return
    width = int(kv.shape[3])
    if not page_first:
        why = "page_first must be true"
    elif width <= 0 or width % 2:
        why = "packed content dimension must be positive and even"
    elif kv.stride(3) != 1:
        why = "packed content feature stride must equal 1"
    elif rotary_dim <= 0 or rotary_dim % 2 or rotary_dim > width // 2:
        why = "rotary_dim must be positive, even, and no greater than the packed K head dimension"
    else:
        return
    raise ValueError(f"Invalid 4D KV cache for rerotate: layer={layer_name}, shape={tuple(kv.shape)}, "
                     f"stride={tuple(kv.stride())}, dtype={kv.dtype}, rotary_dim={rotary_dim}, "
                     f"constraint={why}")


def _process_local_config():
    """DARIC's ProcessLocalConfig class, whose cache_topo attribute holds the
    worker's layer topology; RuntimeError when it is not available."""
    try:
        from daric.configs import ProcessLocalConfig
    except ImportError as e:
        raise RuntimeError(
            "Adapter(config) reads the layer topology from daric.configs.ProcessLocalConfig.cache_topo, "
            f"but daric.configs cannot be imported ({e}); pass cache_topo= explicitly") from e
    if getattr(ProcessLocalConfig, "cache_topo", None) is None:
        raise RuntimeError(
            "Adapter(config) reads the layer topology from daric.configs.ProcessLocalConfig.cache_topo, "
            "which is not set yet; construct the Adapter after the process-local config is registered, "
            "or pass cache_topo= explicitly")
    return ProcessLocalConfig


class Adapter:
    def __init__(self, config: AdaptionConfig, cache_topo=None):
        self.config = config
        self._topo = cache_topo
        self._plc = _process_local_config() if cache_topo is None else None
        self.num_layers = len(self.cache_topo.get_all_layer_names())
        self.kvcaches: dict = {}
        self.rotary_embeds: dict = {}
        self._inv_cache: dict = {}
        self._layers: dict = {}
        self._groups: dict = {}
        self._bt_cache: dict = {}
        if config.recompute_policy == "daric":
            self.recompute_policy = DARICPolicy(config.recompute_avg_num, function=config.function,
                                                r=config.r)
        else:
            self.recompute_policy = None
        self.rerotate = config.rerotate

    @property
    def cache_topo(self):
        """The explicit topology, else ProcessLocalConfig.cache_topo as it is now."""
        return self._topo if self._topo is not None else self._plc.cache_topo

    # ------------------------------------------------------------ registration
    def register_kvcaches(self, kvcaches: dict) -> None:
        self.kvcaches = kvcaches
        self._layers.clear()

    def register_rotary_embed(self, layer_name: str, rotary_embed) -> None:
        if layer_name not in self.rotary_embeds:
            self.rotary_embeds[layer_name] = rotary_embed

    def register_done(self) -> bool:
        return len(self.rotary_embeds) == self.num_layers

    # ------------------------------------------------------------ rotation
    def _host_inv_freq(self, rotary) -> torch.Tensor:
        """_inv_freq(rotary), checked against the module's table once per
        (module, table storage)."""
        table = getattr(rotary, "cos_sin_cache", None)
        key = (id(rotary), table.data_ptr() if isinstance(table, torch.Tensor) else None)
        hit = self._inv_cache.get(key)
        if hit is None or hit[0] is not rotary:
            hit = (rotary, _inv_freq(rotary), {})
            self._inv_cache[key] = hit
        return hit

    def _device_inv_freq(self, rotary, device) -> torch.Tensor:
        hit = self._host_inv_freq(rotary)
        dev = hit[2].get(str(device))
        if dev is None:
            dev = hit[2][str(device)] = hit[1].to(device).contiguous()
        return dev

    def _group_idx(self, name: str, topo) -> int:
        hit = self._groups.get(name)
        if hit is None or hit[0] is not topo:
            hit = self._groups[name] = (topo, topo.get_group_idx(name))
        return hit[1]

    def _layer_info(self, name: str, topo):
        """(batch key, rotary, page_first) of a layer: its layout checked with
        the reference's errors and its rotary table proven, once per (cache
        tensor, rotary module, page_first); a per-layer call (the worker's
        layer-wise load, worker.py:230-231) then costs a few dictionary
        lookups instead of the checks."""
        kv = self.kvcaches[name]
        rotary = self.rotary_embeds[name]
        page_first = bool(topo.layers[name].page_first)
        hit = self._layers.get(name)
        if hit is not None and hit[0] is kv and hit[1] is rotary and hit[2] == page_first:
            return hit[3]
        check_rerotate_layout(name, kv, page_first, int(rotary.rotary_dim))
        self._host_inv_freq(rotary)     # a table the kernels cannot reproduce raises here
        key = (tuple(kv.shape), kv.stride(), kv.dtype, page_first, id(rotary),
               int(rotary.rotary_dim), bool(rotary.is_neox_style))
        info = (key, rotary, page_first)
        self._layers[name] = (kv, rotary, page_first, info)
        return info

    def _device_block_table(self, group_idx: int, bt: np.ndarray, device) -> torch.Tensor:
        """The block table on the device. The worker's layer-wise load plans
        the same metas for every layer, so the last table of each group is
        kept and reused while the planned ids are equal (no copy per layer)."""
        last = self._bt_cache.get(group_idx)
        if last is not None and last[0] == device and last[1].tobytes() == bt.tobytes():
            return last[2]
        bt_dev = torch.from_numpy(bt).to(device, non_blocking=True)
        self._bt_cache[group_idx] = (device, bt, bt_dev)
        return bt_dev

    def _rotate(self, layer_names: Sequence[str], plan) -> None:
        """Runs `plan(group_idx) -> (block table, segments)` for every KV-cache
        group and rotates the group's layers, batching the layers that share a
        geometry and a rotary embedding into one call."""
        topo = self.cache_topo
        by_group: dict = {}
        for name in layer_names:
            if name in self.kvcaches:
                by_group.setdefault(self._group_idx(name, topo), []).append(name)
        work = []
        for group_idx, names in by_group.items():
            bt, segs = plan(group_idx)
            if not segs:
                continue
            kv0 = self.kvcaches[names[0]]
            if kv0.ndim not in (3, 4, 5):      # the reference sizes pages from the first layer
                raise ValueError(f"Unsupported KV cache rank for rerotate: {kv0.ndim}")
            batches: dict = {}
            for name in names:
                key, rotary, page_first = self._layer_info(name, topo)
                batches.setdefault(key, (rotary, page_first, []))[2].append(self.kvcaches[name])
            work.append((group_idx, kv0.device, bt, segs, batches))
        # every layout is checked before any layer is rotated
        for group_idx, device, bt, segs, batches in work:
            bt_dev = self._device_block_table(group_idx, bt, device)
            for rotary, page_first, kvs in batches.values():
                cache_ops.rerotate_pages(kvs, page_first, bt_dev, segs,
                                         self._device_inv_freq(rotary, device),
                                         int(rotary.rotary_dim), bool(rotary.is_neox_style))

    def apply_rerotate_multi(self, group_ptrs: List[List[int]], block_ids_list) -> None:
        if not self.rerotate:
            return
        assert len(group_ptrs) == len(block_ids_list)
        self._rotate(list(self.kvcaches.keys()),
                     lambda g: plan_multi_segments(group_ptrs, block_ids_list, g))

    def apply_rerotate_load(self, metas, layer_name: Optional[str] = None) -> None:
        if not self.rerotate:
            return
        names = [layer_name] if layer_name is not None else list(self.kvcaches.keys())
        self._rotate(names, lambda g: plan_load_segments(metas, g))

    # ------------------------------------------------------------ recompute
    def get_recompute_length(self, group_ptr: List[int]) -> List[int]:
        if self.recompute_policy is None:
            return []
        return self.recompute_policy.get_recompute_ptrs(group_ptr)

    def plan_recompute_selection(self, group_ptrs, block_ids_list, group_idx: int = 0,
                                 no_recompute_lengths=None):
        """(block table int32, chunks int64 [n, 5], rows) for a batch of
        requests: each group of each request is one selection chunk whose k is
        the number of tokens get_recompute_length's ranges put in it
        (policy.plan_selection), over the requests' block lists of KV-cache
        group `group_idx`. None without a recompute policy."""
        if self.recompute_policy is None:
            return None
        return plan_selection(self.recompute_policy, group_ptrs,
                              [b[group_idx] for b in block_ids_list], no_recompute_lengths)
