"""RoPE re-rotation of cached K rows (CPU restatement).

Follows reference daric/adaption/adapter.py:
  - pairing and rotation formula of _fused_rerotate_kernel (:57-88): NeoX pairs
    (i, i + R/2), GPT-J pairs (2i, 2i+1), i < R/2;
      out1 = x1*cos - x2*sin,  out2 = x2*cos + x1*sin;
    dims >= R and the V half are untouched;
  - token -> slot mapping slot = block_ids[j // PS] * PS + j % PS
    (apply_rerotate_load :258-264, apply_rerotate_multi :162-170);
  - which tokens move and by how much: apply_rerotate_load moves token j of a
    meta from saved_pos + j to ptr[0] + j (:208-236), skipping metas with
    old == new; apply_rerotate_multi moves groups 1..n-2 by
    group_ptr[i] - group_ptr[0] (:127-150).

The reference forms the combined angle from vLLM's cos_sin_cache rows
(cos(new)cos(old) + sin(new)sin(old), :276-283), in the table's dtype. That
table is vLLM's and is parity unpinned here (vLLM is absent). This oracle uses
the defined quantity instead: the angle of pair i for a shift of d positions
is the float32 product float32(d) * inv_freq[i]; cos/sin and the rotation are
evaluated in float64 and the result is rounded to float32, then to the cache
dtype (fp8: dequantised with the per-head scale first and requantised after).
"""
from __future__ import annotations

import numpy as np
import torch

from . import fp8
from .layout import rope_geometry


def default_inv_freq(rotary_dim: int, base: float) -> np.ndarray:
    """inv_freq[i] = 1 / base^(2i/R) in float32 (vLLM RotaryEmbedding._compute_inv_freq)."""
    exps = torch.arange(0, rotary_dim, 2, dtype=torch.float) / rotary_dim
    return (1.0 / (base ** exps)).numpy().astype(np.float32)


def angles(delta: int, inv_freq: np.ndarray) -> np.ndarray:
    """float32(delta) * inv_freq, rounded to float32."""
    return (np.float32(delta) * np.asarray(inv_freq, dtype=np.float32)).astype(np.float32)


def rotate_rows(x: np.ndarray, delta: int, inv_freq: np.ndarray, rotary_dim: int,
                is_neox: bool) -> np.ndarray:
    """Rotate the last axis of x (float64) by delta positions; returns float64."""
    x = np.asarray(x, dtype=np.float64)
    R = int(rotary_dim)
    ang = angles(delta, inv_freq).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    out = x.copy()
    if is_neox:
        x1, x2 = x[..., : R // 2], x[..., R // 2: R]
        out[..., : R // 2] = x1 * c - x2 * s
        out[..., R // 2: R] = x2 * c + x1 * s
    else:
        x1, x2 = x[..., 0:R:2], x[..., 1:R:2]
        out[..., 0:R:2] = x1 * c - x2 * s
        out[..., 1:R:2] = x2 * c + x1 * s
    return out


def k_view(layer: torch.Tensor, page_first: bool, rotary_dim: int) -> torch.Tensor:
    """A [num_blocks, PS, H, D] view of the K head rows of a KV layer tensor,
    resolved as adapter.py:311-368 resolves them."""
    g = rope_geometry(tuple(layer.shape), tuple(layer.stride()), page_first, rotary_dim,
                      str(layer.dtype))
    nb = int(layer.shape[0] if (page_first or layer.dim() != 5) else layer.shape[1])
    return torch.as_strided(layer, (nb, g.page_size, g.num_heads, g.head_dim),
                            (g.stride_b, g.stride_s, g.stride_h, 1),
                            layer.storage_offset() + g.k_offset)


def _to_values(x: torch.Tensor, scale) -> np.ndarray:
    """Cache elements -> float64 values (fp8: code value times per-head scale)."""
    if x.dtype == torch.uint8:
        v = fp8.decode(x.numpy()).astype(np.float64)
        return v * np.asarray(scale, dtype=np.float64)[:, None]
    return x.to(torch.float64).numpy()


def _from_values(v: np.ndarray, dtype: torch.dtype, scale) -> torch.Tensor:
    """float64 values -> cache elements, rounding through float32."""
    if dtype == torch.uint8:
        q = v / np.asarray(scale, dtype=np.float64)[:, None]
        return torch.from_numpy(fp8.encode(q.astype(np.float32)))
    return torch.from_numpy(v.astype(np.float32)).to(dtype)


def rotate_slots(layer: torch.Tensor, page_first: bool, slots, delta: int,
                 inv_freq: np.ndarray, rotary_dim: int, is_neox: bool,
                 k_scale=None) -> None:
    """Rotate in place the K rows (all heads) of the given slots by delta."""
    kv = k_view(layer, page_first, rotary_dim)
    ps, h = kv.shape[1], kv.shape[2]
    scale = np.ones(h) if k_scale is None else np.asarray(k_scale, dtype=np.float64)
    slots = np.asarray(list(slots), dtype=np.int64)
    if slots.size == 0:
        return
    if np.unique(slots).size != slots.size:
        # a slot listed twice is rotated twice, one after the other
        for slot in slots:
            blk, s = int(slot) // ps, int(slot) % ps
            rows = kv[blk, s]                   # [H, D] view
            vals = _to_values(rows.clone(), scale)
            out = rotate_rows(vals, delta, inv_freq, rotary_dim, is_neox)
            rows.copy_(_from_values(out, layer.dtype, scale))
        return
    blk, s = torch.from_numpy(slots // ps), torch.from_numpy(slots % ps)
    vals = _to_values(kv[blk, s], scale)        # [n, H, D]
    out = rotate_rows(vals, delta, inv_freq, rotary_dim, is_neox)
    kv[blk, s] = _from_values(out, layer.dtype, scale)


def table_cos_sin_load(cos_sin_cache, old_pos, new_pos):
    """Per-token combined cos/sin [n, R/2] of apply_rerotate_load as the
    reference forms them from the rotary table (adapter.py:271-283):
    cos = cos(new)cos(old) + sin(new)sin(old), sin = sin(new)cos(old) -
    cos(new)sin(old), here in float64 from the table's values. The table is
    first divided by its own scale m = cos_sin_cache[0, 0]: the reference's
    combined values carry m squared, the re-rotation here is the unit rotation
    (rows keep their norm)."""
    t = _unit_table(cos_sin_cache)
    half = t.shape[1] // 2
    o, n = t[np.asarray(old_pos, dtype=np.int64)], t[np.asarray(new_pos, dtype=np.int64)]
    oc, os_, nc, ns = o[:, :half], o[:, half:], n[:, :half], n[:, half:]
    return nc * oc + ns * os_, ns * oc - nc * os_


def table_cos_sin_multi(cos_sin_cache, deltas):
    """Per-token cos/sin [n, R/2] of apply_rerotate_multi: the table row of
    the shift itself (adapter.py:147-150, 176-181), divided by m as above."""
    t = _unit_table(cos_sin_cache)
    half = t.shape[1] // 2
    r = t[np.asarray(deltas, dtype=np.int64)]
    return r[:, :half], r[:, half:]


def _unit_table(cos_sin_cache) -> np.ndarray:
    t = torch.as_tensor(cos_sin_cache).detach().to("cpu", torch.float64)
    t = t.reshape(t.shape[0], -1).numpy()
    return t / t[0, 0]


def rotate_slots_cs(layer: torch.Tensor, page_first: bool, slots, cos, sin, rotary_dim: int,
                    is_neox: bool) -> None:
    """Rotate in place the K rows (all heads) of slot i by its own (cos[i],
    sin[i]) rows, with the pairing and formula of _fused_rerotate_kernel
    (adapter.py:57-88), in float64. An fp8 (uint8) cache has its e4m3 codes
    rotated as values and re-encoded with saturating round-to-nearest-even, no
    scale applied, as that kernel rotates a uint8 cache viewed as
    float8_e4m3fn (adapter.py:370-373). Slots must be distinct."""
    kv = k_view(layer, page_first, rotary_dim)
    ps = kv.shape[1]
    slots = np.asarray(list(slots), dtype=np.int64)
    if slots.size == 0:
        return
    assert np.unique(slots).size == slots.size
    R = int(rotary_dim)
    blk, s = torch.from_numpy(slots // ps), torch.from_numpy(slots % ps)
    ones = np.ones(kv.shape[2])
    x = _to_values(kv[blk, s], ones)                 # [n, H, D]
    c = np.asarray(cos, dtype=np.float64)[:, None, :]
    sn = np.asarray(sin, dtype=np.float64)[:, None, :]
    out = x.copy()
    if is_neox:
        x1, x2 = x[..., : R // 2], x[..., R // 2: R]
        out[..., : R // 2] = x1 * c - x2 * sn
        out[..., R // 2: R] = x2 * c + x1 * sn
    else:
        x1, x2 = x[..., 0:R:2], x[..., 1:R:2]
        out[..., 0:R:2] = x1 * c - x2 * sn
        out[..., 1:R:2] = x2 * c + x1 * sn
    kv[blk, s] = _from_values(out, layer.dtype, ones)


def segment_slots(block_table, bt_offset: int, tok_start: int, n_tokens: int,
                  page_size: int) -> list[int]:
    """Slots of a run of tokens (adapter.py:164-170, 258-264)."""
    bt = np.asarray(block_table)
    pos = np.arange(tok_start, tok_start + n_tokens)
    return (bt[bt_offset + pos // page_size].astype(np.int64) * page_size + pos % page_size).tolist()


def rerotate_pages(layers, page_first: bool, block_table, segments, inv_freq,
                   rotary_dim: int, is_neox: bool, k_scales=None) -> None:
    """In-place re-rotation of every segment (bt_offset, tok_start, n_tokens,
    delta) in every layer: the counterpart of one _launch_triton_rerotate per
    layer over the concatenated gather_idx of the segments. A segment with
    delta 0 is left alone, as apply_rerotate_load leaves a chunk whose saved
    and new positions agree (adapter.py:212); rotating it by the identity
    would still turn some -0 values into +0."""
    for li, layer in enumerate(layers):
        ps = k_view(layer, page_first, rotary_dim).shape[1]
        ks = None if k_scales is None else np.asarray(k_scales[li])
        for bt_offset, tok_start, n_tokens, delta in segments:
            if int(delta) == 0:
                continue
            slots = segment_slots(block_table, bt_offset, tok_start, n_tokens, ps)
            rotate_slots(layer, page_first, slots, delta, inv_freq, rotary_dim, is_neox, ks)


def load_segments(metas):
    """apply_rerotate_load planning (adapter.py:208-220, 258-265): one segment per
    meta with chunk_len > 0 and saved_pos != ptr[0]. Each meta is
    (ptr0, ptr1, saved_pos, block_ids). Returns (block_table, segments)."""
    bt, segs = [], []
    for ptr0, ptr1, saved_pos, block_ids in metas:
        n = int(ptr1) - int(ptr0)
        if n <= 0 or int(saved_pos) == int(ptr0):
            continue
        segs.append((len(bt), 0, n, int(ptr0) - int(saved_pos)))
        bt.extend(int(b) for b in block_ids)
    return np.asarray(bt, dtype=np.int32), segs


def multi_segments(group_ptrs, block_ids_list):
    """apply_rerotate_multi planning (adapter.py:127-171): for requests with more
    than two groups, groups 1..n-2 of non-zero length move by
    group_ptr[i] - group_ptr[0]; token offsets are relative to group_ptr[0]."""
    bt, segs = [], []
    for group_ptr, blocks in zip(group_ptrs, block_ids_list):
        n_groups = len(group_ptr) - 1
        if n_groups <= 2:
            continue
        base = group_ptr[0]
        off = len(bt)
        used = False
        for i in range(1, n_groups - 1):
            glen = group_ptr[i + 1] - group_ptr[i]
            if glen > 0:
                segs.append((off, group_ptr[i] - base, glen, group_ptr[i] - base))
                used = True
        if used:
            bt.extend(int(b) for b in blocks)
    return np.asarray(bt, dtype=np.int32), segs
