"""Recompute selection: deviation keys, per-chunk top-k, merge (CPU restatement).

The reference has no such kernels: its "distribution-aware recomputation" is the
positional DARICPolicy (reference daric/adaption/policy.py:45-103) and the merge
is vLLM's own reshape_and_cache writing recomputed rows into the same slots
(daric/integration/vllm/worker.py:336-345, utils.py:406-427). The spec followed
here is the selection workload of the task's configuration 3:

  key[l, t] = sum over (h, d) of (K_new[l, t, h, d] - K_cache[l, slot(t), h, d])^2

in float32, in this fixed order (the HIP kernel sums in exactly this order, so
the keys and therefore the selected indices are bit-exact):
  - the token's H*D elements are taken in (h, d) order and cut into vectors of
    VEC = 8 consecutive elements; vector v belongs to lane v % 64 of a 64-lane
    wavefront and is visited in round v // 64;
  - each lane accumulates acc = acc + diff*diff element by element (each
    operation rounded to float32, no fused multiply-add), rounds ascending,
    elements of a vector ascending;
  - the 64 lane sums are combined by a butterfly: for off in 32,16,8,4,2,1:
    acc[l] = acc[l] + acc[l ^ off]; the key is acc[0].
Cached fp8 values are dequantised as float32(code value * k_scale[h]).
Keys are ranked by their float32 bit pattern as an unsigned integer (keys are
>= +0; any NaN is stored as 0x7FC00000 and ranks above +inf). Ties go to the
lower token index. The k selected chunk-local indices are returned ascending.
"""
from __future__ import annotations

import numpy as np
import torch

from . import fp8
from .layout import rope_geometry

VEC = 8
LANES = 64
NAN_KEY = np.uint32(0x7FC00000)


def v_view(layer: torch.Tensor, page_first: bool) -> torch.Tensor | None:
    """[num_blocks, PS, H, D] view of the V head rows (None for a 3-D MLA cache)."""
    nd = layer.dim()
    if nd == 5:
        return layer[:, 1] if page_first else layer[1]
    if nd == 4:
        d = layer.shape[3] // 2
        return layer.permute(0, 2, 1, 3)[..., d:]
    return None


def k_rows_view(layer: torch.Tensor, page_first: bool) -> torch.Tensor:
    """[num_blocks, PS, H, D] view of the full K head rows."""
    nd = layer.dim()
    if nd == 5:
        return layer[:, 0] if page_first else layer[0]
    if nd == 4:
        d = layer.shape[3] // 2
        return layer.permute(0, 2, 1, 3)[..., :d]
    return layer.unsqueeze(2)


def _as_f32(x: torch.Tensor, k_scale=None) -> np.ndarray:
    if x.dtype == torch.uint8:
        v = fp8.decode(x.numpy()).astype(np.float32)
        s = np.ones(x.shape[-2], np.float32) if k_scale is None else np.asarray(k_scale, np.float32)
        return (v * s[:, None]).astype(np.float32)
    return x.to(torch.float32).numpy()


def fixed_order_sumsq(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Keys of rows a, b: [T, N] float32 -> [T] float32, in the order above."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    t, n = a.shape
    with np.errstate(invalid="ignore", over="ignore"):   # inf - inf and overflow give NaN / inf, as on the GPU
        d = (a - b).astype(np.float32)
        sq = (d * d).astype(np.float32)
    n_vec = -(-n // VEC)
    rounds = -(-n_vec // LANES)
    padded = np.zeros((t, rounds * LANES * VEC), np.float32)
    padded[:, :n] = sq
    padded = padded.reshape(t, rounds, LANES, VEC)
    acc = np.zeros((t, LANES), np.float32)
    for r in range(rounds):
        for i in range(VEC):
            acc = (acc + padded[:, r, :, i]).astype(np.float32)
    lanes = np.arange(LANES)
    for off in (32, 16, 8, 4, 2, 1):
        acc = (acc + acc[:, lanes ^ off]).astype(np.float32)
    key = acc[:, 0].copy()
    key[np.isnan(key)] = NAN_KEY.view(np.float32)
    return key


def _fields(chunk):
    """(bt_offset, row_offset, n_tokens, k, tok_start) of a 4- or 5-field chunk."""
    c = [int(x) for x in chunk]
    return tuple(c) if len(c) == 5 else tuple(c) + (0,)


def chunk_slots(block_table, bt_offset, n_tokens, page_size, tok_start=0):
    """(block id, place in page) of chunk-local tokens 0..n_tokens-1: token j is
    token tok_start + j of the block list at block_table[bt_offset]."""
    bt = np.asarray(block_table)
    p = tok_start + np.arange(n_tokens)
    return bt[bt_offset + p // page_size].astype(np.int64), p % page_size


def deviation(layers, page_first, block_table, k_new, chunks, k_scales=None) -> np.ndarray:
    """keys [L, T] for chunks (bt_offset, row_offset, n_tokens, k[, tok_start]); rows of T
    not covered by any chunk are left 0, and so are tokens whose block id lies
    outside [0, num_blocks)."""
    L, T = len(layers), k_new.shape[1]
    keys = np.zeros((L, T), np.float32)
    for l, layer in enumerate(layers):
        kv = k_rows_view(layer, page_first)
        ps, h, d = kv.shape[1], kv.shape[2], kv.shape[3]
        ks = None if k_scales is None else k_scales[l]
        nb = kv.shape[0]
        for chunk in chunks:
            bt_offset, row_offset, n_tokens, _k, tok_start = _fields(chunk)
            blk, s = chunk_slots(block_table, bt_offset, n_tokens, ps, tok_start)
            ok = (blk >= 0) & (blk < nb)        # other block ids: not read, key 0
            cached = _as_f32(kv[torch.as_tensor(np.where(ok, blk, 0)), torch.as_tensor(s)], ks)
            cached = cached.reshape(n_tokens, h * d)
            new = k_new[l, row_offset: row_offset + n_tokens].to(torch.float32).numpy().reshape(n_tokens, h * d)
            key = fixed_order_sumsq(new, cached)
            keys[l, row_offset: row_offset + n_tokens] = np.where(ok, key, np.float32(0.0))
    return keys


def topk_chunk(keys: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest keys (by uint32 bit pattern), ties to the lower
    index, returned ascending. Uses numpy's stable lexsort."""
    bits = np.asarray(keys, np.float32).view(np.uint32).astype(np.int64)
    order = np.lexsort((np.arange(len(bits)), -bits))
    return np.sort(order[: min(k, len(bits))])


def topk_per_chunk(keys: np.ndarray, chunks, kmax: int) -> np.ndarray:
    L = keys.shape[0]
    out = np.full((L, len(chunks), kmax), -1, np.int32)
    for l in range(L):
        for c, chunk in enumerate(chunks):
            _bt, row_offset, n_tokens, k, _ts = _fields(chunk)
            sel = topk_chunk(keys[l, row_offset: row_offset + n_tokens], int(k))
            out[l, c, : len(sel)] = sel
    return out


def quantise_rows(rows: torch.Tensor, scales) -> torch.Tensor:
    """bf16/fp16 rows [..., H, D] -> e4m3 codes (uint8) of float32(x) / scale[h],
    the quotient correctly rounded to float32, then saturating RTNE. This is the
    fp8 write of vLLM's reshape_and_cache for the recompute sub-requests'
    rows (daric/integration/vllm/worker.py:336-345, utils.py:406-427)."""
    x = rows.to(torch.float32).numpy()
    s = np.asarray(scales, np.float32).reshape(-1, 1)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):   # saturating cases
        q = (x / s).astype(np.float32)
    return torch.from_numpy(fp8.encode(q)).view(rows.shape)


def merge_rows(layers, page_first, block_table, k_new, v_new, chunks, sel_idx,
               k_scales=None, v_scales=None) -> None:
    """Write selected K/V rows into their slots (block 0 / out of range skipped).
    Rows in the cache's element type are copied; bf16/fp16 rows for an fp8
    (uint8) cache are quantised with k_scales / v_scales [L, H]. The selected
    slots of one call are distinct (as for the kernel, whose workgroups write
    them concurrently)."""
    quant = layers[0].dtype == torch.uint8 and k_new.dtype in (torch.bfloat16, torch.float16)
    bt = np.asarray(block_table)
    sel_idx = np.asarray(sel_idx)
    for l, layer in enumerate(layers):
        kv = k_rows_view(layer, page_first)
        vv = v_view(layer, page_first)
        nb, ps = kv.shape[0], kv.shape[1]
        rows, blks, slots = [], [], []
        for c, chunk in enumerate(chunks):
            bt_offset, row_offset, n_tokens, _k, tok_start = _fields(chunk)
            j = sel_idx[l, c].astype(np.int64)
            j = j[(j >= 0) & (j < n_tokens)]
            p = tok_start + j
            blk = bt[bt_offset + p // ps].astype(np.int64)
            keep = (blk > 0) & (blk < nb)
            rows.append(row_offset + j[keep])
            blks.append(blk[keep])
            slots.append(p[keep] % ps)
        if not rows:
            continue
        r = torch.from_numpy(np.concatenate(rows))
        b = torch.from_numpy(np.concatenate(blks))
        s = torch.from_numpy(np.concatenate(slots))
        if r.numel() == 0:
            continue
        if quant:
            kv[b, s] = quantise_rows(k_new[l, r], k_scales[l])
            if vv is not None:
                vv[b, s] = quantise_rows(v_new[l, r], v_scales[l])
        else:
            kv[b, s] = k_new[l, r].view(kv.dtype)
            if vv is not None:
                vv[b, s] = v_new[l, r].view(vv.dtype)
