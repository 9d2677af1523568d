"""`daric.cache_ops` API on the gfx950 HIP library.

Drop-in for the reference's pybind11 module (stub daric/cache_ops.pyi:1-53,
bindings csrc/cache_ops/bindings.cpp:7-31): `CacheCopier` with
register_layer / register_store / gather_pages / scatter_pages, and the free
functions batched_memcpy_d2h / batched_memcpy_h2d keep their signatures,
argument meaning and errors (RuntimeError with the reference's message text).

Additions (no reference counterpart; the .pyi grows, nothing changes):
  CacheCopier.register_k_scale, CacheCopier.scatter_pages_rerotate (and its
  allocation-free form scatter_pages_rerotate_noalloc),
  CacheCopier.gather_tokens / scatter_tokens (token-major staging for any
  cache layout), rerotate_pages, kv_deviation, topk_per_chunk, merge_rows,
  select_merge (the three selection calls in one), kernel timing.

Every call is asynchronous on `stream` (0 = the current torch stream of the
first layer's device, as in reference copier.cpp:27-30). The wrapper keeps
strong references to registered tensors (copier.cpp:10, 21-24) and records
temporary inputs on the launch stream (kernels.cu:202, copier.cpp:69).
"""
from __future__ import annotations

import ctypes
from collections.abc import Sequence
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import I64, DaricChunk, DaricRope, DaricRopeSegment, check, desc, load, str_array

__all__ = [
    "CacheCopier", "batched_memcpy_d2h", "batched_memcpy_h2d", "rerotate_pages",
    "kv_deviation", "topk_per_chunk", "merge_rows", "select_merge", "SELECT_KEYS_READY",
    "SELECT_ONE_PASS", "timing_enable", "timing_read",
]


# The current stream's raw handle without building a torch.cuda.Stream object
# (0.1 us against 2 us per call on MI355X); the public call is the fallback.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _resolve_stream(stream: int, device: Optional[torch.device]) -> int:
    if stream:
        return int(stream)
    if device is None or device.type != "cuda":
        return 0
    if _RAW_STREAM is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return int(_RAW_STREAM(idx))
    return torch.cuda.current_stream(device).cuda_stream


_EXT_STREAMS: dict = {}


def _ext_stream(stream: int, device: torch.device):
    key = (int(stream), device.index)
    s = _EXT_STREAMS.get(key)
    if s is None:
        if len(_EXT_STREAMS) > 64:
            _EXT_STREAMS.clear()
        s = _EXT_STREAMS[key] = torch.cuda.ExternalStream(stream, device=device)
    return s


def _record(stream: int, device: torch.device, *tensors) -> None:
    """Keep caching-allocator memory of temporaries alive until `stream` has
    consumed them (the reference's record_tensor_on_external_stream). Not
    while a graph is being captured: a captured graph's inputs must outlive
    its replays, which is the caller's to ensure, as for any graph."""
    if device is None or device.type != "cuda":
        return
    if torch.cuda.is_current_stream_capturing():
        return
    ext = _ext_stream(stream, device)
    for t in tensors:
        if t is not None and t.is_cuda:
            t.record_stream(ext)


def _rope(inv_freq: torch.Tensor, rotary_dim: int, is_neox_style: bool, device) -> DaricRope:
    if not isinstance(inv_freq, torch.Tensor) or not inv_freq.is_cuda:
        raise RuntimeError("inv_freq must be a float32 device tensor")
    if inv_freq.dtype != torch.float32 or not inv_freq.is_contiguous():
        raise RuntimeError("inv_freq must be a contiguous float32 tensor")
    if inv_freq.numel() < int(rotary_dim) // 2:
        raise RuntimeError(f"inv_freq has {inv_freq.numel()} entries, rotary_dim/2 = {int(rotary_dim) // 2}")
    if device is not None and inv_freq.device != device:
        raise RuntimeError("inv_freq must be on the KV cache's device")
    r = DaricRope()
    r.inv_freq = inv_freq.data_ptr()
    r.rotary_dim = int(rotary_dim)
    r.is_neox = 1 if is_neox_style else 0
    return r


class CacheCopier:
    """Staged KV-cache gather/scatter (reference csrc/cache_ops/copier.cpp)."""

    def __init__(self) -> None:
        self._lib = load()
        h = ctypes.c_void_p()
        check(self._lib.daric_copier_create(ctypes.byref(h)))
        self._h = h
        self._layers: dict[str, torch.Tensor] = {}
        self._scales: dict[str, torch.Tensor] = {}
        self._store: Optional[torch.Tensor] = None

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.daric_copier_destroy(h)
            self._h = None

    # -------------------------------------------------------------- register
    def register_layer(self, name: str, tensor: torch.Tensor, is_page_first: bool) -> None:
        d = desc(tensor)
        check(self._lib.daric_copier_register_layer(self._h, str(name).encode(), ctypes.byref(d),
                                                    1 if is_page_first else 0))
        self._layers[str(name)] = tensor

    def register_store(self, buffer: torch.Tensor) -> None:
        d = desc(buffer)
        check(self._lib.daric_copier_register_store(self._h, ctypes.byref(d)))
        self._store = buffer

    def register_k_scale(self, name: str, k_scale: Optional[torch.Tensor]) -> None:
        """Per-head fp32 K scales of an fp8 layer (None clears them)."""
        d = desc(k_scale) if k_scale is not None else None
        check(self._lib.daric_copier_register_k_scale(
            self._h, str(name).encode(), ctypes.byref(d) if d is not None else None))
        if k_scale is None:
            self._scales.pop(str(name), None)
        else:
            self._scales[str(name)] = k_scale

    # -------------------------------------------------------------- copies
    def _device(self, layer_names) -> Optional[torch.device]:
        if len(layer_names) == 0:
            return None
        t = self._layers.get(str(layer_names[0]))
        return t.device if t is not None else None

    def _copy(self, fn, layer_names, offsets, byte_sizes, indices_flat, indices_offsets, stream,
              extra=()):
        names = list(layer_names)
        dev = self._device(names)
        st = _resolve_stream(stream, dev)
        idx = desc(indices_flat)
        off, sz, ioff = I64(offsets), I64(byte_sizes), I64(indices_offsets)
        status = fn(self._h, str_array(names), len(names), off.ptr, off.n, sz.ptr, sz.n,
                    ctypes.byref(idx), ioff.ptr, ioff.n, *extra, ctypes.c_uint64(st))
        check(status)
        if names:
            _record(st, dev, indices_flat)

    def gather_pages(self, layer_names: Sequence[str], offsets: Sequence[int],
                     byte_sizes: Sequence[int], indices_flat: torch.Tensor,
                     indices_offsets: Sequence[int], stream: int = 0) -> None:
        self._copy(self._lib.daric_copier_gather_pages, layer_names, offsets, byte_sizes,
                   indices_flat, indices_offsets, stream)

    def scatter_pages(self, layer_names: Sequence[str], offsets: Sequence[int],
                      byte_sizes: Sequence[int], indices_flat: torch.Tensor,
                      indices_offsets: Sequence[int], stream: int = 0) -> None:
        self._copy(self._lib.daric_copier_scatter_pages, layer_names, offsets, byte_sizes,
                   indices_flat, indices_offsets, stream)

    def gather_tokens(self, layer_names: Sequence[str], offsets: Sequence[int],
                      byte_sizes: Sequence[int], indices_flat: torch.Tensor,
                      indices_offsets: Sequence[int], stream: int = 0) -> None:
        """gather_pages into token-major rows: job i's store range becomes
        [n_kv][n_sel * PS][H][D] (K rows then V rows) for any cache layout
        (see include/daric_cache_ops.h). byte_sizes[i] = n_kv * n_sel * PS *
        H * D * element size. No counterpart in the reference."""
        self._copy(self._lib.daric_copier_gather_tokens, layer_names, offsets, byte_sizes,
                   indices_flat, indices_offsets, stream)

    def scatter_tokens(self, layer_names: Sequence[str], offsets: Sequence[int],
                       byte_sizes: Sequence[int], indices_flat: torch.Tensor,
                       indices_offsets: Sequence[int], stream: int = 0) -> None:
        """Inverse of gather_tokens. No counterpart in the reference."""
        self._copy(self._lib.daric_copier_scatter_tokens, layer_names, offsets, byte_sizes,
                   indices_flat, indices_offsets, stream)

    def scatter_pages_rerotate(self, layer_names: Sequence[str], offsets: Sequence[int],
                               byte_sizes: Sequence[int], indices_flat: torch.Tensor,
                               indices_offsets: Sequence[int], deltas: Sequence[int],
                               num_tokens: Sequence[int], inv_freq: torch.Tensor,
                               rotary_dim: int, is_neox_style: bool = True,
                               stream: int = 0) -> None:
        """scatter_pages + re-rotation of the first num_tokens[i] tokens of job
        i by deltas[i] positions, in one pass (see include/daric_cache_ops.h)."""
        self._fused(self._lib.daric_copier_scatter_pages_rerotate, layer_names, offsets, byte_sizes,
                    indices_flat, indices_offsets, deltas, num_tokens, inv_freq, rotary_dim,
                    is_neox_style, stream)

    def scatter_pages_rerotate_noalloc(self, layer_names: Sequence[str], offsets: Sequence[int],
                                       byte_sizes: Sequence[int], indices_flat: torch.Tensor,
                                       indices_offsets: Sequence[int], deltas: Sequence[int],
                                       num_tokens: Sequence[int], inv_freq: torch.Tensor,
                                       rotary_dim: int, is_neox_style: bool = True,
                                       stream: int = 0) -> None:
        """scatter_pages_rerotate without allocating device or pinned memory:
        large job lists are staged in a static per-GPU array of 3276 jobs.
        Calls that overlap on one GPU race on that array (see
        include/daric_cache_ops.h). No counterpart in the reference."""
        self._fused(self._lib.daric_copier_scatter_pages_rerotate_noalloc, layer_names, offsets,
                    byte_sizes, indices_flat, indices_offsets, deltas, num_tokens, inv_freq,
                    rotary_dim, is_neox_style, stream)

    def _fused(self, fn, layer_names, offsets, byte_sizes, indices_flat, indices_offsets, deltas,
               num_tokens, inv_freq, rotary_dim, is_neox_style, stream):
        names = list(layer_names)
        if len(deltas) != len(names) or len(num_tokens) != len(names):
            if names:
                raise RuntimeError("deltas and num_tokens must have one entry per job")
        dev = self._device(names)
        rope = _rope(inv_freq, rotary_dim, is_neox_style, dev) if names else DaricRope()
        dl, nt = I64(deltas), I64(num_tokens)
        self._copy(fn, names, offsets, byte_sizes, indices_flat, indices_offsets, stream,
                   extra=(dl.ptr, nt.ptr, ctypes.byref(rope)))
        if names and dev is not None:
            _record(_resolve_stream(stream, dev), dev, inv_freq)


def _memcpy(fn, dev_t, host_t, dev_offsets, host_offsets, sizes, stream, d2h):
    n = len(sizes)
    if len(dev_offsets) != n or len(host_offsets) != n:
        raise RuntimeError("offset and size lists must have the same length")
    if n == 0:
        return
    dev = dev_t.device if dev_t.is_cuda else None
    st = _resolve_stream(stream, dev)
    a, b = desc(dev_t), desc(host_t)
    do, ho, sz = I64(dev_offsets), I64(host_offsets), I64(sizes)
    if d2h:
        check(fn(ctypes.byref(a), ctypes.byref(b), do.ptr, ho.ptr, sz.ptr, n, ctypes.c_uint64(st)))
    else:
        check(fn(ctypes.byref(b), ctypes.byref(a), ho.ptr, do.ptr, sz.ptr, n, ctypes.c_uint64(st)))


def batched_memcpy_d2h(staging: torch.Tensor, shm: torch.Tensor, stg_offsets: Sequence[int],
                       shm_offsets: Sequence[int], sizes: Sequence[int], stream: int = 0) -> None:
    """One hipMemcpyAsync per (stg_offset, shm_offset, size) region (reference
    helpers.cu:187-217). shm must be page-locked host memory."""
    _memcpy(load().daric_batched_memcpy_d2h, staging, shm, stg_offsets, shm_offsets, sizes, stream, True)


def batched_memcpy_h2d(shm: torch.Tensor, staging: torch.Tensor, shm_offsets: Sequence[int],
                       stg_offsets: Sequence[int], sizes: Sequence[int], stream: int = 0) -> None:
    """Mirror of batched_memcpy_d2h (reference helpers.cu:219-248)."""
    _memcpy(load().daric_batched_memcpy_h2d, staging, shm, stg_offsets, shm_offsets, sizes, stream, False)


_LAYER_ARRAYS: dict = {}


def _layer_array(layers: Sequence[torch.Tensor]):
    """daric_tensor array of `layers`, cached per (address, shape, strides,
    dtype, device) signature: callers pass the same cache tensors every call."""
    key = tuple((t.data_ptr(), t.shape, t.stride(), t.dtype, t.device) for t in layers)
    arr = _LAYER_ARRAYS.get(key)
    if arr is None:
        arr = (_lib.DaricTensor * max(len(layers), 1))()
        for i, t in enumerate(layers):
            arr[i] = desc(t)
        if len(_LAYER_ARRAYS) >= 64:
            _LAYER_ARRAYS.clear()
        _LAYER_ARRAYS[key] = arr
    return arr


def rerotate_pages(layers: Sequence[torch.Tensor], page_first: bool, block_table: torch.Tensor,
                   segments: Sequence[tuple[int, int, int, int]], inv_freq: torch.Tensor,
                   rotary_dim: int, is_neox_style: bool = True,
                   k_scales: Optional[torch.Tensor] = None, stream: int = 0) -> None:
    """In-place re-rotation of the K rows of every segment
    (bt_offset, tok_start, n_tokens, delta) in every layer: the counterpart of
    the reference's per-layer _launch_triton_rerotate (adapter.py:297-396).
    k_scales ([L, H] fp32, positive) is checked but leaves the result
    unchanged: fp8 codes are rotated as stored, since a per-head scale cancels
    in a linear rotation (the reference's kernel rotates the raw fp8 values)."""
    layers = list(layers)
    segs = list(segments)
    if not layers or not segs:
        return
    dev = layers[0].device
    st = _resolve_stream(stream, dev)
    rope = _rope(inv_freq, rotary_dim, is_neox_style, dev)
    seg_np = np.ascontiguousarray(np.asarray(segs, dtype=np.int64).reshape(-1, 4))
    sarr = ctypes.cast(seg_np.ctypes.data, ctypes.POINTER(DaricRopeSegment))
    bt = desc(block_table)
    ks = desc(k_scales) if k_scales is not None else None
    check(load().daric_rerotate_pages(_layer_array(layers), len(layers), 1 if page_first else 0,
                                      ctypes.byref(bt), sarr, len(segs), ctypes.byref(rope),
                                      ctypes.byref(ks) if ks is not None else None,
                                      ctypes.c_uint64(st)))
    _record(st, dev, block_table, inv_freq, k_scales)


def _chunks(chunks):
    """(pointer to daric_chunk[n], n, keep-alive) from a sequence of
    (bt_offset, row_offset, n_tokens, k[, tok_start]) tuples or an int64
    [n, 4] / [n, 5] array; tok_start defaults to 0."""
    a = np.asarray(chunks, dtype=np.int64)
    if a.size == 0:
        a = np.zeros((1, 5), np.int64)
        return ctypes.cast(a.ctypes.data, ctypes.POINTER(DaricChunk)), 0, a
    if a.ndim != 2 or a.shape[1] not in (4, 5):
        raise ValueError("chunks must be (bt_offset, row_offset, n_tokens, k[, tok_start]) entries")
    if a.shape[1] == 4:
        a = np.concatenate([a, np.zeros((a.shape[0], 1), np.int64)], axis=1)
    a = np.ascontiguousarray(a)
    return ctypes.cast(a.ctypes.data, ctypes.POINTER(DaricChunk)), a.shape[0], a


def kv_deviation(layers: Sequence[torch.Tensor], page_first: bool, block_table: torch.Tensor,
                 k_new: torch.Tensor, chunks, keys: Optional[torch.Tensor] = None,
                 stream: int = 0, k_scales: Optional[torch.Tensor] = None) -> torch.Tensor:
    """keys[l, row] = sum over (h, d) of (k_new - cached K)^2 in the fixed
    order of daric_amd/csrc/select_kernels.hip. chunks: (bt_offset,
    row_offset, n_tokens, k[, tok_start]); token j of a chunk is token
    tok_start + j of the block list at block_table[bt_offset]. k_scales: [L, H] fp32 per-head scales of an fp8
    cache (None: scale 1)."""
    layers = list(layers)
    dev = layers[0].device
    st = _resolve_stream(stream, dev)
    if keys is None:
        # zeroed on the launch stream: rows outside every chunk stay 0, and the
        # fill is ordered before the kernel whatever stream the caller passed
        shape = (len(layers), k_new.shape[1])
        if st == _resolve_stream(0, dev):
            keys = torch.zeros(shape, dtype=torch.float32, device=dev)
        else:
            with torch.cuda.stream(_ext_stream(st, dev)):
                keys = torch.zeros(shape, dtype=torch.float32, device=dev)
    carr, n, _keep = _chunks(chunks)
    bt, kn, kd = desc(block_table), desc(k_new), desc(keys)
    ks = desc(k_scales) if k_scales is not None else None
    check(load().daric_kv_deviation(_layer_array(layers), len(layers), 1 if page_first else 0,
                                    ctypes.byref(bt), ctypes.byref(kn), carr, n,
                                    ctypes.byref(ks) if ks is not None else None, ctypes.byref(kd),
                                    ctypes.c_uint64(st)))
    _record(st, dev, block_table, k_new, keys, k_scales)
    return keys


def topk_per_chunk(keys: torch.Tensor, chunks, kmax: Optional[int] = None,
                   out: Optional[torch.Tensor] = None, stream: int = 0) -> torch.Tensor:
    """Per (layer, chunk) the k largest keys, ties to the lower index; chunk-
    local indices ascending, padded with -1 to kmax."""
    ch = list(chunks)
    if kmax is None:
        kmax = max([min(int(c[3]), int(c[2])) for c in ch] + [0])
    if out is None:
        out = torch.empty(keys.shape[0], len(ch), kmax, dtype=torch.int32, device=keys.device)
    st = _resolve_stream(stream, keys.device)
    carr, n, _keep = _chunks(ch)
    kd, od = desc(keys), desc(out)
    check(load().daric_topk_per_chunk(ctypes.byref(kd), carr, n, ctypes.byref(od), ctypes.c_uint64(st)))
    _record(st, keys.device, keys, out)
    return out


def merge_rows(layers: Sequence[torch.Tensor], page_first: bool, block_table: torch.Tensor,
               k_new: torch.Tensor, v_new: Optional[torch.Tensor], chunks, sel_idx: torch.Tensor,
               stream: int = 0, k_scales: Optional[torch.Tensor] = None,
               v_scales: Optional[torch.Tensor] = None) -> None:
    """Write the selected recomputed K/V rows into their paged-cache slots.
    Rows in the cache's element type are copied; bf16/fp16 rows for an fp8
    (e4m3) cache are quantised as sat_rtne(x / scale) with the [L, H] fp32
    k_scales / v_scales (the fp8 write of vLLM's reshape_and_cache)."""
    layers = list(layers)
    dev = layers[0].device
    st = _resolve_stream(stream, dev)
    carr, n, _keep = _chunks(chunks)
    bt, kn, si = desc(block_table), desc(k_new), desc(sel_idx)
    vn = desc(v_new) if v_new is not None else None
    ks = desc(k_scales) if k_scales is not None else None
    vs = desc(v_scales) if v_scales is not None else None
    check(load().daric_merge_rows(_layer_array(layers), len(layers), 1 if page_first else 0,
                                  ctypes.byref(bt), ctypes.byref(kn),
                                  ctypes.byref(vn) if vn is not None else None, carr, n,
                                  ctypes.byref(si), ctypes.byref(ks) if ks is not None else None,
                                  ctypes.byref(vs) if vs is not None else None, ctypes.c_uint64(st)))
    _record(st, dev, block_table, k_new, v_new, sel_idx, k_scales, v_scales)


SELECT_KEYS_READY = 1       # DARIC_SELECT_KEYS_READY
SELECT_ONE_PASS = 2         # DARIC_SELECT_ONE_PASS


def select_merge(layers: Sequence[torch.Tensor], page_first: bool, block_table: torch.Tensor,
                 k_new: torch.Tensor, v_new: Optional[torch.Tensor], chunks, kmax: Optional[int] = None,
                 keys: Optional[torch.Tensor] = None, sel_idx: Optional[torch.Tensor] = None,
                 keys_ready: bool = False, k_scales: Optional[torch.Tensor] = None,
                 v_scales: Optional[torch.Tensor] = None, stream: int = 0, one_pass: bool = False):
    """kv_deviation + topk_per_chunk + merge_rows in one call: returns
    (keys [L, T] fp32, sel_idx [L, n_chunks, kmax] int32), equal to what the
    three calls return, and merges the selected rows the same way. Where the
    chunks fit, the top-k and merge run fused, one workgroup per (layer,
    chunk). For an fp8 cache, k_scales / v_scales are its [L, H] per-head K / V
    scales. keys_ready: `keys` already holds the deviation keys. one_pass: the
    fused workgroups compute the keys too (one launch; measured slower)."""
    layers = list(layers)
    dev = layers[0].device
    st = _resolve_stream(stream, dev)
    ch = list(chunks) if not isinstance(chunks, np.ndarray) else chunks.tolist()
    if kmax is None:
        kmax = max([min(int(c[3]), int(c[2])) for c in ch] + [0])
    carr, n, _keep = _chunks(ch)
    shape = (len(layers), k_new.shape[1])
    if keys is None:
        if keys_ready:
            raise ValueError("keys_ready needs keys")
        # zeroed on the launch stream: rows outside every chunk stay 0
        with torch.cuda.stream(_ext_stream(st, dev)):
            keys = torch.zeros(shape, dtype=torch.float32, device=dev)
    if sel_idx is None:
        with torch.cuda.stream(_ext_stream(st, dev)):
            sel_idx = torch.empty(len(layers), n, kmax, dtype=torch.int32, device=dev)
    bt, kn, kd, si = desc(block_table), desc(k_new), desc(keys), desc(sel_idx)
    vn = desc(v_new) if v_new is not None else None
    ks = desc(k_scales) if k_scales is not None else None
    vs = desc(v_scales) if v_scales is not None else None
    check(load().daric_select_merge(_layer_array(layers), len(layers), 1 if page_first else 0,
                                    ctypes.byref(bt), ctypes.byref(kn),
                                    ctypes.byref(vn) if vn is not None else None, carr, n,
                                    ctypes.byref(ks) if ks is not None else None,
                                    ctypes.byref(vs) if vs is not None else None,
                                    ctypes.byref(kd), ctypes.byref(si),
                                    (SELECT_KEYS_READY if keys_ready else 0) | (SELECT_ONE_PASS if one_pass else 0),
                                    ctypes.c_uint64(st)))
    _record(st, dev, block_table, k_new, v_new, keys, sel_idx, k_scales, v_scales)
    return keys, sel_idx


def timing_enable(enable: bool = True) -> None:
    check(load().daric_timing_enable(1 if enable else 0))


def timing_read() -> tuple[float, int]:
    """(summed kernel milliseconds, launches) since the last read."""
    ms = ctypes.c_double()
    n = ctypes.c_int64()
    check(load().daric_timing_read(ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value
