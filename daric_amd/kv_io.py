"""Store/load of reused KV chunks between a GPU's paged cache and pinned host
records: the per-GPU part of the daric-store's GPU I/O (reference
daric/management/service/gpu_kv_io.py:130-205 RankIPCContext, :318-409 copy
plan and record header, :424-584 _do_store/_do_load) on the gfx950 kernels.

Record format (byte-compatible with the reference): for each meta, the
gather_pages bytes of every layer in registration order (the reference
registers layers in sorted name order, configs/engine.py:25-27), followed by a
4096-byte header whose first 8 bytes hold the little-endian int64 saved
position.

Pipeline: the reference gathers a batch into one staging buffer, copies it to
host, and only then gathers the next batch, with a full stream synchronisation
per load chunk. Here each direction has two staging buffers of staging_bytes
(the reference's one, DARIC_KV_IPC_STAGING_MB, default 256 MiB): the copy
kernels run on a kernel stream and the host DMA on a DMA stream, so batch
b+1's gather (scatter) overlaps batch b's device-to-host (host-to-device)
copy; events order each buffer's reuse. All streams keep the default
priority. Batching keeps the reference's limits: at most MAX_BATCH_SIZE metas
and staging_bytes per batch on store, load chunks of at most staging_bytes,
and a meta larger than staging_bytes is refused, as the reference refuses it
(gpu_kv_io.py:445-462).

Store and load have separate staging buffers and streams, as the reference's
staging and read_staging (gpu_kv_io.py:150-151), so one thread may store while
another loads. Two stores (or two loads) on one context take turns: each
direction has a lock, where the reference lets concurrent calls share one
staging buffer. close() drains the context as the reference's
RankIPCContext.close does (gpu_kv_io.py:157-205).

The host buffer must be page-locked memory so the DMA engines can reach it:
torch pin_memory or hipHostMalloc, or an existing buffer (the store's shared
memory) registered with HostMemoryRegistration, as the reference registers its
shm (gpu_kv_io.py:40-100, 236-260).
"""
from __future__ import annotations

import ctypes
import os
import threading
from contextlib import contextmanager
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import cache_ops
from .host_runtime import HOST_MEMORY_ALREADY_REGISTERED

__all__ = ["POSITION_SIZE", "REGISTRATION_CHUNK_BYTES", "KVIOContext", "HostMemoryRegistration",
           "split_registration_copies", "build_copy_plan", "per_meta_cache_size"]

POSITION_SIZE = 4096
INT64_SIZE = 8
REGISTRATION_CHUNK_BYTES = 1 << 30


def _staging_bytes_from_env() -> int:
    """The reference's staging size setting (gpu_kv_io.py:30-34):
    DARIC_KV_IPC_STAGING_MB, default 256, must be positive."""
    mb = int(os.environ.get("DARIC_KV_IPC_STAGING_MB", "256"))
    if mb <= 0:
        raise ValueError(f"DARIC_KV_IPC_STAGING_MB must be positive, got {mb}")
    return mb << 20


DEFAULT_STAGING_BYTES = _staging_bytes_from_env()


def split_registration_copies(stg_offsets, shm_offsets, sizes, chunk_bytes=REGISTRATION_CHUNK_BYTES):
    """(staging offsets, host offsets, sizes) of the copies, each region cut
    where its host range crosses a multiple of chunk_bytes: the reference
    registers host memory in 1 GiB pieces and no copy may span two of them
    (gpu_kv_io.py:110-127). Region r touches registration chunks
    host[r] // chunk .. (host[r] + size[r] - 1) // chunk; its k-th piece is its
    intersection with the k-th of them. Empty regions give no copy."""
    stg = np.asarray(stg_offsets, dtype=np.int64).reshape(-1)
    host = np.asarray(shm_offsets, dtype=np.int64).reshape(-1)
    size = np.asarray(sizes, dtype=np.int64).reshape(-1)
    if not stg.size == host.size == size.size:
        raise ValueError(f"{stg.size} staging offsets, {host.size} host offsets and {size.size} sizes: "
                         "one of each per region is needed")
    if chunk_bytes <= 0:
        raise ValueError(f"chunk_bytes must be positive, got {chunk_bytes}")
    if (stg < 0).any() or (host < 0).any() or (size < 0).any():
        raise ValueError("staging offsets, host offsets and sizes must be non-negative")
    first = host // chunk_bytes
    pieces = np.where(size > 0, (host + size - 1) // chunk_bytes - first + 1, 0)
    region = np.repeat(np.arange(size.size), pieces)
    k = np.arange(region.size) - np.repeat(np.cumsum(pieces) - pieces, pieces)
    lo = np.maximum(host[region], (first[region] + k) * chunk_bytes)
    hi = np.minimum(host[region] + size[region], (first[region] + k + 1) * chunk_bytes)
    return (stg[region] + (lo - host[region])).tolist(), lo.tolist(), (hi - lo).tolist()


class HostMemoryRegistration:
    """Page-locks an existing host buffer (the store's shared-memory record
    pool) in pieces of chunk_bytes through a host runtime
    (host_runtime.get_gpu_host_runtime()), as the reference's
    HostMemoryRegistration does (gpu_kv_io.py:40-100); the batched host copies
    are then cut at the same piece boundaries (split_registration_copies).

    register(buf) takes a writable buffer (e.g. SharedMemory.buf) or a CPU
    tensor whose start and chunk_bytes are page-aligned. A piece the runtime
    reports as already registered, or any other failure, raises RuntimeError
    after the pieces locked so far are unlocked (pieces that cannot be
    unlocked stay listed in `addresses`; the first error is the one raised).
    unregister() unlocks in reverse order and raises RuntimeError if any
    piece stays locked, keeping those in `addresses`."""

    def __init__(self, runtime, chunk_bytes: int = REGISTRATION_CHUNK_BYTES):
        self.runtime = runtime
        self.chunk_bytes = int(chunk_bytes)
        self.addresses: List[int] = []

    @staticmethod
    def _span(buf):
        if isinstance(buf, torch.Tensor):
            if buf.is_cuda or not buf.is_contiguous():
                raise ValueError("host buffer must be a contiguous CPU tensor")
            return buf.data_ptr(), buf.numel() * buf.element_size()
        view = memoryview(buf)
        if view.readonly:
            raise ValueError("host buffer must be writable")
        if view.nbytes == 0:
            raise ValueError("host buffer must not be empty")
        return ctypes.addressof(ctypes.c_char.from_buffer(view)), view.nbytes

    def register(self, buf) -> None:
        if self.addresses:
            raise RuntimeError("host buffer is still registered; unregister() it first")
        address, size = self._span(buf)
        page = os.sysconf("SC_PAGE_SIZE")
        if address % page or self.chunk_bytes <= 0 or self.chunk_bytes % page:
            raise ValueError("host buffer start and registration chunk size must be page-aligned")
        if size <= 0:
            raise ValueError("host buffer must not be empty")
        try:
            for off in range(0, size, self.chunk_bytes):
                status = self.runtime.register(address + off, min(self.chunk_bytes, size - off))
                if status == HOST_MEMORY_ALREADY_REGISTERED:
                    raise RuntimeError(f"host buffer piece at offset {off} overlaps memory that is "
                                       "already page-locked")
                if status != 0:
                    raise RuntimeError(f"{self.runtime.prefix}HostRegister failed at offset {off} "
                                       f"with status {status}")
                self.addresses.append(address + off)
        except BaseException:
            try:
                self.unregister()
            except RuntimeError:
                pass
            raise

    def unregister(self) -> None:
        kept = []
        for address in reversed(self.addresses):
            try:
                status = self.runtime.unregister(address)
            except Exception:
                status = -1
            if status != 0:
                kept.append(address)
        self.addresses = kept[::-1]
        if kept:
            raise RuntimeError(f"{len(kept)} piece(s) of the host buffer could not be unregistered")


def per_meta_cache_size(layer_names, group_idxs, layer_bpbs, block_ids_list, layer_name=None):
    """Cache bytes of each meta's record (header excluded)."""
    if layer_name is not None:
        li = layer_names.index(layer_name)
        return [layer_bpbs[li] * len(b[group_idxs[li]]) for b in block_ids_list]
    return [sum(bpb * len(b[g]) for g, bpb in zip(group_idxs, layer_bpbs)) for b in block_ids_list]


def build_copy_plan(layer_names, group_idxs, layer_bpbs, offsets, block_ids_list, layer_name=None):
    """Jobs of a batch of metas: (flat int32 block ids, job offsets, indices
    offsets, job layer names, job sizes), one job per (meta, layer)."""
    flat: list = []
    ioff = [0]
    job_off, job_sz, job_names = [], [], []
    if layer_name is not None:
        li = layer_names.index(layer_name)
        sel = [(li, layer_name)]
    else:
        sel = list(enumerate(layer_names))
    for base, blocks in zip(offsets, block_ids_list):
        run = 0
        for li, name in sel:
            ids = blocks[group_idxs[li]]
            if isinstance(ids, torch.Tensor):
                ids = ids.tolist()
            flat.extend(int(x) for x in ids)
            ioff.append(len(flat))
            nbytes = layer_bpbs[li] * len(ids)
            job_off.append(base + run)
            job_sz.append(nbytes)
            job_names.append(name)
            run += nbytes
    return np.asarray(flat, dtype=np.int32), job_off, ioff, job_names, job_sz


class _Pipe:
    """One direction's double-buffered staging: two buffers ("halves") of
    `half` bytes in one allocation, a stream for the copy kernels, a stream
    for the host DMA, and per buffer the event after which it may be
    overwritten."""

    def __init__(self, half: int, device: torch.device):
        self.half = half
        self.staging = torch.empty(2 * half, dtype=torch.uint8, device=device)
        self.kernels = torch.cuda.Stream(device=device)
        self.dma = torch.cuda.Stream(device=device)
        self.half_free = [None, None]


class KVIOContext:
    """One GPU's store/load context: a write copier (gathers into the store
    staging) and a read copier (scatters from the load staging), each direction
    with two staging buffers of staging_bytes, a kernel stream and a DMA
    stream."""

    MAX_BATCH_SIZE = 4

    def __init__(self, layer_names: Sequence[str], group_idxs: Sequence[int],
                 layer_bpbs: Sequence[int], page_firsts: Sequence[bool],
                 kv_caches: dict, host: torch.Tensor, staging_bytes: int = DEFAULT_STAGING_BYTES,
                 device: Optional[torch.device] = None, host_registered: bool = False):
        if host.dtype != torch.uint8 or host.dim() != 1 or host.is_cuda:
            raise ValueError("host records must be a 1-D uint8 CPU tensor")
        # host_registered: the caller page-locked the buffer itself
        # (HostMemoryRegistration); torch's is_pinned() is then not consulted,
        # as the reference's batched copies do not consult it (bindings.cpp:17-29)
        if not host_registered and not host.is_pinned():
            raise ValueError("host records must be page-locked (pin_memory=True, or registered with "
                             "HostMemoryRegistration and host_registered=True)")
        self.layer_names = list(layer_names)
        self.group_idxs = list(group_idxs)
        self.layer_bpbs = list(layer_bpbs)
        self.page_firsts = list(page_firsts)
        first = kv_caches[self.layer_names[0]]
        self.device = device if device is not None else first.device
        self.host = host
        self.half = int(staging_bytes) // 256 * 256
        if self.half <= 0:
            raise ValueError("staging_bytes too small")
        self._store = _Pipe(self.half, self.device)
        self._load = _Pipe(self.half, self.device)
        self.write_copier = cache_ops.CacheCopier()
        self.read_copier = cache_ops.CacheCopier()
        for name, pf in zip(self.layer_names, self.page_firsts):
            self.write_copier.register_layer(name, kv_caches[name], bool(pf))
            self.read_copier.register_layer(name, kv_caches[name], bool(pf))
        self.write_copier.register_store(self._store.staging)
        self.read_copier.register_store(self._load.staging)
        self.done = None   # after load(): event marking the end of its device work
        self._lifecycle = threading.Condition()
        self._inflight = 0
        self._closed = False
        self._store_lock = threading.Lock()
        self._load_lock = threading.Lock()

    # ------------------------------------------------------------ lifecycle
    @property
    def closed(self) -> bool:
        return self._closed

    @contextmanager
    def _operation(self, lock: threading.Lock):
        with self._lifecycle:
            if self._closed:
                raise RuntimeError("KV IO: context is closed")
            self._inflight += 1
        try:
            with lock:
                yield
        finally:
            with self._lifecycle:
                self._inflight -= 1
                if self._inflight == 0:
                    self._lifecycle.notify_all()

    def close(self) -> None:
        """Refuses further stores and loads, waits for the running ones and
        for their queued device work, then drops the copiers and staging
        buffers (the reference's RankIPCContext.close, gpu_kv_io.py:182-205).
        Calling it again does nothing."""
        with self._lifecycle:
            self._closed = True
            while self._inflight > 0:
                self._lifecycle.wait()
            pipes = [p for p in (self._store, self._load) if p is not None]
            self._store = self._load = None
        for pipe in pipes:
            pipe.kernels.synchronize()
            pipe.dma.synchronize()
        self.write_copier = None
        self.read_copier = None

    def _upload_indices(self, flats, stream) -> List[torch.Tensor]:
        """Block ids of every batch of a call in one pinned, non-blocking copy
        on `stream`, issued before the call's waits, so the host never blocks
        on a batch's DMA to upload the next batch's ids."""
        sizes = [len(f) for f in flats]
        host = torch.from_numpy(np.concatenate(flats) if flats else np.zeros(0, np.int32)).pin_memory()
        with torch.cuda.stream(stream):
            dev = host.to(self.device, non_blocking=True)
        out, o = [], 0
        for n in sizes:
            out.append(dev[o:o + n])
            o += n
        return out

    # ------------------------------------------------------------ helpers
    def cache_sizes(self, block_ids_list, layer_name=None) -> List[int]:
        return per_meta_cache_size(self.layer_names, self.group_idxs, self.layer_bpbs,
                                   block_ids_list, layer_name)

    def record_size(self, block_ids, layer_name=None) -> int:
        """Bytes a record of one meta occupies in host memory (header included)."""
        return self.cache_sizes([block_ids], layer_name)[0] + POSITION_SIZE

    def _write_positions(self, position_offsets, saved_positions):
        host = self.host.numpy()
        for off, pos in zip(position_offsets, saved_positions):
            host[off: off + POSITION_SIZE] = 0
            host[off: off + INT64_SIZE] = np.frombuffer(np.int64(pos).tobytes(), np.uint8)

    def read_positions(self, position_offsets) -> List[int]:
        host = self.host.numpy()
        return [int(host[o: o + INT64_SIZE].view(np.int64)[0]) for o in position_offsets]

    def _batches(self, sizes, cap, max_count):
        i, n = 0, len(sizes)
        while i < n:
            j, acc = i, 0
            while j < n and j - i < max_count and acc + sizes[j] <= cap:
                acc += sizes[j]
                j += 1
            if j == i:
                raise RuntimeError(f"KV IO: single meta is {sizes[i]} bytes, larger than the "
                                   f"{cap}-byte staging buffer; raise staging_bytes "
                                   f"(DARIC_KV_IPC_STAGING_MB)")
            yield i, j
            i = j

    # ------------------------------------------------------------ store
    def store(self, offsets: Sequence[int], block_ids_list, saved_positions: Sequence[int],
              layer_name: Optional[str] = None, wait_stream: Optional[torch.cuda.Stream] = None) -> None:
        """Writes one record per meta at host offset offsets[i] (the reference's
        _do_store after allocation). Returns once the records, headers included,
        are in host memory."""
        with self._operation(self._store_lock):
            self._store_records(offsets, block_ids_list, saved_positions, layer_name, wait_stream)

    def _store_records(self, offsets, block_ids_list, saved_positions, layer_name, wait_stream):
        offsets = [int(o) for o in offsets]
        sizes = self.cache_sizes(block_ids_list, layer_name)
        pipe = self._store
        per_meta = 1 if layer_name is not None else len(self.layer_names)
        plans = [(i, j, build_copy_plan(self.layer_names, self.group_idxs, self.layer_bpbs, offsets[i:j],
                                        block_ids_list[i:j], layer_name))
                 for i, j in self._batches(sizes, self.half, self.MAX_BATCH_SIZE)]
        idxs = self._upload_indices([p[2][0] for p in plans], pipe.kernels)
        if wait_stream is not None:
            pipe.kernels.wait_stream(wait_stream)
        for b, ((i, j, (flat, host_off, ioff, names, job_sz)), idx) in enumerate(zip(plans, idxs)):
            h = b % 2
            base = h * self.half
            stg = np.cumsum([0] + job_sz[:-1]).astype(np.int64) + base
            if pipe.half_free[h] is not None:
                pipe.kernels.wait_event(pipe.half_free[h])
            self.write_copier.gather_pages(names, stg.tolist(), job_sz, idx, ioff,
                                           pipe.kernels.cuda_stream)
            gathered = torch.cuda.Event()
            gathered.record(pipe.kernels)
            pipe.dma.wait_event(gathered)
            meta_stg = [int(stg[k * per_meta]) for k in range(j - i)]
            cs, ch, cn = split_registration_copies(meta_stg, offsets[i:j], sizes[i:j])
            cache_ops.batched_memcpy_d2h(pipe.staging, self.host, cs, ch, cn, pipe.dma.cuda_stream)
            ev = torch.cuda.Event()
            ev.record(pipe.dma)
            pipe.half_free[h] = ev
        pipe.dma.synchronize()
        self._write_positions([o + s for o, s in zip(offsets, sizes)], saved_positions)

    # ------------------------------------------------------------ load
    def load(self, offsets: Sequence[int], block_ids_list, layer_name: Optional[str] = None,
             wait_stream: Optional[torch.cuda.Stream] = None, rerotate=None) -> List[int]:
        """Scatters each meta's record back into the paged cache (the
        reference's _do_load) and returns the saved positions. With
        rerotate = (new_positions, num_tokens, inv_freq, rotary_dim, is_neox),
        the K rows of each meta's first num_tokens[i] tokens are moved from the
        saved position to new_positions[i] in the same pass
        (scatter_pages_rerotate); the saved positions are read from the headers
        first, which live in host memory. Device work is left queued on the
        load's kernel stream; self.done, an event recorded after it, marks its
        end."""
        with self._operation(self._load_lock):
            return self._load_records(offsets, block_ids_list, layer_name, wait_stream, rerotate)

    def _load_records(self, offsets, block_ids_list, layer_name, wait_stream, rerotate):
        offsets = [int(o) for o in offsets]
        sizes = self.cache_sizes(block_ids_list, layer_name)
        saved = self.read_positions([o + s for o, s in zip(offsets, sizes)])
        pipe = self._load
        per_meta = 1 if layer_name is not None else len(self.layer_names)
        plans = [(i, j, build_copy_plan(self.layer_names, self.group_idxs, self.layer_bpbs, offsets[i:j],
                                        block_ids_list[i:j], layer_name))
                 for i, j in self._batches(sizes, self.half, 1 << 30)]
        idxs = self._upload_indices([p[2][0] for p in plans], pipe.kernels)
        if wait_stream is not None:
            pipe.dma.wait_stream(wait_stream)
        for b, ((i, j, (flat, host_off, ioff, names, job_sz)), idx) in enumerate(zip(plans, idxs)):
            h = b % 2
            base = h * self.half
            stg = np.cumsum([0] + job_sz[:-1]).astype(np.int64) + base
            if pipe.half_free[h] is not None:
                pipe.dma.wait_event(pipe.half_free[h])
            meta_stg = [int(stg[k * per_meta]) for k in range(j - i)]
            cs, ch, cn = split_registration_copies(meta_stg, offsets[i:j], sizes[i:j])
            cache_ops.batched_memcpy_h2d(self.host, pipe.staging, ch, cs, cn, pipe.dma.cuda_stream)
            arrived = torch.cuda.Event()
            arrived.record(pipe.dma)
            pipe.kernels.wait_event(arrived)
            if rerotate is None:
                self.read_copier.scatter_pages(names, stg.tolist(), job_sz, idx, ioff,
                                               pipe.kernels.cuda_stream)
            else:
                new_pos, ntok, inv, rdim, neox = rerotate
                deltas = [int(new_pos[k]) - int(saved[k]) for k in range(i, j) for _ in range(per_meta)]
                nt = [int(ntok[k]) for k in range(i, j) for _ in range(per_meta)]
                self.read_copier.scatter_pages_rerotate(names, stg.tolist(), job_sz, idx, ioff, deltas,
                                                        nt, inv, rdim, neox, pipe.kernels.cuda_stream)
            ev = torch.cuda.Event()
            ev.record(pipe.kernels)
            pipe.half_free[h] = ev
        self.done = torch.cuda.Event()
        self.done.record(pipe.kernels)
        return saved
