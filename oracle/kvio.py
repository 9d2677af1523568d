"""Store/load record format and copy plan of the daric-store GPU I/O (CPU
restatement) -- TEST INFRASTRUCTURE ONLY.

Follows reference daric/management/service/gpu_kv_io.py:
  - _split_registration_copies (:110-127): a DMA region is cut where the host
    offset crosses a multiple of the registration chunk (1 GiB);
  - _per_meta_cache_size (:318-332) and _build_copy_plan (:334-379): one job
    per (meta, layer) in the registered layer order (sorted names,
    configs/engine.py:25-27), offsets base + running sum of the previous
    layers' bytes, size bytes_per_block * len(block_ids[group]);
  - _position_offsets / _write_positions / _read_positions (:381-409): a
    record is the meta's layer spans followed by a 4096-byte header whose first
    8 bytes are the little-endian int64 saved position;
  - _do_store (:424-503): gather the jobs into staging, copy each meta's span
    to its record, then write the header; _do_load (:518-584): the reverse,
    returning the saved positions.
"""
from __future__ import annotations

import numpy as np
import torch

from .copy import OracleCopier

POSITION_SIZE = 4096
INT64_SIZE = 8
REGISTRATION_CHUNK_BYTES = 1 << 30


def split_registration_copies(stg_offsets, shm_offsets, sizes, chunk_bytes=REGISTRATION_CHUNK_BYTES):
    if not (len(stg_offsets) == len(shm_offsets) == len(sizes)):
        raise ValueError("Copy offsets and sizes must have the same length.")
    if chunk_bytes <= 0:
        raise ValueError("Registration chunk size must be positive.")
    out_stg, out_shm, out_sz = [], [], []
    for s, h, n in zip(stg_offsets, shm_offsets, sizes):
        if s < 0 or h < 0 or n < 0:
            raise ValueError("Copy offsets and sizes must be non-negative.")
        while n:
            piece = min(n, chunk_bytes - h % chunk_bytes)
            out_stg.append(s)
            out_shm.append(h)
            out_sz.append(piece)
            s, h, n = s + piece, h + piece, n - piece
    return out_stg, out_shm, out_sz


def per_meta_cache_size(layer_names, group_idxs, layer_bpbs, block_ids_list, layer_name=None):
    if layer_name is not None:
        li = layer_names.index(layer_name)
        return [layer_bpbs[li] * len(b[group_idxs[li]]) for b in block_ids_list]
    return [sum(layer_bpbs[li] * len(b[group_idxs[li]]) for li in range(len(layer_names)))
            for b in block_ids_list]


def build_copy_plan(layer_names, group_idxs, layer_bpbs, offsets, block_ids_list, layer_name=None):
    """(flat int32 ids, job offsets, indices_offsets, job layer names, job sizes)."""
    flat, ioff, job_off, job_sz, job_names = [], [0], [], [], []
    if layer_name is not None:
        li = layer_names.index(layer_name)
        for base, b in zip(offsets, block_ids_list):
            ids = list(b[group_idxs[li]])
            flat += ids
            ioff.append(len(flat))
            job_off.append(base)
            job_sz.append(layer_bpbs[li] * len(ids))
            job_names.append(layer_name)
    else:
        for base, b in zip(offsets, block_ids_list):
            run = 0
            for li, name in enumerate(layer_names):
                ids = list(b[group_idxs[li]])
                flat += ids
                ioff.append(len(flat))
                sz = layer_bpbs[li] * len(ids)
                job_off.append(base + run)
                job_sz.append(sz)
                job_names.append(name)
                run += sz
    return np.asarray(flat, dtype=np.int32), job_off, ioff, job_names, job_sz


def write_positions(shm: torch.Tensor, position_offsets, saved_positions) -> None:
    for off, pos in zip(position_offsets, saved_positions):
        header = np.zeros(POSITION_SIZE, np.uint8)
        header[:INT64_SIZE] = np.frombuffer(np.int64(pos).tobytes(), np.uint8)
        shm[off: off + POSITION_SIZE] = torch.from_numpy(header)


def read_positions(shm: torch.Tensor, position_offsets):
    return [int(np.frombuffer(shm[o: o + INT64_SIZE].numpy().tobytes(), np.int64)[0])
            for o in position_offsets]


class OracleKVIO:
    """Single-process store/load over CPU layer tensors and a CPU 'shm' buffer."""

    def __init__(self, layer_names, group_idxs, layer_bpbs, page_firsts, layers, shm):
        self.layer_names = list(layer_names)
        self.group_idxs = list(group_idxs)
        self.layer_bpbs = list(layer_bpbs)
        self.shm = shm
        self.copier = OracleCopier()
        for n, pf in zip(self.layer_names, page_firsts):
            self.copier.register_layer(n, layers[n], bool(pf))

    def store(self, offsets, block_ids_list, saved_positions, layer_name=None):
        sizes = per_meta_cache_size(self.layer_names, self.group_idxs, self.layer_bpbs,
                                    block_ids_list, layer_name)
        flat, job_off, ioff, names, job_sz = build_copy_plan(
            self.layer_names, self.group_idxs, self.layer_bpbs, offsets, block_ids_list, layer_name)
        # gathering straight into the records is what staging + DMA amounts to
        self.copier.register_store(self.shm)
        self.copier.gather_pages(names, job_off, job_sz, torch.from_numpy(flat), ioff)
        write_positions(self.shm, [o + s for o, s in zip(offsets, sizes)], saved_positions)

    def load(self, offsets, block_ids_list, layer_name=None, rerotate=None):
        """rerotate: None, or (new_positions, num_tokens, inv_freq, rotary_dim, is_neox):
        each meta's K rows are then moved by new_position - saved_position."""
        sizes = per_meta_cache_size(self.layer_names, self.group_idxs, self.layer_bpbs,
                                    block_ids_list, layer_name)
        saved = read_positions(self.shm, [o + s for o, s in zip(offsets, sizes)])
        flat, job_off, ioff, names, job_sz = build_copy_plan(
            self.layer_names, self.group_idxs, self.layer_bpbs, offsets, block_ids_list, layer_name)
        self.copier.register_store(self.shm)
        if rerotate is None:
            self.copier.scatter_pages(names, job_off, job_sz, torch.from_numpy(flat), ioff)
            return saved
        new_pos, ntok, inv, rdim, neox = rerotate
        per_meta = len(names) // max(len(offsets), 1)
        deltas = [int(new_pos[k]) - int(saved[k]) for k in range(len(offsets)) for _ in range(per_meta)]
        nt = [int(ntok[k]) for k in range(len(offsets)) for _ in range(per_meta)]
        self.copier.scatter_pages_rerotate(names, job_off, job_sz, torch.from_numpy(flat), ioff,
                                           deltas, nt, inv, rdim, neox)
        return saved
