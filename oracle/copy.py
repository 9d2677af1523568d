"""CacheCopier gather/scatter byte semantics (CPU restatement).

Follows reference csrc/cache_ops/copier.cpp:7-111 (registration, check order)
and csrc/cache_ops/kernels.cu (index math of the copy kernels, :7-123, and the
byte-size check of the launchers, :127-292):

  gather : store[off + (p*n_sel + s)*span + b] = layer[p*prefix_stride + idx[s]*page_stride + b]
  scatter: layer[p*prefix_stride + idx[s]*page_stride + b] = store[off + (p*n_sel + s)*span + b]

for prefix index p, selected page s, byte b < span; pages with idx[s] == 0
(vLLM's null block) are neither read nor written (kernels.cu:26,39,69,79,104,117).

One deliberate difference: a block id outside [0, num_pages) is skipped like
block 0. The reference reads/writes out of bounds there (undefined behaviour);
the HIP kernels skip such pages instead of faulting, and so does this oracle.

Layers are CPU torch tensors of any strides; byte offsets are taken from the
address of element [0,...,0], as the reference takes them from data_ptr().
"""
from __future__ import annotations

import numpy as np
import torch

from . import rope
from .layout import (OracleError, _check, page_copy_shape, validate_common_job_inputs,
                     validate_store_ranges)


def byte_view(t: torch.Tensor):
    """(uint8 view of t's whole storage, byte offset of element [0,...,0])."""
    u8 = torch.empty(0, dtype=torch.uint8)
    u8.set_(t.untyped_storage())
    return u8, t.storage_offset() * t.element_size()


class OracleCopier:
    def __init__(self):
        self.layers = {}
        self.store = None
        self.k_scales = {}

    def register_layer(self, name, tensor: torch.Tensor, is_page_first: bool):
        self.layers[name] = (tensor, bool(is_page_first))

    def register_store(self, buffer: torch.Tensor):
        _check(buffer.dim() == 1, "store buffer must be 1D")
        _check(buffer.dtype == torch.uint8, "store buffer must be uint8")
        _check(buffer.is_contiguous(), "store buffer must be contiguous")
        self.store = buffer

    def register_k_scale(self, name, k_scale):
        self.k_scales[name] = np.asarray(k_scale, dtype=np.float64)

    # ------------------------------------------------------------------ #
    def _plan(self, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        """Check order of copier.cpp:46-66 and the launcher's byte-size check."""
        _check(self.store is not None, "store buffer not registered; call register_store() first")
        n = len(layer_names)
        if n == 0:
            return None
        idx = torch.as_tensor(indices_flat)
        validate_common_job_inputs(n, list(offsets), list(byte_sizes), list(indices_offsets),
                                   idx.numel(), (True, idx.dim() == 1, idx.dtype == torch.int32,
                                                 idx.is_contiguous()))
        validate_store_ranges(list(offsets), list(byte_sizes), self.store.numel())
        jobs = []
        for name in layer_names:
            _check(name in self.layers, "layer not registered: ", name)
        for i, name in enumerate(layer_names):
            t, pf = self.layers[name]
            shp = page_copy_shape(tuple(t.shape), tuple(t.stride()), t.element_size(), pf)
            n_sel = int(indices_offsets[i + 1] - indices_offsets[i])
            num = shp.prefix_size * n_sel * shp.suffix_size
            if int(byte_sizes[i]) != num:
                raise OracleError(
                    f"byte_size mismatch at job {i} | C++ expected bytes: {num} | "
                    f"Python passed bytes: {int(byte_sizes[i])} | Tensor shape: "
                    f"[{', '.join(str(x) for x in t.shape)}] | Tensor strides: "
                    f"[{', '.join(str(x) for x in t.stride())}]")
            sel = idx[int(indices_offsets[i]): int(indices_offsets[i + 1])].tolist()
            jobs.append((name, t, pf, shp, int(offsets[i]), sel))
        return jobs

    @staticmethod
    def _pages(shp, sel):
        for p in range(shp.prefix_size):
            for s, page in enumerate(sel):
                if page <= 0 or page >= shp.num_pages:
                    continue
                yield p, s, page

    def gather_pages(self, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        jobs = self._plan(layer_names, offsets, byte_sizes, indices_flat, indices_offsets)
        if not jobs:
            return
        for name, t, pf, shp, off, sel in jobs:
            mem, base = byte_view(t)
            span, n_sel = shp.suffix_size, len(sel)
            for p, s, page in self._pages(shp, sel):
                src = base + p * shp.prefix_stride + page * shp.page_stride
                dst = off + (p * n_sel + s) * span
                self.store[dst: dst + span] = mem[src: src + span]

    def scatter_pages(self, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        jobs = self._plan(layer_names, offsets, byte_sizes, indices_flat, indices_offsets)
        if not jobs:
            return
        for name, t, pf, shp, off, sel in jobs:
            mem, base = byte_view(t)
            span, n_sel = shp.suffix_size, len(sel)
            for p, s, page in self._pages(shp, sel):
                dst = base + p * shp.prefix_stride + page * shp.page_stride
                src = off + (p * n_sel + s) * span
                mem[dst: dst + span] = self.store[src: src + span]

    def scatter_pages_rerotate(self, layer_names, offsets, byte_sizes, indices_flat,
                               indices_offsets, deltas, num_tokens, inv_freq, rotary_dim,
                               is_neox):
        """scatter_pages, then the K rows of the first num_tokens[i] tokens of
        job i are rotated by deltas[i] (token j = slot j % PS of page j // PS of
        the job, pages with block id 0 or out of range excluded), i.e. the
        reference's scatter (gpu_kv_io.py:569-572) followed by its worker-side
        apply_rerotate_load (adapter.py:196-295) restricted to the loaded pages."""
        jobs = self._plan(layer_names, offsets, byte_sizes, indices_flat, indices_offsets)
        if not jobs:
            return
        self.scatter_pages(layer_names, offsets, byte_sizes, indices_flat, indices_offsets)
        for i, (name, t, pf, shp, off, sel) in enumerate(jobs):
            d, nt = int(deltas[i]), int(num_tokens[i])
            if d == 0 or nt <= 0:
                continue
            ps = rope.k_view(t, pf, rotary_dim).shape[1]
            slots = []
            for j in range(min(nt, len(sel) * ps)):
                page = sel[j // ps]
                if 0 < page < shp.num_pages:
                    slots.append(page * ps + j % ps)
            rope.rotate_slots(t, pf, slots, d, inv_freq, rotary_dim, is_neox,
                              self.k_scales.get(name))

    # ------------------------------------------------------------------ #
    # Token-major copies. No counterpart in the reference, whose staging is
    # the physical page span (kernels.cu:20-44); the checks before the layout
    # are gather_pages' (copier.cpp:46-66).
    @staticmethod
    def token_rows(t: torch.Tensor, page_first: bool):
        """[K rows, V rows] of a layer as [num_blocks, PS, H, D] views (V
        absent for a 3-D MLA cache): 5-D [2, NB, PS, H, D] / page-first
        [NB, 2, PS, H, D] with any strides, packed [NB, H, PS, 2D] (K in
        [0, D), V in [D, 2D)), MLA [NB, PS, hidden]."""
        nd = t.dim()
        if nd == 5:
            kv_dim = 1 if page_first else 0
            _check(t.shape[kv_dim] == 2, "token-major copies need a K/V dimension of size 2, got shape=",
                   str(list(t.shape)))
            _check(t.stride(4) == 1 or t.shape[4] == 1,
                   "KV cache head_dim stride must equal 1 for token-major copies")
            views = [t[:, 0], t[:, 1]] if page_first else [t[0], t[1]]
        elif nd == 4:
            _check(page_first, "a 4-D (packed) KV cache must be page_first")
            _check(t.shape[3] > 0 and t.shape[3] % 2 == 0 and t.stride(3) == 1,
                   "packed KV rows must have an even, contiguous last dimension")
            d = t.shape[3] // 2
            p = t.permute(0, 2, 1, 3)
            views = [p[..., :d], p[..., d:]]
        elif nd == 3:
            _check(t.stride(2) == 1 or t.shape[2] == 1,
                   "KV cache hidden stride must equal 1 for token-major copies")
            views = [t.unsqueeze(2)]
        else:
            raise OracleError(f"Unsupported KV cache rank for token-major copies: {nd}")
        _check(all(int(x) > 0 for x in views[0].shape[1:]), "token-major copies need non-empty pages")
        return views

    def _plan_tokens(self, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        _check(self.store is not None, "store buffer not registered; call register_store() first")
        n = len(layer_names)
        if n == 0:
            return None
        idx = torch.as_tensor(indices_flat)
        validate_common_job_inputs(n, list(offsets), list(byte_sizes), list(indices_offsets),
                                   idx.numel(), (True, idx.dim() == 1, idx.dtype == torch.int32,
                                                 idx.is_contiguous()))
        validate_store_ranges(list(offsets), list(byte_sizes), self.store.numel())
        for name in layer_names:
            _check(name in self.layers, "layer not registered: ", name)
        jobs = []
        for i, name in enumerate(layer_names):
            t, pf = self.layers[name]
            page_copy_shape(tuple(t.shape), tuple(t.stride()), t.element_size(), pf)
            views = self.token_rows(t, pf)
            _, ps, h, d = (int(x) for x in views[0].shape)
            n_sel = int(indices_offsets[i + 1] - indices_offsets[i])
            num = len(views) * n_sel * ps * h * d * t.element_size()
            if int(byte_sizes[i]) != num:
                raise OracleError(
                    f"byte_size mismatch at job {i} | C++ expected bytes: {num} | "
                    f"Python passed bytes: {int(byte_sizes[i])} | Tensor shape: "
                    f"[{', '.join(str(x) for x in t.shape)}] | Tensor strides: "
                    f"[{', '.join(str(x) for x in t.stride())}]")
            sel = idx[int(indices_offsets[i]): int(indices_offsets[i + 1])].tolist()
            jobs.append((t, views, int(offsets[i]), sel, num))
        return jobs

    def gather_tokens(self, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        """store[off_i ...] = the selected pages' rows as [n_kv][n_sel * PS][H][D]
        (K rows then V rows); skipped pages (id 0 or out of range) leave their
        rows of the store untouched."""
        jobs = self._plan_tokens(layer_names, offsets, byte_sizes, indices_flat, indices_offsets)
        for t, views, off, sel, num in jobs or []:
            nb, ps, h, d = (int(x) for x in views[0].shape)
            out = self.store[off: off + num].clone().view(t.dtype).view(len(views), len(sel), ps, h, d)
            for kv, v in enumerate(views):
                for s, page in enumerate(sel):
                    if 0 < page < nb:
                        out[kv, s] = v[page]
            self.store[off: off + num] = out.reshape(-1).view(torch.uint8)

    def scatter_tokens(self, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        """Inverse of gather_tokens: skipped pages are not written."""
        jobs = self._plan_tokens(layer_names, offsets, byte_sizes, indices_flat, indices_offsets)
        for t, views, off, sel, num in jobs or []:
            nb, ps, h, d = (int(x) for x in views[0].shape)
            src = self.store[off: off + num].clone().view(t.dtype).view(len(views), len(sel), ps, h, d)
            for kv, v in enumerate(views):
                for s, page in enumerate(sel):
                    if 0 < page < nb:
                        v[page] = src[kv, s]
