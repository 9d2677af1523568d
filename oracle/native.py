"""ctypes front of the C restatement (oracle/c/oracle_copy.c) -- TEST
INFRASTRUCTURE ONLY.

NativeOracleCopier is an OracleCopier whose page copies and fused
scatter + re-rotation run in C with OpenMP threads. The job plan and every
argument check stay the numpy oracle's (OracleCopier._plan), so both oracles
accept and reject the same calls; tests/test_oracle_native.py checks that they
also produce the same bytes. bench.py times it as the multithreaded CPU
baseline.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

from . import rope
from .copy import OracleCopier
from .layout import page_copy_shape, rope_geometry

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "liboracle_copy.so")

_KIND = {torch.bfloat16: 0, torch.float16: 1, torch.uint8: 2}


class OcLayer(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("prefix", ctypes.c_int64),
                ("num_pages", ctypes.c_int64), ("page_stride", ctypes.c_int64),
                ("prefix_stride", ctypes.c_int64), ("suffix", ctypes.c_int64),
                ("k_base", ctypes.c_void_p), ("sb", ctypes.c_int64), ("ss", ctypes.c_int64),
                ("sh", ctypes.c_int64), ("page_size", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("kind", ctypes.c_int32), ("pad", ctypes.c_int32),
                ("k_scale", ctypes.POINTER(ctypes.c_double))]


_lib = None


def load():
    """The built C library (raises if oracle/build.py has not been run)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing; build it with `python -m oracle.build`")
        lib = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        lib.oc_copy_pages.argtypes = [P, P, P, P, P, ctypes.c_int64, P, ctypes.c_int, ctypes.c_int]
        lib.oc_copy_pages.restype = None
        lib.oc_scatter_rerotate.argtypes = [P, P, P, P, P, P, P, ctypes.c_int64, P, P,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.oc_scatter_rerotate.restype = None
        lib.oc_convert.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, P, P]
        lib.oc_convert.restype = None
        _lib = lib
    return _lib


def available() -> bool:
    return os.path.exists(LIB_PATH)


def convert_to_codes(values: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """float32 values -> cache codes (uint16 for bf16/fp16, uint8 for fp8)."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(v.size, dtype=np.uint8 if dtype == torch.uint8 else np.uint16)
    load().oc_convert(_KIND[dtype], 0, v.size, v.ctypes.data, out.ctypes.data)
    return out


def convert_to_values(codes: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """cache codes -> float64 values."""
    c = np.ascontiguousarray(codes, dtype=np.uint8 if dtype == torch.uint8 else np.uint16)
    out = np.empty(c.size, dtype=np.float64)
    load().oc_convert(_KIND[dtype], 1, c.size, c.ctypes.data, out.ctypes.data)
    return out


class NativeOracleCopier(OracleCopier):
    def __init__(self, threads: int = 1):
        super().__init__()
        self.threads = max(1, int(threads))

    def _tables(self, jobs, rotary_dim=None):
        names = []
        for name, *_ in jobs:
            if name not in names:
                names.append(name)
        layers = (OcLayer * len(names))()
        keep = []
        for k, name in enumerate(names):
            t, pf = self.layers[name]
            shp = page_copy_shape(tuple(t.shape), tuple(t.stride()), t.element_size(), pf)
            L = layers[k]
            L.data = t.data_ptr()
            L.prefix, L.num_pages = shp.prefix_size, shp.num_pages
            L.page_stride, L.prefix_stride, L.suffix = shp.page_stride, shp.prefix_stride, shp.suffix_size
            L.kind = _KIND.get(t.dtype, -1)
            if rotary_dim is not None:
                g = rope_geometry(tuple(t.shape), tuple(t.stride()), pf, rotary_dim, str(t.dtype))
                L.k_base = t.data_ptr() + g.k_offset * t.element_size()
                L.sb, L.ss, L.sh = g.stride_b, g.stride_s, g.stride_h
                L.page_size, L.heads = g.page_size, g.num_heads
                sc = self.k_scales.get(name)
                if sc is not None and t.dtype == torch.uint8:
                    arr = np.ascontiguousarray(sc, dtype=np.float64)
                    keep.append(arr)
                    L.k_scale = arr.ctypes.data_as(ctypes.POINTER(ctypes.c_double))
        pos = {n: k for k, n in enumerate(names)}
        job_layer = np.array([pos[j[0]] for j in jobs], dtype=np.int32)
        offsets = np.array([j[4] for j in jobs], dtype=np.int64)
        flat = [np.asarray(j[5], dtype=np.int32) for j in jobs]
        ioff = np.zeros(len(jobs) + 1, dtype=np.int64)
        ioff[1:] = np.cumsum([f.size for f in flat])
        idx = np.concatenate(flat) if flat else np.zeros(0, np.int32)
        idx = np.ascontiguousarray(idx, dtype=np.int32)
        keep += [layers, job_layer, offsets, ioff, idx]
        return layers, job_layer, offsets, ioff, idx, keep

    def _copy(self, gather, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        jobs = self._plan(layer_names, offsets, byte_sizes, indices_flat, indices_offsets)
        if not jobs:
            return
        layers, jl, off, ioff, idx, keep = self._tables(jobs)
        load().oc_copy_pages(ctypes.addressof(layers), jl.ctypes.data, off.ctypes.data,
                             idx.ctypes.data, ioff.ctypes.data, len(jobs), self.store.data_ptr(),
                             1 if gather else 0, self.threads)

    def gather_pages(self, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        self._copy(True, layer_names, offsets, byte_sizes, indices_flat, indices_offsets)

    def scatter_pages(self, layer_names, offsets, byte_sizes, indices_flat, indices_offsets):
        self._copy(False, layer_names, offsets, byte_sizes, indices_flat, indices_offsets)

    def scatter_pages_rerotate(self, layer_names, offsets, byte_sizes, indices_flat,
                               indices_offsets, deltas, num_tokens, inv_freq, rotary_dim,
                               is_neox):
        jobs = self._plan(layer_names, offsets, byte_sizes, indices_flat, indices_offsets)
        if not jobs:
            return
        for name, t, *_ in jobs:
            if t.dtype not in _KIND:
                raise ValueError(f"unsupported KV cache dtype for rerotate: {t.dtype}")
            rope.k_view(t, self.layers[name][1], rotary_dim)   # layout checks of the numpy path
        layers, jl, off, ioff, idx, keep = self._tables(jobs, rotary_dim)
        d = np.ascontiguousarray(deltas, dtype=np.int64)
        nt = np.ascontiguousarray(num_tokens, dtype=np.int64)
        inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
        load().oc_scatter_rerotate(ctypes.addressof(layers), jl.ctypes.data, off.ctypes.data,
                                   idx.ctypes.data, ioff.ctypes.data, d.ctypes.data, nt.ctypes.data,
                                   len(jobs), self.store.data_ptr(), inv.ctypes.data,
                                   int(rotary_dim), 1 if is_neox else 0, self.threads)
