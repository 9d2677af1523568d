"""ctypes binding of libdaric_cache_ops.so (include/daric_cache_ops.h).

torch is imported before the library is loaded so that the library binds to
the HIP runtime torch already loaded (both carry the soname libamdhip64.so.7):
device pointers and hipStream_t values from torch are then valid in it.
"""
from __future__ import annotations

import array
import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_int, c_int32, c_int64, c_uint64, c_void_p

import torch

# DARIC_AMD_LIB selects another build of the same library (the host-sanitized
# build of `python -m daric_amd.build --sanitize`); unset, the in-tree build.
LIB_PATH = os.environ.get("DARIC_AMD_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "_lib", "libdaric_cache_ops.so")
MAX_DIMS = 8
ABI_VERSION = 5
ERR_VALUE = 5

DTYPE_CODES = {
    torch.uint8: 0,
    torch.int32: 1,
    torch.int64: 2,
    torch.float16: 3,
    torch.bfloat16: 4,
    torch.float32: 5,
    torch.float8_e4m3fn: 6,
}


class DaricTensor(ctypes.Structure):
    _fields_ = [
        ("data", c_void_p),
        ("ndim", c_int32),
        ("elem_size", c_int32),
        ("device", c_int32),
        ("dtype", c_int32),
        ("sizes", c_int64 * MAX_DIMS),
        ("strides", c_int64 * MAX_DIMS),
    ]


class DaricRope(ctypes.Structure):
    _fields_ = [("inv_freq", c_void_p), ("rotary_dim", c_int32), ("is_neox", c_int32)]


class DaricRopeSegment(ctypes.Structure):
    _fields_ = [("bt_offset", c_int64), ("tok_start", c_int64), ("n_tokens", c_int64),
                ("delta", c_int64)]


class DaricChunk(ctypes.Structure):
    _fields_ = [("bt_offset", c_int64), ("row_offset", c_int64), ("n_tokens", c_int64),
                ("k", c_int64), ("tok_start", c_int64)]


P = POINTER
T = P(DaricTensor)
I64P = c_void_p  # address of an I64 buffer
STRS = P(c_char_p)

# name -> (restype, argtypes); mirrors include/daric_cache_ops.h
SIGNATURES = {
    "daric_abi_version": (c_int, []),
    "daric_last_error": (c_char_p, []),
    "daric_timing_enable": (c_int, [c_int]),
    "daric_timing_read": (c_int, [P(c_double), I64P]),
    "daric_debug_counters": (c_int, [I64P, I64P, I64P]),
    "daric_copier_create": (c_int, [P(c_void_p)]),
    "daric_copier_destroy": (c_int, [c_void_p]),
    "daric_copier_register_layer": (c_int, [c_void_p, c_char_p, T, c_int]),
    "daric_copier_register_store": (c_int, [c_void_p, T]),
    "daric_copier_register_k_scale": (c_int, [c_void_p, c_char_p, T]),
    "daric_copier_gather_pages": (c_int, [c_void_p, STRS, c_int64, I64P, c_int64, I64P, c_int64, T, I64P,
                                          c_int64, c_uint64]),
    "daric_copier_scatter_pages": (c_int, [c_void_p, STRS, c_int64, I64P, c_int64, I64P, c_int64, T, I64P,
                                           c_int64, c_uint64]),
    "daric_copier_gather_tokens": (c_int, [c_void_p, STRS, c_int64, I64P, c_int64, I64P, c_int64, T, I64P,
                                           c_int64, c_uint64]),
    "daric_copier_scatter_tokens": (c_int, [c_void_p, STRS, c_int64, I64P, c_int64, I64P, c_int64, T, I64P,
                                            c_int64, c_uint64]),
    "daric_copier_scatter_pages_rerotate": (c_int, [c_void_p, STRS, c_int64, I64P, c_int64, I64P, c_int64, T,
                                                    I64P, c_int64, I64P, I64P, P(DaricRope), c_uint64]),
    "daric_copier_scatter_pages_rerotate_noalloc": (c_int, [c_void_p, STRS, c_int64, I64P, c_int64, I64P,
                                                            c_int64, T, I64P, c_int64, I64P, I64P,
                                                            P(DaricRope), c_uint64]),
    "daric_batched_memcpy_d2h": (c_int, [T, T, I64P, I64P, I64P, c_int64, c_uint64]),
    "daric_batched_memcpy_h2d": (c_int, [T, T, I64P, I64P, I64P, c_int64, c_uint64]),
    "daric_rerotate_pages": (c_int, [T, c_int64, c_int, T, P(DaricRopeSegment), c_int64, P(DaricRope), T,
                                     c_uint64]),
    "daric_kv_deviation": (c_int, [T, c_int64, c_int, T, T, P(DaricChunk), c_int64, T, T, c_uint64]),
    "daric_topk_per_chunk": (c_int, [T, P(DaricChunk), c_int64, T, c_uint64]),
    "daric_merge_rows": (c_int, [T, c_int64, c_int, T, T, T, P(DaricChunk), c_int64, T, T, T, c_uint64]),
    "daric_select_merge": (c_int, [T, c_int64, c_int, T, T, T, P(DaricChunk), c_int64, T, T, T, T, c_int,
                                   c_uint64]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Loads the HIP library; raises ImportError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"daric_amd HIP library not found at {LIB_PATH}; build it with `python -m daric_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.daric_abi_version() != ABI_VERSION:
        raise ImportError("daric_amd HIP library ABI version mismatch")
    _lib = lib
    return lib


def check(status: int) -> None:
    """Raises the library's message for a non-zero status: RuntimeError, as
    TORCH_CHECK and std::runtime_error surface in the reference's pybind11
    module, or ValueError for the cache layouts the reference's rotation
    rejects with ValueError (daric/adaption/adapter.py:20-27, 336-368)."""
    if status != 0:
        msg = load().daric_last_error()
        text = msg.decode() if msg else f"daric error {status}"
        raise (ValueError if status == ERR_VALUE else RuntimeError)(text)


def desc(t: torch.Tensor) -> DaricTensor:
    n = t.dim()
    if n > MAX_DIMS:
        raise RuntimeError(f"tensor rank {n} exceeds {MAX_DIMS}")
    d = DaricTensor()
    d.data = t.data_ptr()
    d.ndim = n
    d.elem_size = t.element_size()
    dv = t.device
    if dv.type == "cuda":
        d.device = dv.index if dv.index is not None else torch.cuda.current_device()
    else:
        d.device = -1
    d.dtype = DTYPE_CODES.get(t.dtype, 15)
    if n:
        d.sizes[:n] = tuple(t.shape)
        d.strides[:n] = t.stride()
    return d


class I64:
    """Contiguous int64 copy of a sequence of ints for an `const int64_t*`
    argument; `ptr` stays valid while the object is alive. Non-integer values
    raise TypeError (the reference's pybind11 list<int64> conversion refuses
    them too)."""
    __slots__ = ("buf", "ptr", "n")

    def __init__(self, values):
        buf = array.array("q", values)
        self.n = len(buf)
        if self.n == 0:
            buf = array.array("q", [0])
        self.buf = buf
        self.ptr = buf.buffer_info()[0]


_NAME_CACHE: dict = {}
_NAME_CACHE_MAX = 256


def str_array(names) -> ctypes.Array:
    """NUL-terminated C strings of `names` as a `const char* const*` array.
    Arrays are cached per distinct name tuple: callers pass the same layer
    name lists on every call, and encoding them dominated the call cost."""
    key = tuple(names)
    hit = _NAME_CACHE.get(key)
    if hit is not None:
        return hit
    enc = [str(n).encode() for n in key]
    arr = (c_char_p * max(len(enc), 1))(*enc)
    if len(_NAME_CACHE) >= _NAME_CACHE_MAX:
        _NAME_CACHE.clear()
    _NAME_CACHE[key] = arr
    return arr
