"""Layout normalisation and argument validation (CPU restatement).

Follows reference csrc/cache_ops/helpers.cu:15-174 (get_page_copy_shape,
get_dense_span_elements, validate_outer_regions, validate_common_job_inputs),
csrc/cache_ops/copier.cpp:32-39 (validate_store_ranges) and the rotary layout
resolution of daric/adaption/adapter.py:297-373. Errors are raised as
OracleError carrying the reference's message text.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

INT64_MAX = (1 << 63) - 1
INT_MAX = (1 << 31) - 1


class OracleError(RuntimeError):
    pass


def _fmt(v: Sequence[int]) -> str:
    return "[" + ", ".join(str(int(x)) for x in v) + "]"


def _check(cond: bool, *msg) -> None:
    if not cond:
        raise OracleError("".join(str(m) for m in msg))


def checked_multiply(lhs: int, rhs: int, context: str) -> int:
    """helpers.cu:15-20."""
    _check(lhs >= 0 and rhs >= 0, context, " must be non-negative")
    _check(lhs == 0 or rhs <= INT64_MAX // lhs, context, " exceeds int64 range")
    return lhs * rhs


def dense_span_elements(sizes, strides, first_dim: int) -> int:
    """helpers.cu:22-64: the dims from first_dim on must cover a dense span in
    memory order (sorted by stride, singleton dims ignored)."""
    dims = []
    for d in range(first_dim, len(sizes)):
        size, stride = int(sizes[d]), int(strides[d])
        _check(size > 0, "KV cache copy dimensions must be non-empty",
               " | shape=", _fmt(sizes), " | stride=", _fmt(strides), " | failed_dim=", d)
        if size == 1:
            continue
        _check(stride > 0, "KV cache non-singleton dimensions must have positive strides",
               " | shape=", _fmt(sizes), " | stride=", _fmt(strides), " | failed_dim=", d,
               " | actual_stride=", stride)
        dims.append((d, size, stride))
    dims.sort(key=lambda t: t[2])  # std::sort by stride; ties keep no particular order
    expected = 1
    for d, size, stride in dims:
        _check(stride == expected, "KV cache copy dimensions must form a dense physical span",
               " | shape=", _fmt(sizes), " | stride=", _fmt(strides), " | failed_dim=", d,
               " | expected_stride=", expected, " | actual_stride=", stride,
               " | relation=", "hole" if stride > expected else "overlap")
        expected = checked_multiply(expected, size, "KV cache dense span")
    return expected


def validate_outer_regions(sizes, strides, prefix_size, num_pages, prefix_stride,
                           page_stride, suffix_size) -> None:
    """helpers.cu:66-90."""
    axes = []
    if prefix_size > 1:
        axes.append((prefix_stride, prefix_size))
    if num_pages > 1:
        axes.append((page_stride, num_pages))
    axes.sort()
    occupied = suffix_size
    for stride, size in axes:
        _check(stride >= occupied, "KV cache prefix/page regions overlap",
               " | shape=", _fmt(sizes), " | stride=", _fmt(strides),
               " | region_size=", suffix_size, " | required_stride=", occupied,
               " | actual_stride=", stride)
        extent = checked_multiply(size - 1, stride, "KV cache outer span")
        _check(extent <= INT64_MAX - occupied, "KV cache outer span exceeds int64 range")
        occupied += extent


@dataclass(frozen=True)
class PageCopyShape:
    num_pages: int
    prefix_size: int
    page_stride: int      # bytes
    suffix_size: int      # bytes of one page span
    prefix_stride: int    # bytes


def page_copy_shape(sizes, strides, elem_size: int, is_page_first: bool,
                    on_device: bool = True) -> PageCopyShape:
    """helpers.cu:94-148: reduce a KV tensor to (prefix, pages, strides, span)."""
    _check(on_device, "KV cache tensor must be on CUDA")
    _check(len(sizes) >= 1, "KV cache tensor must have at least one dimension")
    e = int(elem_size)
    if is_page_first:
        _check(sizes[0] > 0, "page dimension must be non-zero")
        _check(sizes[0] <= INT_MAX, "number of pages exceeds int range: ", sizes[0])
        num_pages, prefix_size, prefix_stride = int(sizes[0]), 1, 0
        page_stride = checked_multiply(int(strides[0]), e, "KV cache page stride")
        suffix = checked_multiply(dense_span_elements(sizes, strides, 1), e, "KV cache page span")
        if num_pages > 1:
            _check(page_stride >= suffix, "KV cache pages overlap",
                   " | shape=", _fmt(sizes), " | stride=", _fmt(strides),
                   " | page_stride=", page_stride, " | page_span=", suffix)
    else:
        _check(len(sizes) >= 2, "non-page-first KV cache tensor must have at least two dimensions")
        _check(sizes[0] > 0, "prefix dimension must be non-zero")
        _check(sizes[1] > 0, "page dimension must be non-zero")
        _check(sizes[0] <= INT_MAX, "prefix size exceeds int range: ", sizes[0])
        _check(sizes[1] <= INT_MAX, "number of pages exceeds int range: ", sizes[1])
        prefix_size, num_pages = int(sizes[0]), int(sizes[1])
        prefix_stride = checked_multiply(int(strides[0]), e, "KV cache prefix stride")
        page_stride = checked_multiply(int(strides[1]), e, "KV cache page stride")
        suffix = checked_multiply(dense_span_elements(sizes, strides, 2), e, "KV cache suffix span")
        validate_outer_regions(sizes, strides, prefix_size, num_pages, prefix_stride,
                               page_stride, suffix)
    _check(page_stride > 0, "page_stride must be positive")
    return PageCopyShape(num_pages, prefix_size, page_stride, suffix, prefix_stride)


def validate_common_job_inputs(num_jobs, offsets, byte_sizes, indices_offsets,
                               indices_numel, indices_ok=(True, True, True, True)) -> None:
    """helpers.cu:150-174. indices_ok = (on device, 1-D, int32, contiguous)."""
    _check(len(offsets) == num_jobs, "offsets length mismatch")
    _check(len(byte_sizes) == num_jobs, "byte_sizes length mismatch")
    _check(len(indices_offsets) == num_jobs + 1, "indices_offsets size must be num_jobs + 1")
    _check(indices_ok[0], "indices_flat must be on CUDA")
    _check(indices_ok[1], "indices_flat must be 1D")
    _check(indices_ok[2], "indices_flat must be int32")
    _check(indices_ok[3], "indices_flat must be contiguous")
    _check(indices_offsets[0] >= 0, "indices_offsets[0] must be non-negative")
    _check(indices_offsets[-1] <= indices_numel, "indices_offsets.back() exceeds indices_flat.numel()")
    for i in range(num_jobs):
        _check(offsets[i] >= 0, "negative store offset at job ", i)
        _check(byte_sizes[i] >= 0, "negative byte size at job ", i)
        _check(indices_offsets[i] >= 0, "negative indices offset at job ", i)
        _check(indices_offsets[i] <= indices_offsets[i + 1],
               "indices_offsets must be non-decreasing at job ", i)


def validate_store_ranges(offsets, byte_sizes, store_size) -> None:
    """copier.cpp:32-39."""
    for i in range(len(offsets)):
        _check(offsets[i] >= 0, "negative store offset at job ", i)
        _check(byte_sizes[i] >= 0, "negative store byte size at job ", i)
        _check(offsets[i] <= store_size, "store offset out of range at job ", i)
        _check(byte_sizes[i] <= store_size - offsets[i], "store range out of bounds at job ", i)


@dataclass(frozen=True)
class RopeGeometry:
    """Where the K head rows of a KV layer live, in elements.

    K element (block b, slot s, head h, dim d) is at
    k_offset + b*stride_b + s*stride_s + h*stride_h + d from element [0,...,0].
    """
    page_size: int
    num_heads: int
    head_dim: int
    stride_b: int
    stride_s: int
    stride_h: int
    k_offset: int


def rope_geometry(sizes, strides, page_first: bool, rotary_dim: int,
                  dtype_name: str = "") -> RopeGeometry:
    """adapter.py:311-368 (_launch_triton_rerotate layout resolution)."""
    nd = len(sizes)
    if nd == 5:
        _, _, ps, h, d = (int(x) for x in sizes)
        if page_first:
            return RopeGeometry(ps, h, d, int(strides[0]), int(strides[2]), int(strides[3]), 0)
        # kv_layer[0]: element 0 of the K half, strides of dims 1..3
        return RopeGeometry(ps, h, d, int(strides[1]), int(strides[2]), int(strides[3]), 0)
    if nd == 4:
        constraint = None
        if not page_first:
            constraint = "page_first must be true"
        elif sizes[3] <= 0 or sizes[3] % 2 != 0:
            constraint = "packed content dimension must be positive and even"
        elif strides[3] != 1:
            constraint = "packed content feature stride must equal 1"
        _, h, ps, packed = (int(x) for x in sizes)
        d = packed // 2
        if constraint is None and (rotary_dim <= 0 or rotary_dim % 2 != 0 or rotary_dim > d):
            constraint = ("rotary_dim must be positive, even, and no greater than "
                          "the packed K head dimension")
        if constraint is not None:
            raise ValueError(
                "Invalid 4D KV cache for rerotate: "
                f"shape={tuple(int(x) for x in sizes)}, stride={tuple(int(x) for x in strides)}, "
                f"dtype={dtype_name}, rotary_dim={rotary_dim}, constraint={constraint}")
        return RopeGeometry(ps, h, d, int(strides[0]), int(strides[2]), int(strides[1]), 0)
    if nd == 3:
        _, ps, hidden = (int(x) for x in sizes)
        return RopeGeometry(ps, 1, hidden, int(strides[0]), int(strides[1]), 0, 0)
    raise ValueError(f"Unsupported KV cache rank for rerotate: {nd}")
