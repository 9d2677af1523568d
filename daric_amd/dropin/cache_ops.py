"""Copy to daric/cache_ops.py in a DARIC tree (and drop the CUDAExtension of
setup.py:8-27): the store's `from ... import cache_ops`
(daric/management/service/gpu_kv_io.py:9) then binds the gfx950 library.

The names of the reference's type stub (daric/cache_ops.pyi:6-53) keep their
signatures; the rest are additions.
"""
from daric_amd.cache_ops import (  # noqa: F401
    CacheCopier,
    batched_memcpy_d2h,
    batched_memcpy_h2d,
    kv_deviation,
    merge_rows,
    rerotate_pages,
    select_merge,
    timing_enable,
    timing_read,
    topk_per_chunk,
)
