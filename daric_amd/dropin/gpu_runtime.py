"""Copy over daric/utils/gpu_runtime.py in a DARIC tree: the package's
`from .gpu_runtime import get_gpu_host_runtime, HOST_MEMORY_ALREADY_REGISTERED`
(daric/utils/__init__.py:17) and the store's shm registration
(daric/management/service/gpu_kv_io.py:40-100, 236-260) then page-lock through
the HIP runtime (libamdhip64.so) instead of looking for libcudart.so.
"""
from daric_amd.host_runtime import (  # noqa: F401
    HOST_MEMORY_ALREADY_REGISTERED,
    HOST_MEMORY_NOT_REGISTERED,
    GpuHostRuntime,
    get_gpu_host_runtime,
)
