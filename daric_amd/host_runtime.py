"""Page-locking existing host memory for the GPU, through the HIP runtime: the
counterpart of the reference's host-runtime loader
(daric/utils/gpu_runtime.py:1-114), which looks only for libcudart.so and so
finds nothing on ROCm. The daric-store pins its shared-memory record pool with
it before the batched host copies (gpu_kv_io.py:40-100, 236-260).

Same interface: get_gpu_host_runtime() returns one process-wide object with
register(address, size) -> status, unregister(address) -> status, `prefix`
and `path`; HOST_MEMORY_ALREADY_REGISTERED is the status a register call
returns for memory that is already page-locked. Statuses are HIP's
(hipError_t), whose codes for these cases equal CUDA's: 712 already
registered, 713 not registered (the reference's HOST_MEMORY_NOT_REGISTERED
reads 708, which is not the runtime's code for that case).

Registration is portable (hipHostRegisterPortable): the pages count as pinned
for every device of the process, as the reference asks of CUDA."""
from __future__ import annotations

import ctypes
import os
import threading

__all__ = ["GpuHostRuntime", "get_gpu_host_runtime", "HOST_MEMORY_ALREADY_REGISTERED",
           "HOST_MEMORY_NOT_REGISTERED", "HOST_REGISTER_PORTABLE"]

HOST_MEMORY_ALREADY_REGISTERED = 712   # hipErrorHostMemoryAlreadyRegistered
HOST_MEMORY_NOT_REGISTERED = 713       # hipErrorHostMemoryNotRegistered
HOST_REGISTER_PORTABLE = 0x1           # hipHostRegisterPortable

SONAME = "libamdhip64.so"


class GpuHostRuntime:
    """hipHostRegister / hipHostUnregister of one loaded HIP runtime library."""

    def __init__(self, lib, prefix: str, path: str):
        reg = getattr(lib, prefix + "HostRegister")
        unreg = getattr(lib, prefix + "HostUnregister")
        reg.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint]
        reg.restype = ctypes.c_int
        unreg.argtypes = [ctypes.c_void_p]
        unreg.restype = ctypes.c_int
        self._reg, self._unreg = reg, unreg
        self.prefix = prefix
        self.path = path

    def register(self, address: int, size: int) -> int:
        """Page-locks [address, address + size); returns the runtime's status."""
        return int(self._reg(ctypes.c_void_p(int(address)), ctypes.c_size_t(int(size)),
                             ctypes.c_uint(HOST_REGISTER_PORTABLE)))

    def unregister(self, address: int) -> int:
        """Unlocks the range registered at `address`; returns the runtime's status."""
        return int(self._unreg(ctypes.c_void_p(int(address))))


def _mapped_path(soname: str):
    """Path of `soname` if this process has it mapped already (PyTorch-ROCm
    loads the HIP runtime when it initialises), so the same copy is used."""
    try:
        with open("/proc/self/maps") as maps:
            for line in maps:
                path = line.rsplit(None, 1)[-1] if "/" in line else ""
                if os.path.basename(path).startswith(soname) and os.path.exists(path):
                    return path
    except OSError:
        pass
    return None


def _candidates():
    mapped = _mapped_path(SONAME)
    if mapped:
        yield mapped
    for env in ("ROCM_PATH", "ROCM_HOME", "HIP_PATH"):
        root = os.environ.get(env)
        if root:
            yield os.path.join(root, "lib", SONAME)
    yield os.path.join("/opt/rocm", "lib", SONAME)
    yield SONAME                                  # the dynamic linker's search path


_runtime = None
_runtime_lock = threading.Lock()


def get_gpu_host_runtime() -> GpuHostRuntime:
    """The process's HIP host-registration runtime (loaded once); RuntimeError
    when no HIP runtime with hipHostRegister can be loaded."""
    global _runtime
    with _runtime_lock:
        if _runtime is None:
            tried = []
            for path in _candidates():
                tried.append(path)
                try:
                    lib = ctypes.CDLL(path)
                    _runtime = GpuHostRuntime(lib, "hip", path)
                    break
                except (OSError, AttributeError):
                    continue
            if _runtime is None:
                raise RuntimeError("No HIP runtime found (looked for " + ", ".join(tried) +
                                   "); cannot register host memory for GPU access.")
        return _runtime
