"""Host-memory registration for the store's record pool (CPU only; no
register call reaches a HIP runtime here, and none may on the GPU boxes, whose
runtime refuses to page-lock existing memory).

- host_runtime.get_gpu_host_runtime() finds the HIP runtime PyTorch-ROCm
  loaded and binds hipHostRegister / hipHostUnregister (the reference's
  loader, daric/utils/gpu_runtime.py:13-114, looks only for libcudart.so);
- GpuHostRuntime passes (address, size, hipHostRegisterPortable) and the
  address through ctypes as the C functions take them;
- kv_io.HostMemoryRegistration locks a buffer in page-aligned pieces and
  unlocks them again, as gpu_kv_io.py:40-100 does, against a recording
  runtime: piece addresses and sizes, refusal of misaligned or empty
  buffers, rollback after an already-registered piece or a failing status,
  and reverse-order unregistration that keeps the pieces it could not unlock.
"""
import ctypes
import mmap
import os

import pytest
import torch

from daric_amd import host_runtime as hr
from daric_amd.kv_io import REGISTRATION_CHUNK_BYTES, HostMemoryRegistration

PAGE = os.sysconf("SC_PAGE_SIZE")


def test_loads_the_hip_runtime():
    rt = hr.get_gpu_host_runtime()
    assert rt is hr.get_gpu_host_runtime()               # one per process
    assert rt.prefix == "hip"
    assert os.path.basename(rt.path).startswith("libamdhip64.so")
    assert rt._reg.argtypes == [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint]
    assert rt._unreg.argtypes == [ctypes.c_void_p]
    assert hr.HOST_MEMORY_ALREADY_REGISTERED == 712 and hr.HOST_MEMORY_NOT_REGISTERED == 713


def test_runtime_passes_its_arguments_through_ctypes():
    calls = []
    reg_t = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint)
    unreg_t = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)

    class FakeLib:
        hipHostRegister = reg_t(lambda a, n, f: calls.append(("reg", a, n, f)) or 0)
        hipHostUnregister = unreg_t(lambda a: calls.append(("unreg", a)) or 713)

    rt = hr.GpuHostRuntime(FakeLib(), "hip", "fake")
    assert rt.register(0x7F0000001000, 3 << 30) == 0
    assert rt.unregister(0x7F0000001000) == 713
    assert calls == [("reg", 0x7F0000001000, 3 << 30, hr.HOST_REGISTER_PORTABLE), ("unreg", 0x7F0000001000)]


class Recorder:
    """A runtime that records calls; `statuses` maps a call index to the
    status it returns (0 otherwise)."""
    prefix = "hip"

    def __init__(self, reg_statuses=None, unreg_statuses=None):
        self.reg, self.unreg = [], []
        self.reg_statuses = reg_statuses or {}
        self.unreg_statuses = unreg_statuses or {}

    def register(self, address, size):
        self.reg.append((address, size))
        return self.reg_statuses.get(len(self.reg) - 1, 0)

    def unregister(self, address):
        self.unreg.append(address)
        return self.unreg_statuses.get(len(self.unreg) - 1, 0)


def buffer(pages):
    m = mmap.mmap(-1, pages * PAGE)         # page-aligned, writable
    return m, ctypes.addressof(ctypes.c_char.from_buffer(m))


def test_registers_in_page_aligned_pieces_and_unregisters_in_reverse():
    m, base = buffer(5)
    rt = Recorder()
    r = HostMemoryRegistration(rt, 2 * PAGE)
    r.register(m)
    assert rt.reg == [(base, 2 * PAGE), (base + 2 * PAGE, 2 * PAGE), (base + 4 * PAGE, PAGE)]
    assert r.addresses == [base, base + 2 * PAGE, base + 4 * PAGE]
    with pytest.raises(RuntimeError, match="still registered"):
        r.register(m)
    r.unregister()
    assert rt.unreg == [base + 4 * PAGE, base + 2 * PAGE, base] and r.addresses == []
    # a CPU tensor over the same memory registers the same pieces
    t = torch.frombuffer(m, dtype=torch.uint8)
    r.register(t)
    assert rt.reg[3:] == rt.reg[:3]
    r.unregister()
    assert REGISTRATION_CHUNK_BYTES == 1 << 30


def test_refuses_misaligned_or_empty_buffers():
    m, base = buffer(4)
    with pytest.raises(ValueError, match="page-aligned"):
        HostMemoryRegistration(Recorder(), PAGE + 1).register(m)
    with pytest.raises(ValueError, match="page-aligned"):
        HostMemoryRegistration(Recorder(), PAGE).register(memoryview(m)[16:])
    with pytest.raises(ValueError, match="empty"):
        HostMemoryRegistration(Recorder(), PAGE).register(bytearray(0))
    with pytest.raises(ValueError, match="writable"):
        HostMemoryRegistration(Recorder(), PAGE).register(bytes(PAGE))


@pytest.mark.parametrize("status,match", [(hr.HOST_MEMORY_ALREADY_REGISTERED, "already page-locked"),
                                          (1, "hipHostRegister failed at offset")])
def test_a_failing_piece_unlocks_the_pieces_before_it(status, match):
    m, base = buffer(6)
    rt = Recorder(reg_statuses={2: status})
    r = HostMemoryRegistration(rt, 2 * PAGE)
    with pytest.raises(RuntimeError, match=match):
        r.register(m)
    assert rt.reg == [(base, 2 * PAGE), (base + 2 * PAGE, 2 * PAGE), (base + 4 * PAGE, 2 * PAGE)]
    assert rt.unreg == [base + 2 * PAGE, base] and r.addresses == []


def test_pieces_that_stay_locked_are_kept_and_reported():
    m, base = buffer(6)
    rt = Recorder(unreg_statuses={1: hr.HOST_MEMORY_NOT_REGISTERED})
    r = HostMemoryRegistration(rt, 2 * PAGE)
    r.register(m)
    with pytest.raises(RuntimeError, match="1 piece"):
        r.unregister()
    assert r.addresses == [base + 2 * PAGE]
    # the original error wins when the rollback itself fails
    rt2 = Recorder(reg_statuses={1: 5}, unreg_statuses={0: 9})
    r2 = HostMemoryRegistration(rt2, 2 * PAGE)
    with pytest.raises(RuntimeError, match="failed at offset"):
        r2.register(m)
    assert r2.addresses == [base]
