"""Builds the gfx950 HIP library of the KV-reuse hot path.

  python -m daric_amd.build            # -> daric_amd/_lib/libdaric_cache_ops.so

Every source is compiled by hipcc for gfx950 only; objects go to _build/.
Also builds libdaric_hosttest.so, host-only entry points that let the CPU
test suite check the element conversions and the fast divider exhaustively.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "_lib")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(LIBDIR, "libdaric_cache_ops.so")
HOSTTEST_LIB = os.path.join(LIBDIR, "libdaric_hosttest.so")

SOURCES = ["capi.cpp", "runtime.cpp", "copy_kernels.hip", "rope_kernels.hip", "select_kernels.hip",
           "token_kernels.hip", "noalloc.hip"]

ARCH = "gfx950"
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wshadow", "-Wno-unused-result",
          f"-I{os.path.join(ROOT, 'include')}"]
# Keep the compiler from emitting packed fp32 VALU ops (v_pk_*_f32).
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build daric_amd)")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def _compile(src: str, extra=()) -> str:
    out = os.path.join(BUILD, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [hipcc(), *lang, f"--offload-arch={ARCH}", *COMMON, *NO_PACKED_FP32, *extra,
           "-c", os.path.join(CSRC, src), "-o", out]
    _run(cmd)
    return out


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    # host-only test hooks (no device code)
    tmp = HOSTTEST_LIB + ".tmp"
    _run([hipcc(), *COMMON, "-shared", "-o", tmp, os.path.join(CSRC, "hosttest.cpp")])
    os.replace(tmp, HOSTTEST_LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
