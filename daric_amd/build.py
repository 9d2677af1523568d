"""Builds the gfx950 HIP library of the KV-reuse hot path.

  python -m daric_amd.build            # -> daric_amd/_lib/libdaric_cache_ops.so

Every source is compiled by hipcc for gfx950 only; objects go to _build/.
Also builds libdaric_hosttest.so, host-only entry points that let the CPU
test suite check the element conversions and the fast divider exhaustively.

  python -m daric_amd.build --sanitize # -> daric_amd/_lib/sanitize/libdaric_cache_ops.so

builds the same library with AddressSanitizer and UndefinedBehaviorSanitizer
on its host code only (device code is compiled as usual), for the CPU tests
of the C ABI's validation paths (tests/test_sanitized_host.py). Load it with
DARIC_AMD_LIB pointing at it and sanitizer_runtime() preloaded.
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
# Host-side sanitizers only: every flag reaches the host compilation alone.
SANITIZE = ("-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined "
            "-Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer").split()
SANITIZE_LINK = "-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -shared-libasan".split()
SANITIZE_DIR = os.path.join(LIBDIR, "sanitize")
SANITIZE_LIB = os.path.join(SANITIZE_DIR, "libdaric_cache_ops.so")


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


def _compile(src: str, extra=(), build_dir: str = BUILD, common=COMMON) -> str:
    out = os.path.join(build_dir, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [hipcc(), *lang, f"--offload-arch={ARCH}", *common, *NO_PACKED_FP32, *extra,
           "-c", os.path.join(CSRC, src), "-o", out]
    _run(cmd)
    return out


def sanitizer_runtime() -> str:
    """The shared AddressSanitizer runtime the sanitized library links to
    (preload it into a process that loads that library)."""
    r = subprocess.run([os.path.join(os.path.dirname(os.path.realpath(hipcc())), "..", "llvm", "bin", "clang"),
                        "--print-resource-dir"], capture_output=True, text=True)
    base = r.stdout.strip() if r.returncode == 0 else ""
    for cand in (os.path.join(base, "lib", "linux", "libclang_rt.asan-x86_64.so"),
                 os.path.join(base, "lib", "x86_64-unknown-linux-gnu", "libclang_rt.asan.so")):
        if base and os.path.exists(cand):
            return cand
    raise RuntimeError("clang's shared AddressSanitizer runtime was not found")


def build_sanitized(verbose: bool = True) -> str:
    """The library with host-side ASan + UBSan (-O1 -g), rebuilt only when a
    source is newer than it."""
    sources = [os.path.join(CSRC, f) for f in os.listdir(CSRC)] + [os.path.join(ROOT, "include", "daric_cache_ops.h")]
    if os.path.exists(SANITIZE_LIB) and os.path.getmtime(SANITIZE_LIB) >= max(os.path.getmtime(f) for f in sources):
        return SANITIZE_LIB
    bdir = os.path.join(BUILD, "sanitize")
    os.makedirs(bdir, exist_ok=True)
    os.makedirs(SANITIZE_DIR, exist_ok=True)
    common = [("-O1" if f == "-O3" else f) for f in COMMON] + ["-g"]
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda f: _compile(f, SANITIZE, bdir, common), SOURCES))
    tmp = SANITIZE_LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *SANITIZE_LINK, "-o", tmp, *objs])
    os.replace(tmp, SANITIZE_LIB)
    if verbose:
        print(f"built {SANITIZE_LIB}")
    return SANITIZE_LIB


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
    if "--sanitize" in sys.argv[1:]:
        build_sanitized()
    else:
        build()
    sys.exit(0)
