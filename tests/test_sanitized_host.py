"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only): the library is rebuilt with both sanitizers on its host side
(python -m daric_amd.build --sanitize) and the C-ABI validation suites,
tests/test_capi_cpu.py and tests/test_capi_fuzz.py, run against it in a
subprocess. Their cases drive every validation path with fake device
pointers and fail before any HIP call, so no kernel runs. Any sanitizer
report fails the run (UBSan halts on error). The C-consumer link test is
left out: it links the library by name without the sanitizer runtime."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_capi_suites_under_asan_and_ubsan():
    from daric_amd import build
    try:
        build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc is not available")
    lib = build.build_sanitized(verbose=False)
    env = dict(os.environ)
    env.update(DARIC_AMD_LIB=lib, LD_PRELOAD=build.sanitizer_runtime(),
               ASAN_OPTIONS="detect_leaks=0:alloc_dealloc_mismatch=0:detect_odr_violation=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    probe = subprocess.run([sys.executable, "-c",
                            "from daric_amd import _lib; _lib.load(); print(open('/proc/self/maps').read())"],
                           cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    assert probe.returncode == 0, probe.stderr[-2000:]
    assert lib in probe.stdout and "libclang_rt.asan" in probe.stdout, "the sanitized library was not loaded"
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        "tests/test_capi_cpu.py", "tests/test_capi_fuzz.py", "-k", "not c_consumer"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert " passed" in out
