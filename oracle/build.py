"""Builds the C restatement of the oracle (oracle/c/oracle_copy.c) with gcc.

  python -m oracle.build            # -> oracle/_lib/liboracle_copy.so

Test infrastructure: used by tests/ (checked against the numpy oracle) and by
bench.py's CPU baseline; never by the product path.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "c", "oracle_copy.c")
LIBDIR = os.path.join(HERE, "_lib")
LIB = os.path.join(LIBDIR, "liboracle_copy.so")

# -ffp-contract=off: the double products and sums are rounded one by one, as
# numpy rounds them.
FLAGS = ["-O3", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-Wall",
         "-Wextra", "-Wno-unused-parameter"]


def build(verbose: bool = True) -> str:
    cc = os.environ.get("CC") or shutil.which("gcc") or "cc"
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = LIB + ".tmp"
    r = subprocess.run([cc, *FLAGS, "-o", tmp, SRC, "-lm"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle C build failed ({r.returncode}):\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
