"""CPU oracle for the KV-reuse hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with torch/numpy, the algorithm of every
function on the path, each citing the reference file:line it follows:

  layout.py  page-copy shape normalisation and argument validation
             (reference csrc/cache_ops/helpers.cu, copier.cpp) and the rotary
             layout resolution (daric/adaption/adapter.py:297-373)
  copy.py    CacheCopier gather/scatter byte semantics (csrc/cache_ops/kernels.cu)
             and the fused scatter + re-rotate
  rope.py    RoPE re-rotation (adapter.py:30-88, 118-295)
  fp8.py     OCP e4m3 encode/decode used by the fp8 path
  select.py  deviation keys, per-chunk top-k and merge (spec of the selection
             kernels; the reference has no such kernel)
  kvio.py    store/load record format and copy plan of the daric-store GPU I/O
             (daric/management/service/gpu_kv_io.py)
  c/oracle_copy.c + native.py
             a second, independent restatement in C (OpenMP) of the page
             copies and the fused scatter + re-rotation, built by build.py;
             byte-identical to copy.py on every layout and dtype
             (tests/test_oracle_native.py) and timed as bench.py's CPU baseline

The recompute budget (daric/adaption/policy.py) is host logic of the product
(daric_amd/policy.py) and is pinned by vectors of the reference's own function
(tests/golden/policy_vectors.json), not restated here.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker or as the timed CPU baseline. The
product path (daric_amd) never imports it and fails loudly when its HIP library
is missing.

Pinning: every function here is checked in tests/test_oracle_*.py against
facts that do not restate its formula (brute-force byte loops, torch indexing
semantics, complex-number RoPE, composition/identity invariants, torch's own
float8 cast, numpy's stable sort, fp64 sums). The reference ships no tests or
golden vectors for this path. Functions that only an import of the reference
could pin are marked "parity unpinned" in their docstrings.
"""
