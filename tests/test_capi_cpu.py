"""CPU-side checks of the C-ABI library (no GPU needed, no kernel launched).

- the built library loads and exports every function include/daric_cache_ops.h
  declares;
- host validation rejects bad jobs with the same message, in the same order,
  as the oracle's restatement of the reference's checks (descriptors carry fake
  device pointers; every case fails before any HIP call);
- the element conversions and the fast divider used by the kernels, compiled
  for the host from the same headers, agree with torch / exact division.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from daric_amd import _lib
from oracle import fp8 as ofp8
from oracle.copy import OracleCopier
from oracle.layout import OracleError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "daric_cache_ops.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from daric_amd import build
        build.build(verbose=False)
    return _lib.load()


@pytest.fixture(scope="module")
def hosttest(lib):
    from daric_amd import build
    h = ctypes.CDLL(build.HOSTTEST_LIB)
    h.daric_hosttest_encode_e4m3.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    h.daric_hosttest_encode_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    h.daric_hosttest_e4m3_to_f32.argtypes = [ctypes.c_uint32]
    h.daric_hosttest_e4m3_to_f32.restype = ctypes.c_float
    h.daric_hosttest_f32_to_f16.argtypes = [ctypes.c_float]
    h.daric_hosttest_f32_to_f16.restype = ctypes.c_uint32
    h.daric_hosttest_fastdiv_errors.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
    h.daric_hosttest_fastdiv_errors.restype = ctypes.c_int64
    h.daric_hosttest_quant_quotients.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                                 ctypes.c_int64, ctypes.c_void_p]
    h.daric_hosttest_layer_minor.argtypes = [ctypes.c_int, ctypes.c_int64]
    h.daric_hosttest_layer_minor.restype = ctypes.c_int64
    return h


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(daric_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must cover the header"
    assert lib.daric_abi_version() == _lib.ABI_VERSION == 5


def fake(shape, dtype, device=0, strides=None, ptr=0x10000000):
    t = torch.empty(0, dtype=dtype)
    d = _lib.DaricTensor()
    d.data = ptr
    d.ndim = len(shape)
    d.elem_size = t.element_size()
    d.device = device
    d.dtype = _lib.DTYPE_CODES[dtype]
    if strides is None:
        strides, acc = [], 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    for i, (s, st) in enumerate(zip(shape, strides)):
        d.sizes[i] = s
        d.strides[i] = st
    return d


class CCopier:
    """Direct ctypes driver of the C copier (the Python shim needs real tensors)."""

    def __init__(self, lib):
        self.lib = lib
        self.h = ctypes.c_void_p()
        assert lib.daric_copier_create(ctypes.byref(self.h)) == 0

    def err(self, status):
        return None if status == 0 else self.lib.daric_last_error().decode()

    def register_layer(self, name, d, pf):
        return self.err(self.lib.daric_copier_register_layer(self.h, name.encode(), ctypes.byref(d), pf))

    def register_store(self, d):
        return self.err(self.lib.daric_copier_register_store(self.h, ctypes.byref(d)))

    def gather(self, names, offsets, sizes, idx, idx_off, fn="daric_copier_gather_pages"):
        off, sz, io = _lib.I64(offsets), _lib.I64(sizes), _lib.I64(idx_off)
        return self.err(getattr(self.lib, fn)(
            self.h, _lib.str_array(names), len(names), off.ptr, off.n, sz.ptr, sz.n,
            ctypes.byref(idx), io.ptr, io.n, ctypes.c_uint64(0)))


def oracle_error(fn):
    try:
        fn()
    except OracleError as e:
        return str(e)
    return None


LAYER_SHAPE = (2, 4, 2, 2, 4)


def test_validation_matches_oracle(lib):
    c = CCopier(lib)
    o = OracleCopier()
    layer = torch.zeros(LAYER_SHAPE, dtype=torch.float16)
    assert c.register_layer("a", fake(LAYER_SHAPE, torch.float16), 0) is None
    o.register_layer("a", layer, False)
    idx = fake((1,), torch.int32, ptr=0x20000000)
    oidx = torch.tensor([1], dtype=torch.int32)

    def both(names, offs, sizes, idx_off, i=idx, oi=oidx):
        return c.gather(names, offs, sizes, i, idx_off), oracle_error(
            lambda: o.gather_pages(names, offs, sizes, oi, idx_off))

    e_c, e_o = both(["a"], [0], [64], [0, 1])
    assert e_c == e_o and "store buffer not registered" in e_c
    assert c.register_store(fake((128,), torch.uint8, ptr=0x30000000)) is None
    o.register_store(torch.zeros(128, dtype=torch.uint8))
    assert both([], [], [], [0]) == (None, None)
    cases = [
        (["a"], [], [64], [0, 1]),
        (["a"], [0], [64, 1], [0, 1]),
        (["a"], [0], [64], [0]),
        (["a"], [0], [64], [0, 2]),
        (["a", "a"], [0, 0], [0, 0], [1, 0, 1]),
        (["a"], [-1], [64], [0, 1]),
        (["a"], [100], [64], [0, 1]),
        (["a"], [200], [0], [0, 1]),
        (["b"], [0], [64], [0, 1]),
        (["a"], [0], [63], [0, 1]),
    ]
    for case in cases:
        e_c, e_o = both(*case)
        assert e_c is not None and e_c == e_o, (case, e_c, e_o)
    # indices tensor properties
    e_c = c.gather(["a"], [0], [64], fake((1,), torch.int64, ptr=0x20000000), [0, 1])
    assert e_c == "indices_flat must be int32"
    e_c = c.gather(["a"], [0], [64], fake((1,), torch.int32, device=-1), [0, 1])
    assert e_c == "indices_flat must be on CUDA"
    e_c = c.gather(["a"], [0], [64], fake((1,), torch.int32, device=1), [0, 1])
    assert e_c == "indices_flat must be on the same device as kvcache"


@pytest.mark.parametrize("fn", ["daric_copier_gather_tokens", "daric_copier_scatter_tokens"])
def test_token_copy_validation_matches_oracle(lib, fn):
    """gather/scatter_tokens: gather_pages' checks in the same order, then the
    token-major byte size and layout checks, with the oracle's messages."""
    c = CCopier(lib)
    o = OracleCopier()
    shapes = {"a": ((2, 4, 2, 2, 4), False), "p": ((4, 2, 8), True), "m": ((4, 2, 8), False),
              "q": ((4, 8), False)}
    for name, (shape, pf) in shapes.items():
        assert c.register_layer(name, fake(shape, torch.float16), int(pf)) is None
        o.register_layer(name, torch.zeros(shape, dtype=torch.float16), pf)
    idx = fake((2,), torch.int32, ptr=0x20000000)
    oidx = torch.tensor([1, 2], dtype=torch.int32)
    ofn = o.gather_tokens if "gather" in fn else o.scatter_tokens

    def both(names, offs, sizes, idx_off):
        return c.gather(names, offs, sizes, idx, idx_off, fn), oracle_error(
            lambda: ofn(names, offs, sizes, oidx, idx_off))

    e_c, e_o = both(["a"], [0], [64], [0, 1])
    assert e_c == e_o and "store buffer not registered" in e_c
    assert c.register_store(fake((4096,), torch.uint8, ptr=0x30000000)) is None
    o.register_store(torch.zeros(4096, dtype=torch.uint8))
    assert both([], [], [], [0]) == (None, None)
    # every case below fails validation, so no HIP call is reached with the
    # fake pointers
    cases = [
        (["a"], [0], [63], [0, 1]),          # token-major bytes are 2*1*2*2*4*2 = 64
        (["a"], [0], [100], [0, 2]),         # two pages: 128
        (["p"], [0], [64], [0, 1]),          # 3-D (MLA-like) layer, K only: 1*1*2*1*8*2 = 32
        (["q"], [0], [16], [0, 1]),          # 2-D tensor: no token-major layout
        (["b"], [0], [64], [0, 1]),
        (["a"], [4090], [64], [0, 1]),
    ]
    for names, offs, sizes, io in cases:
        e_c, e_o = both(names, offs, sizes, io)
        assert e_o is not None and e_c == e_o, (names, sizes, e_c, e_o)
    # the sizes the oracle accepts (checked on the oracle only)
    for names, sizes, io in ((["a"], [64], [0, 1]), (["a"], [128], [0, 2]), (["p"], [32], [0, 1])):
        assert oracle_error(lambda: ofn(names, [0], sizes, oidx, io)) is None


def test_layout_errors_match_oracle(lib):
    from oracle.layout import page_copy_shape
    cases = [
        ((2, 5, 16, 4, 32), (5 * 16 * 4 * 64, 16 * 4 * 64, 4 * 64, 64, 1), False),   # hole
        ((2, 5, 16, 4, 32), (5 * 16 * 32, 16 * 32, 32, 0, 1), False),                # stride 0
        ((2, 5, 16, 4, 32), (0, 16 * 4 * 32, 4 * 32, 32, 1), False),                 # K/V overlap
        ((5, 2, 16, 4, 32), (16 * 4 * 32, 16 * 4 * 32, 4 * 32, 32, 1), True),        # pages overlap
    ]
    for shape, strides, pf in cases:
        c = CCopier(lib)
        assert c.register_layer("x", fake(shape, torch.float16, strides=strides), int(pf)) is None
        assert c.register_store(fake((1 << 20,), torch.uint8, ptr=0x30000000)) is None
        e_c = c.gather(["x"], [0], [64], fake((1,), torch.int32, ptr=0x20000000), [0, 1])
        e_o = oracle_error(lambda: page_copy_shape(shape, strides, 2, pf))
        assert e_o is not None and e_c == e_o, (shape, e_c, e_o)


def test_register_errors(lib):
    c = CCopier(lib)
    assert c.register_layer("a", fake(LAYER_SHAPE, torch.float16, device=-1), 0) == \
        "kvcache tensor must be on GPU: a"
    assert c.register_store(fake((4, 4), torch.uint8)) == "store buffer must be 1D"
    assert c.register_store(fake((16,), torch.int32)) == "store buffer must be uint8"
    assert c.register_store(fake((16,), torch.uint8, device=-1)) == "staging buffer must be on CUDA"
    assert c.register_store(fake((16,), torch.uint8, strides=(2,))) == "store buffer must be contiguous"
    # as torch: a tensor without elements is contiguous whatever its strides
    assert c.register_store(fake((0,), torch.uint8, strides=(2,))) is None


def test_rerotate_layout_errors(lib):
    rope = _lib.DaricRope()
    rope.inv_freq = 0x40000000
    rope.rotary_dim = 16
    rope.is_neox = 1
    bt = fake((4,), torch.int32, ptr=0x20000000)
    seg = (_lib.DaricRopeSegment * 1)(_lib.DaricRopeSegment(0, 0, 16, 5))

    def run(shape, pf, dtype=torch.bfloat16, rd=16, nseg_tokens=16):
        rope.rotary_dim = rd
        seg[0].n_tokens = nseg_tokens
        arr = (_lib.DaricTensor * 1)(fake(shape, dtype))
        st = lib.daric_rerotate_pages(arr, 1, pf, ctypes.byref(bt), seg, 1, ctypes.byref(rope), None,
                                      ctypes.c_uint64(0))
        if not st:
            return None
        msg = lib.daric_last_error().decode()
        # the layouts the reference's rotation rejects with ValueError carry their
        # own status, which the Python wrapper raises as ValueError
        with pytest.raises(ValueError if st == _lib.ERR_VALUE else RuntimeError, match=re.escape(msg)):
            _lib.check(st)
        return st, msg

    assert run((8, 2, 4, 32), 0) == (
        _lib.ERR_VALUE, "Invalid 4D KV cache for rerotate: shape=[8, 2, 4, 32], stride=[256, 128, 32, 1], "
        "rotary_dim=16, constraint=page_first must be true")
    st, msg = run((8, 2, 4, 32), 1, rd=32)
    assert st == _lib.ERR_VALUE and "rotary_dim must be positive, even, and no greater" in msg
    assert run((8, 32), 1) == (_lib.ERR_VALUE, "Unsupported KV cache rank for rerotate: 2")
    st, msg = run((2, 8, 4, 2, 16), 0, dtype=torch.float32)
    assert st == 1 and "unsupported KV cache dtype" in msg
    st, msg = run((2, 8, 4, 2, 16), 0, nseg_tokens=17)
    assert st == 1 and "reads past the end of block_table" in msg


def test_noalloc_rejects_job_lists_beyond_its_scratch(lib):
    """The allocation-free fused entry point stages descriptors in a static
    262144-byte array per GPU: 3276 jobs of 80 bytes fit; one more is refused
    before any device work (every pointer here is fake)."""
    c = CCopier(lib)
    span = 16 * 8 * 128 * 2
    assert c.register_layer("L", fake((2, 8, 16, 8, 128), torch.bfloat16), 0) is None
    assert c.register_store(fake((2 * span,), torch.uint8, ptr=0x30000000)) is None
    idx = fake((1,), torch.int32, ptr=0x20000000)
    rope = _lib.DaricRope(0x40000000, 64, 1)

    def run(n):
        names = ["L"] * n
        sizes = [2 * span] + [0] * (n - 1)          # job 0 moves one page, the others none
        off, sz, io = _lib.I64([0] * n), _lib.I64(sizes), _lib.I64([0] + [1] * n)
        dl, nt = _lib.I64([5] * n), _lib.I64([16] * n)
        st = lib.daric_copier_scatter_pages_rerotate_noalloc(
            c.h, _lib.str_array(names), n, off.ptr, off.n, sz.ptr, sz.n, ctypes.byref(idx), io.ptr, io.n,
            dl.ptr, nt.ptr, ctypes.byref(rope), ctypes.c_uint64(0))
        return st, lib.daric_last_error().decode()

    st, msg = run(3277)
    assert st == 1 and "need 262400 bytes of scratch, more than the 262144 bytes (3276 jobs)" in msg


def test_host_fp8_conversion_matches_oracle(hosttest):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(50),
        rng.standard_normal(50000).astype(np.float32) * np.float32(1e-2),
        (rng.random(50000).astype(np.float32) * 600 - 300),
        np.array([0.0, -0.0, 448, 449, 463.99, 464, 464.01, 1e9, -1e9, np.inf, -np.inf,
                  2 ** -9, 2 ** -10, 3 * 2 ** -11, 2 ** -6, 2 ** -6 * 0.999], np.float32),
    ]).astype(np.float32)
    # every midpoint between adjacent e4m3 values (rounding ties)
    pos = np.unique(ofp8.decode(np.arange(0x7f)))
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    vals = np.concatenate([vals, mids, -mids]).astype(np.float32)
    out = np.empty(vals.shape, np.uint8)
    hosttest.daric_hosttest_encode_e4m3(vals.ctypes.data, out.ctypes.data, len(vals))
    want = ofp8.encode(vals)
    assert np.array_equal(out, want)
    for c in range(256):
        got = hosttest.daric_hosttest_e4m3_to_f32(c)
        ref = float(ofp8.decode([c])[0])
        assert (np.isnan(got) and np.isnan(ref)) or got == ref


def test_quant_quotient_is_correctly_rounded_division(hosttest):
    """The quantising merge's x / scale (one reciprocal per scale and two FMAs
    per element for scales in [2^-60, 2^60], a division otherwise) against
    numpy's IEEE float32 division, for every bf16 and every fp16 value of x
    (zeros, subnormals, infinities and NaNs included) and 320 scales: random
    ones over the whole fast range and over typical fp8 scales, significands of
    all ones and of 1 + a few ulps (where a reciprocal rounds worst), powers of
    two, and scales outside the fast range. The float32 quotient must be the
    correctly rounded one wherever |x / scale| lies in [2^-11, 480] (the e4m3
    codes depend on its bits only there), and the e4m3 code must be equal for
    every x."""
    bits = np.arange(65536, dtype=np.uint32)
    x = np.ascontiguousarray(np.concatenate([
        (bits << 16).view(np.float32),
        bits.astype(np.uint16).view(np.float16).astype(np.float32)]))
    rng = np.random.default_rng(11)
    n = 40
    scales = np.concatenate([
        np.exp2(rng.uniform(-60, 60, n)),
        np.exp(rng.uniform(np.log(1e-5), np.log(1e3), n)),
        np.float32(2 - 2.0 ** -23) * np.exp2(rng.integers(-40, 40, n).astype(np.float64)),
        (np.uint32(0x3f800000) + rng.integers(1, 16, n).astype(np.uint32)).view(np.float32)
        * np.exp2(rng.integers(-30, 30, n).astype(np.float64)),
        (np.uint32(0x3fffffff) - rng.integers(0, 16, n).astype(np.uint32)).view(np.float32)
        * np.exp2(rng.integers(-30, 30, n).astype(np.float64)),
        np.exp2(rng.integers(-60, 61, n).astype(np.float64)),
        np.array([2.0 ** -60, 2.0 ** 60, 2.0 ** -61, 2.0 ** 61, 2.0 ** -70, 2.0 ** 70, 1e-30, 1e30,
                  0.0017, 0.25, 1.0, 3.0, 448.0, 0.007, 1.1754944e-38, 3.0e38] * (n // 16)),
        np.exp2(rng.uniform(-80, 80, n)),
    ]).astype(np.float32)
    scales = np.ascontiguousarray(scales)
    for i in range(0, len(scales), 32):
        sc = np.ascontiguousarray(scales[i:i + 32])
        got = np.empty((len(sc), len(x)), np.float32)
        hosttest.daric_hosttest_quant_quotients(x.ctypes.data, len(x), sc.ctypes.data, len(sc),
                                                got.ctypes.data)
        with np.errstate(all="ignore"):
            want = (x[None, :] / sc[:, None]).astype(np.float32)
            region = (np.abs(want) >= 2.0 ** -11) & (np.abs(want) <= 480)
        bad = region & (got.view(np.uint32) != want.view(np.uint32))
        assert not bad.any(), (sc[np.nonzero(bad)[0][0]], x[np.nonzero(bad)[1][0]])
        assert np.array_equal(ofp8.encode(got.ravel()), ofp8.encode(want.ravel()))


def test_host_bf16_f16_conversion_matches_torch(hosttest):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, 400000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[~np.isnan(vals)]
    out = np.empty(vals.shape, np.uint16)
    hosttest.daric_hosttest_encode_bf16(vals.ctypes.data, out.ctypes.data, len(vals))
    want = torch.from_numpy(vals.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(out, want)
    sample = rng.standard_normal(2000).astype(np.float32) * 1e3
    got = np.array([hosttest.daric_hosttest_f32_to_f16(float(v)) for v in sample], np.uint16)
    want = torch.from_numpy(sample).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("d", [1, 2, 3, 7, 8, 16, 68, 100, 128, 1000, 65535, 2 ** 20 + 7])
def test_host_fastdiv(hosttest, d):
    assert hosttest.daric_hosttest_fastdiv_errors(d, 0, 1 << 20) == 0
    assert hosttest.daric_hosttest_fastdiv_errors(d, (1 << 31) - (1 << 18), 1 << 31) == 0


C_CONSUMER = r"""
#include <stdio.h>
#include <string.h>
#include "daric_cache_ops.h"

int main(void) {
    daric_copier* c = NULL;
    if (daric_abi_version() != DARIC_ABI_VERSION) { puts("abi"); return 1; }
    if (daric_copier_create(&c) != DARIC_OK || c == NULL) { puts("create"); return 2; }
    /* no store registered: the reference's first check (copier.cpp:46) */
    int64_t off = 0, size = 16, ioff[2] = {0, 1};
    const char* names[1] = {"model.layers.0.self_attn.attn"};
    daric_tensor idx;
    memset(&idx, 0, sizeof idx);
    int st = daric_copier_gather_pages(c, names, 1, &off, 1, &size, 1, &idx, ioff, 2, 0);
    if (st == DARIC_OK) { puts("gather accepted a call without a store"); return 3; }
    printf("status %d: %s\n", st, daric_last_error());
    if (daric_copier_destroy(c) != DARIC_OK) { puts("destroy"); return 4; }
    return 0;
}
"""


def test_c_consumer_compiles_and_links(lib, tmp_path):
    # the header is plain C99 and the library links and runs from a C program
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    src = tmp_path / "consumer.c"
    src.write_text(C_CONSUMER)
    exe = tmp_path / "consumer"
    libdir = os.path.dirname(_lib.LIB_PATH)
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src),
                    "-o", str(exe), "-L", libdir, "-ldaric_cache_ops", f"-Wl,-rpath,{libdir}"],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "store buffer not registered" in out.stdout


def test_merge_of_nothing_makes_no_device_call(lib):
    """merge_rows with empty recomputed rows (null data pointer) or chunks
    without tokens returns before any HIP call: with no GPU here, any launch
    or device call would fail the call."""
    layer = (_lib.DaricTensor * 1)(fake((2, 8, 16, 4, 64), torch.bfloat16))
    bt = fake((8,), torch.int32, ptr=0x20000000)
    empty = fake((1, 0, 4, 64), torch.bfloat16, ptr=0)
    chunks = (_lib.DaricChunk * 2)(_lib.DaricChunk(0, 0, 0, 4, 0), _lib.DaricChunk(1, 0, 0, 5, 3))
    sel = fake((1, 2, 5), torch.int32, ptr=0x50000000)
    st = lib.daric_merge_rows(layer, 1, 0, ctypes.byref(bt), ctypes.byref(empty), ctypes.byref(empty),
                              chunks, 2, ctypes.byref(sel), None, None, ctypes.c_uint64(0))
    assert st == 0, lib.daric_last_error().decode()
    # rows present but no chunk has tokens: still nothing to merge
    rows = fake((1, 6, 4, 64), torch.bfloat16, ptr=0x60000000)
    st = lib.daric_merge_rows(layer, 1, 0, ctypes.byref(bt), ctypes.byref(rows), ctypes.byref(rows),
                              chunks, 2, ctypes.byref(sel), None, None, ctypes.c_uint64(0))
    assert st == 0, lib.daric_last_error().decode()
    # a chunk with tokens does reach the device (and fails here, without a GPU)
    chunks[1].n_tokens = 6
    st = lib.daric_merge_rows(layer, 1, 0, ctypes.byref(bt), ctypes.byref(rows), ctypes.byref(rows),
                              chunks, 2, ctypes.byref(sel), None, None, ctypes.c_uint64(0))
    assert st != 0


def test_chunk_start_inside_a_page_is_checked_against_the_block_table(lib):
    """tok_start moves a chunk's tokens along its block list: a chunk whose
    last token falls past the block table is refused."""
    layer = (_lib.DaricTensor * 1)(fake((2, 8, 16, 4, 64), torch.bfloat16))
    bt = fake((4,), torch.int32, ptr=0x20000000)
    rows = fake((1, 64, 4, 64), torch.bfloat16, ptr=0x60000000)
    keys = fake((1, 64), torch.float32, ptr=0x70000000)

    def run(bo, n, ts):
        ch = (_lib.DaricChunk * 1)(_lib.DaricChunk(bo, 0, n, 1, ts))
        st = lib.daric_kv_deviation(layer, 1, 0, ctypes.byref(bt), ctypes.byref(rows), ch, 1, None,
                                    ctypes.byref(keys), ctypes.c_uint64(0))
        return lib.daric_last_error().decode() if st else None

    assert "reads past the end of block_table" in run(0, 49, 16)       # tokens 16..64: page 4
    assert "reads past the end of block_table" in run(1, 40, 9)        # pages 1.. + (9 + 39) // 16 = 4
    assert "negative chunk field" in run(0, 4, -1)
    assert "reads past the end" not in (run(0, 48, 16) or "")           # tokens 16..63: pages 1-3


def test_select_merge_validation(lib):
    """daric_select_merge refuses bad arguments before any device call (fake
    device pointers; every case fails in validation)."""
    bf = (_lib.DaricTensor * 1)(fake((2, 8, 16, 4, 64), torch.bfloat16))
    f8 = (_lib.DaricTensor * 1)(fake((2, 8, 16, 4, 64), torch.uint8))
    bt = fake((8,), torch.int32, ptr=0x20000000)
    rows = fake((1, 64, 4, 64), torch.bfloat16, ptr=0x60000000)
    keys = fake((1, 64), torch.float32, ptr=0x70000000)
    sel = fake((1, 1, 4), torch.int32, ptr=0x50000000)
    sc = fake((1, 4), torch.float32, ptr=0x80000000)
    ch = (_lib.DaricChunk * 1)(_lib.DaricChunk(0, 0, 64, 4, 0))

    def run(layers, k_sc=None, v_sc=None, flags=0, sel_t=sel, chunk=ch):
        st = lib.daric_select_merge(layers, 1, 0, ctypes.byref(bt), ctypes.byref(rows), ctypes.byref(rows),
                                    chunk, 1, ctypes.byref(k_sc) if k_sc is not None else None,
                                    ctypes.byref(v_sc) if v_sc is not None else None, ctypes.byref(keys),
                                    ctypes.byref(sel_t), flags, ctypes.c_uint64(0))
        assert st != 0
        return st, lib.daric_last_error().decode()

    assert "unknown select_merge flags 4" in run(bf, flags=4)[1]
    assert "apply only to an fp8 cache" in run(bf, k_sc=sc, v_sc=sc)[1]
    assert "needs k_scales" in run(f8)[1]
    assert "needs v_scales" in run(f8, k_sc=sc)[1]
    small = fake((1, 1, 3), torch.int32, ptr=0x50000000)
    assert "smaller than a chunk's k" in run(bf, sel_t=small)[1]
    past = (_lib.DaricChunk * 1)(_lib.DaricChunk(6, 0, 40, 4, 5))   # tokens 5..44 from page 6: page 8
    assert "reads past the end of block_table" in run(bf, chunk=past)[1]


# (layers, items, launches): the merge at configs 3 and 5 (items = row batches x
# chunks), the in-place kernel at config 2 (page parts), one layer and one
# item, and grids past 2^24 - 1 blocks cut into launches by items or by layers.
@pytest.mark.parametrize("n_layers,n_items,launches", [
    (32, 1920, 1), (80, 416, 1), (32, 896, 1), (1, 1, 1), (3, 7, 1), (7, 5, 1),
    (80, 300_000, 2), (2, (1 << 24) - 1, 3), (1, 1 << 24, 2), ((1 << 24) + 5, 2, 4),
])
def test_layer_minor_grid_covers_every_pair_once(hosttest, n_layers, n_items, launches):
    """The layer-minor block order of the merge, the fused top-k + merge and
    the in-place lane kernel: every (layer, work item) pair is taken by
    exactly one block of exactly one launch, no launch passes 2^24 - 1 blocks
    (grid.x x 256 lanes < 2^32), and the grid is cut only when it must be."""
    assert hosttest.daric_hosttest_layer_minor(n_layers, n_items) == launches

