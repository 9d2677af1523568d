"""Property test of the C library's host validation against the oracle's
restatement of the reference's checks (csrc/cache_ops/helpers.cu:15-174,
copier.cpp:32-66, kernels.cu:135-161): random KV layouts (dimension orders,
padding holes, overlaps, page-first or not) and random job lists must be
rejected with the same message, or accepted by both. No GPU is used: an
accepted call fails afterwards at its first HIP call, which this container
has no device for (or succeeds on a machine that has one), and is counted as
accepted."""
import ctypes

import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from daric_amd import _lib
from oracle.copy import OracleCopier
from oracle.layout import OracleError
from tests.test_capi_cpu import CCopier, fake


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def layouts():
    @st.composite
    def build(draw):
        page_first = draw(st.booleans())
        nb = draw(st.integers(1, 6))
        ps = draw(st.sampled_from([1, 2, 4]))
        h = draw(st.integers(1, 3))
        d = draw(st.sampled_from([2, 4, 8]))
        shape = (nb, 2, ps, h, d) if page_first else (2, nb, ps, h, d)
        order = draw(st.permutations(range(5)))           # physical dim order, innermost last
        pads = draw(st.lists(st.sampled_from([0, 0, 0, 1, 3]), min_size=5, max_size=5))
        strides = [0] * 5
        acc = 1
        for dim in reversed(order):
            strides[dim] = acc
            acc *= shape[dim] + pads[dim]
        if draw(st.integers(0, 9)) == 0:                   # occasionally an overlap
            strides[draw(st.integers(0, 4))] = 0
        return page_first, shape, tuple(strides)
    return build()


@settings(max_examples=150, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(lay=layouts(), data=st.data())
def test_validation_agrees_with_oracle(lib, lay, data):
    page_first, shape, strides = lay
    elem = 2
    c = CCopier(lib)
    assert c.register_layer("L", fake(shape, torch.float16, strides=strides), int(page_first)) is None
    o = OracleCopier()
    o.register_layer("L", torch.empty_strided(shape, strides, dtype=torch.float16), page_first)
    store_n = data.draw(st.integers(0, 4096))
    assert c.register_store(fake((store_n,), torch.uint8, ptr=0x30000000)) is None
    o.register_store(torch.zeros(store_n, dtype=torch.uint8))
    n_jobs = data.draw(st.integers(0, 3))
    names = [data.draw(st.sampled_from(["L", "L", "L", "M"])) for _ in range(n_jobs)]
    offs = [data.draw(st.integers(-2, 4096)) for _ in range(n_jobs + data.draw(st.sampled_from([0, 0, 1])))]
    sizes = [data.draw(st.integers(-1, 2048)) for _ in range(n_jobs)]
    n_idx = data.draw(st.integers(0, 8))
    ioff = sorted(data.draw(st.integers(0, n_idx)) for _ in range(n_jobs + 1))
    if n_jobs and data.draw(st.integers(0, 7)) == 0:
        ioff = list(reversed(ioff))
    idx = fake((n_idx,), torch.int32, ptr=0x20000000)
    e_c = c.gather(names, offs, sizes, idx, ioff)
    if e_c is not None and e_c.startswith("HIP error"):
        e_c = None                    # passed validation, stopped at the first device call
    try:
        o.gather_pages(names, offs, sizes, torch.zeros(n_idx, dtype=torch.int32), ioff)
        e_o = None
    except OracleError as e:
        e_o = str(e)
    except (IndexError, ValueError):
        e_o = "oracle-rejected"
    if e_o == "oracle-rejected":
        assert e_c is not None
    else:
        assert e_c == e_o, (shape, strides, page_first, names, offs, sizes, ioff, e_c, e_o)
