"""Pins the CPU oracle's gather/scatter and layout normalisation.

Checks use torch's own indexing on the logical tensor (not the byte formula the
oracle restates), the physical-span rule on permuted layouts, round trips and
the reference's validation messages (csrc/cache_ops/helpers.cu, copier.cpp).
"""
import pytest
import torch

from oracle.copy import OracleCopier, byte_view
from oracle.layout import OracleError, page_copy_shape


def rand_bytes(shape, dtype, gen):
    n = 1
    for s in shape:
        n *= s
    e = torch.empty(0, dtype=dtype).element_size()
    return torch.randint(0, 256, (n * e,), dtype=torch.uint8, generator=gen).view(dtype).view(shape)


def as_bytes(t):
    return t.contiguous().view(torch.uint8).reshape(-1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.uint8])
def test_shape_standard_layouts(dtype):
    e = torch.empty(0, dtype=dtype).element_size()
    nb, ps, h, d = 7, 16, 4, 32
    t = torch.empty(2, nb, ps, h, d, dtype=dtype)
    s = page_copy_shape(t.shape, t.stride(), e, False)
    span = ps * h * d * e
    assert (s.prefix_size, s.num_pages, s.page_stride, s.suffix_size, s.prefix_stride) == \
        (2, nb, span, span, nb * span)
    t = torch.empty(nb, 2, ps, h, d, dtype=dtype)
    s = page_copy_shape(t.shape, t.stride(), e, True)
    assert (s.prefix_size, s.num_pages, s.page_stride, s.suffix_size, s.prefix_stride) == \
        (1, nb, 2 * span, 2 * span, 0)


def test_shape_errors():
    t = torch.empty(2, 5, 16, 4, 64, dtype=torch.float16)[..., :32]  # hole
    with pytest.raises(OracleError, match="dense physical span.*relation=hole"):
        page_copy_shape(t.shape, t.stride(), 2, False)
    t = torch.empty(2, 5, 16, 1, 32).expand(2, 5, 16, 4, 32)          # stride 0
    with pytest.raises(OracleError, match="positive strides"):
        page_copy_shape(t.shape, t.stride(), 4, False)
    t = torch.empty(5, 16, 4, 32).unsqueeze(0).expand(2, 5, 16, 4, 32)  # K/V share memory
    with pytest.raises(OracleError, match="prefix/page regions overlap"):
        page_copy_shape(t.shape, t.stride(), 4, False)
    with pytest.raises(OracleError, match="must be on CUDA"):
        page_copy_shape((2, 3), (3, 1), 2, False, on_device=False)


def _copier(layers, store_bytes):
    c = OracleCopier()
    for name, (t, pf) in layers.items():
        c.register_layer(name, t, pf)
    store = torch.full((store_bytes,), 0xAB, dtype=torch.uint8)
    c.register_store(store)
    return c, store


@pytest.mark.parametrize("page_first", [False, True])
def test_gather_matches_torch_indexing(page_first):
    g = torch.Generator().manual_seed(1)
    nb, ps, h, d = 9, 4, 2, 8
    shape = (nb, 2, ps, h, d) if page_first else (2, nb, ps, h, d)
    t = rand_bytes(shape, torch.bfloat16, g)
    idx = torch.tensor([3, 0, 8, 1, 5], dtype=torch.int32)
    span = (2 if page_first else 1) * ps * h * d * 2
    nbytes = len(idx) * span * (1 if page_first else 2)
    c, store = _copier({"a": (t, page_first)}, nbytes + 64)
    c.gather_pages(["a"], [64], [nbytes], idx, [0, len(idx)])
    out = store[64:].view(-1, span) if page_first else store[64:].view(2, len(idx), span)
    for s, page in enumerate(idx.tolist()):
        if page_first:
            want = as_bytes(t[page]) if page else torch.full((span,), 0xAB, dtype=torch.uint8)
            assert torch.equal(out[s], want)
        else:
            for p in range(2):
                want = as_bytes(t[p, page]) if page else torch.full((span,), 0xAB, dtype=torch.uint8)
                assert torch.equal(out[p, s], want)
    assert torch.equal(store[:64], torch.full((64,), 0xAB, dtype=torch.uint8))


def test_gather_hnd_physical_span():
    # logical [2, NB, PS, H, D] over a physical [2, NB, H, PS, D] cache: the staged
    # page is the page's memory span in memory order (helpers.cu:22-64)
    g = torch.Generator().manual_seed(2)
    phys = rand_bytes((2, 6, 3, 4, 8), torch.float16, g)
    t = phys.permute(0, 1, 3, 2, 4)
    idx = torch.tensor([5, 2], dtype=torch.int32)
    span = 3 * 4 * 8 * 2
    c, store = _copier({"a": (t, False)}, 2 * 2 * span)
    c.gather_pages(["a"], [0], [2 * 2 * span], idx, [0, 2])
    out = store.view(2, 2, span)
    for p in range(2):
        for s, page in enumerate(idx.tolist()):
            assert torch.equal(out[p, s], as_bytes(phys[p, page]))


def test_scatter_roundtrip_and_null_block():
    g = torch.Generator().manual_seed(3)
    src = rand_bytes((2, 10, 4, 2, 8), torch.bfloat16, g)
    dst = torch.zeros_like(src)
    idx = torch.tensor([4, 0, 9, 2], dtype=torch.int32)
    span = 4 * 2 * 8 * 2
    n = 2 * len(idx) * span
    c = OracleCopier()
    c.register_layer("src", src, False)
    c.register_layer("dst", dst, False)
    c.register_store(torch.zeros(n, dtype=torch.uint8))
    c.gather_pages(["src"], [0], [n], idx, [0, 4])
    c.scatter_pages(["dst"], [0], [n], idx, [0, 4])
    for page in range(10):
        if page in (4, 9, 2):
            assert torch.equal(as_bytes(dst[:, page]), as_bytes(src[:, page]))
        else:
            assert torch.count_nonzero(dst[:, page].view(torch.int16)) == 0


def test_multi_job_offsets_and_order():
    # jobs of several layers land at their own offsets (gpu_kv_io.py:355-373 layout)
    g = torch.Generator().manual_seed(4)
    layers = {f"l{i}": (rand_bytes((2, 8, 2, 2, 4), torch.float16, g), False) for i in range(3)}
    span = 2 * 2 * 4 * 2
    idx = torch.tensor([1, 7, 3, 6], dtype=torch.int32)
    sizes = [2 * 2 * span, 2 * 2 * span, 2 * 2 * span]
    offs = [0, sizes[0], sizes[0] + sizes[1]]
    c, store = _copier(layers, sum(sizes))
    c.gather_pages(["l2", "l0", "l1"], offs, sizes, idx[[0, 1, 2, 3, 0, 1]], [0, 2, 4, 6])
    sel = [[1, 7], [3, 6], [1, 7]]
    for j, name in enumerate(["l2", "l0", "l1"]):
        t = layers[name][0]
        want = as_bytes(t[:, sel[j]])
        assert torch.equal(store[offs[j]: offs[j] + sizes[j]], want)


def test_validation_order_and_messages():
    t = torch.zeros(2, 4, 2, 2, 4, dtype=torch.float16)
    c = OracleCopier()
    c.register_layer("a", t, False)
    idx = torch.tensor([1], dtype=torch.int32)
    with pytest.raises(OracleError, match="store buffer not registered"):
        c.gather_pages(["a"], [0], [64], idx, [0, 1])
    c.register_store(torch.zeros(128, dtype=torch.uint8))
    c.gather_pages([], [], [], idx, [0])  # empty job list returns first
    with pytest.raises(OracleError, match="offsets length mismatch"):
        c.gather_pages(["a"], [], [64], idx, [0, 1])
    with pytest.raises(OracleError, match="indices_offsets size must be num_jobs \\+ 1"):
        c.gather_pages(["a"], [0], [64], idx, [0])
    with pytest.raises(OracleError, match="indices_flat must be int32"):
        c.gather_pages(["a"], [0], [64], idx.long(), [0, 1])
    with pytest.raises(OracleError, match="exceeds indices_flat.numel"):
        c.gather_pages(["a"], [0], [64], idx, [0, 2])
    with pytest.raises(OracleError, match="non-decreasing at job 0"):
        c.gather_pages(["a", "a"], [0, 0], [0, 0], torch.tensor([1, 1], dtype=torch.int32), [1, 0, 2])
    with pytest.raises(OracleError, match="store range out of bounds at job 0"):
        c.gather_pages(["a"], [100], [64], idx, [0, 1])
    with pytest.raises(OracleError, match="layer not registered: b"):
        c.gather_pages(["b"], [0], [64], idx, [0, 1])
    with pytest.raises(OracleError, match="byte_size mismatch at job 0 \\| C\\+\\+ expected bytes: 64"):
        c.gather_pages(["a"], [0], [63], idx, [0, 1])


def test_byte_view_offset():
    base = torch.arange(64, dtype=torch.int16)
    t = base[5:]
    mem, off = byte_view(t)
    assert off == 10 and mem[off] == 5


def _elem(t, layout, kv, page, p, h, d):
    """Element (kv, page, token p, head h, dim d) of a layer by explicit index
    arithmetic on its logical shape (independent of the oracle's views)."""
    if layout in ("nhd", "hnd"):          # logical [2, NB, PS, H, D]
        return t[kv, page, p, h, d]
    if layout in ("pf", "pf_hnd"):        # logical [NB, 2, PS, H, D]
        return t[page, kv, p, h, d]
    if layout == "packed":                # [NB, H, PS, 2D]
        return t[page, h, p, kv * (t.shape[3] // 2) + d]
    return t[page, p, d]                  # mla [NB, PS, hidden]


@pytest.mark.parametrize("layout", ["nhd", "hnd", "pf", "pf_hnd", "packed", "mla"])
def test_gather_tokens_brute_force_and_round_trip(layout):
    from tests.gpu_util import make_layer
    g = torch.Generator().manual_seed(21)
    nb, ps, h, d = 9, 4, 3, 5
    t, pf = make_layer(layout, nb, ps, h, d, torch.float16, g)
    n_kv = 1 if layout == "mla" else 2
    H, D = (1, h * d) if layout == "mla" else (h, d)
    sel = [4, 0, 8, nb + 2, 2]                      # null and out-of-range pages are skipped
    n = n_kv * len(sel) * ps * H * D * 2
    base = torch.randint(0, 256, (n + 8,), dtype=torch.uint8, generator=g)
    oc = OracleCopier()
    oc.register_layer("x", t, pf)
    oc.register_store(base.clone())
    idx = torch.tensor(sel, dtype=torch.int32)
    oc.gather_tokens(["x"], [8], [n], idx, [0, len(sel)])
    out = oc.store[8:].view(torch.float16).view(n_kv, len(sel), ps, H, D)
    keep = base[8:].view(torch.float16).view(n_kv, len(sel), ps, H, D)
    for kv in range(n_kv):
        for s, page in enumerate(sel):
            for p in range(ps):
                for hh in range(H):
                    for dd in range(D):
                        got = out[kv, s, p, hh, dd].view(torch.int16)
                        if 0 < page < nb:
                            want = _elem(t, layout, kv, page, p, hh, dd).view(torch.int16)
                        else:
                            want = keep[kv, s, p, hh, dd].view(torch.int16)
                        assert int(got) == int(want), (kv, s, p, hh, dd)
    assert torch.equal(oc.store[:8], base[:8])
    # scatter_tokens of the gathered rows into a zeroed copy restores exactly
    # the listed pages and leaves everything else zero
    z = torch.zeros_like(t)
    oc2 = OracleCopier()
    oc2.register_layer("x", z, pf)
    oc2.register_store(oc.store.clone())
    oc2.scatter_tokens(["x"], [8], [n], idx, [0, len(sel)])
    for page in range(nb):
        for kv in range(n_kv):
            for p in range(ps):
                for hh in range(H):
                    for dd in range(D):
                        got = _elem(z, layout, kv, page, p, hh, dd).view(torch.int16)
                        want = _elem(t, layout, kv, page, p, hh, dd).view(torch.int16) if page in (4, 8, 2) else 0
                        assert int(got) == int(want), (page, kv, p, hh, dd)


def test_gather_tokens_equals_gather_pages_for_nhd():
    # vLLM's [2, NB, PS, H, D] pages are token-major already: both gathers agree
    g = torch.Generator().manual_seed(22)
    t = torch.randn(2, 12, 16, 4, 8, generator=g).to(torch.bfloat16)
    sel = torch.tensor([3, 0, 11, 7], dtype=torch.int32)
    n = 2 * 4 * 16 * 4 * 8 * 2
    a, b = OracleCopier(), OracleCopier()
    for c in (a, b):
        c.register_layer("x", t, False)
        c.register_store(torch.full((n,), 7, dtype=torch.uint8))
    a.gather_pages(["x"], [0], [n], sel, [0, 4])
    b.gather_tokens(["x"], [0], [n], sel, [0, 4])
    assert torch.equal(a.store, b.store)
