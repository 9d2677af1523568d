"""The C restatement of the oracle (oracle/c/oracle_copy.c) against the numpy
oracle and against torch/numpy's own conversions.

The two oracles were written separately (numpy float64 arrays and torch casts
on one side; scalar C with hand-written conversions on the other), so
byte-for-byte agreement on every layout, dtype and pairing pins each against
the other. The C conversions are also checked exhaustively (decoding) and on
ties, subnormals and saturation (encoding) against torch's and numpy's casts.
"""
import numpy as np
import pytest
import torch

from oracle import build as obuild
from oracle import fp8 as ofp8
from oracle import native
from oracle import rope as orope
from oracle.copy import OracleCopier
from oracle.layout import page_copy_shape
from tests.gpu_util import make_layer


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not native.available():
        obuild.build(verbose=False)
    native.load()


def _edge_floats():
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(4.0),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),     # fp16 / e4m3 subnormals
        (rng.standard_normal(5000) * 1e4).astype(np.float32),      # fp16 overflow region
        np.array([0.0, -0.0, 448.0, -448.0, 464.0, 465.0, 1e6, 65504.0, 65519.0, 65520.0,
                  2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -6, 2.0 ** -9,
                  2.0 ** -10, 3 * 2.0 ** -11, np.inf, -np.inf], dtype=np.float32)])
    # exact ties between neighbouring codes of each format
    b = np.arange(-3000, 3000, dtype=np.int64)
    bf_ties = ((b.astype(np.uint32) << 16) | 0x8000).astype(np.uint32).view(np.float32)
    f16 = np.arange(0, 0x7bff, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    f16_ties = ((f16 + np.nextafter(f16.astype(np.float16), np.float16(np.inf)).astype(np.float64)) / 2)
    e4 = ofp8.decode(np.arange(0, 0x7e, dtype=np.uint8)).astype(np.float64)
    e4_ties = (e4[:-1] + e4[1:]) / 2
    ties = np.concatenate([bf_ties[np.isfinite(bf_ties)], f16_ties.astype(np.float32),
                           e4_ties.astype(np.float32), -e4_ties.astype(np.float32)])
    return np.concatenate([x, ties]).astype(np.float32)


def test_bf16_conversions():
    codes = np.arange(65536, dtype=np.uint16)
    got = native.convert_to_values(codes, torch.bfloat16)
    want = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).double().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    x = _edge_floats()
    enc = native.convert_to_codes(x, torch.bfloat16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(enc, ref)


def test_f16_conversions():
    codes = np.arange(65536, dtype=np.uint16)
    got = native.convert_to_values(codes, torch.float16)
    want = codes.view(np.float16).astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    x = _edge_floats()
    enc = native.convert_to_codes(x, torch.float16)
    with np.errstate(over="ignore"):
        assert np.array_equal(enc, x.astype(np.float16).view(np.uint16))


def test_e4m3_conversions():
    codes = np.arange(256, dtype=np.uint8)
    got = native.convert_to_values(codes, torch.uint8)
    want = ofp8.decode(codes).astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    x = _edge_floats()
    x = x[~np.isnan(x)]
    enc = native.convert_to_codes(x, torch.uint8)
    ref = ofp8.encode(x)
    # -0 and +0 both decode to zero; torch may keep or drop the sign of tiny negatives
    canon = lambda c: np.where(c == 0x80, 0, c)  # noqa: E731
    assert np.array_equal(canon(enc), canon(ref))


def _fused_case(layout, dtype, neox, rotary_dim, d=64, h=4, ps=16, nb=40, L=2, threads=4, seed=0,
                repeat_page=False):
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g) for _ in range(L)]
    pf = layers[0][1]
    t0 = layers[0][0]
    s = page_copy_shape(tuple(t0.shape), tuple(t0.stride()), t0.element_size(), pf)
    perm = np.random.default_rng(seed).permutation(np.arange(1, nb)).tolist()
    chunk_tokens, deltas = (37, 64, 16, 5, 20), (1024, 30720, 0, -300, 7)
    chunks, k = [], 0
    for n in chunk_tokens:
        npg = -(-n // ps)
        chunks.append(perm[k:k + npg])
        k += npg
    chunks[0][0] = 0                      # the null block
    chunks[3][0] = nb + 5                 # out of range: skipped
    if repeat_page:
        chunks[4] = [chunks[4][0], chunks[4][0]]
    names, offsets, sizes, flat, ioff, dl, nt = [], [], [], [], [0], [], []
    off = 0
    for c, bids in enumerate(chunks):
        for li in range(L):
            names.append(f"l{li}")
            offsets.append(off)
            sz = s.prefix_size * len(bids) * s.suffix_size
            sizes.append(sz)
            flat.extend(bids)
            ioff.append(len(flat))
            dl.append(deltas[c])
            nt.append(chunk_tokens[c])
            off += sz
    inv = orope.default_inv_freq(rotary_dim, 500000.0)
    gs = torch.Generator().manual_seed(seed + 1)
    if dtype == torch.uint8:
        store = torch.from_numpy(ofp8.encode(torch.randn(off, generator=gs).numpy()))
    else:
        e = torch.empty(0, dtype=dtype).element_size()
        store = torch.randn(off // e, generator=gs).to(dtype).view(torch.uint8)
    a, b = OracleCopier(), native.NativeOracleCopier(threads)
    la = [t.clone() for t, _ in layers]
    lb = [t.clone() for t, _ in layers]
    for li in range(L):
        a.register_layer(f"l{li}", la[li], pf)
        b.register_layer(f"l{li}", lb[li], pf)
        if dtype == torch.uint8:
            sc = (0.5 + torch.rand(h if layout != "mla" else 1, generator=gs)).float().numpy()
            a.register_k_scale(f"l{li}", sc)
            b.register_k_scale(f"l{li}", sc)
    a.register_store(store.clone())
    b.register_store(store.clone())
    idx = torch.tensor(flat, dtype=torch.int32)
    a.scatter_pages_rerotate(names, offsets, sizes, idx, ioff, dl, nt, inv, rotary_dim, neox)
    b.scatter_pages_rerotate(names, offsets, sizes, idx, ioff, dl, nt, inv, rotary_dim, neox)
    for x, y in zip(la, lb):
        assert torch.equal(x.contiguous().view(torch.uint8), y.contiguous().view(torch.uint8))
    return la


@pytest.mark.parametrize("layout", ["nhd", "hnd", "pf", "pf_hnd", "packed", "mla"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.uint8])
@pytest.mark.parametrize("neox", [True, False])
def test_fused_matches_numpy_oracle(layout, dtype, neox):
    _fused_case(layout, dtype, neox, 64, d=128 if dtype == torch.uint8 else 64)


@pytest.mark.parametrize("rotary_dim", [24, 10])
@pytest.mark.parametrize("threads", [1, 3])
def test_fused_partial_rotary_and_threads(rotary_dim, threads):
    _fused_case("nhd", torch.bfloat16, True, rotary_dim, threads=threads, seed=4)
    _fused_case("pf", torch.float16, False, rotary_dim, threads=threads, seed=5)


def test_fused_page_listed_twice_rotates_twice():
    # a job naming the same page twice: the numpy oracle rotates its slots
    # twice in order; the C path must run that job sequentially and agree
    _fused_case("nhd", torch.bfloat16, True, 64, threads=4, repeat_page=True)


@pytest.mark.parametrize("gather", [True, False])
def test_page_copies_match_numpy_oracle(gather):
    g = torch.Generator().manual_seed(11)
    nb, ps, h, d = 24, 16, 2, 32
    for layout in ("nhd", "hnd", "pf", "packed", "mla"):
        t, pf = make_layer(layout, nb, ps, h, d, torch.bfloat16, g, kind="bytes")
        s = page_copy_shape(tuple(t.shape), tuple(t.stride()), t.element_size(), pf)
        sel = [[3, 0, 7], [5, 5, 2], [nb + 1, 9]]      # null, repeated and out-of-range pages
        off, offsets, sizes, flat, ioff = 0, [], [], [], [0]
        for p in sel:
            offsets.append(off)
            sz = s.prefix_size * len(p) * s.suffix_size
            sizes.append(sz)
            flat.extend(p)
            ioff.append(len(flat))
            off += sz
        store = torch.randint(0, 256, (off + 64,), dtype=torch.uint8, generator=g)
        ta, tb = t.clone(), t.clone()
        a, b = OracleCopier(), native.NativeOracleCopier(4)
        a.register_layer("x", ta, pf)
        b.register_layer("x", tb, pf)
        a.register_store(store.clone())
        b.register_store(store.clone())
        idx = torch.tensor(flat, dtype=torch.int32)
        fn = "gather_pages" if gather else "scatter_pages"
        getattr(a, fn)(["x"] * 3, offsets, sizes, idx, ioff)
        getattr(b, fn)(["x"] * 3, offsets, sizes, idx, ioff)
        assert torch.equal(a.store, b.store), layout
        assert torch.equal(ta.contiguous().view(torch.uint8), tb.contiguous().view(torch.uint8)), layout


def test_same_checks_as_numpy_oracle():
    # the plan and every check are the numpy oracle's: a wrong byte size fails alike
    t = torch.zeros(2, 4, 16, 2, 32, dtype=torch.bfloat16)
    for c in (OracleCopier(), native.NativeOracleCopier(2)):
        c.register_layer("x", t, False)
        c.register_store(torch.zeros(1 << 16, dtype=torch.uint8))
        with pytest.raises(Exception, match="byte_size mismatch"):
            c.scatter_pages(["x"], [0], [100], torch.tensor([1], dtype=torch.int32), [0, 1])
