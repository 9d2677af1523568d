"""GPU parity of the recompute-selection kernels against the CPU oracle:
deviation keys bit-exact (fixed reduction order), selected indices bit-exact
(ties to the lower index), merge bit-exact."""
import numpy as np
import pytest
import torch

from daric_amd import cache_ops
from oracle import select as osel
from tests.gpu_util import make_layer, same_bytes, to_dev

pytestmark = pytest.mark.gpu


def setup_case(dev, layout="nhd", dtype=torch.bfloat16, nb=64, ps=16, h=4, d=64, L=2,
               chunk_tokens=(100, 64, 37), k_frac=0.15, seed=0):
    g = torch.Generator().manual_seed(seed)
    layers = [make_layer(layout, nb, ps, h, d, dtype, g) for _ in range(L)]
    pf = layers[0][1]
    perm = np.random.default_rng(seed).permutation(np.arange(1, nb)).tolist()
    bt, chunks, p, row = [], [], 0, 0
    for n in chunk_tokens:
        npg = -(-n // ps)
        chunks.append((len(bt), row, n, max(1, int(round(k_frac * n)))))
        bt.extend(perm[p:p + npg])
        p += npg
        row += n
    T = row
    bt = np.asarray(bt, np.int32)
    # recomputed K = cached K + heavy-tailed noise (config 3 style)
    kv = osel.k_rows_view(layers[0][0], pf)
    hh = kv.shape[2]
    rng = np.random.default_rng(seed + 1)
    k_new = torch.empty(L, T, hh, d if layout != "mla" else h * d, dtype=torch.bfloat16)
    v_new = torch.randn(L, T, hh, k_new.shape[3], generator=g).to(torch.bfloat16)
    for l, (t, _) in enumerate(layers):
        kvl = osel.k_rows_view(t, pf)
        for (bo, ro, n, _k) in chunks:
            blk, s = osel.chunk_slots(bt, bo, n, kvl.shape[1])
            base = kvl[torch.as_tensor(blk), torch.as_tensor(s)].float()
            noise = torch.from_numpy(0.1 * rng.standard_t(3, size=tuple(base.shape))).float()
            k_new[l, ro:ro + n] = (base + noise).to(torch.bfloat16)
    return layers, pf, bt, chunks, k_new, v_new


@pytest.mark.parametrize("layout", ["nhd", "hnd", "pf", "packed"])
def test_deviation_topk_merge_parity(dev, layout):
    layers, pf, bt, chunks, k_new, v_new = setup_case(dev, layout)
    cpu = [t for t, _ in layers]
    gpu = [to_dev(t, dev) for t in cpu]
    btd = torch.from_numpy(bt).to(dev)
    keys_o = osel.deviation(cpu, pf, bt, k_new, chunks)
    keys_g = cache_ops.kv_deviation(gpu, pf, btd, k_new.to(dev), chunks)
    torch.cuda.synchronize()
    kg = keys_g.cpu().numpy()
    assert np.array_equal(kg.view(np.uint32), keys_o.view(np.uint32)), \
        f"{int((kg != keys_o).sum())} keys differ"
    kmax = max(c[3] for c in chunks) + 3
    sel_o = osel.topk_per_chunk(keys_o, chunks, kmax)
    sel_g = cache_ops.topk_per_chunk(keys_g, chunks, kmax=kmax)
    torch.cuda.synchronize()
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    osel.merge_rows(cpu, pf, bt, k_new, v_new, chunks, sel_o)
    cache_ops.merge_rows(gpu, pf, btd, k_new.to(dev), v_new.to(dev), chunks, sel_g)
    torch.cuda.synchronize()
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)


@pytest.mark.parametrize("layout", ["nhd", "hnd", "pf", "packed", "mla"])
@pytest.mark.parametrize("row_dtype", [torch.bfloat16, torch.float16])
def test_quantising_merge_parity(dev, layout, row_dtype):
    """bf16/fp16 recomputed rows merged into an fp8 (e4m3) cache: codes of
    x / scale[l, h] (K and V scales differ per layer and head), bit-exact
    against the oracle; every other byte of the cache unchanged."""
    layers, pf, bt, chunks, _k, _v = setup_case(dev, layout, dtype=torch.uint8, d=64, h=4, L=3)
    cpu = [t for t, _ in layers]
    gpu = [to_dev(t, dev) for t in cpu]
    kv = osel.k_rows_view(cpu[0], pf)
    L, H, D = len(cpu), kv.shape[2], kv.shape[3]
    T = chunks[-1][1] + chunks[-1][2]
    g = torch.Generator().manual_seed(21)
    k_new = (torch.randn(L, T, H, D, generator=g) * 5).to(row_dtype)
    v_new = (torch.randn(L, T, H, D, generator=g) * 5).to(row_dtype)
    k_new[0, 0, 0, :4] = torch.tensor([1e4, -1e4, 0.0, -0.0])        # saturation and signed zero
    k_new[0, 0, 0, 4:8] = torch.tensor([float("inf"), -float("inf"), 1e-39, 3e38]).to(row_dtype)
    k_new[0, 0, 0, 8:10] = torch.tensor([float("nan"), -float("nan")]).to(row_dtype)   # NaN codes keep the sign
    ks = (0.004 + 0.03 * torch.rand(L, H, generator=g)).float()
    vs = (0.004 + 0.03 * torch.rand(L, H, generator=g)).float()
    # scales outside [2^-60, 2^60] take the kernel's dividing path: rows scaled
    # alike keep bf16 codes in range (fp16 rows saturate or vanish)
    hv = min(1, H - 1)
    ks[1, 0] = 2.0 ** -70
    vs[2, hv] = 2.0 ** 62
    v_new[2, :, hv] = (v_new[2, :, hv].float() * 2.0 ** 62).to(row_dtype)
    kmax = max(c[3] for c in chunks)
    sel = np.full((L, len(chunks), kmax), -1, np.int32)
    rng = np.random.default_rng(5)
    for l in range(L):
        for c, (_bo, _ro, n, k) in enumerate(chunks):
            sel[l, c, :k] = np.sort(rng.choice(n, size=k, replace=False))
    sel[0, 0, 0] = 0
    osel.merge_rows(cpu, pf, bt, k_new, v_new, chunks, sel, k_scales=ks.numpy(), v_scales=vs.numpy())
    cache_ops.merge_rows(gpu, pf, torch.from_numpy(bt).to(dev), k_new.to(dev), v_new.to(dev), chunks,
                         torch.from_numpy(sel).to(dev), k_scales=ks.to(dev), v_scales=vs.to(dev))
    torch.cuda.synchronize()
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)


def test_quantising_merge_argument_errors(dev):
    layers, pf, bt, chunks, _k, _v = setup_case(dev, "nhd", dtype=torch.uint8, L=1)
    gpu = [to_dev(t, dev) for t, _ in layers]
    T = chunks[-1][1] + chunks[-1][2]
    k_new = torch.zeros(1, T, 4, 64, dtype=torch.bfloat16, device=dev)
    sel = torch.zeros(1, len(chunks), 1, dtype=torch.int32, device=dev)
    btd = torch.from_numpy(bt).to(dev)
    sc = torch.ones(1, 4, device=dev)
    with pytest.raises(RuntimeError, match="needs k_scales"):
        cache_ops.merge_rows(gpu, pf, btd, k_new, k_new, chunks, sel)
    with pytest.raises(RuntimeError, match="needs v_scales"):
        cache_ops.merge_rows(gpu, pf, btd, k_new, k_new, chunks, sel, k_scales=sc)
    with pytest.raises(RuntimeError, match="contiguous float32"):
        cache_ops.merge_rows(gpu, pf, btd, k_new, k_new, chunks, sel, k_scales=sc[:, :2], v_scales=sc)
    bf = [torch.zeros(2, 8, 16, 4, 64, dtype=torch.bfloat16, device=dev)]
    with pytest.raises(RuntimeError, match="element type"):
        cache_ops.merge_rows(bf, False, btd, k_new.half(), k_new.half(), chunks, sel)
    with pytest.raises(RuntimeError, match="apply only"):
        cache_ops.merge_rows(bf, False, btd, k_new, k_new, chunks, sel, k_scales=sc, v_scales=sc)


def test_topk_ties_and_edge_k(dev):
    rng = np.random.default_rng(7)
    L, T = 2, 3000
    keys = rng.integers(0, 4, (L, T)).astype(np.float32)    # massive ties
    keys[0, 17] = np.inf
    keys[1, 5] = np.array([0x7FC00000], np.uint32).view(np.float32)[0]
    chunks = [(0, 0, 512, 77), (0, 512, 2048, 205), (0, 2560, 400, 0), (0, 2960, 40, 40),
              (0, 2999, 1, 5)]
    kmax = 205
    want = osel.topk_per_chunk(keys, chunks, kmax)
    got = cache_ops.topk_per_chunk(torch.from_numpy(keys).to(dev), chunks, kmax=kmax)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want)


def test_topk_random_distinct(dev):
    rng = np.random.default_rng(8)
    keys = rng.random((3, 8192)).astype(np.float32)
    chunks = [(0, 0, 8192, 1229), (0, 0, 100, 1)]
    want = osel.topk_per_chunk(keys, chunks, 1229)
    got = cache_ops.topk_per_chunk(torch.from_numpy(keys).to(dev), chunks, kmax=1229)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want)


def test_deviation_llama_shape(dev):
    # H*D = 1024 (two reduction rounds per lane), as benchmark configuration 3
    layers, pf, bt, chunks, k_new, v_new = setup_case(dev, "nhd", nb=80, h=8, d=128, L=2,
                                                      chunk_tokens=(512, 512), seed=3)
    cpu = [t for t, _ in layers]
    keys_o = osel.deviation(cpu, pf, bt, k_new, chunks)
    keys_g = cache_ops.kv_deviation([to_dev(t, dev) for t in cpu], pf, torch.from_numpy(bt).to(dev),
                                    k_new.to(dev), chunks)
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))


@pytest.mark.parametrize("layout", ["nhd", "pf"])
def test_deviation_fp8_with_scales(dev, layout):
    """fp8 (e4m3) cache with per-(layer, head) scales: cached K is dequantised
    as float32(code * scale) before the fixed-order sum (configuration 5's
    selection on an fp8 cache). Keys and indices bit-exact."""
    from oracle import fp8 as ofp8
    g = torch.Generator().manual_seed(11)
    L, nb, ps, h, d = 2, 40, 16, 4, 64
    layers = [make_layer(layout, nb, ps, h, d, torch.uint8, g) for _ in range(L)]
    pf = layers[0][1]
    cpu = [t for t, _ in layers]
    scales = (torch.rand(L, h, generator=g) * 0.05 + 0.01).float()
    perm = np.random.default_rng(11).permutation(np.arange(1, nb)).tolist()
    chunk_tokens = (200, 97)
    bt, chunks, p, row = [], [], 0, 0
    for n in chunk_tokens:
        npg = -(-n // ps)
        chunks.append((len(bt), row, n, max(1, int(round(0.1 * n)))))
        bt.extend(perm[p:p + npg])
        p += npg
        row += n
    bt = np.asarray(bt, np.int32)
    T = row
    rng = np.random.default_rng(12)
    k_new = torch.empty(L, T, h, d, dtype=torch.bfloat16)
    for l in range(L):
        kv = osel.k_rows_view(cpu[l], pf)
        for (bo, ro, n, _k) in chunks:
            blk, s = osel.chunk_slots(bt, bo, n, ps)
            codes = kv[torch.as_tensor(blk), torch.as_tensor(s)].numpy()
            vals = ofp8.decode(codes) * scales[l].numpy()[:, None]
            noise = 0.01 * rng.standard_t(3, size=vals.shape)
            k_new[l, ro:ro + n] = torch.from_numpy((vals + noise).astype(np.float32)).to(torch.bfloat16)
    keys_o = osel.deviation(cpu, pf, bt, k_new, chunks, k_scales=scales.numpy())
    keys_g = cache_ops.kv_deviation([to_dev(t, dev) for t in cpu], pf, torch.from_numpy(bt).to(dev),
                                    k_new.to(dev), chunks, k_scales=scales.to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    kmax = max(c[3] for c in chunks)
    sel_o = osel.topk_per_chunk(keys_o, chunks, kmax)
    sel_g = cache_ops.topk_per_chunk(keys_g, chunks, kmax=kmax)
    torch.cuda.synchronize()
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)


def test_deviation_allocated_keys_on_a_side_stream(dev):
    """kv_deviation allocating its own keys while launching on another stream:
    the zero fill is ordered before the kernel, so the rows outside every
    chunk read 0 and the chunk rows match the oracle."""
    layers, pf, bt, chunks, k_new, v_new = setup_case(dev, "nhd", chunk_tokens=(100, 64, 37))
    cpu = [t for t, _ in layers]
    gpu = [to_dev(t, dev) for t in cpu]
    # leave rows 0..9 and the rows after the last chunk outside every chunk
    T = k_new.shape[1] + 24
    kn = torch.zeros(k_new.shape[0], T, *k_new.shape[2:], dtype=k_new.dtype)
    kn[:, 10:10 + k_new.shape[1]] = k_new
    moved = [(bo, ro + 10, n, k) for (bo, ro, n, k) in chunks]
    side = torch.cuda.Stream()
    btd, knd = torch.from_numpy(bt).to(dev), kn.to(dev)
    torch.cuda.synchronize()
    keys = cache_ops.kv_deviation(gpu, pf, btd, knd, moved, stream=side.cuda_stream)
    side.synchronize()
    want = osel.deviation(cpu, pf, bt, kn, moved)
    assert np.array_equal(keys.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert not keys[:, :10].any() and not keys[:, 10 + k_new.shape[1]:].any()


def test_topk_chunk_longer_than_lds_budget(dev):
    """A 20000-token chunk (past the 8192 tokens whose keys the kernel stages
    in LDS) and a short one in the same call: the long chunk's keys are read
    from global memory in every pass; indices bit-exact, ties to the lower
    index (the keys repeat every 97 tokens)."""
    rng = np.random.default_rng(11)
    n_long, n_short = 20000, 300
    base = rng.standard_normal(97).astype(np.float32) ** 2
    keys = np.concatenate([np.tile(base, n_long // 97 + 1)[:n_long],
                           rng.standard_normal(n_short).astype(np.float32) ** 2])[None, :].repeat(2, 0)
    keys[1] = keys[1][::-1]
    chunks = [(0, 0, n_long, 3001), (0, n_long, n_short, 45)]
    want = osel.topk_per_chunk(keys, chunks, 3001)
    got = cache_ops.topk_per_chunk(torch.from_numpy(keys.copy()).to(dev), chunks, kmax=3001)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want)


def test_selection_over_more_than_65535_chunks(dev):
    """70000 chunks (past the 65535 a grid dimension holds): deviation, top-k
    and merge cut their grids into slices; keys, indices and merged bytes
    bit-exact against the oracle."""
    g = torch.Generator().manual_seed(13)
    n_chunks, ps, h, d = 70000, 1, 2, 64
    nb = n_chunks + 8
    layer = torch.randn(2, nb, ps, h, d, generator=g).to(torch.bfloat16)
    # one-token chunks, each on a page of its own: every merged slot is distinct
    bt = (torch.randperm(nb - 1, generator=g)[:n_chunks] + 1).numpy().astype(np.int32)
    chunks = [(c, c, 1, 1) for c in range(n_chunks)]
    k_new = torch.randn(1, n_chunks, h, d, generator=g).to(torch.bfloat16)
    v_new = torch.randn(1, n_chunks, h, d, generator=g).to(torch.bfloat16)
    gl = [layer.to(dev)]
    btd = torch.from_numpy(bt).to(dev)
    keys = cache_ops.kv_deviation(gl, False, btd, k_new.to(dev), chunks)
    sel = cache_ops.topk_per_chunk(keys, chunks, kmax=1)
    torch.cuda.synchronize()
    keys_o = osel.deviation([layer], False, bt, k_new, chunks)
    assert np.array_equal(keys.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    sel_o = osel.topk_per_chunk(keys_o, chunks, 1)
    assert np.array_equal(sel.cpu().numpy(), sel_o)
    cache_ops.merge_rows(gl, False, btd, k_new.to(dev), v_new.to(dev), chunks, sel)
    torch.cuda.synchronize()
    osel.merge_rows([layer], False, bt, k_new, v_new, chunks, sel_o)
    assert same_bytes(gl[0], layer)


def _oracle_selection(cpu, pf, bt, k_new, v_new, chunks, kmax, ks=None, vs=None):
    keys = osel.deviation(cpu, pf, bt, k_new, chunks, k_scales=ks)
    sel = osel.topk_per_chunk(keys, chunks, kmax)
    osel.merge_rows(cpu, pf, bt, k_new, v_new, chunks, sel, k_scales=ks, v_scales=vs)
    return keys, sel


@pytest.mark.parametrize("layout", ["nhd", "hnd", "pf", "packed", "mla"])
@pytest.mark.parametrize("mode", ["default", "keys_ready", "one_pass"])
def test_select_merge_matches_oracle(dev, layout, mode):
    """The whole selection in one call (the deviation kernel, then one
    workgroup per (layer, chunk) for top-k and merge; keys_ready: keys from an
    earlier kv_deviation; one_pass: those workgroups compute the keys too):
    keys, indices and merged bytes bit-exact against the oracle's three steps.
    Chunks start inside pages (tok_start) and one has k = 0."""
    keys_ready = mode == "keys_ready"
    layers, pf, bt, chunks, k_new, v_new = setup_case(dev, layout, chunk_tokens=(100, 64, 37, 300), seed=4)
    chunks = [c + (0,) for c in chunks]
    chunks[1] = (chunks[1][0], chunks[1][1], 50, chunks[1][3], 14)      # starts at token 14 of its pages
    chunks[2] = chunks[2][:3] + (0, 3)                                    # nothing selected
    cpu = [t for t, _ in layers]
    gpu = [to_dev(t, dev) for t in cpu]
    btd = torch.from_numpy(bt).to(dev)
    kmax = max(c[3] for c in chunks) + 2
    if layout == "mla":
        v_new = None
    keys_o, sel_o = _oracle_selection(cpu, pf, bt, k_new, v_new, chunks, kmax)
    keys = None
    if keys_ready:
        keys = cache_ops.kv_deviation(gpu, pf, btd, k_new.to(dev), chunks)
    keys_g, sel_g = cache_ops.select_merge(gpu, pf, btd, k_new.to(dev), None if v_new is None else v_new.to(dev),
                                           chunks, kmax=kmax, keys=keys, keys_ready=keys_ready,
                                           one_pass=mode == "one_pass")
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)


@pytest.mark.parametrize("layout", ["nhd", "pf"])
def test_select_merge_head_dim_256(dev, layout):
    """256-wide heads (two per token: 1 KiB rows): select_merge against the
    oracle's three steps, bit-exact."""
    layers, pf, bt, chunks, k_new, v_new = setup_case(dev, layout, h=2, d=256, chunk_tokens=(100, 64, 37),
                                                      seed=37)
    cpu = [t for t, _ in layers]
    gpu = [to_dev(t, dev) for t in cpu]
    btd = torch.from_numpy(bt).to(dev)
    kmax = max(c[3] for c in chunks)
    keys_o, sel_o = _oracle_selection(cpu, pf, bt, k_new, v_new, chunks, kmax)
    keys_g, sel_g = cache_ops.select_merge(gpu, pf, btd, k_new.to(dev), v_new.to(dev), chunks, kmax=kmax)
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)


@pytest.mark.parametrize("row_dtype,one_pass", [(torch.bfloat16, False), (torch.float16, False),
                                                (torch.bfloat16, True)])
def test_select_merge_fp8_cache(dev, row_dtype, one_pass):
    """fp8 (e4m3) cache: keys from cached K dequantised with the per-head K
    scales, rows quantised with the same K scales and the V scales."""
    layers, pf, bt, chunks, _k, _v = setup_case(dev, "nhd", dtype=torch.uint8, chunk_tokens=(100, 64, 37), L=2)
    cpu = [t for t, _ in layers]
    gpu = [to_dev(t, dev) for t in cpu]
    L, H, D = 2, 4, 64
    T = chunks[-1][1] + chunks[-1][2]
    g = torch.Generator().manual_seed(23)
    ks = (0.01 + 0.03 * torch.rand(L, H, generator=g)).float()
    vs = (0.01 + 0.03 * torch.rand(L, H, generator=g)).float()
    k_new = torch.randn(L, T, H, D, generator=g).to(row_dtype)
    v_new = torch.randn(L, T, H, D, generator=g).to(row_dtype)
    kmax = max(c[3] for c in chunks)
    keys_o, sel_o = _oracle_selection(cpu, pf, bt, k_new, v_new, chunks, kmax, ks.numpy(), vs.numpy())
    keys_g, sel_g = cache_ops.select_merge(gpu, pf, torch.from_numpy(bt).to(dev), k_new.to(dev), v_new.to(dev),
                                           chunks, k_scales=ks.to(dev), v_scales=vs.to(dev), one_pass=one_pass)
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)


def test_select_merge_long_chunk_takes_three_launches(dev):
    """A 9000-token chunk (past the 8192 keys the fused kernel holds in LDS)
    beside a short one: the call runs deviation, top-k and merge in turn, with
    the same results."""
    layers, pf, bt, chunks, k_new, v_new = setup_case(dev, "nhd", nb=600, h=2, d=64, L=1,
                                                      chunk_tokens=(9000, 120), seed=9)
    cpu = [t for t, _ in layers]
    gpu = [to_dev(t, dev) for t in cpu]
    kmax = max(c[3] for c in chunks)
    keys_o, sel_o = _oracle_selection(cpu, pf, bt, k_new, v_new, chunks, kmax)
    keys_g, sel_g = cache_ops.select_merge(gpu, pf, torch.from_numpy(bt).to(dev), k_new.to(dev), v_new.to(dev),
                                           chunks)
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    assert same_bytes(gpu[0], cpu[0])


@pytest.mark.parametrize("one_pass", [False, True])
def test_select_merge_many_selected_rows(dev, one_pass):
    """Chunks whose selected rows take more merge rounds than a fused
    workgroup handles well (Llama-3-8B rows, k = 154 of 1024): the call runs
    the three kernels, unless one_pass asks for the fused launch; results
    bit-exact either way."""
    layers, pf, bt, chunks, k_new, v_new = setup_case(dev, "nhd", nb=200, h=8, d=128, L=2,
                                                      chunk_tokens=(1024, 700), seed=5)
    cpu = [t for t, _ in layers]
    gpu = [to_dev(t, dev) for t in cpu]
    kmax = max(c[3] for c in chunks)
    keys_o, sel_o = _oracle_selection(cpu, pf, bt, k_new, v_new, chunks, kmax)
    keys_g, sel_g = cache_ops.select_merge(gpu, pf, torch.from_numpy(bt).to(dev), k_new.to(dev), v_new.to(dev),
                                           chunks, one_pass=one_pass)
    torch.cuda.synchronize()
    assert np.array_equal(keys_g.cpu().numpy().view(np.uint32), keys_o.view(np.uint32))
    assert np.array_equal(sel_g.cpu().numpy(), sel_o)
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)
