"""Pins the CPU oracle's deviation keys, top-k and merge.

Independent facts: the fixed-order float32 sum agrees with a float64 sum to
float32 accuracy and with a scalar float32 walk in the documented order on tiny
rows (brute force); top-k agrees with Python's stable sorted() on (-key, index);
merge lands rows where torch indexing says.
"""
import numpy as np
import torch

from oracle import select


def scalar_walk(a, b):
    """Brute force in np.float32 scalars, following the documented order."""
    n = len(a)
    acc = [np.float32(0)] * 64
    v = 0
    while v * 8 < n:
        lane = v % 64
        for i in range(8):
            e = v * 8 + i
            if e < n:
                d = np.float32(np.float32(a[e]) - np.float32(b[e]))
                acc[lane] = np.float32(acc[lane] + np.float32(d * d))
        v += 1
    for off in (32, 16, 8, 4, 2, 1):
        acc = [np.float32(acc[l] + acc[l ^ off]) for l in range(64)]
    return acc[0]


def test_sumsq_matches_float64_and_scalar_walk():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((6, 1024)).astype(np.float32)
    b = (a + 0.1 * rng.standard_t(3, size=a.shape)).astype(np.float32)
    k = select.fixed_order_sumsq(a, b)
    ref = ((a.astype(np.float64) - b.astype(np.float64)) ** 2).sum(1)
    assert np.all(np.abs(k - ref) <= 1e-5 * ref)
    for n in (8, 40, 130, 600):
        x = rng.standard_normal((1, n)).astype(np.float32) * np.float32(1e3) ** rng.integers(-2, 3, n)
        y = rng.standard_normal((1, n)).astype(np.float32)
        assert select.fixed_order_sumsq(x.astype(np.float32), y)[0] == scalar_walk(x[0], y[0])


def test_sumsq_exact_counts_and_nan():
    a = np.ones((2, 1024), np.float32)
    b = np.zeros((2, 1024), np.float32)
    b[1, 5] = np.inf
    a[1, 5] = np.inf
    k = select.fixed_order_sumsq(a, b)
    assert k[0] == 1024.0
    assert k.view(np.uint32)[1] == 0x7FC00000


def test_topk_matches_stable_sort():
    rng = np.random.default_rng(1)
    for n, k in ((512, 77), (2048, 205), (37, 5), (10, 10), (5, 9)):
        keys = rng.integers(0, 6, n).astype(np.float32)  # heavy ties
        keys[rng.integers(0, n)] = np.inf
        want = sorted(sorted(range(n), key=lambda i: (-keys[i], i))[:k])
        assert select.topk_chunk(keys, k).tolist() == want
    keys = np.array([1.0, 3.0, 3.0, 2.0, 3.0], np.float32)
    assert select.topk_chunk(keys, 2).tolist() == [1, 2]
    nan = np.array([0x7FC00000], np.uint32).view(np.float32)[0]
    keys = np.array([np.inf, nan, 5.0], np.float32)
    assert select.topk_chunk(keys, 1).tolist() == [1]


def test_merge_rows_land_in_slots():
    nb, ps, h, d = 6, 4, 2, 8
    layer = torch.zeros(2, nb, ps, h, d, dtype=torch.bfloat16)
    k_new = torch.randn(1, 10, h, d).to(torch.bfloat16)
    v_new = torch.randn(1, 10, h, d).to(torch.bfloat16)
    bt = np.array([3, 0, 5], np.int32)
    chunks = [(0, 0, 10, 3)]
    sel = np.array([[[1, 4, 9]]], np.int32)
    select.merge_rows([layer], False, bt, k_new, v_new, chunks, sel)
    assert torch.equal(layer[0, 3, 1], k_new[0, 1]) and torch.equal(layer[1, 3, 1], v_new[0, 1])
    assert torch.equal(layer[0, 5, 1], k_new[0, 9]) and torch.equal(layer[1, 5, 1], v_new[0, 9])
    assert layer[:, 0].abs().sum() == 0  # token 4 maps to block 0: skipped
    assert int((layer != 0).sum()) == 4 * h * d - int((k_new[0, [1, 9]] == 0).sum() + (v_new[0, [1, 9]] == 0).sum())


def test_deviation_uses_slots():
    g = torch.Generator().manual_seed(2)
    nb, ps, h, d = 5, 4, 2, 8
    layer = torch.randn(2, nb, ps, h, d, generator=g).to(torch.bfloat16)
    bt = np.array([4, 1], np.int32)
    k_new = torch.randn(1, 8, h, d, generator=g).to(torch.bfloat16)
    keys = select.deviation([layer], False, bt, k_new, [(0, 0, 8, 2)])
    for j in range(8):
        cached = layer[0, bt[j // ps], j % ps].double()
        ref = ((k_new[0, j].double() - cached) ** 2).sum().item()
        assert abs(keys[0, j] - ref) <= 1e-5 * ref


def test_deviation_out_of_range_block_gives_zero_key():
    # block ids outside [0, num_blocks) are not read and give key 0 (negative
    # ids must not wrap around as Python indexing would); block 0 is read
    g = torch.Generator().manual_seed(3)
    nb, ps, h, d = 5, 4, 2, 8
    layer = torch.randn(2, nb, ps, h, d, generator=g).to(torch.bfloat16)
    bt = np.array([-1, 0, nb, 3], np.int32)
    k_new = torch.randn(1, 16, h, d, generator=g).to(torch.bfloat16)
    keys = select.deviation([layer], False, bt, k_new, [(0, 0, 16, 2)])
    for j in range(16):
        blk = int(bt[j // ps])
        if blk < 0 or blk >= nb:
            assert keys[0, j] == 0.0
        else:
            ref = ((k_new[0, j].double() - layer[0, blk, j % ps].double()) ** 2).sum().item()
            assert abs(keys[0, j] - ref) <= 1e-5 * ref


def test_deviation_fp8_dequantises_with_per_head_scale():
    """fp8 cache: cached K is code value x scale[layer, head] (float64 check,
    independent of the fixed order); no scales means scale 1."""
    from oracle import fp8
    rng = np.random.default_rng(4)
    nb, ps, h, d = 6, 4, 3, 16
    codes = fp8.encode(rng.standard_normal(2 * nb * ps * h * d).astype(np.float32))
    layer = torch.from_numpy(codes).view(2, nb, ps, h, d)
    bt = np.array([5, 2], np.int32)
    k_new = torch.randn(1, 8, h, d).to(torch.bfloat16)
    scales = np.array([[0.5, 0.031, 2.0]], np.float32)
    keys = select.deviation([layer], False, bt, k_new, [(0, 0, 8, 2)], k_scales=scales)
    keys1 = select.deviation([layer], False, bt, k_new, [(0, 0, 8, 2)])
    for j in range(8):
        q = fp8.decode(layer[0, bt[j // ps], j % ps].numpy()).astype(np.float64)
        kn = k_new[0, j].double().numpy()
        ref = ((kn - q * scales[0][:, None].astype(np.float64)) ** 2).sum()
        ref1 = ((kn - q) ** 2).sum()
        assert abs(keys[0, j] - ref) <= 1e-5 * ref
        assert abs(keys1[0, j] - ref1) <= 1e-5 * ref1


def test_quantising_merge_is_pinned():
    """bf16/fp16 rows merged into an fp8 cache: codes of x / scale[l, h].
    Pinned by (1) scale 1 reducing to the e4m3 encoder, (2) power-of-two scales
    scaling exactly, (3) an independent path -- float64 division rounded once
    to float32 (which, for division, equals the correctly rounded float32
    quotient) and torch's float8 cast after clamping -- with scales that differ
    per head and between K and V, so a wrong head or K/V scale fails."""
    from oracle import fp8
    g = torch.Generator().manual_seed(9)
    nb, ps, h, d, L, T = 7, 4, 3, 16, 2, 12
    for dtype in (torch.bfloat16, torch.float16):
        k_new = (torch.randn(L, T, h, d, generator=g) * 3).to(dtype)
        v_new = (torch.randn(L, T, h, d, generator=g) * 3).to(dtype)
        bt = np.array([3, 6, 1], np.int32)
        chunks = [(0, 0, T, 5)]
        sel = np.array([[[0, 2, 5, 9, 11]], [[1, 4, 6, 8, 10]]], np.int32)
        for case in ("one", "pow2", "general"):
            if case == "one":
                ks = np.ones((L, h), np.float32)
                vs = np.ones((L, h), np.float32)
            elif case == "pow2":
                ks = np.exp2(np.array([[-3, 0, 2], [1, -5, 4]], np.float32))
                vs = np.exp2(np.array([[2, -1, 0], [-2, 3, -4]], np.float32))
            else:
                ks = np.array([[0.011, 0.0093, 0.0071], [0.013, 0.0088, 0.0102]], np.float32)
                vs = np.array([[0.007, 0.0121, 0.0099], [0.0081, 0.0066, 0.0143]], np.float32)
            layer = [torch.zeros(2, nb, ps, h, d, dtype=torch.uint8) for _ in range(L)]
            select.merge_rows(layer, False, bt, k_new, v_new, chunks, sel, k_scales=ks, v_scales=vs)
            for l in range(L):
                for j in sel[l, 0]:
                    blk, s = int(bt[j // ps]), int(j % ps)
                    for kvi, (rows, sc) in enumerate(((k_new, ks), (v_new, vs))):
                        got = layer[l][kvi, blk, s].numpy()
                        x = rows[l, j].to(torch.float64)
                        if case == "one":
                            want = fp8.encode(rows[l, j].to(torch.float32).numpy())
                        elif case == "pow2":
                            want = fp8.encode((x * torch.from_numpy(1.0 / sc[l]).double()[:, None]).numpy())
                        else:
                            q = (x / torch.from_numpy(sc[l]).double()[:, None]).to(torch.float32)
                            want = q.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
                        assert np.array_equal(got, want), (dtype, case, l, int(j), kvi)
            # unselected slots stay zero
            touched = {(int(bt[j // ps]), int(j % ps)) for l in range(L) for j in sel[l, 0]}
            for b in range(nb):
                for s in range(ps):
                    if (b, s) not in touched:
                        assert all(int(t[:, b, s].abs().sum()) == 0 for t in layer)


def test_chunk_slots_with_a_start_inside_a_page():
    """Token j of a chunk starting at token ts of its block list lives in page
    bt[bo + (ts + j) // PS] at place (ts + j) % PS: against a token-by-token
    walk over the pages."""
    bt = np.array([7, 3, 9, 4, 11, 2], np.int32)
    for ps in (1, 4, 16):
        for bo, ts, n in ((0, 0, 5), (1, 3, 9), (2, ps - 1, 2 * ps), (0, 2 * ps + 1, ps)):
            if bo + (ts + n - 1) // ps >= bt.size:
                continue
            walk = []
            page, place = bo, 0
            for _ in range(ts):                 # skip ts tokens
                place += 1
                if place == ps:
                    page, place = page + 1, 0
            for _ in range(n):
                walk.append((int(bt[page]), place))
                place += 1
                if place == ps:
                    page, place = page + 1, 0
            blk, s = select.chunk_slots(bt, bo, n, ps, ts)
            assert list(zip(blk.tolist(), s.tolist())) == walk


def test_four_and_five_field_chunks_agree():
    """A chunk given without tok_start is the chunk with tok_start 0."""
    g = torch.Generator().manual_seed(3)
    layer = torch.randn(2, 12, 16, 2, 16, generator=g).to(torch.bfloat16)
    bt = np.array([5, 2, 9, 1], np.int32)
    k_new = torch.randn(1, 40, 2, 16, generator=g).to(torch.bfloat16)
    k4 = select.deviation([layer], False, bt, k_new, [(0, 0, 20, 3), (2, 20, 20, 4)])
    k5 = select.deviation([layer], False, bt, k_new, [(0, 0, 20, 3, 0), (2, 20, 20, 4, 0)])
    assert np.array_equal(k4.view(np.uint32), k5.view(np.uint32))
    shifted = select.deviation([layer], False, bt, k_new, [(0, 0, 20, 3, 16)])   # starts on page 1
    same = select.deviation([layer], False, bt, k_new, [(1, 0, 20, 3, 0)])
    assert np.array_equal(shifted.view(np.uint32), same.view(np.uint32))
