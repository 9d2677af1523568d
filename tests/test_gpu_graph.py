"""HIP graph capture of the entry points. A call whose descriptors fit in the
kernel arguments (at most 2816 bytes: e.g. one layer's re-rotation, or a
gather of up to 35 jobs) launches only its kernel, with the descriptors by
value, so it can be captured and replayed; a larger call is refused while
capturing. Every replay is checked against the same call run eagerly, with
eager work and synchronisation between the replays."""
import numpy as np
import pytest
import torch

from daric_amd import cache_ops
from oracle import rope as orope

pytestmark = pytest.mark.gpu


def _layers(dev, n, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(2, 64, 16, 8, 128, generator=g).to(torch.bfloat16).to(dev) for _ in range(n)]


def test_layerwise_rerotate_replays_match_eager(dev):
    layers = _layers(dev, 4, 0)
    ref = [t.clone() for t in layers]
    bt = torch.tensor([5, 9, 2, 40], dtype=torch.int32, device=dev)
    # PS = 16: tokens 3..31 lie in blocks 5 and 9, tokens 0..19 from offset 2 in
    # blocks 2 and 40; segments of one call must name distinct slots
    segs = [(0, 3, 29, 300), (2, 0, 20, -77)]
    inv = torch.from_numpy(orope.default_inv_freq(128, 500000.0)).to(dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):      # warm-up outside the capture, as torch asks
        for t in ref:
            cache_ops.rerotate_pages([t], False, bt, segs, inv, 128, True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for t, r in zip(layers, ref):   # bring both copies to the same state
        t.copy_(r)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for t in layers:            # the Adapter's layerwise mode: one call per layer
            cache_ops.rerotate_pages([t], False, bt, segs, inv, 128, True)
    torch.cuda.synchronize()
    for t, r in zip(layers, ref):   # capturing ran nothing
        assert torch.equal(t.view(torch.int16), r.view(torch.int16))
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for r in ref:
            cache_ops.rerotate_pages([r], False, bt, segs, inv, 128, True)
        torch.cuda.synchronize()
        for li, (t, r) in enumerate(zip(layers, ref)):
            assert torch.equal(t.view(torch.int16), r.view(torch.int16)), f"replay {rep} layer {li}"
        _ = float(torch.randn(4096, device=dev).abs().sum())   # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")   # the refused capture
def test_gather_replays_match_eager_and_large_calls_refuse_capture(dev):
    layers = _layers(dev, 3, 1)
    cp = cache_ops.CacheCopier()
    names = [f"l{i}" for i in range(3)]
    for n, t in zip(names, layers):
        cp.register_layer(n, t, False)
    span = 16 * 8 * 128 * 2
    per = 2 * 4 * span
    store = torch.zeros(3 * per, dtype=torch.uint8, device=dev)
    cp.register_store(store)
    idx = torch.tensor([3, 7, 0, 60] * 3, dtype=torch.int32, device=dev)
    args = (names, [0, per, 2 * per], [per] * 3, idx, [0, 4, 8, 12])
    cp.gather_pages(*args)
    torch.cuda.synchronize()
    want = store.clone()
    store.zero_()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cp.gather_pages(*args)
    torch.cuda.synchronize()
    assert int(store.count_nonzero()) == 0
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(store, want), f"replay {rep}"
        store.zero_()
        _ = float(torch.randn(4096, device=dev).abs().sum())
        torch.cuda.synchronize()
    # 40 jobs = 3200 bytes of descriptors: too large to travel by value
    many = [names[i % 3] for i in range(40)]
    idx40 = torch.tensor([1 + i // 3 for i in range(40)], dtype=torch.int32, device=dev)
    big = torch.zeros(40 * 2 * span, dtype=torch.uint8, device=dev)
    cp.register_store(big)
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="cannot be captured in a graph"):
        with torch.cuda.graph(g2):
            cp.gather_pages(many, [i * 2 * span for i in range(40)], [2 * span] * 40, idx40,
                            list(range(41)))
    torch.cuda.synchronize()
    # the same call runs eagerly
    cp.gather_pages(many, [i * 2 * span for i in range(40)], [2 * span] * 40, idx40, list(range(41)))
    torch.cuda.synchronize()
    got = big.view(40, 2, span)
    for i in range(40):
        src = layers[i % 3][:, 1 + i // 3].contiguous().view(torch.uint8).reshape(2, span)
        assert torch.equal(got[i], src), i


def test_fused_and_selection_replays_match_eager(dev):
    # a two-job fused scatter + re-rotation, then deviation -> top-k -> merge
    # over two chunks: every call small enough to carry its descriptors by value
    g = torch.Generator().manual_seed(2)
    L, NB, PS, H, D = 2, 32, 16, 8, 128
    base = [torch.randn(2, NB, PS, H, D, generator=g).to(torch.bfloat16) for _ in range(L)]
    span = PS * H * D * 2
    per = 2 * 3 * span
    store_cpu = torch.randn(L * per // 2, generator=g).to(torch.bfloat16).view(torch.uint8)
    T = 64
    k_new = torch.randn(L, T, H, D, generator=g).to(torch.bfloat16).to(dev)
    v_new = torch.randn(L, T, H, D, generator=g).to(torch.bfloat16).to(dev)
    bt = torch.tensor([4, 9, 2, 17], dtype=torch.int32, device=dev)
    chunks = [(0, 0, 32, 5), (2, 32, 32, 7)]
    inv = torch.from_numpy(orope.default_inv_freq(D, 500000.0)).to(dev)
    idx = torch.tensor([3, 11, 20, 5, 6, 30], dtype=torch.int32, device=dev)
    names = ["a", "b"]

    def make():
        layers = [t.to(dev) for t in base]
        cp = cache_ops.CacheCopier()
        for n, t in zip(names, layers):
            cp.register_layer(n, t, False)
        store = store_cpu.to(dev)
        cp.register_store(store)
        keys = torch.zeros(L, T, dtype=torch.float32, device=dev)
        sel = torch.zeros(L, 2, 7, dtype=torch.int32, device=dev)
        return dict(layers=layers, cp=cp, store=store, keys=keys, sel=sel)

    def run(s):
        s["cp"].scatter_pages_rerotate(names, [0, per], [per, per], idx, [0, 3, 6], [100, -37], [48, 40],
                                       inv, D, True)
        cache_ops.kv_deviation(s["layers"], False, bt, k_new, chunks, keys=s["keys"])
        cache_ops.topk_per_chunk(s["keys"], chunks, kmax=7, out=s["sel"])
        cache_ops.merge_rows(s["layers"], False, bt, k_new, v_new, chunks, s["sel"])

    eager, cap = make(), make()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):       # warm-up outside the capture
        run(make())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(cap)
    torch.cuda.synchronize()
    for t, b in zip(cap["layers"], base):      # capturing ran nothing
        assert torch.equal(t.cpu().view(torch.int16), b.view(torch.int16))
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        run(eager)
        torch.cuda.synchronize()
        for li in range(L):
            assert torch.equal(cap["layers"][li].view(torch.int16), eager["layers"][li].view(torch.int16)), \
                f"replay {rep} layer {li}"
        assert torch.equal(cap["keys"], eager["keys"]), f"replay {rep} keys"
        assert torch.equal(cap["sel"], eager["sel"]), f"replay {rep} sel"
        _ = float(torch.randn(4096, device=dev).abs().sum())
        torch.cuda.synchronize()


def test_select_merge_replays_match_eager(dev):
    """select_merge (the deviation kernel, then the fused top-k and merge) of
    three chunks, one starting inside a page, captured in a graph: every
    replay equals the same call run eagerly."""
    g = torch.Generator().manual_seed(5)
    L, NB, PS, H, D = 2, 32, 16, 8, 128
    base = [torch.randn(2, NB, PS, H, D, generator=g).to(torch.bfloat16) for _ in range(L)]
    T = 96
    k_new = torch.randn(L, T, H, D, generator=g).to(torch.bfloat16).to(dev)
    v_new = torch.randn(L, T, H, D, generator=g).to(torch.bfloat16).to(dev)
    bt = torch.tensor([4, 9, 2, 17, 23, 6], dtype=torch.int32, device=dev)
    chunks = [(0, 0, 32, 5, 0), (2, 32, 30, 7, 2), (4, 62, 32, 0, 0)]

    def make():
        return dict(layers=[t.to(dev) for t in base],
                    keys=torch.zeros(L, T, dtype=torch.float32, device=dev),
                    sel=torch.zeros(L, 3, 7, dtype=torch.int32, device=dev))

    def run(s):
        cache_ops.select_merge(s["layers"], False, bt, k_new, v_new, chunks, kmax=7, keys=s["keys"],
                               sel_idx=s["sel"])

    eager, cap = make(), make()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):       # warm-up outside the capture
        run(make())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(cap)
    torch.cuda.synchronize()
    for t, b in zip(cap["layers"], base):      # capturing ran nothing
        assert torch.equal(t.cpu().view(torch.int16), b.view(torch.int16))
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        run(eager)
        torch.cuda.synchronize()
        for li in range(L):
            assert torch.equal(cap["layers"][li].view(torch.int16), eager["layers"][li].view(torch.int16)), \
                f"replay {rep} layer {li}"
        assert torch.equal(cap["keys"].view(torch.int32), eager["keys"].view(torch.int32)), f"replay {rep} keys"
        assert torch.equal(cap["sel"], eager["sel"]), f"replay {rep} sel"
        _ = float(torch.randn(4096, device=dev).abs().sum())
        torch.cuda.synchronize()
