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
