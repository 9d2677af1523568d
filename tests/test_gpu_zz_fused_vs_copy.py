"""Performance guard: the fused scatter + re-rotation kernel against a plain
scatter of the same jobs, timed alternately in one process (kernel durations
from the dispatch packets' own events). The rotation should cost little over
the copy of the same access pattern: on MI355X the fused kernel runs at
98-99.6% of the plain scatter's rate; the guard fails below 80%, which would
mean a lost occupancy or access-pattern regression, not box-to-box noise.
Named to run after the parity tests."""
import numpy as np
import pytest
import torch

from daric_amd import cache_ops

pytestmark = pytest.mark.gpu


def _kernel_ms(fn, n=6):
    cache_ops.timing_enable(True)
    cache_ops.timing_read()
    for _ in range(n):
        fn()
    torch.cuda.synchronize()
    ms, launches = cache_ops.timing_read()
    cache_ops.timing_enable(False)
    return ms / max(launches, 1)


def test_fused_kernel_keeps_pace_with_plain_scatter(dev):
    L, NB, PS, H, D, C, CT = 8, 8192, 16, 8, 128, 8, 1024     # 512 MiB moved per call
    g = torch.Generator().manual_seed(0)
    ids = (torch.randperm(NB - 1, generator=g)[: C * CT // PS] + 1).to(torch.int32)
    cache = [torch.empty(2, NB, PS, H, D, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    span = PS * H * D * 2
    job = 2 * (CT // PS) * span
    staging = torch.randn(C * L * job // 2, device=dev).to(torch.bfloat16).view(torch.uint8)
    cp = cache_ops.CacheCopier()
    names = [f"layer.{i}" for i in range(L)]
    for n, t in zip(names, cache):
        cp.register_layer(n, t, False)
    cp.register_store(staging)
    jn, offs, sizes, flat, ioff, deltas, ntok = [], [], [], [], [0], [], []
    for c in range(C):
        bids = ids[c * (CT // PS):(c + 1) * (CT // PS)].tolist()
        for n in names:
            jn.append(n); offs.append(len(offs) * job); sizes.append(job); flat.extend(bids)
            ioff.append(len(flat)); deltas.append(c * CT); ntok.append(CT)
    idx = torch.tensor(flat, dtype=torch.int32, device=dev)
    inv = (1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))).to(dev)

    def fused():
        cp.scatter_pages_rerotate(jn, offs, sizes, idx, ioff, deltas, ntok, inv, D, True)

    def plain():
        cp.scatter_pages(jn, offs, sizes, idx, ioff)

    fused(); plain()
    torch.cuda.synchronize()
    tf, tp = [], []
    for r in range(4):
        order = (fused, plain) if r % 2 == 0 else (plain, fused)
        for fn in order:
            (tf if fn is fused else tp).append(_kernel_ms(fn))
    ratio = float(np.median(tp)) / float(np.median(tf))
    print(f"fused {np.median(tf) * 1e3:.1f} us, plain scatter {np.median(tp) * 1e3:.1f} us, ratio {ratio:.3f}")
    assert ratio > 0.8, f"fused kernel at {ratio:.1%} of the plain scatter of the same jobs"
