"""Descriptor ring at its limits: calls whose job descriptors exceed a slot's
initial 1 MiB (the slot grows) on both hand-over paths -- the upload kernel
(gather/scatter_pages) and direct reads of the pinned slot (the fused path) --
and back-to-back calls that reuse grown slots with different contents, all
checked against the CPU oracle."""
import numpy as np
import pytest
import torch

from daric_amd import cache_ops
from oracle import native
from oracle import rope as orope
from oracle.copy import OracleCopier
from tests.gpu_util import assert_rotation_parity, rotation_region, same_bytes

pytestmark = pytest.mark.gpu

N_LAYERS, NB, PS, H, D = 400, 64, 4, 1, 16     # 20,000 one-page jobs: 1.6 MB of descriptors
PAGES_PER_LAYER = 50


def _setup(dev, seed):
    g = torch.Generator().manual_seed(seed)
    layers = [torch.randn(2, NB, PS, H, D, generator=g).to(torch.bfloat16) for _ in range(N_LAYERS)]
    names = [f"layer.{i}" for i in range(N_LAYERS)]
    rng = np.random.default_rng(seed)
    jobs = []
    for li in range(N_LAYERS):
        for p in rng.permutation(np.arange(1, NB))[:PAGES_PER_LAYER]:
            jobs.append((li, int(p)))
    rng.shuffle(jobs)
    span = PS * H * D * 2
    offsets = [i * 2 * span for i in range(len(jobs))]
    sizes = [2 * span] * len(jobs)
    flat = [p for _, p in jobs]
    ioff = list(range(len(jobs) + 1))
    jn = [names[li] for li, _ in jobs]
    return g, layers, names, jobs, jn, offsets, sizes, flat, ioff


def _oracle(threads=8):
    return native.NativeOracleCopier(threads) if native.available() else OracleCopier()


def test_gather_with_grown_upload_slot(dev):
    for seed in (0, 1):     # the second call reuses the grown slots with new contents
        g, layers, names, jobs, jn, offsets, sizes, flat, ioff = _setup(dev, seed)
        oc, gc = _oracle(), cache_ops.CacheCopier()
        for n, t in zip(names, layers):
            oc.register_layer(n, t, False)
            gc.register_layer(n, t.to(dev), False)
        total = offsets[-1] + sizes[-1]
        oc.register_store(torch.zeros(total, dtype=torch.uint8))
        gstore = torch.zeros(total, dtype=torch.uint8, device=dev)
        gc.register_store(gstore)
        idx = torch.tensor(flat, dtype=torch.int32)
        oc.gather_pages(jn, offsets, sizes, idx, ioff)
        gc.gather_pages(jn, offsets, sizes, idx.to(dev), ioff)
        torch.cuda.synchronize()
        assert torch.equal(gstore.cpu(), oc.store), f"seed {seed}"


def test_fused_with_grown_direct_slot(dev):
    R = D
    inv = orope.default_inv_freq(R, 500000.0)
    for seed in (2, 3):
        g, layers, names, jobs, jn, offsets, sizes, flat, ioff = _setup(dev, seed)
        deltas = [(7 * i) % 5000 - 1000 for i in range(len(jobs))]
        ntok = [PS] * len(jobs)
        oc, gc = _oracle(), cache_ops.CacheCopier()
        dev_layers = []
        for n, t in zip(names, layers):
            oc.register_layer(n, t, False)
            td = t.to(dev)
            dev_layers.append(td)
            gc.register_layer(n, td, False)
        total = offsets[-1] + sizes[-1]
        store = torch.randn(total // 2, generator=g).to(torch.bfloat16).view(torch.uint8)
        oc.register_store(store.clone())
        gc.register_store(store.to(dev))
        idx = torch.tensor(flat, dtype=torch.int32)
        oc.scatter_pages_rerotate(jn, offsets, sizes, idx, ioff, deltas, ntok, inv, R, True)
        gc.scatter_pages_rerotate(jn, offsets, sizes, idx.to(dev), ioff, deltas, ntok,
                                  torch.from_numpy(inv).to(dev), R, True)
        torch.cuda.synchronize()
        slots = {li: [] for li in range(N_LAYERS)}
        for (li, p), dl in zip(jobs, deltas):
            if dl != 0:
                slots[li] += [p * PS + j for j in range(PS)]
        for li in range(0, N_LAYERS, 7):          # a spread subset of the 400 layers
            mask, pn = rotation_region(layers[li], False, R, slots[li], True)
            assert_rotation_parity(dev_layers[li], layers[li], mask, pn)
        # every layer's V half is a plain copy: bit-exact
        for li in range(N_LAYERS):
            assert same_bytes(dev_layers[li][1], layers[li][1]), f"seed {seed} layer {li}"


def test_back_to_back_calls_reuse_slots_safely(dev):
    # 40 fused calls with no synchronisation between them, each with 48 jobs
    # (3840 bytes of descriptors: a ring slot, read directly by the kernels).
    # The 16 slots are reused 2.5 times; every call writes its own pages with
    # its own shifts, so a slot rewritten before its kernel finished would
    # show up as a wrong rotation. Each slot's reuse waits for the event its
    # call's kernel carries.
    n_calls, n_jobs, nb, ps, h, d = 40, 48, 2048, 4, 1, 16
    R = d
    inv = orope.default_inv_freq(R, 10000.0)
    g = torch.Generator().manual_seed(11)
    layer = torch.randn(2, nb, ps, h, d, generator=g).to(torch.bfloat16)
    span = ps * h * d * 2
    pages = np.random.default_rng(11).permutation(np.arange(1, nb))[: n_calls * n_jobs].tolist()
    store = torch.randn(n_calls * n_jobs * span, generator=g).to(torch.bfloat16).view(torch.uint8)
    oc, gc = _oracle(), cache_ops.CacheCopier()
    oc.register_layer("l", layer, False)
    dl = layer.to(dev)
    gc.register_layer("l", dl, False)
    oc.register_store(store.clone())
    gc.register_store(store.to(dev))
    invd = torch.from_numpy(inv).to(dev)
    calls = []
    for c in range(n_calls):
        jp = pages[c * n_jobs:(c + 1) * n_jobs]
        offs = [(c * n_jobs + j) * 2 * span for j in range(n_jobs)]
        deltas = [1 + 97 * c + j for j in range(n_jobs)]
        calls.append((["l"] * n_jobs, offs, [2 * span] * n_jobs, torch.tensor(jp, dtype=torch.int32),
                      list(range(n_jobs + 1)), deltas, [ps] * n_jobs))
    idx_dev = [ci[3].to(dev) for ci in calls]
    torch.cuda.synchronize()
    # a bounded spin ahead of the calls keeps their kernels queued, so the
    # 17th call must wait for the first call's kernel to release slot 0
    torch.cuda._sleep(50_000_000)
    for ci, idd in zip(calls, idx_dev):
        gc.scatter_pages_rerotate(ci[0], ci[1], ci[2], idd, ci[4], ci[5], ci[6], invd, R, True)
    for ci in calls:
        oc.scatter_pages_rerotate(ci[0], ci[1], ci[2], ci[3], ci[4], ci[5], ci[6], inv, R, True)
    torch.cuda.synchronize()
    slots = [p * ps + j for p in pages for j in range(ps)]
    mask, pn = rotation_region(layer, False, R, slots, True)
    assert_rotation_parity(dl, layer, mask, pn)
    assert same_bytes(dl[1], layer[1])
