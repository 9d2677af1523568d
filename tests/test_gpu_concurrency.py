"""Concurrent use from several host threads, as the daric-store does (one
read and one write copier per rank, separate streams, 16 RPC worker threads;
reference gpu_kv_io.py:138-141, main.py:24): calls on different copiers and
streams interleave through the shared per-device descriptor ring and still
produce the oracle's bytes."""
import threading

import numpy as np
import pytest
import torch

from daric_amd import cache_ops
from oracle.copy import OracleCopier
from tests.gpu_util import make_layer, same_bytes, to_dev

pytestmark = pytest.mark.gpu


def test_threads_streams_and_copiers(dev):
    g = torch.Generator().manual_seed(5)
    L, nb = 4, 96
    src_layers = [make_layer("nhd", nb, 16, 4, 64, torch.bfloat16, g)[0] for _ in range(L)]
    names = [f"l{i}" for i in range(L)]
    from oracle.layout import page_copy_shape
    s = page_copy_shape(tuple(src_layers[0].shape), tuple(src_layers[0].stride()), 2, False)
    per_page = s.prefix_size * s.suffix_size
    n_threads, rounds = 6, 20
    results = {}
    errors = []

    def worker(tid):
        try:
            stream = torch.cuda.Stream(device=dev)
            pages = np.random.default_rng(100 + tid).choice(np.arange(1, nb), 8, replace=False).tolist()
            cache = [to_dev(t, dev) for t in src_layers]
            stage = torch.zeros(L * 8 * per_page, dtype=torch.uint8, device=dev)
            cp = cache_ops.CacheCopier()
            for n, t in zip(names, cache):
                cp.register_layer(n, t, False)
            cp.register_store(stage)
            idx = torch.tensor(pages * L, dtype=torch.int32, device=dev)
            offs = [i * 8 * per_page for i in range(L)]
            ioff = [i * 8 for i in range(L + 1)]
            for _ in range(rounds):
                cp.gather_pages(names, offs, [8 * per_page] * L, idx, ioff, stream.cuda_stream)
                # scatter the gathered pages back one page-slot later (a permutation)
                cp.scatter_pages(names, offs, [8 * per_page] * L,
                                 torch.tensor((pages[1:] + pages[:1]) * L, dtype=torch.int32, device=dev),
                                 ioff, stream.cuda_stream)
            stream.synchronize()
            results[tid] = (pages, [t.cpu() for t in cache], stage.cpu())
        except Exception as e:  # surfaced below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(n_threads)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    # replay each thread's sequence on the oracle
    for tid, (pages, got_cache, got_stage) in results.items():
        oc = OracleCopier()
        cache = [t.clone() for t in src_layers]
        for n, t in zip(names, cache):
            oc.register_layer(n, t, False)
        stage = torch.zeros(L * 8 * per_page, dtype=torch.uint8)
        oc.register_store(stage)
        offs = [i * 8 * per_page for i in range(L)]
        ioff = [i * 8 for i in range(L + 1)]
        for _ in range(rounds):
            oc.gather_pages(names, offs, [8 * per_page] * L, torch.tensor(pages * L, dtype=torch.int32), ioff)
            oc.scatter_pages(names, offs, [8 * per_page] * L,
                             torch.tensor((pages[1:] + pages[:1]) * L, dtype=torch.int32), ioff)
        assert torch.equal(got_stage, stage), f"thread {tid} staging differs"
        for a, b in zip(got_cache, cache):
            assert same_bytes(a, b), f"thread {tid} cache differs"
