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


def test_sixteen_threads_share_the_descriptor_ring(dev):
    """16 threads, as the store's RPC workers, each with its own copiers and
    stream, issue calls of 48 jobs: too many descriptors for the kernel
    arguments, so every call takes one of the ring's 16 slots. Each thread runs
    a fused scatter + re-rotation of its own pages and a gather of them back,
    8 rounds, gathering round r into its own region; every region must equal
    what the same two calls gave when run alone beforehand."""
    L, NB, PS, H, D = 4, 1024, 16, 4, 64
    n_threads, rounds, chunks, ppc = 16, 8, 12, 4
    span = PS * H * D * 2
    job = 2 * ppc * span
    n_jobs = chunks * L
    g = torch.Generator(device=dev).manual_seed(3)
    layers = [torch.randn(2, NB, PS, H, D, generator=g, device=dev).to(torch.bfloat16) for _ in range(L)]
    names = [f"layer.{l}" for l in range(L)]
    inv = (1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))).to(dev)

    def setup(t):
        pages = [1 + t * chunks * ppc + i for i in range(chunks * ppc)]
        flat, ioff, deltas, ntok = [], [0], [], []
        for c in range(chunks):
            for _ in range(L):
                flat.extend(pages[c * ppc:(c + 1) * ppc])
                ioff.append(len(flat))
                deltas.append(c * ppc * PS + 1 + t)
                ntok.append(ppc * PS - t % 3)
        staging = torch.randn(n_jobs * job // 2, generator=g, device=dev).to(torch.bfloat16).view(torch.uint8)
        out = torch.zeros(rounds * n_jobs * job, dtype=torch.uint8, device=dev)
        wcp, rcp = cache_ops.CacheCopier(), cache_ops.CacheCopier()
        for n, lt in zip(names * 1, layers):
            wcp.register_layer(n, lt, False)
            rcp.register_layer(n, lt, False)
        wcp.register_store(staging)
        rcp.register_store(out)
        jn = [names[i % L] for i in range(n_jobs)]
        offs = [i * job for i in range(n_jobs)]
        idx = torch.tensor(flat, dtype=torch.int32, device=dev)
        return dict(wcp=wcp, rcp=rcp, jn=jn, offs=offs, idx=idx, ioff=ioff, deltas=deltas, ntok=ntok,
                    staging=staging, out=out)

    def run(s, r, st):
        s["wcp"].scatter_pages_rerotate(s["jn"], s["offs"], [job] * n_jobs, s["idx"], s["ioff"], s["deltas"],
                                        s["ntok"], inv, D, True, st)
        s["rcp"].gather_pages(s["jn"], [r * n_jobs * job + o for o in s["offs"]], [job] * n_jobs, s["idx"],
                              s["ioff"], st)

    work = [setup(t) for t in range(n_threads)]
    expected = []
    for s in work:
        run(s, 0, torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize()
        expected.append(s["out"][: n_jobs * job].clone())
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        try:
            st = torch.cuda.Stream(device=dev)
            st.wait_stream(torch.cuda.current_stream(dev))
            for r in range(rounds):
                run(work[t], r, st.cuda_stream)
            st.synchronize()
        except Exception as e:  # surfaced below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(n_threads)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for t, s in enumerate(work):
        got = s["out"].view(rounds, n_jobs * job)
        for r in range(rounds):
            assert torch.equal(got[r], expected[t]), f"thread {t} round {r}"
