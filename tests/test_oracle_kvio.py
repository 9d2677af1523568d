"""Pins the oracle's store/load record format (reference gpu_kv_io.py) with
hand-built expectations on tiny inputs, and checks the product's host-side
planning helpers against it."""
import numpy as np
import torch

from daric_amd import kv_io
from oracle import kvio as okv


def test_split_registration_copies_cuts_at_chunk_boundaries():
    s, h, n = okv.split_registration_copies([0, 100], [90, 300], [30, 10], chunk_bytes=100)
    # region 1: host 90..120 crosses 100 -> 10 + 20 bytes; region 2 inside one chunk
    assert (s, h, n) == ([0, 10, 100], [90, 100, 300], [10, 20, 10])
    assert okv.split_registration_copies([5], [0], [250], chunk_bytes=100) == \
        ([5, 105, 205], [0, 100, 200], [100, 100, 50])
    for args in (([0], [0], [0]), ([7], [199], [1])):
        assert kv_io.split_registration_copies(*args, chunk_bytes=100) == \
            okv.split_registration_copies(*args, chunk_bytes=100)


def test_copy_plan_order_and_sizes():
    names = ["a.attn", "b.attn", "c.attn"]            # registration (sorted) order
    groups = [0, 1, 0]
    bpb = [10, 20, 10]
    blocks = [([1, 2], [7]), ([3], [8, 9])]
    flat, off, ioff, jn, sz = okv.build_copy_plan(names, groups, bpb, [1000, 5000], blocks)
    assert flat.tolist() == [1, 2, 7, 1, 2, 3, 8, 9, 3]
    assert ioff == [0, 2, 3, 5, 6, 8, 9]
    assert jn == names * 2
    assert sz == [20, 20, 20, 10, 40, 10]
    assert off == [1000, 1020, 1040, 5000, 5010, 5050]
    assert okv.per_meta_cache_size(names, groups, bpb, blocks) == [60, 60]
    # layerwise: one job per meta, that layer only
    flat, off, ioff, jn, sz = okv.build_copy_plan(names, groups, bpb, [1000, 5000], blocks, "b.attn")
    assert (flat.tolist(), off, ioff, jn, sz) == ([7, 8, 9], [1000, 5000], [0, 1, 3], ["b.attn"] * 2, [20, 40])
    for ln in (None, "b.attn"):
        p = kv_io.build_copy_plan(names, groups, bpb, [1000, 5000], blocks, ln)
        q = okv.build_copy_plan(names, groups, bpb, [1000, 5000], blocks, ln)
        assert p[0].tolist() == q[0].tolist() and p[1:] == q[1:]
        assert kv_io.per_meta_cache_size(names, groups, bpb, blocks, ln) == \
            okv.per_meta_cache_size(names, groups, bpb, blocks, ln)


def test_record_bytes_and_header():
    """A record is the layers' page spans in order, then a 4096-byte header
    with the int64 saved position at +0 (little endian)."""
    g = torch.Generator().manual_seed(0)
    names = ["l0", "l1"]
    layers = {n: torch.randint(0, 256, (2, 6, 4, 8), dtype=torch.uint8, generator=g) for n in names}
    span = 4 * 8
    bpb = [2 * span, 2 * span]
    shm = torch.zeros(4 * bpb[0] * 2 + 2 * okv.POSITION_SIZE + 64, dtype=torch.uint8)
    io = okv.OracleKVIO(names, [0, 0], bpb, [False, False], layers, shm)
    blocks = [([3, 1],)]
    io.store([16], blocks, [123456789012])
    off = 16
    for n in names:
        for p in range(2):              # K half then V half (prefix dim)
            for b in (3, 1):
                want = layers[n][p, b].reshape(-1)
                assert torch.equal(shm[off: off + span], want)
                off += span
    assert int(np.frombuffer(shm[off: off + 8].numpy().tobytes(), np.int64)[0]) == 123456789012
    assert int(shm[off + 8: off + okv.POSITION_SIZE].sum()) == 0
    assert okv.read_positions(shm, [off]) == [123456789012]
    # load into zeroed layers restores the listed pages only
    fresh = {n: torch.zeros_like(t) for n, t in layers.items()}
    io2 = okv.OracleKVIO(names, [0, 0], bpb, [False, False], fresh, shm)
    assert io2.load([16], blocks) == [123456789012]
    for n in names:
        for b in range(6):
            same = torch.equal(fresh[n][:, b], layers[n][:, b])
            assert same == (b in (1, 3)) or (b not in (1, 3) and int(fresh[n][:, b].sum()) == 0)


def test_split_registration_copies_product_matches_oracle_on_random_regions():
    rng = np.random.default_rng(8)
    for _ in range(300):
        n = int(rng.integers(0, 6))
        chunk = int(rng.integers(1, 64))
        stg = rng.integers(0, 500, n).tolist()
        host = rng.integers(0, 500, n).tolist()
        size = rng.integers(0, 200, n).tolist()
        assert kv_io.split_registration_copies(stg, host, size, chunk_bytes=chunk) == \
            okv.split_registration_copies(stg, host, size, chunk_bytes=chunk)
    for bad in (([0], [0, 1], [1]), ([-1], [0], [1]), ([0], [0], [-4])):
        for fn in (kv_io.split_registration_copies, okv.split_registration_copies):
            try:
                fn(*bad, chunk_bytes=8)
            except ValueError:
                continue
            raise AssertionError(f"{fn.__module__} accepted {bad}")
