"""Store/load pipeline (daric_amd.kv_io.KVIOContext) against the oracle's
restatement of the daric-store GPU I/O (oracle/kvio.py): host record bytes
and headers bit-exact after store, cache bytes bit-exact after load, the
fused re-rotating load within the rotation bar; small staging halves force
multi-batch pipelining and reuse of both halves."""
import time

import numpy as np
import pytest
import torch

from daric_amd import kv_io
from oracle import kvio as okv
from oracle import rope as orope
from tests.gpu_util import assert_rotation_parity, make_layer, rotation_region, same_bytes, to_dev

pytestmark = pytest.mark.gpu


def setup(dev, n_layers=3, nb=64, layout="nhd", dtype=torch.bfloat16, two_groups=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    names = sorted(f"model.layers.{i}.self_attn.attn" for i in range(n_layers))
    cpu, pf = {}, False
    for n in names:
        cpu[n], pf = make_layer(layout, nb, 16, 4, 64, dtype, g)
    t0 = cpu[names[0]]
    from oracle.layout import page_copy_shape
    s = page_copy_shape(tuple(t0.shape), tuple(t0.stride()), t0.element_size(), pf)
    bpb = [s.prefix_size * s.suffix_size] * n_layers
    groups = [i % 2 if two_groups else 0 for i in range(n_layers)]
    return names, cpu, pf, bpb, groups


def metas_blocks(rng, n_meta, nb, two_groups):
    """Per meta 1-5 block ids per group, disjoint across metas (no null block)."""
    p0 = rng.permutation(np.arange(1, nb)).tolist()
    p1 = rng.permutation(np.arange(1, nb)).tolist()
    out = []
    for _ in range(n_meta):
        k0, k1 = int(rng.integers(1, 6)), int(rng.integers(1, 6))
        g0, p0 = p0[:k0], p0[k0:]
        g1, p1 = p1[:k1], p1[k1:]
        out.append((g0, g1) if two_groups else (g0,))
    return out


def record_offsets(ctx, blocks, gap=4096 + 256):
    offs, o = [], 8192
    for b in blocks:
        offs.append(o)
        o += ctx.record_size(b) + gap
    return offs, o


@pytest.mark.parametrize("two_groups,staging", [(False, 512 << 10), (True, 300 << 10)])
def test_store_then_load_matches_oracle(dev, two_groups, staging):
    names, cpu, pf, bpb, groups = setup(dev, two_groups=two_groups)
    rng = np.random.default_rng(1)
    blocks = metas_blocks(rng, 7, 64, two_groups)
    dev_caches = {n: to_dev(t, dev) for n, t in cpu.items()}
    host_size = 64 << 20
    host = torch.zeros(host_size, dtype=torch.uint8, pin_memory=True)
    ctx = kv_io.KVIOContext(names, groups, bpb, [pf] * len(names), dev_caches, host, staging_bytes=staging)
    offs, end = record_offsets(ctx, blocks)
    assert end < host_size
    saved = [int(x) for x in rng.integers(0, 1 << 40, len(blocks))]
    ctx.store(offs, blocks, saved)
    shm = torch.zeros(host_size, dtype=torch.uint8)
    okv.OracleKVIO(names, groups, bpb, [pf] * len(names), cpu, shm).store(offs, blocks, saved)
    assert torch.equal(host, shm), "host records differ from the oracle's"
    # load into zeroed caches
    fresh_cpu = {n: torch.zeros_like(t) for n, t in cpu.items()}
    fresh_dev = {n: to_dev(t, dev) for n, t in fresh_cpu.items()}
    ctx2 = kv_io.KVIOContext(names, groups, bpb, [pf] * len(names), fresh_dev, host, staging_bytes=staging)
    got = ctx2.load(offs, blocks)
    torch.cuda.synchronize()
    want = okv.OracleKVIO(names, groups, bpb, [pf] * len(names), fresh_cpu, shm).load(offs, blocks)
    assert got == want == saved
    for n in names:
        assert same_bytes(fresh_dev[n], fresh_cpu[n])


def test_layerwise_and_null_blocks(dev):
    names, cpu, pf, bpb, groups = setup(dev, layout="pf")
    rng = np.random.default_rng(2)
    blocks = metas_blocks(rng, 3, 64, False)
    host = torch.zeros(8 << 20, dtype=torch.uint8, pin_memory=True)
    shm = torch.zeros(8 << 20, dtype=torch.uint8)
    dev_caches = {n: to_dev(t, dev) for n, t in cpu.items()}
    ctx = kv_io.KVIOContext(names, groups, bpb, [pf] * 3, dev_caches, host, staging_bytes=512 << 10)
    offs = [4096 + i * (1 << 20) for i in range(3)]
    ctx.store(offs, blocks, [5, 6, 7], layer_name=names[1])
    okv.OracleKVIO(names, groups, bpb, [pf] * 3, cpu, shm).store(offs, blocks, [5, 6, 7], layer_name=names[1])
    assert torch.equal(host, shm)
    # load with a null block (id 0) in the list: that page is neither read nor written
    blocks0 = [([0] + b[0][1:],) for b in blocks]
    fresh_cpu = {n: torch.full_like(t, 7) for n, t in cpu.items()}
    fresh_dev = {n: to_dev(t, dev) for n, t in fresh_cpu.items()}
    ctx2 = kv_io.KVIOContext(names, groups, bpb, [pf] * 3, fresh_dev, host, staging_bytes=512 << 10)
    assert ctx2.load(offs, blocks0, layer_name=names[1]) == [5, 6, 7]
    torch.cuda.synchronize()
    okv.OracleKVIO(names, groups, bpb, [pf] * 3, fresh_cpu, shm).load(offs, blocks0, layer_name=names[1])
    for n in names:
        assert same_bytes(fresh_dev[n], fresh_cpu[n])


@pytest.mark.parametrize("two_groups,layerwise,layout", [(False, False, "nhd"), (False, True, "nhd"),
                                                          (True, False, "pf"), (True, True, "nhd")])
def test_load_rerotate_matches_oracle(dev, two_groups, layerwise, layout):
    """The fused load (records scattered and K moved from the saved position
    to the new one in one pass) against the oracle's load then rotation:
    whole records or one layer's record (the reference's per-layer load,
    worker.py:219-231), one KV-cache group or two (each layer's pages are its
    group's block list)."""
    names, cpu, pf, bpb, groups = setup(dev, n_layers=4, layout=layout, two_groups=two_groups)
    rng = np.random.default_rng(3)
    blocks = metas_blocks(rng, 5, 64, two_groups)
    host = torch.zeros(32 << 20, dtype=torch.uint8, pin_memory=True)
    shm = torch.zeros(32 << 20, dtype=torch.uint8)
    dev_caches = {n: to_dev(t, dev) for n, t in cpu.items()}
    L = len(names)
    ctx = kv_io.KVIOContext(names, groups, bpb, [pf] * L, dev_caches, host, staging_bytes=320 << 10)
    offs, _ = record_offsets(ctx, blocks)
    saved = [0, 512, 77, 3000, 9]
    layer = names[2] if layerwise else None
    ctx.store(offs, blocks, saved, layer_name=layer)
    okv.OracleKVIO(names, groups, bpb, [pf] * L, cpu, shm).store(offs, blocks, saved, layer_name=layer)
    assert torch.equal(host, shm)
    R = 64
    inv = orope.default_inv_freq(R, 500000.0)
    new_pos = [100, 512, 4000, 0, 20000]
    # tokens per meta: within the shorter group's pages when there are two
    ntok = [min(len(g) for g in b) * 16 - 3 for b in blocks]
    fresh_cpu = {n: torch.zeros_like(t) for n, t in cpu.items()}
    fresh_dev = {n: to_dev(t, dev) for n, t in fresh_cpu.items()}
    ctx2 = kv_io.KVIOContext(names, groups, bpb, [pf] * L, fresh_dev, host, staging_bytes=320 << 10)
    got = ctx2.load(offs, blocks, layer_name=layer,
                    rerotate=(new_pos, ntok, torch.from_numpy(inv).to(dev), R, True))
    torch.cuda.synchronize()
    want = okv.OracleKVIO(names, groups, bpb, [pf] * L, fresh_cpu, shm).load(
        offs, blocks, layer_name=layer, rerotate=(new_pos, ntok, inv, R, True))
    assert got == want == saved
    for n, gi in zip(names, groups):
        slots = []
        if layer is None or n == layer:
            for b, nt, np_, sp in zip(blocks, ntok, new_pos, saved):
                if np_ != sp:
                    slots += [b[gi][j // 16] * 16 + j % 16 for j in range(nt)]
        mask, pn = rotation_region(fresh_cpu[n], pf, R, slots, True)
        assert_rotation_parity(fresh_dev[n], fresh_cpu[n], mask, pn)
        if layer is not None and n != layer:
            assert not bool(fresh_dev[n].view(torch.int16).any()), f"layer {n} was not loaded"


def test_store_and_load_from_two_threads(dev):
    # One context, one thread storing records of some blocks while another loads
    # earlier records into other blocks: store and load have their own staging
    # halves and streams, as the reference's staging and read_staging
    # (gpu_kv_io.py:150-151). Small staging halves make both pipelines run
    # several batches at once.
    import threading
    names, cpu, pf, bpb, groups = setup(dev, nb=160)
    rng = np.random.default_rng(4)
    perm = rng.permutation(np.arange(1, 160)).tolist()
    cut = lambda lo, n: [(perm[lo + 3 * k: lo + 3 * k + 3],) for k in range(n)]
    src_y, blk_x, dst_l = cut(0, 12), cut(36, 12), cut(72, 12)     # disjoint block sets
    host = torch.zeros(64 << 20, dtype=torch.uint8, pin_memory=True)
    dev_caches = {n: to_dev(t, dev) for n, t in cpu.items()}
    ctx = kv_io.KVIOContext(names, groups, bpb, [pf] * 3, dev_caches, host, staging_bytes=160 << 10)
    rec = ctx.record_size(src_y[0])
    offs_y = [8192 + k * (rec + 512) for k in range(12)]
    offs_x = [(16 << 20) + k * (rec + 512) for k in range(12)]
    saved_y, saved_x = list(range(100, 112)), list(range(200, 212))
    ctx.store(offs_y, src_y, saved_y)
    torch.cuda.synchronize()
    shm = host.clone()
    errors = []

    def run(fn):
        try:
            for _ in range(3):
                fn()
        except Exception as e:      # surfaced below
            errors.append(e)

    got = {}
    t1 = threading.Thread(target=run, args=(lambda: ctx.store(offs_x, blk_x, saved_x),))
    t2 = threading.Thread(target=run, args=(lambda: got.__setitem__("pos", ctx.load(offs_y, dst_l)),))
    t1.start(); t2.start(); t1.join(); t2.join()
    torch.cuda.synchronize()
    assert not errors, errors
    assert got["pos"] == saved_y
    ocpu = {n: t.clone() for n, t in cpu.items()}
    ok = okv.OracleKVIO(names, groups, bpb, [pf] * 3, ocpu, shm)
    ok.store(offs_x, blk_x, saved_x)
    ok.load(offs_y, dst_l)
    assert torch.equal(host, shm), "stored records differ from the oracle's"
    for n in names:
        assert same_bytes(dev_caches[n], ocpu[n])


KV_FUZZ = None
try:
    from hypothesis import HealthCheck, given, settings
    from hypothesis import strategies as st
    KV_FUZZ = settings(max_examples=25, deadline=None, derandomize=True, database=None,
                       suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture])
except ImportError:      # hypothesis is part of the image; keep the module importable without it
    pass


if KV_FUZZ is not None:
    @KV_FUZZ
    @given(data=st.data())
    def test_store_load_fuzz(dev, data):
        # drawn layout, dtype, group count, meta count, blocks per meta (null
        # ids included), layerwise or whole records and staging size; host
        # records bit-exact after store, caches bit-exact after load
        layout = data.draw(st.sampled_from(["nhd", "hnd", "pf", "pf_hnd", "packed", "mla"]), label="layout")
        dtype = data.draw(st.sampled_from([torch.bfloat16, torch.float16, torch.uint8]), label="dtype")
        two = data.draw(st.booleans(), label="two_groups") and layout != "mla"
        n_layers = data.draw(st.integers(1, 4), label="layers")
        n_meta = data.draw(st.integers(1, 9), label="metas")
        seed = data.draw(st.integers(0, 1 << 20), label="seed")
        names, cpu, pf, bpb, groups = setup(dev, n_layers=n_layers, nb=96, layout=layout, dtype=dtype,
                                            two_groups=two, seed=seed)
        rng = np.random.default_rng(seed)
        blocks = metas_blocks(rng, n_meta, 96, two)
        # a null id (block 0) only on load: a stored null page would leave its
        # record bytes to whatever staging held, in the reference as here
        load_blocks = list(blocks)
        if data.draw(st.booleans(), label="null_block_on_load"):
            load_blocks[0] = tuple([0] + list(g[1:]) for g in blocks[0])
        layer_name = names[data.draw(st.integers(0, n_layers - 1), label="layer")] \
            if data.draw(st.booleans(), label="layerwise") else None
        host = torch.zeros(32 << 20, dtype=torch.uint8, pin_memory=True)
        dev_caches = {n: to_dev(t, dev) for n, t in cpu.items()}
        ctx = kv_io.KVIOContext(names, groups, bpb, [pf] * n_layers, dev_caches, host,
                                staging_bytes=data.draw(st.sampled_from([160 << 10, 512 << 10, 4 << 20]),
                                                        label="staging"))
        offs, o = [], 4096
        for b in blocks:
            offs.append(o)
            o += ctx.record_size(b, layer_name) + 512
        saved = [int(x) for x in rng.integers(0, 1 << 40, n_meta)]
        try:
            ctx.store(offs, blocks, saved, layer_name=layer_name)
        except RuntimeError as e:           # a meta larger than a staging buffer: refused up front
            assert "staging buffer" in str(e)
            return
        shm = torch.zeros(32 << 20, dtype=torch.uint8)
        okv.OracleKVIO(names, groups, bpb, [pf] * n_layers, cpu, shm).store(offs, blocks, saved,
                                                                            layer_name=layer_name)
        assert torch.equal(host, shm)
        fresh_cpu = {n: torch.zeros_like(t) for n, t in cpu.items()}
        fresh_dev = {n: to_dev(t, dev) for n, t in fresh_cpu.items()}
        ctx2 = kv_io.KVIOContext(names, groups, bpb, [pf] * n_layers, fresh_dev, host, staging_bytes=512 << 10)
        # the fused re-rotating load: K of each meta's first tokens moved from
        # the saved position to a drawn one
        rerot = None
        if data.draw(st.booleans(), label="rerotate"):
            R = data.draw(st.sampled_from([16, 32, 64]), label="rotary_dim")
            neox = data.draw(st.booleans(), label="neox")
            new_pos = [int(saved[k]) + int(d) for k, d in enumerate(rng.integers(-5000, 5000, n_meta))]
            if n_meta > 1:
                new_pos[1] = saved[1]                       # a meta that does not move
            ntok = [int(rng.integers(0, min(len(g) for g in b) * 16 + 1)) for b in load_blocks]
            inv = orope.default_inv_freq(R, 500000.0)
            rerot = (new_pos, ntok, inv, R, neox)
        got = ctx2.load(offs, load_blocks, layer_name=layer_name,
                        rerotate=None if rerot is None else
                        (rerot[0], rerot[1], torch.from_numpy(rerot[2]).to(dev), rerot[3], rerot[4]))
        torch.cuda.synchronize()
        want = okv.OracleKVIO(names, groups, bpb, [pf] * n_layers, fresh_cpu, shm).load(
            offs, load_blocks, layer_name=layer_name, rerotate=rerot)
        assert got == want == saved
        for n, gi in zip(names, groups):
            if rerot is None:
                assert same_bytes(fresh_dev[n], fresh_cpu[n])
                continue
            slots = []
            if layer_name is None or n == layer_name:
                for b, nt, npos, sp in zip(load_blocks, rerot[1], rerot[0], saved):
                    if npos != sp:
                        slots += [b[gi][j // 16] * 16 + j % 16 for j in range(nt) if b[gi][j // 16] != 0]
            mask, pn = rotation_region(fresh_cpu[n], pf, rerot[3], slots, rerot[4])
            assert_rotation_parity(fresh_dev[n], fresh_cpu[n], mask, pn)


def test_concurrent_stores_take_turns_and_close_drains(dev):
    """Four threads store disjoint records through one context at once: the
    store lock makes them take turns on the shared staging, so every record
    matches the oracle's. close() then waits for a running load and its device
    work; afterwards store and load raise, and a second close() does nothing."""
    import threading
    names, cpu, pf, bpb, groups = setup(dev, n_layers=2)
    rng = np.random.default_rng(3)
    blocks = metas_blocks(rng, 12, 64, False)
    dev_caches = {n: to_dev(t, dev) for n, t in cpu.items()}
    host_size = 64 << 20
    host = torch.zeros(host_size, dtype=torch.uint8, pin_memory=True)
    ctx = kv_io.KVIOContext(names, groups, bpb, [pf] * len(names), dev_caches, host,
                            staging_bytes=256 << 10)
    offs, end = record_offsets(ctx, blocks)
    saved = [int(x) for x in rng.integers(0, 1 << 40, len(blocks))]
    errors = []

    def store(part):
        try:
            sel = list(range(part, len(blocks), 4))
            ctx.store([offs[i] for i in sel], [blocks[i] for i in sel], [saved[i] for i in sel])
        except Exception as e:  # surfaced below
            errors.append(repr(e))

    threads = [threading.Thread(target=store, args=(p,)) for p in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    shm = torch.zeros(host_size, dtype=torch.uint8)
    okv.OracleKVIO(names, groups, bpb, [pf] * len(names), cpu, shm).store(offs, blocks, saved)
    assert torch.equal(host, shm)
    # close while a load is running in another thread
    fresh = {n: torch.zeros_like(t, device=dev) for n, t in cpu.items()}
    ctx2 = kv_io.KVIOContext(names, groups, bpb, [pf] * len(names), fresh, host, staging_bytes=256 << 10)
    got = {}
    loader = threading.Thread(target=lambda: got.setdefault("saved", ctx2.load(offs, blocks)))
    loader.start()
    while not got and ctx2._inflight == 0 and loader.is_alive():
        time.sleep(0.0005)
    ctx2.close()
    loader.join()
    assert ctx2.closed and got["saved"] == saved
    loaded = sorted({b for bl in blocks for b in bl[0]})
    for n in names:
        assert torch.equal(fresh[n][:, loaded].cpu().view(torch.int16), cpu[n][:, loaded].view(torch.int16))
    with pytest.raises(RuntimeError, match="closed"):
        ctx2.load(offs, blocks)
    with pytest.raises(RuntimeError, match="closed"):
        ctx2.store(offs, blocks, saved)
    ctx2.close()
