"""GPU parity of the token-major copies (CacheCopier.gather_tokens /
scatter_tokens) against the CPU oracle: bit-exact staging and cache bytes on
every layout, with null and out-of-range pages, on the row kernel (16-byte and
byte accesses) and the LDS-transpose kernel (head-major pages with rows of
>= 128 bytes)."""
import numpy as np
import pytest
import torch

from daric_amd import cache_ops
from oracle.copy import OracleCopier
from tests.gpu_util import make_layer, same_bytes, to_dev

pytestmark = pytest.mark.gpu

LAYOUTS = ["nhd", "hnd", "pf", "pf_hnd", "packed", "mla"]


def _case(dev, layouts, dtype, nb=24, ps=16, h=4, d=64, sels=None, seed=0, gather=True, base=16):
    g = torch.Generator().manual_seed(seed)
    names, offsets, sizes, flat, ioff = [], [], [], [], [0]
    oc, gc = OracleCopier(), cache_ops.CacheCopier()
    cpu, gpu = [], []
    off = base
    rng = np.random.default_rng(seed)
    for li, layout in enumerate(layouts):
        t, pf = make_layer(layout, nb, ps, h, d, dtype, g, kind="bytes")
        td = to_dev(t, dev)
        cpu.append(t)
        gpu.append(td)
        name = f"layer.{li}"
        oc.register_layer(name, t, pf)
        gc.register_layer(name, td, pf)
        sel = sels[li] if sels is not None else [int(x) for x in rng.permutation(np.arange(1, nb))[:5]] + [0, nb + 1]
        n_kv = 1 if layout == "mla" else 2
        sz = n_kv * len(sel) * ps * h * d * t.element_size()
        names.append(name)
        offsets.append(off)
        sizes.append(sz)
        flat.extend(sel)
        ioff.append(len(flat))
        off += sz
    store = torch.randint(0, 256, (off + 32,), dtype=torch.uint8, generator=g)
    oc.register_store(store.clone())
    gstore = store.to(dev)
    gc.register_store(gstore)
    idx = torch.tensor(flat, dtype=torch.int32)
    if gather:
        oc.gather_tokens(names, offsets, sizes, idx, ioff)
        gc.gather_tokens(names, offsets, sizes, idx.to(dev), ioff)
    else:
        oc.scatter_tokens(names, offsets, sizes, idx, ioff)
        gc.scatter_tokens(names, offsets, sizes, idx.to(dev), ioff)
    torch.cuda.synchronize()
    assert torch.equal(gstore.cpu(), oc.store)
    for t, td in zip(cpu, gpu):
        assert same_bytes(td, t)


@pytest.mark.parametrize("gather", [True, False])
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.uint8])
def test_token_copies_layouts(dev, layout, dtype, gather):
    # d = 64: bf16/fp16 rows of 128 bytes take the LDS kernel on head-major
    # pages (hnd, pf_hnd); fp8 rows of 64 bytes and the rest take the row kernel
    _case(dev, [layout], dtype, gather=gather)


@pytest.mark.parametrize("gather", [True, False])
@pytest.mark.parametrize("d", [5, 24])
def test_token_copies_byte_path(dev, d, gather):
    # rows of 10 or 48 bytes in odd sizes: 1-byte accesses (d = 5) and the
    # 16-byte row kernel with small rows (d = 24)
    _case(dev, ["hnd", "pf"], torch.float16, d=d, h=3, ps=3, gather=gather, seed=1)


@pytest.mark.parametrize("gather", [True, False])
def test_token_copies_mixed_layers_and_misaligned_store(dev, gather):
    # layers of different layouts in one call, and a store offset that is not
    # 16-byte aligned: the whole call takes 1-byte accesses
    _case(dev, ["nhd", "hnd", "packed"], torch.bfloat16, gather=gather, base=3, seed=2)


@pytest.mark.parametrize("gather", [True, False])
def test_token_copies_llama3_8b_hnd(dev, gather):
    # H = 8, D = 128 bf16 head-major pages (32 KiB, 4-token parts of 8 KiB)
    _case(dev, ["hnd", "pf_hnd"], torch.bfloat16, nb=40, h=8, d=128, gather=gather, seed=3,
          sels=[list(range(1, 33)), [5, 0, 7, 39, 41]])


@pytest.mark.parametrize("n_sel", [33, 35, 40])
def test_token_gather_xcd_runs_with_tail(dev, n_sel):
    # 8 KiB parts, 2 * n_sel * 4 per job: runs of 32 parts per XCD cover the
    # largest multiple of 256 and the tail (8, 24 or 64 parts) keeps its place;
    # a null page and an out-of-range page sit in both regions
    sel = list(range(1, n_sel + 1))
    sel[3], sel[-2] = 0, 99
    _case(dev, ["hnd", "pf_hnd"], torch.bfloat16, nb=48, h=8, d=128, gather=True, seed=7 + n_sel,
          sels=[sel, sel[: n_sel - 5]])


def test_gather_tokens_canonical_rows_at_size(dev):
    """An HND cache gathered token-major equals torch's own permute of the
    selected pages (2 layers x 256 pages of [H=8, PS=16, D=128] bf16)."""
    g = torch.Generator().manual_seed(4)
    nb, ps, h, d, n = 1024, 16, 8, 128, 256
    phys = [torch.randn(2, nb, h, ps, d, generator=g).to(torch.bfloat16) for _ in range(2)]
    sel = torch.randperm(nb - 1, generator=g)[:n] + 1
    gc = cache_ops.CacheCopier()
    per = 2 * n * ps * h * d * 2
    store = torch.zeros(2 * per, dtype=torch.uint8, device=dev)
    for i, p in enumerate(phys):
        gc.register_layer(f"l{i}", p.to(dev).permute(0, 1, 3, 2, 4), False)
    gc.register_store(store)
    idx = sel.to(torch.int32).to(dev)
    gc.gather_tokens(["l0", "l1"], [0, per], [per, per], torch.cat([idx, idx]), [0, n, 2 * n])
    torch.cuda.synchronize()
    got = store.cpu().view(torch.bfloat16).view(2, 2, n * ps, h, d)
    for i, p in enumerate(phys):
        want = p[:, sel].permute(0, 1, 3, 2, 4).reshape(2, n * ps, h, d)
        assert torch.equal(got[i].view(torch.int16), want.contiguous().view(torch.int16))
