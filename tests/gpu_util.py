"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle import rope as orope

INT_VIEW = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.uint8: torch.uint8,
            torch.float32: torch.int32}


def make_layer(layout: str, nb: int, ps: int, h: int, d: int, dtype, gen, kind="normal"):
    """A CPU KV layer tensor of the named vLLM layout, filled with N(0,1) values
    (fp8: codes of N(0,1) values) or random bytes (kind="bytes")."""
    if layout == "nhd":          # [2, NB, PS, H, D]
        phys, perm, pf = (2, nb, ps, h, d), None, False
    elif layout == "hnd":        # logical [2, NB, PS, H, D] over physical [2, NB, H, PS, D]
        phys, perm, pf = (2, nb, h, ps, d), (0, 1, 3, 2, 4), False
    elif layout == "pf":         # [NB, 2, PS, H, D]
        phys, perm, pf = (nb, 2, ps, h, d), None, True
    elif layout == "pf_hnd":     # logical [NB, 2, PS, H, D] over physical [NB, 2, H, PS, D]
        phys, perm, pf = (nb, 2, h, ps, d), (0, 1, 3, 2, 4), True
    elif layout == "packed":     # [NB, H, PS, 2D]
        phys, perm, pf = (nb, h, ps, 2 * d), None, True
    elif layout == "mla":        # [NB, PS, hidden]
        phys, perm, pf = (nb, ps, h * d), None, True
    elif layout == "nhd_pad":    # [2, NB, PS, H, D] with 16 padding elements after each head row
        phys, perm, pf = (2, nb, ps, h, d + 16), None, False
    else:
        raise ValueError(layout)
    n = int(np.prod(phys))
    if kind == "bytes":
        e = torch.empty(0, dtype=dtype).element_size()
        t = torch.randint(0, 256, (n * e,), dtype=torch.uint8, generator=gen).view(dtype).view(phys)
    elif dtype == torch.uint8:
        v = torch.randn(n, generator=gen)
        t = torch.from_numpy(ofp8.encode(v.numpy())).view(phys)
    else:
        t = torch.randn(n, generator=gen).to(dtype).view(phys)
    if perm is not None:
        t = t.permute(*perm)
    if layout == "nhd_pad":
        t = t[..., :d]
    return t, pf


def to_dev(t: torch.Tensor, dev) -> torch.Tensor:
    """Device copy with the same strides (permuted layouts stay permuted)."""
    out = torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device=dev)
    out.copy_(t)
    return out


def same_bytes(a: torch.Tensor, b: torch.Tensor) -> bool:
    a = a.cpu().contiguous()
    b = b.cpu().contiguous()
    return torch.equal(a.view(INT_VIEW[a.dtype]), b.view(INT_VIEW[b.dtype]))


def rotation_region(want: torch.Tensor, page_first: bool, rotary_dim: int, slots, is_neox=True):
    """(mask of rotated elements, float64 norm of each rotated element's pair
    in `want`) for the K rows of `slots`."""
    R = rotary_dim
    mask = torch.zeros_like(want, dtype=torch.bool)
    pnorm = torch.zeros_like(want, dtype=torch.float64)
    km, kp = orope.k_view(mask, page_first, R), orope.k_view(pnorm, page_first, R)
    kw = orope.k_view(want, page_first, R)
    ps = km.shape[1]
    for s in slots:
        b, j = int(s) // ps, int(s) % ps
        km[b, j, :, :R] = True
        w = values(kw[b, j, :, :R].clone())
        if is_neox:
            n = np.sqrt(w[:, : R // 2] ** 2 + w[:, R // 2:] ** 2)
            norm = np.concatenate([n, n], axis=1)
        else:
            n = np.sqrt(w[:, 0::2] ** 2 + w[:, 1::2] ** 2)
            norm = np.repeat(n, 2, axis=1)
        kp[b, j, :, :R] = torch.from_numpy(norm)
    return mask, pnorm


def values(x: torch.Tensor) -> np.ndarray:
    if x.dtype == torch.uint8:
        return ofp8.decode(x.numpy()).astype(np.float64)
    return x.to(torch.float64).numpy()


def ulp(v: np.ndarray, dtype) -> np.ndarray:
    a = np.abs(v)
    if dtype == torch.bfloat16:
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
        return np.exp2(e - 7)
    if dtype == torch.float16:
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
        return np.exp2(e - 10)
    if dtype == torch.uint8:
        return ofp8.quantum(a)
    raise ValueError(dtype)


def assert_rotation_parity(got: torch.Tensor, want: torch.Tensor, mask: torch.Tensor,
                           pnorm: torch.Tensor, max_ulps=1, angle_tol=0.0):
    """Bit-exact outside `mask`. Inside: within max_ulps of the target dtype of
    the oracle value, plus an fp32 arithmetic allowance of 2^-20 times the
    pair's norm (the float32 rounding of x1*c - x2*s when it cancels; 2^12
    below the bf16 resolution of the pair), plus angle_tol (radians) times the
    pair's norm where the oracle's angles come from another rounding of the
    same angle (a rotary table's float32 entries)."""
    got = got.cpu()
    want = want.cpu()
    gi, wi = got.view(INT_VIEW[got.dtype]), want.view(INT_VIEW[want.dtype])
    bad = (gi != wi) & ~mask
    assert not bool(bad.any()), f"{int(bad.sum())} elements differ outside the rotated region"
    gv, wv = values(got[mask]), values(want[mask])
    tol = max_ulps * ulp(np.maximum(np.abs(gv), np.abs(wv)), got.dtype) + \
        (2.0 ** -20 + angle_tol) * pnorm[mask].numpy()
    err = np.abs(gv - wv)
    worst = float((err / tol).max()) if err.size else 0.0
    if not (err <= tol).all():
        i = np.nonzero(err > tol)[0][:6]
        raise AssertionError(f"rotation error {worst:.2f} x tolerance; {int((err > tol).sum())}/{err.size} "
                             f"elements; got {gv[i].tolist()} want {wv[i].tolist()}")
    return worst
