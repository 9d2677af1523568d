"""Pins the CPU oracle's RoPE re-rotation.

Independent facts used: RoPE as complex multiplication z * exp(i*p*theta)
(NeoX pairs (i, i+R/2), GPT-J pairs (2i, 2i+1) via numpy's complex view),
re-rotation of RoPE(x, p) by d equals RoPE(x, p + d), identity at d = 0,
composition, norm preservation, untouched tail dims, and the layout views of
reference adapter.py:311-368 checked against torch slicing.
"""
import math

import numpy as np
import pytest
import torch

from oracle import rope


def rope_forward_complex(x, pos, inv_freq, R, neox):
    """Textbook RoPE: pair i is the complex number z_i, multiplied by e^{i*pos*theta_i}."""
    x = np.asarray(x, np.float64)
    th = np.asarray(inv_freq, np.float64) * pos
    out = x.copy()
    if neox:
        z = x[..., : R // 2] + 1j * x[..., R // 2: R]
        z = z * np.exp(1j * th)
        out[..., : R // 2], out[..., R // 2: R] = z.real, z.imag
    else:
        z = np.ascontiguousarray(x[..., :R]).view(np.complex128)
        z = z * np.exp(1j * th)
        out[..., :R] = z.view(np.float64)
    return out


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("delta", [1, 7, 512, 1536, 30720])
def test_rerotation_moves_rope_position(neox, delta):
    rng = np.random.default_rng(0)
    R, D = 64, 96
    inv = rope.default_inv_freq(R, 500000.0)
    x = rng.standard_normal((5, D))
    p = 37
    cached = rope_forward_complex(x, p, inv, R, neox)
    moved = rope.rotate_rows(cached, delta, inv, R, neox)
    want = rope_forward_complex(x, p + delta, inv, R, neox)
    # the only difference is the float32 rounding of the angle delta*theta
    tol = 4 * np.abs(x).max() * (2.0 ** -24) * (1 + delta * inv.max())
    assert np.abs(moved - want).max() <= tol
    assert np.array_equal(moved[:, R:], cached[:, R:])


def test_identity_composition_norm():
    rng = np.random.default_rng(1)
    R = 128
    inv = rope.default_inv_freq(R, 10000.0)
    x = rng.standard_normal((3, R))
    assert np.array_equal(rope.rotate_rows(x, 0, inv, R, True), x)
    a = rope.rotate_rows(rope.rotate_rows(x, 100, inv, R, True), 250, inv, R, True)
    b = rope.rotate_rows(x, 350, inv, R, True)
    assert np.abs(a - b).max() < 1e-4
    y = rope.rotate_rows(x, 999, inv, R, False)
    n0 = x[:, 0::2] ** 2 + x[:, 1::2] ** 2
    n1 = y[:, 0::2] ** 2 + y[:, 1::2] ** 2
    assert np.allclose(n0, n1, rtol=1e-12)


def test_default_inv_freq_closed_form():
    inv = rope.default_inv_freq(128, 500000.0)
    for i in range(64):
        assert abs(inv[i] - 500000.0 ** (-(2 * i) / 128)) <= 2e-7 * inv[i]
    assert inv[0] == 1.0


def test_angle_is_float32_product():
    inv = np.array([0.3, 1.0, 1e-5], np.float32)
    a = rope.angles(32767, inv)
    assert a.dtype == np.float32
    assert a[1] == np.float32(32767.0)
    assert a[0] == np.float32(np.float32(32767) * np.float32(0.3))


def test_k_view_matches_slicing():
    t5 = torch.arange(2 * 6 * 4 * 3 * 8, dtype=torch.float32).view(2, 6, 4, 3, 8)
    assert torch.equal(rope.k_view(t5, False, 8), t5[0])
    p5 = torch.arange(6 * 2 * 4 * 3 * 8, dtype=torch.float32).view(6, 2, 4, 3, 8)
    assert torch.equal(rope.k_view(p5, True, 8), p5[:, 0])
    t4 = torch.arange(6 * 3 * 4 * 16, dtype=torch.float32).view(6, 3, 4, 16)
    assert torch.equal(rope.k_view(t4, True, 8), t4.permute(0, 2, 1, 3)[..., :8])
    t3 = torch.arange(6 * 4 * 10, dtype=torch.float32).view(6, 4, 10)
    assert torch.equal(rope.k_view(t3, True, 8), t3.unsqueeze(2))
    with pytest.raises(ValueError, match="page_first must be true"):
        rope.k_view(t4, False, 8)
    with pytest.raises(ValueError, match="rotary_dim must be positive"):
        rope.k_view(t4, True, 10)
    with pytest.raises(ValueError, match="Unsupported KV cache rank"):
        rope.k_view(torch.zeros(2, 2), True, 2)


@pytest.mark.parametrize("page_first", [False, True])
def test_rerotate_pages_in_place(page_first):
    g = torch.Generator().manual_seed(5)
    nb, ps, h, d, R = 8, 4, 2, 16, 16
    shape = (nb, 2, ps, h, d) if page_first else (2, nb, ps, h, d)
    layer = torch.randn(shape, generator=g).to(torch.bfloat16)
    before = layer.clone()
    inv = rope.default_inv_freq(R, 10000.0)
    bt = np.array([5, 2, 7], np.int32)
    rope.rerotate_pages([layer], page_first, bt, [(0, 2, 7, 300)], inv, R, True)
    kv_b, kv_a = rope.k_view(before, page_first, R), rope.k_view(layer, page_first, R)
    moved = set()
    for j in range(2, 9):
        blk, s = bt[j // ps], j % ps
        moved.add((blk, s))
        want = rope.rotate_rows(kv_b[blk, s].double().numpy(), 300, inv, R, True)
        got = kv_a[blk, s].double().numpy()
        ulp = np.abs(want) * 2.0 ** -8 + 1e-30
        assert (np.abs(got - want) <= ulp).all()
    for blk in range(nb):
        for s in range(ps):
            if (blk, s) not in moved:
                assert torch.equal(kv_a[blk, s].view(torch.int16), kv_b[blk, s].view(torch.int16))
    v_b = before[:, 1] if page_first else before[1]
    v_a = layer[:, 1] if page_first else layer[1]
    assert torch.equal(v_a.view(torch.int16), v_b.view(torch.int16))


def test_zero_shift_segment_is_untouched():
    # delta 0 leaves every byte alone, -0 codes included (an identity rotation
    # computes -0*1 - (-0)*0 = +0)
    layer = torch.zeros(2, 4, 4, 2, 16, dtype=torch.uint8)
    layer[0] = 0x80                                   # fp8 -0 everywhere in K
    before = layer.clone()
    inv = rope.default_inv_freq(16, 10000.0)
    rope.rerotate_pages([layer], False, np.array([1, 2], np.int32), [(0, 0, 8, 0)], inv, 16, True,
                        np.ones((1, 2)))
    assert torch.equal(layer, before)
    # the same rows rotated by a non-zero shift do change sign of zero somewhere
    rope.rerotate_pages([layer], False, np.array([1, 2], np.int32), [(0, 0, 8, 5)], inv, 16, True,
                        np.ones((1, 2)))
    assert not torch.equal(layer, before)


def test_segment_planning():
    # apply_rerotate_load: metas with saved_pos == ptr[0] or empty are skipped
    bt, segs = rope.load_segments([(0, 32, 0, [4, 5]), (32, 64, 0, [6, 7]),
                                   (64, 64, 3, [8]), (64, 80, 16, [9])])
    assert bt.tolist() == [6, 7, 9] and segs == [(0, 0, 32, 32), (2, 0, 16, 48)]
    # apply_rerotate_multi: groups 1..n-2 move by group_ptr[i] - group_ptr[0]
    bt, segs = rope.multi_segments([[10, 20, 30, 45, 50], [0, 5, 9]], [[1, 2, 3, 4], [9]])
    assert bt.tolist() == [1, 2, 3, 4]
    assert segs == [(0, 10, 10, 10), (0, 20, 15, 20)]
    # relative position 10 with PS 16 is block bt[0] = 1, offset 10 -> slot 26
    assert rope.segment_slots(bt, 0, 10, 10, 16)[:2] == [26, 27]
    assert rope.segment_slots(bt, 0, 20, 15, 16)[-1] == 2 * 16 + 34 - 16


def _complex_table(max_pos, inv_freq, m=1.0):
    """m * cat(cos(p * theta), sin(p * theta)) from complex exponentials in float64."""
    z = np.exp(1j * np.arange(max_pos)[:, None] * np.asarray(inv_freq, np.float64)[None, :])
    return torch.from_numpy(np.concatenate([z.real, z.imag], axis=1) * m)


@pytest.mark.parametrize("m", [1.0, 1.25])
def test_table_cos_sin_is_the_angle_difference(m):
    """The reference's combined rows (adapter.py:276-283) equal cos/sin of
    (new - old) * theta by the angle-subtraction identity; multi's rows are
    the shift's own row; the table scale m is divided out."""
    inv = rope.default_inv_freq(64, 10000.0)
    tab = _complex_table(3000, inv, m)
    rng = np.random.default_rng(4)
    old = rng.integers(0, 3000, 50)
    new = rng.integers(0, 3000, 50)
    c, s = rope.table_cos_sin_load(tab, old, new)
    th = (new - old)[:, None] * inv.astype(np.float64)[None, :]
    np.testing.assert_allclose(c, np.cos(th), atol=1e-12)
    np.testing.assert_allclose(s, np.sin(th), atol=1e-12)
    c2, s2 = rope.table_cos_sin_multi(tab, new)
    th2 = new[:, None] * inv.astype(np.float64)[None, :]
    np.testing.assert_allclose(c2, np.cos(th2), atol=1e-12)
    np.testing.assert_allclose(s2, np.sin(th2), atol=1e-12)


@pytest.mark.parametrize("neox", [True, False])
def test_rotate_slots_cs_is_complex_multiplication(neox):
    """Per-slot rotation by its own angle row equals the textbook complex
    form, slot by slot; V and dims >= R stay as they were."""
    R, D, H = 32, 48, 2
    inv = rope.default_inv_freq(R, 500000.0)
    g = torch.Generator().manual_seed(2)
    layer = torch.randn(2, 6, 16, H, D, generator=g, dtype=torch.float64).to(torch.float32)
    before = layer.clone()
    slots = [3, 17, 40, 95]
    delta = np.array([5, -9, 700, 1])
    th = delta[:, None] * inv.astype(np.float64)[None, :]
    rope.rotate_slots_cs(layer, False, slots, np.cos(th), np.sin(th), R, neox)
    for i, slot in enumerate(slots):
        b, j = slot // 16, slot % 16
        x = before[0, b, j].numpy().astype(np.float64)
        want = rope_forward_complex(x, float(delta[i]), inv, R, neox)
        np.testing.assert_allclose(layer[0, b, j].numpy(), want, rtol=1e-6, atol=1e-6)
    assert torch.equal(layer[1], before[1])
    mask = torch.ones(6 * 16, dtype=torch.bool)
    mask[slots] = False
    assert torch.equal(layer[0].reshape(96, H, D)[mask], before[0].reshape(96, H, D)[mask])


@pytest.mark.parametrize("neox", [True, False])
def test_rotate_slots_cs_on_fp8_codes(neox):
    """On an e4m3 (uint8) cache the per-slot rotation rotates the code values
    and re-encodes them: equal to torch's float8_e4m3fn cast of the complex-form
    rotation of the decoded values (inside +-448, where that cast and
    saturating round-to-nearest-even agree); V, the dims past R and unlisted
    slots keep their codes."""
    R, D, H = 32, 48, 2
    inv = rope.default_inv_freq(R, 500000.0)
    g = torch.Generator().manual_seed(3)
    layer = (torch.randn(2, 6, 16, H, D, generator=g) * 4).to(torch.float8_e4m3fn).view(torch.uint8)
    before = layer.clone()
    slots = [3, 17, 40, 95]
    delta = np.array([5, -9, 700, 1])
    th = delta[:, None] * inv.astype(np.float64)[None, :]
    rope.rotate_slots_cs(layer, False, slots, np.cos(th), np.sin(th), R, neox)
    for i, slot in enumerate(slots):
        b, j = slot // 16, slot % 16
        x = before[0, b, j].view(torch.float8_e4m3fn).to(torch.float64).numpy()
        want = rope_forward_complex(x, float(delta[i]), inv, R, neox)
        codes = torch.from_numpy(want.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8)
        assert torch.equal(layer[0, b, j], codes), slot
    assert torch.equal(layer[1], before[1])
    mask = torch.ones(6 * 16, dtype=torch.bool)
    mask[slots] = False
    assert torch.equal(layer[0].reshape(96, H, D)[mask], before[0].reshape(96, H, D)[mask])


def test_rotation_bar_needs_its_cancellation_allowance():
    """Why the GPU rotation bar (tests.gpu_util.assert_rotation_parity) adds
    2^-20 x the pair norm to 1 ulp. Where x1*cos - x2*sin nearly cancels, even
    the correctly rounded bf16 result (the fp64 rotation rounded once) lies
    more than 1 bf16 ulp from a float32 torch rotation of the same inputs:
    float32's own rounding error, ~2^-24 x the pair norm, exceeds the bf16
    ulp of the tiny result. With the allowance no element of the sample
    fails, and the allowance stays 2^12 below the bf16 resolution of the
    pair."""
    from tests.gpu_util import ulp
    g = torch.Generator().manual_seed(5)
    n = 4_000_000
    x1 = torch.randn(n, generator=g).to(torch.bfloat16).double()
    x2 = torch.randn(n, generator=g).to(torch.bfloat16).double()
    inv = torch.from_numpy(rope.default_inv_freq(128, 500000.0))
    ang = (torch.randint(-8192, 8192, (n,), generator=g).float()
           * inv[torch.randint(0, 64, (n,), generator=g)])
    a = ang.double()
    exact = (x1 * torch.cos(a) - x2 * torch.sin(a)).float().to(torch.bfloat16).double().numpy()
    ref32 = (x1.float() * torch.cos(ang) - x2.float() * torch.sin(ang)).double().numpy()
    pnorm = torch.sqrt(x1 * x1 + x2 * x2).numpy()
    err = np.abs(exact - ref32)
    one_ulp = ulp(np.maximum(np.abs(exact), np.abs(ref32)), torch.bfloat16)
    literal = err > one_ulp
    assert literal.sum() >= 1
    assert (np.abs(ref32[literal]) < 2.0 ** -16 * pnorm[literal]).all()     # all of them cancel
    assert (err <= one_ulp + 2.0 ** -20 * pnorm).all()
