"""Pins the CPU oracle's e4m3 conversion against the OCP e4m3 definition
(sign, 4-bit exponent with bias 7, 3-bit mantissa, no infinities, NaN = S.1111.111)."""
import numpy as np

from oracle import fp8


def textbook_e4m3(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1 + m / 8.0) * 2.0 ** (e - 7)


def test_decode_all_codes():
    got = fp8.decode(np.arange(256))
    for c in range(256):
        want = textbook_e4m3(c)
        if np.isnan(want):
            assert np.isnan(got[c])
        else:
            assert got[c] == want and np.signbit(got[c]) == bool(c & 0x80)


def test_encode_roundtrip_midpoints_saturation():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F])
    vals = fp8.decode(codes)
    assert np.array_equal(fp8.encode(vals).view(np.int8).astype(np.int64) & 0xFF,
                          np.where(vals == 0, codes & 0x80, codes))
    pos = np.sort(np.unique(vals[vals > 0]))
    for a, b in zip(pos[:-1], pos[1:]):
        mid = (a + b) / 2
        ca, cb = fp8.encode([a])[0], fp8.encode([b])[0]
        even = ca if ca % 2 == 0 else cb
        assert fp8.encode([mid])[0] == even
        assert fp8.encode([np.nextafter(np.float32(mid), np.float32(0))])[0] == ca
        assert fp8.encode([np.nextafter(np.float32(mid), np.float32(1e9))])[0] == cb
    assert fp8.encode([448.0, 460.0, 1e6, float("inf"), -1e6])[:5].tolist() == [0x7E] * 4 + [0xFE]
    assert fp8.encode([2.0 ** -10, 2.0 ** -11])[:2].tolist() == [0, 0]
    assert fp8.encode([float("nan")])[0] & 0x7F == 0x7F


def test_quantum():
    assert fp8.quantum(1.0) == 0.125
    assert fp8.quantum(448.0) == 32.0
    assert fp8.quantum(0.001) == 2.0 ** -9
