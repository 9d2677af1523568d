"""OCP float8 e4m3fn encode/decode for the fp8 KV path (CPU restatement).

The reference views a uint8 cache as torch.float8_e4m3fn and lets Triton cast
fp32 results back (reference daric/adaption/adapter.py:370-373, store cast at
:72-73). Triton's fp32->e4m3 store rounding is parity unpinned (it needs the
reference's GPU run); this oracle fixes the conversion as saturating
round-to-nearest-even, which is what torch's cast does once the input has been
clamped to the finite range (torch alone maps overflow to NaN).
"""
from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0


def decode(codes) -> np.ndarray:
    """uint8 codes -> float32 values (exact)."""
    t = torch.as_tensor(np.asarray(codes, dtype=np.uint8))
    return t.view(torch.float8_e4m3fn).float().numpy()


def encode(x) -> np.ndarray:
    """float values -> uint8 codes, saturating RTNE. Values are first rounded to
    float32 (the kernel's arithmetic type), then clamped to +-448 and cast."""
    t = torch.as_tensor(np.asarray(x, dtype=np.float32))
    return t.clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def quantum(v) -> np.ndarray:
    """Spacing of e4m3 values at magnitude |v| (2^-9 in the subnormal range)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -6)))
    return np.exp2(e - 3)
