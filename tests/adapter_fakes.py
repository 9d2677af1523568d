"""Fakes for the Adapter tests (vLLM is absent): rotary embeddings exposing
what the adapter reads (rotary_dim, is_neox_style, base, _compute_inv_freq,
cos_sin_cache) and the KVCache meta of reference daric/reuse_controller/kvcache.py:7-15.

FakeRotary builds its table as vLLM's RotaryEmbedding does:
cat(cos(t * inv_freq), sin(t * inv_freq)) over float32 positions t, cast to
the table dtype. The variants below build tables the re-rotation must refuse
(positions divided by a factor, a base other than .base) or accept (a table
scale m != 1 with YaRN's _compute_inv_freq(scaling_factor) signature)."""
from __future__ import annotations

from dataclasses import dataclass

import torch


class FakeRotary:
    def __init__(self, rotary_dim: int, base: float = 500000.0, is_neox_style: bool = True,
                 max_pos: int = 64, dtype=torch.float32):
        self.rotary_dim = rotary_dim
        self.base = base
        self.is_neox_style = is_neox_style
        self.max_position_embeddings = max_pos
        self.cos_sin_cache = self._table(max_pos).to(dtype)

    def _compute_inv_freq(self, base: float) -> torch.Tensor:
        return 1.0 / (base ** (torch.arange(0, self.rotary_dim, 2, dtype=torch.float) / self.rotary_dim))

    def _positions(self, max_pos: int) -> torch.Tensor:
        return torch.arange(max_pos, dtype=torch.float32)

    def _table(self, max_pos: int) -> torch.Tensor:
        freqs = torch.outer(self._positions(max_pos), self._compute_inv_freq(self.base))
        return torch.cat([freqs.cos(), freqs.sin()], dim=-1)


class ScaledPositionsRotary(FakeRotary):
    """Positions divided by a factor before the angle (linear position
    scaling), with nothing else exposed that says so."""
    factor = 4.0

    def _positions(self, max_pos):
        return torch.arange(max_pos, dtype=torch.float32) / self.factor


class OtherBaseRotary(FakeRotary):
    """The table uses a base adjusted away from .base (as dynamic-NTK scaling
    does)."""

    def _table(self, max_pos):
        freqs = torch.outer(self._positions(max_pos), self._compute_inv_freq(self.base * 3.0))
        return torch.cat([freqs.cos(), freqs.sin()], dim=-1)


class MScaleRotary(FakeRotary):
    """YaRN's form: _compute_inv_freq takes the scaling factor, and the table
    holds m * cos and m * sin."""
    mscale = 1.25

    def __init__(self, rotary_dim, scaling_factor=4.0, **kw):
        self.scaling_factor = scaling_factor
        super().__init__(rotary_dim, **kw)

    def _compute_inv_freq(self, scaling_factor: float) -> torch.Tensor:
        pos_freqs = self.base ** (torch.arange(0, self.rotary_dim, 2, dtype=torch.float) / self.rotary_dim)
        return 1.0 / (scaling_factor * pos_freqs)

    def _table(self, max_pos):
        freqs = torch.outer(self._positions(max_pos), self._compute_inv_freq(self.scaling_factor))
        return torch.cat([freqs.cos() * self.mscale, freqs.sin() * self.mscale], dim=-1)


@dataclass
class FakeMeta:
    cache_id: str
    ptr: list
    saved_pos: int = 0
    block_ids: tuple = None
