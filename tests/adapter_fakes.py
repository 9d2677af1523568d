"""Fakes for the Adapter tests (vLLM is absent): a rotary embedding exposing
what the adapter reads (rotary_dim, is_neox_style, base, _compute_inv_freq,
cos_sin_cache) and the KVCache meta of reference daric/reuse_controller/kvcache.py:7-15."""
from __future__ import annotations

from dataclasses import dataclass

import torch


class FakeRotary:
    def __init__(self, rotary_dim: int, base: float = 500000.0, is_neox_style: bool = True,
                 max_pos: int = 64):
        self.rotary_dim = rotary_dim
        self.base = base
        self.is_neox_style = is_neox_style
        inv = self._compute_inv_freq(base)
        t = torch.arange(max_pos, dtype=torch.float32)
        freqs = torch.outer(t, inv)
        self.cos_sin_cache = torch.cat([freqs.cos(), freqs.sin()], dim=-1)

    def _compute_inv_freq(self, base: float) -> torch.Tensor:
        return 1.0 / (base ** (torch.arange(0, self.rotary_dim, 2, dtype=torch.float) / self.rotary_dim))


@dataclass
class FakeMeta:
    cache_id: str
    ptr: list
    saved_pos: int = 0
    block_ids: tuple = None
