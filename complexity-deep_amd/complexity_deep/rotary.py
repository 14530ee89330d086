"""Rotary position embedding; interface of core/rotary.py:16-86.

Used around the QKV projection but not one of the three kernel pieces: it runs as
PyTorch ops on the GPU.  ``inv_freq`` is a persistent buffer (it is in the
reference's state_dict); the cos/sin tables are non-persistent and grow on demand.
"""

from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn


class RotaryEmbedding(nn.Module):
    def __init__(self, dim: int, max_seq_len: int = 2048, theta: float = 10000.0):
        super().__init__()
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.theta = theta
        exponents = torch.arange(0, dim, 2).float() / dim
        self.register_buffer("inv_freq", 1.0 / (theta ** exponents))
        self._build_cache(max_seq_len)

    def _build_cache(self, seq_len: int) -> None:
        pos = torch.arange(seq_len, device=self.inv_freq.device).float()
        angles = torch.outer(pos, self.inv_freq)
        table = torch.cat([angles, angles], dim=-1)
        self.register_buffer("cos_cached", table.cos(), persistent=False)
        self.register_buffer("sin_cached", table.sin(), persistent=False)

    def forward(self, seq_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if seq_len > self.max_seq_len:
            self._build_cache(seq_len)
            self.max_seq_len = seq_len
        return self.cos_cached[:seq_len], self.sin_cached[:seq_len]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """q, k [B, heads, S, D]; cos, sin [S, D]."""
    cos = cos[None, None]
    sin = sin[None, None]
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin
