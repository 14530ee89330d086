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

    def cos_sin_table(self, n_pos: int, device: torch.device) -> torch.Tensor:
        """fp32 [n, dim/2, 2] table of (cos, sin)(p * inv_freq[j]) for p < n >= n_pos, the
        form the fused QKV + RoPE kernel reads.  The angles are the fp32 products of
        _build_cache; the table stays fp32 whatever dtype the module was cast to.
        Cached per device and inv_freq version; grows geometrically."""
        inv = self.inv_freq
        key = (device, inv.data_ptr(), inv._version, inv.dtype)
        cached = getattr(self, "_cs_table", None)
        if cached is None or cached[0] != key or cached[1].shape[0] < n_pos:
            n = max(n_pos, self.max_seq_len, 2 * cached[1].shape[0] if cached is not None and cached[0] == key else 0)
            pos = torch.arange(n, device=device, dtype=torch.float32)
            angles = torch.outer(pos, inv.to(device=device, dtype=torch.float32))
            table = torch.stack([angles.cos(), angles.sin()], dim=-1).contiguous()
            self._cs_table = (key, table)
        return self._cs_table[1]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """q, k [B, heads, S, D]; cos, sin [S, D]."""
    cos = cos[None, None]
    sin = sin[None, None]
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin
