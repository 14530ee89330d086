"""Rotary position embedding; interface of core/rotary.py:16-86.

Used around the QKV projection but not one of the three kernel pieces: it runs as
PyTorch ops on the GPU.  ``inv_freq`` is a persistent buffer (it is in the
reference's state_dict); the cos/sin tables are non-persistent and grow on demand.

Angles are always formed in fp32 from the exact fp32 inverse frequencies, computed
from ``dim`` and ``theta`` the way the reference's constructor computes them
(core/rotary.py:35-36).  The ``inv_freq`` buffer itself is not used for that: a
``model.to(torch.bfloat16)`` rounds it to bf16, and angles p * bf16(inv_freq) drift
by whole radians at p ~ 2000.  The reference builds its tables once at construction,
in fp32, before any such cast; this module matches that.
"""

from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn


def exact_inv_freq(dim: int, theta: float) -> torch.Tensor:
    """fp32 [dim/2] theta^(-2i/dim), computed on the CPU as at construction."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2).float() / dim))


class RotaryEmbedding(nn.Module):
    def __init__(self, dim: int, max_seq_len: int = 2048, theta: float = 10000.0):
        super().__init__()
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.theta = theta
        self.register_buffer("inv_freq", exact_inv_freq(dim, theta))
        self._build_cache(max_seq_len)

    def _angles(self, n: int, device) -> torch.Tensor:
        """fp32 [n, dim/2] angles p * inv_freq[j] for p < n."""
        pos = torch.arange(n, device=device, dtype=torch.float32)
        return torch.outer(pos, exact_inv_freq(self.dim, self.theta).to(device))

    def _build_cache(self, seq_len: int) -> None:
        angles = self._angles(seq_len, self.inv_freq.device)
        table = torch.cat([angles, angles], dim=-1)
        # Tables take the module's floating dtype (bf16 after model.to(bf16)), rounded
        # once from the fp32 cos/sin, as the reference's cast buffers are.
        dt = self.inv_freq.dtype if self.inv_freq.is_floating_point() else torch.float32
        self.register_buffer("cos_cached", table.cos().to(dt), persistent=False)
        self.register_buffer("sin_cached", table.sin().to(dt), persistent=False)

    def forward(self, seq_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if seq_len > self.max_seq_len:
            self._build_cache(seq_len)
            self.max_seq_len = seq_len
        return self.cos_cached[:seq_len], self.sin_cached[:seq_len]

    def cos_sin_table(self, n_pos: int, device: torch.device) -> torch.Tensor:
        """fp32 [n, dim/2, 2] table of (cos, sin)(p * inv_freq[j]) for p < n >= n_pos, the
        form the fused QKV + RoPE kernel reads.  fp32 whatever dtype the module was cast
        to.  Cached per device; grows geometrically."""
        cached = getattr(self, "_cs_table", None)
        if cached is None or cached[0] != device or cached[1].shape[0] < n_pos:
            grow = 2 * cached[1].shape[0] if cached is not None and cached[0] == device else 0
            n = max(n_pos, self.max_seq_len, grow)
            angles = self._angles(n, device)
            table = torch.stack([angles.cos(), angles.sin()], dim=-1).contiguous()
            self._cs_table = (device, table)
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
