"""Dense SwiGLU MLP; interface of core/mlp.py:19-40.

Only used when ``use_token_routed_mlp=False``.  It runs on the same gfx950 kernel
as the MoE (cdx_moe_swiglu_fwd) with one expert, no shared block and an identity
routing plan, so the dense configuration also stays on MFMA.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ._grad import forward_only
from .token_routed_mlp import RoutePlan, moe_swiglu, pack_moe_weights
from . import _native as nat


def identity_plan(T: int, device) -> RoutePlan:
    """One expert holding every token in order (built on the device: no host copy)."""
    ar = torch.arange(T, dtype=torch.int32, device=device)
    return RoutePlan(expert_id=torch.zeros(T, dtype=torch.int32, device=device), perm=ar, inv_perm=ar,
                     counts=torch.full((1,), T, dtype=torch.int32, device=device),
                     offsets=torch.arange(2, dtype=torch.int32, device=device) * T, num_experts=1)


class SwiGLU(nn.Module):
    """down_proj(silu(gate_proj(x)) * up_proj(x)), bias-free nn.Linear weights."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)
        self._key = None
        self._packed = None

    def refresh_packed_weights(self) -> None:
        """Repack at the next forward (needed after writes through ``.data``, which bump
        no version counter)."""
        self._key = None
        self._packed = None

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``residual`` (same shape, contiguous) receives residual + MLP(x) in place and is
        returned (the block's residual add fused into the down pass)."""
        forward_only("SwiGLU", x, residual, *self.parameters())
        nat.require_device(x, what="SwiGLU")
        ws = (self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws)
        if key != self._key:
            with torch.no_grad():
                # [in, out] expert layout with E = 1
                self._packed = pack_moe_weights(ws[0].t().unsqueeze(0), ws[1].t().unsqueeze(0),
                                                ws[2].t().unsqueeze(0), None, None, None)
            self._key = key
        shape = x.shape
        x2d = x.reshape(-1, shape[-1]).contiguous()
        r2d = None
        if residual is not None:
            if residual.shape != shape or not residual.is_contiguous():
                raise ValueError("SwiGLU: residual must be a contiguous tensor shaped like the input")
            r2d = residual.view(-1, shape[-1])
        out = moe_swiglu(x2d, identity_plan(x2d.shape[0], x.device), *self._packed,
                         self.gate_proj.weight.shape[0], False, residual=r2d)
        return out.view(shape)
