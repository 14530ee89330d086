"""Dense SwiGLU MLP; interface of core/mlp.py:19-40.

Only used when ``use_token_routed_mlp=False``.  It runs on the same gfx950 kernel
as the MoE (cdx_moe_swiglu_fwd) with one expert, no shared block and an identity
routing plan, so the dense configuration also stays on MFMA.  Its three nn.Linear
weights are views of that kernel's operands (MLPOperands), as in TokenRoutedMLP.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from ._grad import forward_only
from .token_routed_mlp import MLPOperands, RoutePlan, moe_swiglu
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
        self._operands = MLPOperands()

    def kernel_weights(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(w_gu [1, 2, P, H], w_down [1, H, P]): the operands the three weights are views of."""
        # One routed expert (block 0) whose weights are nn.Linear weights.
        ws = {"lin_gate": self.gate_proj.weight, "lin_up": self.up_proj.weight, "lin_down": self.down_proj.weight}
        I, H = self.gate_proj.weight.shape
        return self._operands.get(ws, 1, H, I, False)

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``residual`` (same shape, contiguous) receives residual + MLP(x) in place and is
        returned (the block's residual add fused into the down pass)."""
        forward_only("SwiGLU", x, residual, module=self)
        nat.require_device(x, what="SwiGLU")
        w_gu, w_down = self.kernel_weights()
        shape = x.shape
        x2d = x.reshape(-1, shape[-1]).contiguous()
        r2d = None
        if residual is not None:
            if residual.shape != shape or not residual.is_contiguous():
                raise ValueError("SwiGLU: residual must be a contiguous tensor shaped like the input")
            r2d = residual.view(-1, shape[-1])
        out = moe_swiglu(x2d, identity_plan(x2d.shape[0], x.device), w_gu, w_down,
                         self.gate_proj.weight.shape[0], False, residual=r2d)
        return out.view(shape)
