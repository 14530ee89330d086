"""Guard for the forward-only kernels.

The gfx950 kernels implement the forward pass only.  When autograd would record a
graph through one of them (grad mode on and an input that requires grad), the call
raises instead of silently returning an output with no gradient path.
"""

from __future__ import annotations

import torch


def forward_only(what: str, *tensors) -> None:
    if not torch.is_grad_enabled():
        return
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.requires_grad:
            raise NotImplementedError(
                f"{what}: the MI355X kernels are forward-only (no backward); run the model under "
                "torch.no_grad() or torch.inference_mode()")
