"""Guard for the forward-only kernels.

The gfx950 kernels implement the forward pass only.  When autograd would record a
graph through one of them (grad mode on and an input that requires grad), the call
raises instead of silently returning an output with no gradient path.
"""

from __future__ import annotations

from typing import Optional

import torch


def forward_only(what: str, *tensors, module: Optional[torch.nn.Module] = None) -> None:
    """Raise if autograd would record through a kernel call: grad mode on and any of
    ``tensors`` (or of ``module``'s parameters, walked only in grad mode) requiring grad."""
    if not torch.is_grad_enabled():
        return
    params = module.parameters() if module is not None else ()
    for t in (*tensors, *params):
        if isinstance(t, torch.Tensor) and t.requires_grad:
            raise NotImplementedError(
                f"{what}: the MI355X kernels are forward-only (no backward); run the model under "
                "torch.no_grad() or torch.inference_mode()")
