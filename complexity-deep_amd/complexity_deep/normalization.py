"""RMSNorm and fused residual-add + RMSNorm on the gfx950 kernel (piece 3).

Module and operator interfaces follow the reference:
  RMSNorm                    core/normalization.py:15-35
  fused_residual_rmsnorm     cuda/fused_residual.py:333-399
  fused_add_rmsnorm_inplace  cuda/fused_residual.py:478-533
  FusedResidualRMSNorm       cuda/fused_residual.py:540-589 (inference path; the
                             dropout variant is training-only and not provided)
  fused_rmsnorm              cuda/triton_token_routed.py:578-602

Numerics: h = x + residual is rounded to bf16 like the reference's bf16 add; the
norm is computed in fp32 from that h and rounded once (the reference rounds every
sub-step to bf16).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _native as nat
from ._grad import forward_only


def _weight(weight: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    if weight.dtype != like.dtype or weight.device != like.device:
        weight = weight.to(device=like.device, dtype=like.dtype)
    return weight if weight.is_contiguous() else weight.contiguous()


def _check_out(t: Optional[torch.Tensor], x: torch.Tensor, what: str) -> None:
    """A caller-provided output must be a contiguous tensor of x's shape, dtype and device:
    the kernel writes T * H values through its base pointer."""
    if t is None:
        return
    if t.shape != x.shape or t.dtype != x.dtype or t.device != x.device or not t.is_contiguous():
        raise ValueError(f"add_rms_norm: {what} must be a contiguous {x.dtype} tensor of shape "
                         f"{tuple(x.shape)} on {x.device}, got {tuple(t.shape)} {t.dtype} on {t.device}"
                         f"{'' if t.is_contiguous() else ' (not contiguous)'}")


def add_rms_norm(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor,
                 eps: float = 1e-6, *, out: Optional[torch.Tensor] = None,
                 residual_out: Optional[torch.Tensor] = None,
                 store_residual: bool = True) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """(rmsnorm(x + residual) * weight, x + residual) in one pass over HBM.

    residual=None gives a plain RMSNorm (second result None).  ``residual_out`` may
    be ``residual`` itself for an in-place update."""
    forward_only("add_rms_norm", x, residual, weight)
    nat.require_device(x, residual, what="add_rms_norm")
    shape = x.shape
    H = shape[-1]
    # The kernel reads rows base + r * H: contiguous operands need no row view.
    x2 = x if x.is_contiguous() else x.contiguous()
    T = x2.numel() // H if H else 0
    r2 = None
    if residual is not None:
        if residual.shape != shape:
            raise ValueError(f"add_rms_norm: residual shape {tuple(residual.shape)} != {tuple(shape)}")
        r2 = residual if residual.is_contiguous() else residual.contiguous()
    w = _weight(weight, x2)
    if w.numel() != H:
        raise ValueError(f"add_rms_norm: weight has {w.numel()} elements, hidden size is {H}")
    if out is not None:
        _check_out(out, x, "out")
    if residual_out is not None:
        _check_out(residual_out, x, "residual_out")
    y = out if out is not None else torch.empty(shape, dtype=x.dtype, device=x.device)
    h = None
    if residual is not None and store_residual:
        h = residual_out if residual_out is not None else torch.empty(shape, dtype=x.dtype, device=x.device)
    with nat.launch_region("add_rmsnorm" if r2 is not None else "rmsnorm", x.device, T=T, H=H,
                           residual=r2 is not None, store_residual=h is not None):
        nat.check(nat.lib().cdx_add_rmsnorm_fwd(
            x2.data_ptr(), nat.ptr(r2), w.data_ptr(), float(eps), T, H,
            y.data_ptr(), nat.ptr(h), nat.stream_of(x)), "cdx_add_rmsnorm_fwd")
    return y, h


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Plain RMSNorm.  ``out`` may be any [..., H] view whose rows are evenly spaced, e.g.
    the left half of a [T, 2H] buffer (cdx_rmsnorm_ld_fwd writes rows at that stride)."""
    if out is None or out.is_contiguous():
        return add_rms_norm(x, None, weight, eps, out=out)[0]
    forward_only("rms_norm", x, weight)
    nat.require_device(x, out, what="rms_norm")
    H = x.shape[-1]
    if out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError(f"rms_norm: out must be a {x.dtype} tensor of shape {tuple(x.shape)}, "
                         f"got {out.dtype} {tuple(out.shape)}")
    ldo = nat.row_stride(out, H, "rms_norm out")
    x2 = x if x.is_contiguous() else x.contiguous()
    T = x2.numel() // H if H else 0
    w = _weight(weight, x2)
    if w.numel() != H:
        raise ValueError(f"rms_norm: weight has {w.numel()} elements, hidden size is {H}")
    with nat.launch_region("rmsnorm", x.device, T=T, H=H, residual=False, store_residual=False):
        nat.check(nat.lib().cdx_rmsnorm_ld_fwd(x2.data_ptr(), w.data_ptr(), float(eps), T, H, out.data_ptr(), ldo,
                                               nat.stream_of(x)), "cdx_rmsnorm_ld_fwd")
    return out


class RMSNorm(nn.Module):
    """y = weight * x / sqrt(mean(x^2) + eps); core/normalization.py:15-35."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.weight, self.eps)

    def extra_repr(self) -> str:
        return f"{self.weight.shape[0]}, eps={self.eps}"


def fused_residual_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                           eps: float = 1e-6, store_residual: bool = True) -> tuple:
    """Returns (out, x + residual) or (out,); cuda/fused_residual.py:333-399."""
    out, h = add_rms_norm(x, residual, weight, eps, store_residual=store_residual)
    return (out, h) if store_residual else (out,)


def fused_add_rmsnorm_inplace(hidden: torch.Tensor, mlp_out: torch.Tensor, weight: torch.Tensor,
                              eps: float = 1e-6) -> torch.Tensor:
    """hidden += mlp_out (in place); returns rmsnorm(hidden); cuda/fused_residual.py:478-533."""
    if not hidden.is_contiguous():
        raise ValueError("fused_add_rmsnorm_inplace: hidden must be contiguous (it is updated in place)")
    out, _ = add_rms_norm(mlp_out, hidden, weight, eps, residual_out=hidden)
    return out


def fused_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Plain RMSNorm; cuda/triton_token_routed.py:578-602."""
    return rms_norm(x, weight, eps)


class FusedResidualRMSNorm(nn.Module):
    """forward(x, residual) -> (out, new_residual); cuda/fused_residual.py:540-589."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, dropout_p: float = 0.0):
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.dropout_p = dropout_p
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor, residual: torch.Tensor) -> tuple:
        if self.dropout_p > 0 and self.training:
            raise NotImplementedError("FusedResidualRMSNorm: residual dropout is training-only and not "
                                      "part of this forward-only build")
        return fused_residual_rmsnorm(x, residual, self.weight, eps=self.eps, store_residual=True)
