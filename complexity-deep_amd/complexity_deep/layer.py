"""Decoder block and mu guidance; interfaces of core/layer.py:28-190.

``TransformerBlock.forward`` keeps the reference signature and returns
(hidden_states, new_kv, mu) with mu unclamped, as the reference does.  Inside, the
residual add before the MLP's norm is the fused add+RMSNorm kernel.
``ComplexityModel`` drives the blocks through ``forward_fused``, where both residual
adds run inside the kernels that produce the branch outputs (o_proj as hipBLASLt's
GEMM with beta = 1, the MoE down pass's scatter epilogue) and the norms after them are
plain RMSNorms of h; the layer's routing plan comes from the model.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as nat
from ._grad import forward_only
from .attention import ComplexityAttention
from .mlp import SwiGLU
from .normalization import RMSNorm, add_rms_norm, rms_norm
from .token_routed_mlp import RoutePlan, TokenRoutedMLP


def mu_guidance(h: torch.Tensor, w: torch.Tensor, mu: torch.Tensor, mu_lo: float = -math.inf,
                mu_hi: float = math.inf, lo: float = -math.inf, hi: float = math.inf,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """clamp(h @ w^T + clamp(mu, mu_lo, mu_hi), lo, hi) through cdx_mu_guidance_fwd (fp32
    accumulate, one rounding).  h [..., H], w [H, H] and mu [H], all bf16.  ``out`` may be
    any [..., H] view with evenly spaced rows (e.g. the right half of a [T, 2H] buffer)."""
    nat.require_device(h, w, mu, out, what="mu_guidance")
    H = h.shape[-1]
    h2 = h if h.is_contiguous() else h.contiguous()  # rows base + r * H
    T = h2.numel() // H if H else 0
    w = w if w.is_contiguous() else w.contiguous()
    mu = mu if mu.is_contiguous() else mu.contiguous()
    if mu.shape != (H,):
        raise ValueError(f"mu_guidance: mu must be [{H}], got {tuple(mu.shape)}")
    if out is None:
        out = torch.empty(h.shape, dtype=h.dtype, device=h.device)
    elif out.shape != h.shape:
        raise ValueError(f"mu_guidance: out must have shape {tuple(h.shape)}, got {tuple(out.shape)}")
    ldo = nat.row_stride(out, H, "mu_guidance out")
    with nat.launch_region("mu_guidance", h.device, T=T, H=H):
        nat.check(nat.lib().cdx_mu_guidance_fwd(h2.data_ptr(), T, H, w.data_ptr(), mu.data_ptr(),
                                                float(mu_lo), float(mu_hi), float(lo), float(hi), out.data_ptr(),
                                                ldo, nat.stream_of(h)), "cdx_mu_guidance_fwd")
    return out


class MuGuidance(nn.Module):
    """mu = clamp(mu_param, mu_min, mu_max) + mu_proj(h); core/layer.py:28-61.

    Runs as one kernel (cdx_mu_guidance_fwd): the mu_proj GEMM whose epilogue reads the
    mu parameter, clamps it and adds it; ``fused(h, lo, hi)`` also applies the clamp the
    model puts on mu between layers (models/modeling.py:199-200).  Nothing is cached:
    the kernel reads both parameters on every call."""

    def __init__(self, hidden_size: int, mu_min: float = 0.0, mu_max: float = 2.0):
        super().__init__()
        self.mu_min = mu_min
        self.mu_max = mu_max
        self.mu = nn.Parameter(torch.full((hidden_size,), (mu_min + mu_max) / 2))
        self.mu_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        nn.init.zeros_(self.mu_proj.weight)

    def fused(self, hidden_states: torch.Tensor, lo: float = -math.inf, hi: float = math.inf,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
        forward_only("MuGuidance", hidden_states, module=self)
        return mu_guidance(hidden_states, self.mu_proj.weight, self.mu, self.mu_min, self.mu_max, lo, hi, out=out)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return self.fused(hidden_states)


class TransformerBlock(nn.Module):
    """Pre-norm block: attention -> MLP -> mu guidance; core/layer.py:63-190."""

    def __init__(self, hidden_size: int, intermediate_size: int, num_attention_heads: int,
                 num_key_value_heads: int, max_position_embeddings: int = 2048,
                 rms_norm_eps: float = 1e-6, rope_theta: float = 10000.0,
                 attention_dropout: float = 0.0, use_token_routed_mlp: bool = True,
                 num_experts: int = 4, vocab_size: int = 100_000, shared_expert: bool = True,
                 token_frequencies: Optional[torch.Tensor] = None, use_qk_norm: bool = True,
                 use_mu_guidance: bool = True):
        super().__init__()
        self.hidden_size = hidden_size
        self.use_token_routed_mlp = use_token_routed_mlp
        self.input_layernorm = RMSNorm(hidden_size, eps=rms_norm_eps)
        self.self_attn = ComplexityAttention(
            hidden_size=hidden_size, num_attention_heads=num_attention_heads,
            num_key_value_heads=num_key_value_heads, max_position_embeddings=max_position_embeddings,
            rope_theta=rope_theta, attention_dropout=attention_dropout, use_qk_norm=use_qk_norm)
        self.post_attention_layernorm = RMSNorm(hidden_size, eps=rms_norm_eps)
        if use_token_routed_mlp:
            self.mlp = TokenRoutedMLP(hidden_size=hidden_size, intermediate_size=intermediate_size,
                                      num_experts=num_experts, vocab_size=vocab_size,
                                      shared_expert=shared_expert, token_frequencies=token_frequencies)
        else:
            self.mlp = SwiGLU(hidden_size=hidden_size, intermediate_size=intermediate_size)
        self.use_mu_guidance = use_mu_guidance
        self.mu_guidance = MuGuidance(hidden_size=hidden_size) if use_mu_guidance else None

    def _mlp(self, x: torch.Tensor, token_ids, route: Optional[RoutePlan],
             residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.use_token_routed_mlp:
            return self.mlp(x, token_ids=token_ids, route=route, residual=residual)
        return self.mlp(x, residual=residual)

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                past_key_value: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                use_cache: bool = False, token_ids: Optional[torch.Tensor] = None,
                mu_prev: Optional[torch.Tensor] = None):
        normed = self.input_layernorm(hidden_states)
        attn_out, new_kv = self.self_attn(normed, attention_mask=attention_mask,
                                          past_key_value=past_key_value, use_cache=use_cache,
                                          mu_prev=mu_prev)
        ln = self.post_attention_layernorm
        normed, h = add_rms_norm(attn_out, hidden_states, ln.weight, ln.eps)
        h = h + self._mlp(normed, token_ids, None)
        mu = self.mu_guidance(h) if self.mu_guidance is not None else None
        return h, new_kv, mu

    def forward_fused(self, h: torch.Tensor, normed: torch.Tensor, next_norm: RMSNorm,
                      attention_mask=None, past_key_value=None, use_cache: bool = False,
                      token_ids=None, mu_prev=None, route: Optional[RoutePlan] = None,
                      want_mu: bool = True, pair: Optional[torch.Tensor] = None):
        """One block given h (updated in place) and normed = input_layernorm(h).

        Returns (h, next_norm(h_out), new_kv, mu) where mu is already clamped to [-2, 2],
        the model's clamp between layers (modeling.py:199-200).  Both residual adds
        (core/layer.py:174, 183) happen inside the kernels that produce the branch
        outputs: o_proj as a GEMM with beta = 1 and the MoE down pass's scatter
        epilogue; the norms that follow read h alone.  ``want_mu=False`` skips mu for
        the last layer, whose mu the reference computes and then discards.  ``pair``, a
        [..., 2H] buffer, receives next_norm(h_out) in its left half and mu in its right
        half (the returned tensors are those halves), so that the next layer's projection
        reads [x | mu] as one operand; the caller reads them before the next call writes
        the buffer again."""
        if not h.is_contiguous():
            raise ValueError("forward_fused: h must be contiguous (it is updated in place)")
        _, new_kv = self.self_attn(normed, attention_mask=attention_mask, past_key_value=past_key_value,
                                   use_cache=use_cache, mu_prev=mu_prev, residual=h)
        ln = self.post_attention_layernorm
        normed = rms_norm(h, ln.weight, ln.eps)
        self._mlp(normed, token_ids, route, residual=h)
        H = h.shape[-1]
        mu_out = None
        if pair is not None and want_mu and self.mu_guidance is not None:
            normed, mu_out = pair[..., :H], pair[..., H:]
            rms_norm(h, next_norm.weight, next_norm.eps, out=normed)
        else:
            normed = rms_norm(h, next_norm.weight, next_norm.eps)
        mu = self.mu_guidance.fused(h, -2.0, 2.0, out=mu_out) if (want_mu and self.mu_guidance is not None) else None
        return h, normed, new_kv, mu
