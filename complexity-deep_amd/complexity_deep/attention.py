"""GQA attention with the mu-guided QKV projection on the gfx950 kernel (piece 2).

Interfaces follow the reference:
  ComplexityAttention        core/attention.py:33-181 (constructor, parameters and
                             state_dict keys; exported also as MuGuidedAttention)
  fused_mu_qkv_projection    cuda/triton_mu_qkv.py:195-283 (weights [in, out])
  FusedMuQKVProjection       cuda/triton_mu_qkv.py:336-394

The projection is one MFMA contraction over K = 2H: [x | mu_prev] @ W_pack^T with
W_pack = [[Wq; Wk; Wv] | [Wmu_q; Wmu_k; Wmu_v]] packed once (cached per parameter
version) instead of being concatenated on every forward (attention.py:122-124).  q,
k and v are column slices of the packed [T, Nq*D + 2*Nkv*D] output.  Everything
after the projection — QK RMSNorm, RoPE, KV cache, GQA SDPA, o_proj — runs as
PyTorch-ROCm ops, exactly as the reference orders them (attention.py:133-181).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as nat
from ._grad import forward_only
from .rotary import RotaryEmbedding, apply_rotary_pos_emb


def _rows_view(t: torch.Tensor, H: int) -> Tuple[torch.Tensor, int]:
    """Express a [..., H] tensor as rows base + r * ld; ld = 0 for one broadcast row."""
    if t.stride(-1) != 1:
        t = t.contiguous()
    if t.dim() > 1 and all(s == 0 for s in t.stride()[:-1]):
        return t, 0
    try:
        rows = t.view(-1, H)
    except RuntimeError:
        rows = t.contiguous().view(-1, H)
    ld = rows.stride(0) if rows.shape[0] > 1 else H
    if ld < H:
        rows = rows.contiguous()
        ld = H
    return rows, ld


def mu_qkv_project(x: torch.Tensor, mu: Optional[torch.Tensor], w_pack: torch.Tensor,
                   H: int) -> torch.Tensor:
    """[..., N] = [x | mu] @ w_pack^T (cdx_mu_qkv_fwd).

    w_pack is [N, 2H] (or [N, >=H] row-strided when mu is None)."""
    nat.require_device(x, mu, w_pack, what="mu_qkv_project")
    lead = x.shape[:-1]
    x2, ldx = _rows_view(x, H)
    if ldx == 0:
        x2, ldx = x.contiguous(), H
    M = x.numel() // H
    N = w_pack.shape[0]
    if mu is not None:
        if mu.shape[-1] != H:
            raise ValueError(f"mu_qkv_project: mu hidden size {mu.shape[-1]} != {H}")
        mu = mu.expand(*lead, H) if mu.shape[:-1] != lead else mu
        mu2, ldmu = _rows_view(mu, H)
    else:
        mu2, ldmu = None, 0
    if w_pack.stride(-1) != 1:
        raise ValueError("mu_qkv_project: packed weight must be unit-stride in K")
    out = torch.empty(*lead, N, dtype=x.dtype, device=x.device)
    with nat.launch_region("mu_qkv", x.device, M=M, H=H, N=N, mu=mu2 is not None):
        nat.check(nat.lib().cdx_mu_qkv_fwd(x2.data_ptr(), ldx, nat.ptr(mu2), ldmu, w_pack.data_ptr(),
                                           w_pack.stride(0), M, H, N, out.data_ptr(), N,
                                           nat.stream_of(x)), "cdx_mu_qkv_fwd")
    return out


def fused_mu_qkv_projection(x: torch.Tensor, mu: Optional[torch.Tensor], wq: torch.Tensor,
                            wk: torch.Tensor, wv: torch.Tensor, mu_wq: torch.Tensor,
                            mu_wk: torch.Tensor, mu_wv: torch.Tensor
                            ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """q = x@wq + mu@mu_wq (k, v alike) with weights [in, out]; cuda/triton_mu_qkv.py:195-283.
    Returns [B, S, q_dim], [B, S, kv_dim], [B, S, kv_dim] (column views of one buffer)."""
    forward_only("fused_mu_qkv_projection", x, mu, wq, wk, wv, mu_wq, mu_wk, mu_wv)
    H = x.shape[-1]
    q_dim, kv_dim = wq.shape[1], wk.shape[1]
    w_x = torch.cat([wq, wk, wv], dim=1)
    if mu is not None:
        w_mu = torch.cat([mu_wq, mu_wk, mu_wv], dim=1)
        w_pack = torch.cat([w_x, w_mu], dim=0).t().contiguous()
    else:
        w_pack = w_x.t().contiguous()
    out = mu_qkv_project(x, mu, w_pack, H)
    return (out[..., :q_dim], out[..., q_dim:q_dim + kv_dim], out[..., q_dim + kv_dim:])


class FusedMuQKVProjection(nn.Module):
    """Module form of the fused projection; cuda/triton_mu_qkv.py:336-394."""

    def __init__(self, hidden_size: int, num_attention_heads: int, num_key_value_heads: int):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_attention_heads
        self.num_kv_heads = num_key_value_heads
        self.head_dim = hidden_size // num_attention_heads
        self.q_dim = num_attention_heads * self.head_dim
        self.kv_dim = num_key_value_heads * self.head_dim
        self.q_proj = nn.Linear(hidden_size, self.q_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.kv_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.kv_dim, bias=False)
        self.mu_to_q = nn.Linear(hidden_size, self.q_dim, bias=False)
        self.mu_to_k = nn.Linear(hidden_size, self.kv_dim, bias=False)
        self.mu_to_v = nn.Linear(hidden_size, self.kv_dim, bias=False)
        self._cache = _PackCache()

    def forward(self, x: torch.Tensor, mu: Optional[torch.Tensor] = None):
        forward_only("FusedMuQKVProjection", x, mu, *self.parameters())
        w = self._cache.get(self)
        out = mu_qkv_project(x, mu, w if mu is not None else w[:, : self.hidden_size], self.hidden_size)
        return (out[..., : self.q_dim], out[..., self.q_dim: self.q_dim + self.kv_dim],
                out[..., self.q_dim + self.kv_dim:])


class _PackCache:
    """W_pack = [[Wq; Wk; Wv] | [Wmu_q; Wmu_k; Wmu_v]] ([N, 2H]), rebuilt when a weight changes."""

    def __init__(self):
        self.key = None
        self.w = None

    def get(self, m) -> torch.Tensor:
        ws = (m.q_proj.weight, m.k_proj.weight, m.v_proj.weight,
              m.mu_to_q.weight, m.mu_to_k.weight, m.mu_to_v.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws)
        if key != self.key:
            with torch.no_grad():
                self.w = torch.cat([torch.cat(ws[:3], 0), torch.cat(ws[3:], 0)], 1).contiguous()
            self.key = key
        return self.w


class ComplexityAttention(nn.Module):
    """GQA attention with mu guidance and QK normalisation; core/attention.py:33-181."""

    def __init__(self, hidden_size: int, num_attention_heads: int, num_key_value_heads: int,
                 max_position_embeddings: int = 2048, rope_theta: float = 10000.0,
                 attention_dropout: float = 0.0, use_qk_norm: bool = True):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_attention_heads
        self.num_kv_heads = num_key_value_heads
        self.head_dim = hidden_size // num_attention_heads
        self.num_kv_groups = num_attention_heads // num_key_value_heads
        if self.head_dim * num_attention_heads != hidden_size:
            raise ValueError("hidden_size must be divisible by num_attention_heads")
        if num_attention_heads % num_key_value_heads != 0:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        q_dim = num_attention_heads * self.head_dim
        kv_dim = num_key_value_heads * self.head_dim
        # Registration order matters for seeded init parity (one draw per Linear).
        self.q_proj = nn.Linear(hidden_size, q_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, kv_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, kv_dim, bias=False)
        self.o_proj = nn.Linear(q_dim, hidden_size, bias=False)
        self.mu_to_q = nn.Linear(hidden_size, q_dim, bias=False)
        self.mu_to_k = nn.Linear(hidden_size, kv_dim, bias=False)
        self.mu_to_v = nn.Linear(hidden_size, kv_dim, bias=False)
        self.use_qk_norm = use_qk_norm
        if use_qk_norm:
            self.q_norm = nn.RMSNorm(self.head_dim, eps=1e-6)
            self.k_norm = nn.RMSNorm(self.head_dim, eps=1e-6)
        self.rotary_emb = RotaryEmbedding(self.head_dim, max_seq_len=max_position_embeddings, theta=rope_theta)
        self.attention_dropout = attention_dropout
        self._cache = _PackCache()

    def project_qkv(self, hidden_states: torch.Tensor, mu_prev: Optional[torch.Tensor]) -> torch.Tensor:
        """Packed [.., Nq*D + 2*Nkv*D] projection through the gfx950 MFMA kernel."""
        w = self._cache.get(self)
        if mu_prev is None:
            w = w[:, : self.hidden_size]
        return mu_qkv_project(hidden_states, mu_prev, w, self.hidden_size)

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                past_key_value: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                use_cache: bool = False, mu_prev: Optional[torch.Tensor] = None):
        forward_only("ComplexityAttention", hidden_states, mu_prev, *self.parameters())
        B, S, _ = hidden_states.shape
        D = self.head_dim
        q_dim, kv_dim = self.num_heads * D, self.num_kv_heads * D
        qkv = self.project_qkv(hidden_states, mu_prev)
        q = qkv[..., :q_dim].view(B, S, self.num_heads, D).transpose(1, 2)
        k = qkv[..., q_dim:q_dim + kv_dim].view(B, S, self.num_kv_heads, D).transpose(1, 2)
        v = qkv[..., q_dim + kv_dim:].view(B, S, self.num_kv_heads, D).transpose(1, 2)
        if self.use_qk_norm:
            q = self.q_norm(q)
            k = self.k_norm(k)
        kv_seq_len = S + (past_key_value[0].shape[2] if past_key_value is not None else 0)
        cos, sin = self.rotary_emb(kv_seq_len)
        cos = cos.to(q.device, dtype=q.dtype)
        sin = sin.to(q.device, dtype=q.dtype)
        if past_key_value is not None:
            cos, sin = cos[kv_seq_len - S:], sin[kv_seq_len - S:]
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        if past_key_value is not None:
            k = torch.cat([past_key_value[0], k], dim=2)
            v = torch.cat([past_key_value[1], v], dim=2)
        new_kv = (k, v) if use_cache else None
        k = k.repeat_interleave(self.num_kv_groups, dim=1)
        v = v.repeat_interleave(self.num_kv_groups, dim=1)
        # Same SDPA call as the reference, including is_causal=(mask is None).
        attn = F.scaled_dot_product_attention(
            q, k, v, attn_mask=attention_mask,
            dropout_p=self.attention_dropout if self.training else 0.0,
            is_causal=attention_mask is None)
        attn = attn.transpose(1, 2).contiguous().view(B, S, -1)
        return self.o_proj(attn), new_kv


MuGuidedAttention = ComplexityAttention

__all__ = ["ComplexityAttention", "MuGuidedAttention", "FusedMuQKVProjection", "fused_mu_qkv_projection",
           "mu_qkv_project"]
