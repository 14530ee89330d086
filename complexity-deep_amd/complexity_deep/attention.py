"""GQA attention with the mu-guided QKV projection on the gfx950 kernel (piece 2).

Interfaces follow the reference:
  ComplexityAttention        core/attention.py:33-181 (constructor, parameters and
                             state_dict keys; exported also as MuGuidedAttention)
  fused_mu_qkv_projection    cuda/triton_mu_qkv.py:195-283 (weights [in, out])
  FusedMuQKVProjection       cuda/triton_mu_qkv.py:336-394

The projection is one MFMA contraction over K = 2H: [x | mu_prev] @ [W_x | W_mu]^T
with W_x = [Wq; Wk; Wv] and W_mu = [Wmu_q; Wmu_k; Wmu_v], the kernel switching weight
source at K = H.  The module keeps W_x and W_mu side by side in one [N, 2H] buffer
(row n is [W_x[n] | W_mu[n]], the layout of the reference's torch.cat(..., dim=1)) and
its six Linear weights are views of it, so nothing is concatenated per forward
(attention.py:122-124 concatenates every call) and every write to a weight, through
``.data`` or otherwise, reaches the kernel operand.  When x and mu also sit side by
side in one [T, 2H] buffer (the model writes them so), the projection is one plain
K = 2H contraction over single operands.  q, k and v are column slices of
the packed [T, Nq*D + 2*Nkv*D] output.

ComplexityAttention.forward goes one step further for head dims 32/64/128: the
per-head QK RMSNorm and RoPE (attention.py:138-155) run in the projection kernel's
epilogue (cdx_mu_qkv_rope_fwd), which writes q, k, v head-major, in fp32 up to one
final rounding.  The KV cache, GQA SDPA and o_proj stay PyTorch-ROCm ops in the
reference's order (attention.py:157-181).
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
    """Express a [..., H] tensor as rows base + r * ld; ld = 0 for one broadcast row.
    (Only the base pointer and ld are used: a contiguous tensor is returned as is.)"""
    if t.shape[-1] == H and t.is_contiguous():
        return t, H
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


def _weight_sources(w: torch.Tensor, w_mu: Optional[torch.Tensor], mu: Optional[torch.Tensor], H: int,
                    what: str) -> Tuple[int, Optional[int], int]:
    """(x-weight pointer, mu-weight pointer, common row stride) for the kernels.

    ``w`` is [N, >= H] (unit stride in K).  With ``w_mu`` None and a mu operand, ``w``
    is a packed [N, >= 2H] whose columns [H, 2H) are the mu weights; otherwise
    ``w_mu`` is [N, H] with the same row stride as ``w``."""
    if w.dim() != 2 or w.stride(-1) != 1 or w.shape[1] < H:
        raise ValueError(f"{what}: weight must be [N, >= {H}] with unit stride in K")
    ldw = w.stride(0) if w.shape[0] > 1 else w.shape[1]
    if mu is None:
        return w.data_ptr(), None, ldw
    if w_mu is None:
        if w.shape[1] < 2 * H:
            raise ValueError(f"{what}: a packed weight needs 2H = {2 * H} columns, got {w.shape[1]}")
        return w.data_ptr(), w.data_ptr() + H * w.element_size(), ldw
    if w_mu.dim() != 2 or w_mu.shape[0] != w.shape[0] or w_mu.shape[1] < H:
        raise ValueError(f"{what}: mu weight shape {tuple(w_mu.shape)} does not match {tuple(w.shape)}")
    ldm = w_mu.stride(0) if w_mu.shape[0] > 1 else ldw
    if w_mu.stride(-1) != 1 or ldm != ldw or w_mu.dtype != w.dtype or w_mu.device != w.device:
        raise ValueError(f"{what}: x and mu weights must share dtype, device and row stride")
    return w.data_ptr(), w_mu.data_ptr(), ldw


def mu_qkv_project(x: torch.Tensor, mu: Optional[torch.Tensor], w_pack: torch.Tensor,
                   H: int, w_mu: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[..., N] = [x | mu] @ [w_x | w_mu]^T (cdx_mu_qkv_fwd).

    w_pack is [N, 2H] (x weights then mu weights) or, with ``w_mu`` given, the x
    weights [N, H] alone; with mu=None only its first H columns are read."""
    nat.require_device(x, mu, w_pack, w_mu, what="mu_qkv_project")
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
    wx_ptr, wmu_ptr, ldw = _weight_sources(w_pack, w_mu, mu2, H, "mu_qkv_project")
    out = torch.empty(*lead, N, dtype=x.dtype, device=x.device)
    with nat.launch_region("mu_qkv", x.device, M=M, H=H, N=N, mu=mu2 is not None):
        nat.check(nat.lib().cdx_mu_qkv_fwd(x2.data_ptr(), ldx, nat.ptr(mu2), ldmu, wx_ptr, wmu_ptr, ldw,
                                           M, H, N, out.data_ptr(), N, nat.stream_of(x)), "cdx_mu_qkv_fwd")
    return out


def vt_ld_for(S: int) -> int:
    """Row length of the transposed V layout (keys padded to a multiple of 64)."""
    return (S + 63) // 64 * 64


def vt_columns(S: int, device=None) -> torch.Tensor:
    """Column of each token s in the transposed V layout: inside every group of 16 the
    middle two groups of 4 swap places (the key order of the attention kernel's
    P fragments)."""
    s = torch.arange(S, device=device)
    q = (s // 4) % 4
    qs = torch.where(q == 1, 2, torch.where(q == 2, 1, q))
    return (s // 16) * 16 + 4 * qs + s % 4


def to_vt_layout(v: torch.Tensor) -> torch.Tensor:
    """[B, h, S, D] -> the transposed layout [B, h, D, vt_ld] cdx_attention_fwd reads
    (padding columns zero).  The model never calls this: the projection kernel writes
    V in this layout directly."""
    B, h, S, D = v.shape
    vt = torch.zeros(B, h, D, vt_ld_for(S), dtype=v.dtype, device=v.device)
    vt[..., vt_columns(S, v.device)] = v.transpose(-1, -2)
    return vt


def mu_qkv_rope(x: torch.Tensor, mu: Optional[torch.Tensor], w_pack: torch.Tensor, H: int, nq: int,
                nkv: int, hd: int, q_norm_w: Optional[torch.Tensor], k_norm_w: Optional[torch.Tensor],
                eps: float, cos_sin: torch.Tensor, pos0: int = 0, v_transposed: bool = False,
                w_mu: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(q, k, v) head-major [B, heads, S, hd] from x [B, S, H] (cdx_mu_qkv_rope_fwd):
    the mu-QKV projection with per-head RMSNorm of q and k (weights q_norm_w /
    k_norm_w, None = no norm) and RoPE at positions pos0 .. pos0+S-1 fused into one
    kernel.  cos_sin is the fp32 [n_pos, hd/2, 2] table of RotaryEmbedding.  Weights
    as in mu_qkv_project.  v_transposed=True returns V in the layout of to_vt_layout
    instead.  A mu that is one row broadcast to every token (layer 0's mu_init.expand)
    goes through cdx_mu_qkv_rope_bcast_fwd, which folds its product with W_mu into one
    64-column K block (K = H + 64 instead of 2H)."""
    nat.require_device(x, mu, w_pack, w_mu, q_norm_w, k_norm_w, what="mu_qkv_rope")
    B, S, _ = x.shape
    x2, ldx = _rows_view(x, H)
    if ldx == 0:
        x2, ldx = x.contiguous(), H
    if mu is not None:
        mu = mu.expand(B, S, H) if mu.shape[:-1] != (B, S) else mu
        mu2, ldmu = _rows_view(mu, H)
    else:
        mu2, ldmu = None, 0
    wx_ptr, wmu_ptr, ldw = _weight_sources(w_pack, w_mu, mu2, H, "mu_qkv_rope")
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous() or cos_sin.device != x.device:
        raise ValueError("mu_qkv_rope: cos_sin must be a contiguous fp32 table on the input's device")
    if (q_norm_w is None) != (k_norm_w is None):
        raise ValueError("mu_qkv_rope: pass both QK norm weights or neither")
    if q_norm_w is not None:
        q_norm_w = q_norm_w.to(x.dtype).contiguous()
        k_norm_w = k_norm_w.to(x.dtype).contiguous()
    q = torch.empty(B, nq, S, hd, dtype=x.dtype, device=x.device)
    k = torch.empty(B, nkv, S, hd, dtype=x.dtype, device=x.device)
    if v_transposed:
        vt_ld = vt_ld_for(S)
        v = torch.empty(B, nkv, hd, vt_ld, dtype=x.dtype, device=x.device)
        if vt_ld > S:
            # Columns of the key positions S .. vt_ld-1 are masked but must be finite.
            # The order inside a 16-group moves some of them below S, so clear from the
            # last partial group on; the kernel then fills the columns of tokens < S.
            v[..., (S // 16) * 16:].zero_()
    else:
        vt_ld = 0
        v = torch.empty(B, nkv, S, hd, dtype=x.dtype, device=x.device)
    N = (nq + 2 * nkv) * hd
    esz = x.element_size()
    if (mu2 is not None and ldmu != 0 and ldx == ldmu and ldx >= 2 * H and ldw >= 2 * H
            and mu2.data_ptr() == x2.data_ptr() + H * esz and wmu_ptr == wx_ptr + H * esz):
        # x and mu side by side in one buffer, and W_x and W_mu likewise: one K = 2H
        # contraction over single operands (the same sums in the same order).
        with nat.launch_region("mu_qkv", x.device, M=B * S, H=H, N=N, mu=True):
            nat.check(nat.lib().cdx_mu_qkv_rope_fwd(
                x2.data_ptr(), ldx, None, 0, wx_ptr, None, ldw, B, S, 2 * H, nq, nkv, hd,
                nat.ptr(q_norm_w), nat.ptr(k_norm_w), float(eps), cos_sin.data_ptr(), cos_sin.shape[0], pos0,
                q.data_ptr(), k.data_ptr(), v.data_ptr(), vt_ld, nat.stream_of(x)), "cdx_mu_qkv_rope_fwd")
        return q, k, v
    if mu2 is not None and ldmu == 0 and H > 64:
        # One broadcast mu row (layer 0's mu_init.expand): its product with W_mu is one
        # row, folded into a 64-column K block (K = H + 64 instead of 2H).
        work = torch.empty(N * ldw + 64, dtype=x.dtype, device=x.device)
        with nat.launch_region("mu_qkv_bcast", x.device, M=B * S, H=H, N=N):
            nat.check(nat.lib().cdx_mu_qkv_rope_bcast_fwd(
                x2.data_ptr(), ldx, mu2.data_ptr(), wx_ptr, wmu_ptr, ldw, B, S, H, nq, nkv, hd,
                nat.ptr(q_norm_w), nat.ptr(k_norm_w), float(eps), cos_sin.data_ptr(), cos_sin.shape[0], pos0,
                q.data_ptr(), k.data_ptr(), v.data_ptr(), vt_ld, work.data_ptr(), nat.stream_of(x)),
                "cdx_mu_qkv_rope_bcast_fwd")
        return q, k, v
    with nat.launch_region("mu_qkv", x.device, M=B * S, H=H, N=N, mu=mu2 is not None):
        nat.check(nat.lib().cdx_mu_qkv_rope_fwd(
            x2.data_ptr(), ldx, nat.ptr(mu2), ldmu, wx_ptr, wmu_ptr, ldw, B, S, H, nq, nkv, hd,
            nat.ptr(q_norm_w), nat.ptr(k_norm_w), float(eps), cos_sin.data_ptr(), cos_sin.shape[0], pos0,
            q.data_ptr(), k.data_ptr(), v.data_ptr(), vt_ld, nat.stream_of(x)), "cdx_mu_qkv_rope_fwd")
    return q, k, v


def causal_attention(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, scale: Optional[float] = None
                     ) -> torch.Tensor:
    """softmax(q k^T * scale, top-left causal) v for GQA heads (cdx_attention_fwd).

    q [B, nq, S, D], k [B, nkv, S, D], vt = V in the transposed layout
    [B, nkv, D, vt_ld] (to_vt_layout / mu_qkv_rope(v_transposed=True)).  Returns the
    merged [B, S, nq * D] that o_proj consumes.  Equals
    F.scaled_dot_product_attention(q, k.repeat_interleave(nq // nkv, 1),
    v.repeat_interleave(nq // nkv, 1), is_causal=True) (core/attention.py:163-181)."""
    nat.require_device(q, k, vt, what="causal_attention")
    B, nq, S, D = q.shape
    nkv = k.shape[1]
    if k.shape != (B, nkv, S, D) or vt.shape[:3] != (B, nkv, D) or vt.shape[3] < S:
        raise ValueError("causal_attention: q/k/vt shapes do not match")
    if not (q.is_contiguous() and k.is_contiguous() and vt.is_contiguous()):
        raise ValueError("causal_attention: q, k and vt must be contiguous")
    scale = D ** -0.5 if scale is None else scale
    out = torch.empty(B, S, nq * D, dtype=q.dtype, device=q.device)
    with nat.launch_region("attention", q.device, B=B, S=S, nq=nq, D=D):
        nat.check(nat.lib().cdx_attention_fwd(q.data_ptr(), k.data_ptr(), vt.data_ptr(), B, S, nq, nkv, D,
                                              vt.shape[3], float(scale), out.data_ptr(), nat.stream_of(q)),
                  "cdx_attention_fwd")
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
        self._qkv_w = QKVWeights()

    def forward(self, x: torch.Tensor, mu: Optional[torch.Tensor] = None):
        forward_only("FusedMuQKVProjection", x, mu, module=self)
        w_x, w_mu = self._qkv_w.get(self)
        out = mu_qkv_project(x, mu, w_x, self.hidden_size, w_mu=w_mu)
        return (out[..., : self.q_dim], out[..., self.q_dim: self.q_dim + self.kv_dim],
                out[..., self.q_dim + self.kv_dim:])


class QKVWeights:
    """The kernel operands W_x = [Wq; Wk; Wv] and W_mu = [Wmu_q; Wmu_k; Wmu_v] of one
    module, side by side in one [N, 2H] buffer (row n = [W_x[n] | W_mu[n]], the
    reference's torch.cat([q_proj.weight, mu_to_q.weight], dim=1) for each of q, k, v)
    whose column halves the six Linear weights are views of.

    A write to a weight (in place, through ``.data``, by load_state_dict) therefore
    lands in the operand the kernel reads; nothing is cached that could go stale.
    When a weight is no longer its view (the module was moved or cast, a Parameter was
    replaced), ``get`` copies the current weights into a new buffer and re-points them
    at it.  The buffer is made outside inference mode, so that the weights stay
    writable after a forward run under torch.inference_mode()."""

    def __init__(self):
        self.buf: Optional[torch.Tensor] = None
        self.ptrs = None

    @staticmethod
    def _linears(m):
        return (m.q_proj, m.k_proj, m.v_proj, m.mu_to_q, m.mu_to_k, m.mu_to_v)

    def get(self, m) -> Tuple[torch.Tensor, torch.Tensor]:
        ws = [lin.weight for lin in self._linears(m)]
        if self.buf is None or [w.data_ptr() for w in ws] != self.ptrs:
            self._bind(ws, m.hidden_size)
        H = m.hidden_size
        return self.buf[:, :H], self.buf[:, H:]

    def _bind(self, ws, H: int) -> None:
        dt, dev = ws[0].dtype, ws[0].device
        if any(w.dtype != dt or w.device != dev or w.dim() != 2 or w.shape[1] != H for w in ws):
            raise ValueError("ComplexityAttention: the q/k/v and mu_to_q/k/v weights must share one dtype "
                             f"and device and be [out, {H}]")
        xs, mus = ws[:3], ws[3:]
        if [w.shape[0] for w in xs] != [w.shape[0] for w in mus]:
            raise ValueError("ComplexityAttention: mu_to_q/k/v must have the shapes of q/k/v_proj")
        N = sum(w.shape[0] for w in xs)
        with torch.inference_mode(False), torch.no_grad():
            buf = torch.empty(N, 2 * H, dtype=dt, device=dev)
            r = 0
            for wx, wm in zip(xs, mus):
                n = wx.shape[0]
                buf[r:r + n, :H].copy_(wx)
                buf[r:r + n, H:].copy_(wm)
                wx.data = buf[r:r + n, :H]
                wm.data = buf[r:r + n, H:]
                r += n
        self.buf = buf
        self.ptrs = [w.data_ptr() for w in ws]


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
        self._qkv_w = QKVWeights()

    def qkv_weights(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(W_x, W_mu), each [Nq*D + 2*Nkv*D, H]: the two column halves of the [N, 2H]
        buffer the six projection weights are views of, i.e. exactly what the kernels read."""
        return self._qkv_w.get(self)

    def project_qkv(self, hidden_states: torch.Tensor, mu_prev: Optional[torch.Tensor]) -> torch.Tensor:
        """Packed [.., Nq*D + 2*Nkv*D] projection through the gfx950 MFMA kernel."""
        w_x, w_mu = self.qkv_weights()
        return mu_qkv_project(hidden_states, mu_prev, w_x, self.hidden_size, w_mu=w_mu)

    @property
    def fused_prologue(self) -> bool:
        """Whether QK-norm + RoPE run inside the projection kernel (cdx_mu_qkv_rope_fwd
        handles head dims 32, 64 and 128 and H a multiple of 64)."""
        return self.head_dim in (32, 64, 128) and self.hidden_size % 64 == 0

    def _out_proj(self, attn: torch.Tensor, residual: Optional[torch.Tensor]) -> torch.Tensor:
        """o_proj(attn), or with ``residual``: residual + o_proj(attn) written into residual
        (one GEMM with beta = 1, the block's residual add of core/layer.py:174).  o_proj is
        not one of the path's three pieces; hipBLASLt's beta = 1 GEMM ran the 1B forward
        0.8% faster than the tile engine's o_proj + residual kernel (linear_residual_), so
        the model keeps it."""
        if residual is None:
            return self.o_proj(attn)
        if residual.shape[:-1] != attn.shape[:-1] or not residual.is_contiguous():
            raise ValueError("ComplexityAttention: residual must be contiguous and match the input rows")
        residual.view(-1, residual.shape[-1]).addmm_(attn.reshape(-1, attn.shape[-1]), self.o_proj.weight.t())
        return residual

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                past_key_value: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                use_cache: bool = False, mu_prev: Optional[torch.Tensor] = None,
                residual: Optional[torch.Tensor] = None):
        """Returns (o_proj(attention), new_kv); with ``residual`` (the block input h,
        contiguous) the output is added to it in place and residual is returned."""
        forward_only("ComplexityAttention", hidden_states, mu_prev, residual, module=self)
        B, S, _ = hidden_states.shape
        D = self.head_dim
        past_len = past_key_value[0].shape[2] if past_key_value is not None else 0
        if self.fused_prologue and attention_mask is None and past_key_value is None and not use_cache \
                and not (self.training and self.attention_dropout > 0):
            # Whole attention on the kernels: fused projection (V written transposed) and
            # the causal GQA kernel, whose output is already merged over heads.
            w_x, w_mu = self.qkv_weights()
            table = self.rotary_emb.cos_sin_table(S, hidden_states.device)
            qn = (self.q_norm.weight, self.k_norm.weight) if self.use_qk_norm else (None, None)
            eps = self.q_norm.eps if self.use_qk_norm else 0.0
            q, k, vt = mu_qkv_rope(hidden_states, mu_prev, w_x, self.hidden_size, self.num_heads,
                                   self.num_kv_heads, D, qn[0], qn[1], eps, table, 0, v_transposed=True,
                                   w_mu=w_mu)
            return self._out_proj(causal_attention(q, k, vt), residual), None
        if self.fused_prologue:
            # Projection, head split, QK RMSNorm and RoPE in one kernel (attention.py:120-155).
            w_x, w_mu = self.qkv_weights()
            table = self.rotary_emb.cos_sin_table(past_len + S, hidden_states.device)
            qn = (self.q_norm.weight, self.k_norm.weight) if self.use_qk_norm else (None, None)
            eps = self.q_norm.eps if self.use_qk_norm else 0.0
            q, k, v = mu_qkv_rope(hidden_states, mu_prev, w_x, self.hidden_size, self.num_heads,
                                  self.num_kv_heads, D, qn[0], qn[1], eps, table, past_len, w_mu=w_mu)
        else:
            q_dim, kv_dim = self.num_heads * D, self.num_kv_heads * D
            qkv = self.project_qkv(hidden_states, mu_prev)
            q = qkv[..., :q_dim].view(B, S, self.num_heads, D).transpose(1, 2)
            k = qkv[..., q_dim:q_dim + kv_dim].view(B, S, self.num_kv_heads, D).transpose(1, 2)
            v = qkv[..., q_dim + kv_dim:].view(B, S, self.num_kv_heads, D).transpose(1, 2)
            if self.use_qk_norm:
                q = self.q_norm(q)
                k = self.k_norm(k)
            kv_seq_len = S + past_len
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
        return self._out_proj(attn, residual), new_kv


MuGuidedAttention = ComplexityAttention

__all__ = ["ComplexityAttention", "MuGuidedAttention", "FusedMuQKVProjection", "fused_mu_qkv_projection",
           "mu_qkv_project", "mu_qkv_rope", "causal_attention", "to_vt_layout", "vt_columns", "QKVWeights"]
