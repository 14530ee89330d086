"""Token-ID-routed MoE with the shared lexical expert on the gfx950 kernels (piece 1).

Interfaces follow the reference:
  TokenRoutedMLP            core/token_routed_mlp.py:28-194 (same constructor,
                            parameters, buffer and state_dict keys)
  sort_tokens_by_expert     cuda/triton_token_routed.py:37-61
  cggr_grouped_gemm         cuda/triton_token_routed.py:197-231 (and the PyTorch
                            grouped_gemm_pytorch of :64-86)

The forward is: route plan (cdx_route_plan: expert lookup, counts, offsets, stable
permutation) -> cdx_moe_swiglu_fwd (gathered gate/up GEMM with SwiGLU epilogue,
then the down GEMM whose epilogue scatters rows back to token order).  The shared
expert's weights are packed next to every routed expert's, so one fp32 accumulator
sums shared + routed before the single bf16 rounding.  No host synchronisation
happens anywhere in the forward.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _native as nat
from ._grad import forward_only


# ---------------------------------------------------------------------------
# routing plan
# ---------------------------------------------------------------------------

@dataclass
class RoutePlan:
    """Device routing plan for T tokens over E experts (all int32)."""
    expert_id: torch.Tensor  # [T]
    perm: torch.Tensor       # [T] sorted position -> token index
    inv_perm: torch.Tensor   # [T] token index -> sorted position
    counts: torch.Tensor     # [E]
    offsets: torch.Tensor    # [E + 1]
    num_experts: int

    @property
    def num_tokens(self) -> int:
        return self.perm.shape[0]


def route_plan(ids: torch.Tensor, token_map: Optional[torch.Tensor], num_experts: int) -> RoutePlan:
    """Bit-exact routing plan on the GPU (cdx_route_plan).

    ids: int64 token ids (any shape) looked up through ``token_map`` (int64 [V]) after
    clamping to [0, V-1]; with token_map=None ``ids`` are expert ids already."""
    nat.require_device(ids, token_map, dtype=None, what="route_plan")
    ids = ids.reshape(-1)
    if ids.dtype != torch.int64:
        ids = ids.to(torch.int64)
    ids = ids if ids.is_contiguous() else ids.contiguous()
    V = 0
    if token_map is not None:
        if token_map.dtype != torch.int64:
            token_map = token_map.to(torch.int64)
        token_map = token_map.contiguous()
        V = token_map.shape[0]
    T = ids.shape[0]
    dev = ids.device
    i32 = dict(dtype=torch.int32, device=dev)
    expert_id = torch.empty(T, **i32)
    perm = torch.empty(T, **i32)
    inv_perm = torch.empty(T, **i32)
    counts = torch.empty(num_experts, **i32)
    offsets = torch.empty(num_experts + 1, **i32)
    lib = nat.lib()
    ws_bytes = lib.cdx_route_workspace_bytes(T, num_experts)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    with nat.launch_region("route_plan", dev, T=T, E=num_experts, V=V):
        nat.check(lib.cdx_route_plan(ids.data_ptr(), T, nat.ptr(token_map), V, num_experts,
                                     expert_id.data_ptr(), perm.data_ptr(), inv_perm.data_ptr(),
                                     counts.data_ptr(), offsets.data_ptr(), ws.data_ptr(), ws_bytes,
                                     nat.stream_of(ids)), "cdx_route_plan")
    return RoutePlan(expert_id, perm, inv_perm, counts, offsets, num_experts)


def permute_rows(x: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """out[i] = x[perm[i]] for a 2-D tensor (cdx_permute_rows)."""
    x = x.contiguous()
    out = torch.empty_like(x)
    nat.check(nat.lib().cdx_permute_rows(x.data_ptr(), perm.data_ptr(), x.shape[0],
                                         x.shape[1] * x.element_size(), out.data_ptr(),
                                         nat.stream_of(x)), "cdx_permute_rows")
    return out


def unpermute_rows(x: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """out[perm[i]] = x[i] for a 2-D tensor (cdx_unpermute_rows)."""
    x = x.contiguous()
    out = torch.empty_like(x)
    nat.check(nat.lib().cdx_unpermute_rows(x.data_ptr(), perm.data_ptr(), x.shape[0],
                                           x.shape[1] * x.element_size(), out.data_ptr(),
                                           nat.stream_of(x)), "cdx_unpermute_rows")
    return out


def sort_tokens_by_expert(tokens: torch.Tensor, expert_ids: torch.Tensor, num_experts: int
                          ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(sorted_tokens, sorted_indices, expert_offsets [E+1], expert_counts [E]) with int64
    index outputs; cuda/triton_token_routed.py:37-61.  The order inside an expert is the
    original token order (a stable sort)."""
    nat.require_device(tokens, expert_ids, dtype=None, what="sort_tokens_by_expert")
    plan = route_plan(expert_ids, None, num_experts)
    rows = tokens.reshape(tokens.shape[0], -1)
    if (rows.shape[1] * rows.element_size()) % 16 != 0:
        raise ValueError("sort_tokens_by_expert: token rows must be a multiple of 16 bytes")
    sorted_tokens = permute_rows(rows, plan.perm).view_as(tokens)
    return sorted_tokens, plan.perm.to(torch.int64), plan.offsets.to(torch.int64), plan.counts.to(torch.int64)


def cggr_grouped_gemm(sorted_tokens: torch.Tensor, expert_weights: torch.Tensor,
                      expert_offsets: torch.Tensor) -> torch.Tensor:
    """out[o_e:o_{e+1}] = sorted_tokens[o_e:o_{e+1}] @ expert_weights[e];
    cuda/triton_token_routed.py:197-231.  expert_weights is [E, in, out] (bf16)."""
    forward_only("cggr_grouped_gemm", sorted_tokens, expert_weights)
    nat.require_device(sorted_tokens, expert_weights, what="cggr_grouped_gemm")
    T, K = sorted_tokens.shape
    E, K2, N = expert_weights.shape
    if K2 != K:
        raise ValueError(f"cggr_grouped_gemm: in_dim mismatch {K} vs {K2}")
    a = sorted_tokens.contiguous()
    w_t = expert_weights.transpose(1, 2).contiguous()  # [E, N, K], K-contiguous
    offs = expert_offsets.to(device=a.device, dtype=torch.int32).contiguous()
    out = torch.empty(T, N, dtype=a.dtype, device=a.device)
    nat.check(nat.lib().cdx_grouped_gemm_fwd(a.data_ptr(), T, K, N, E, offs.data_ptr(), w_t.data_ptr(),
                                             out.data_ptr(), nat.stream_of(a)), "cdx_grouped_gemm_fwd")
    return out


cggr_grouped_gemm_triton = cggr_grouped_gemm
grouped_gemm = cggr_grouped_gemm


# ---------------------------------------------------------------------------
# weight packing (layouts documented in include/cdx.h, cdx_moe_swiglu_fwd)
# ---------------------------------------------------------------------------

def padded_width(ie: int) -> int:
    return (ie + 63) // 64 * 64


def _interleave_gate_up(gate_rows: torch.Tensor, up_rows: torch.Tensor, P: int) -> torch.Tensor:
    """[Ie, H] gate and up rows -> [2P, H]: groups of 32 gate rows then the matching 32 up rows."""
    ie, H = gate_rows.shape
    g = torch.zeros(P, H, dtype=gate_rows.dtype, device=gate_rows.device)
    u = torch.zeros_like(g)
    g[:ie] = gate_rows
    u[:ie] = up_rows
    return torch.stack([g.view(P // 32, 32, H), u.view(P // 32, 32, H)], dim=1).reshape(2 * P, H)


def pack_moe_weights(gate_w: torch.Tensor, up_w: torch.Tensor, down_w: torch.Tensor,
                     shared_gate: Optional[torch.Tensor], shared_up: Optional[torch.Tensor],
                     shared_down: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Build (w_gu [E, S*2P, H], w_down [E, H, S*P]) from the module's parameters.

    gate_w/up_w [E, H, Ie] and down_w [E, Ie, H] are [in, out]; shared_* are
    nn.Linear weights [out, in]."""
    E, H, ie = gate_w.shape
    P = padded_width(ie)
    has_shared = shared_gate is not None
    blocks_gu, blocks_dn = [], []
    with torch.no_grad():
        if has_shared:
            sg = _interleave_gate_up(shared_gate, shared_up, P)  # [2P, H]
            sd = torch.zeros(H, P, dtype=down_w.dtype, device=down_w.device)
            sd[:, :ie] = shared_down
        for e in range(E):
            rg = _interleave_gate_up(gate_w[e].t(), up_w[e].t(), P)
            rd = torch.zeros(H, P, dtype=down_w.dtype, device=down_w.device)
            rd[:, :ie] = down_w[e].t()
            blocks_gu.append(torch.cat([sg, rg], 0) if has_shared else rg)
            blocks_dn.append(torch.cat([sd, rd], 1) if has_shared else rd)
        w_gu = torch.stack(blocks_gu).contiguous()
        w_down = torch.stack(blocks_dn).contiguous()
    return w_gu, w_down


def moe_swiglu(x2d: torch.Tensor, plan: RoutePlan, w_gu: torch.Tensor, w_down: torch.Tensor,
               ie: int, has_shared: bool, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[T, H] = shared(x) + expert_e(x) through cdx_moe_swiglu_fwd.

    With ``residual`` ([T, H], contiguous) the rows are added to it in place instead
    (cdx_moe_swiglu_residual_fwd) and ``residual`` is returned."""
    T, H = x2d.shape
    E = plan.num_experts
    P = padded_width(ie)
    S = 2 if has_shared else 1
    if w_gu.shape != (E, 2 * S * P, H) or w_down.shape != (E, H, S * P):
        raise ValueError("moe_swiglu: packed weight shapes do not match the plan/hidden size")
    if residual is not None:
        nat.require_device(residual, x2d, what="moe_swiglu residual")
        if residual.shape != x2d.shape or not residual.is_contiguous():
            raise ValueError(f"moe_swiglu: residual must be a contiguous {tuple(x2d.shape)} tensor")
        out, fn, fname = residual, nat.lib().cdx_moe_swiglu_residual_fwd, "cdx_moe_swiglu_residual_fwd"
    else:
        out, fn, fname = torch.empty_like(x2d), nat.lib().cdx_moe_swiglu_fwd, "cdx_moe_swiglu_fwd"
    inter = torch.empty(T, S * P, dtype=x2d.dtype, device=x2d.device)
    with nat.launch_region("moe_swiglu", x2d.device, T=T, H=H, Ie=ie, E=E, shared=has_shared):
        nat.check(fn(x2d.data_ptr(), T, H, ie, E, int(has_shared), plan.perm.data_ptr(), plan.offsets.data_ptr(),
                     w_gu.data_ptr(), w_down.data_ptr(), inter.data_ptr(), out.data_ptr(), nat.stream_of(x2d)),
                  fname)
    return out


# ---------------------------------------------------------------------------
# module
# ---------------------------------------------------------------------------

class TokenRoutedMLP(nn.Module):
    """Deterministic token-ID-routed MoE with a shared lexical expert.

    Same constructor, parameters ([E,H,Ie] gate/up, [E,Ie,H] down, nn.Linear shared
    expert), ``token_to_expert`` buffer and state_dict keys as
    core/token_routed_mlp.py:43-81."""

    def __init__(self, hidden_size: int, intermediate_size: int, num_experts: int = 4,
                 vocab_size: int = 100_000, shared_expert: bool = True,
                 token_frequencies: Optional[torch.Tensor] = None):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_experts = num_experts
        self.vocab_size = vocab_size
        self.expert_intermediate_size = intermediate_size // num_experts
        ie = self.expert_intermediate_size
        # Three draws from the default generator, in this order (seeded-init parity).
        self.gate_proj_w = nn.Parameter(torch.randn(num_experts, hidden_size, ie) * 0.02)
        self.up_proj_w = nn.Parameter(torch.randn(num_experts, hidden_size, ie) * 0.02)
        self.down_proj_w = nn.Parameter(torch.randn(num_experts, ie, hidden_size) * 0.02)
        self.use_shared_expert = shared_expert
        if shared_expert:
            self.shared_gate = nn.Linear(hidden_size, ie, bias=False)
            self.shared_up = nn.Linear(hidden_size, ie, bias=False)
            self.shared_down = nn.Linear(ie, hidden_size, bias=False)
        self.register_buffer("token_to_expert",
                             self._build_token_mapping(vocab_size, num_experts, token_frequencies))
        self._pack_key = None
        self._packed = None

    @staticmethod
    def _build_token_mapping(vocab_size: int, num_experts: int,
                             token_frequencies: Optional[torch.Tensor]) -> torch.Tensor:
        """Greedy Zipf bin-packing (token_routed_mlp.py:87-119) through the native
        builder cdx_binpack_map: tokens in descending frequency (ties: lower id
        first), each to the least-loaded expert (ties: lowest index), loads
        accumulated in double.  Without frequencies: token_id % num_experts."""
        if token_frequencies is None:
            return torch.arange(vocab_size, dtype=torch.long) % num_experts
        freq = torch.as_tensor(token_frequencies).detach().to("cpu", torch.float32).contiguous()
        if freq.shape != (vocab_size,):
            raise ValueError(f"token_frequencies has shape {tuple(freq.shape)}, expected ({vocab_size},)")
        mapping = torch.empty(vocab_size, dtype=torch.long)
        nat.check(nat.lib().cdx_binpack_map(freq.data_ptr(), vocab_size, num_experts, mapping.data_ptr()),
                  "cdx_binpack_map")
        return mapping

    def packed_weights(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Kernel-layout weights, rebuilt only when a parameter changes (never saved)."""
        params = [self.gate_proj_w, self.up_proj_w, self.down_proj_w]
        if self.use_shared_expert:
            params += [self.shared_gate.weight, self.shared_up.weight, self.shared_down.weight]
        key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in params)
        if key != self._pack_key:
            sh = (self.shared_gate.weight, self.shared_up.weight, self.shared_down.weight) \
                if self.use_shared_expert else (None, None, None)
            self._packed = pack_moe_weights(self.gate_proj_w.detach(), self.up_proj_w.detach(),
                                            self.down_proj_w.detach(), *[None if t is None else t.detach() for t in sh])
            self._pack_key = key
        return self._packed

    def plan(self, token_ids: torch.Tensor) -> RoutePlan:
        return route_plan(token_ids, self.token_to_expert, self.num_experts)

    def forward(self, hidden_states: torch.Tensor, token_ids: Optional[torch.Tensor] = None,
                route: Optional[RoutePlan] = None, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """[B, S, H] -> [B, S, H] = SharedMLP(x) + Expert_{map[token_id]}(x).

        ``route`` lets the caller pass a plan computed once for several layers that
        share token ids and map (ComplexityModel does this).  ``residual`` (same shape,
        contiguous) receives residual + MLP(x) in place and is returned: the block's
        residual add (core/layer.py:183) fused into the down pass."""
        forward_only("TokenRoutedMLP", hidden_states, residual, *self.parameters())
        nat.require_device(hidden_states, what="TokenRoutedMLP")
        shape = hidden_states.shape
        H = shape[-1]
        x2d = hidden_states.reshape(-1, H)
        x2d = x2d if x2d.is_contiguous() else x2d.contiguous()
        if token_ids is None and route is None:
            out = self._forward_all_experts(x2d).view(shape)
            return out if residual is None else residual.add_(out)
        if route is None:
            route = self.plan(token_ids)
        if route.num_tokens != x2d.shape[0]:
            raise ValueError(f"TokenRoutedMLP: plan has {route.num_tokens} tokens, input has {x2d.shape[0]}")
        w_gu, w_down = self.packed_weights()
        r2d = None
        if residual is not None:
            if residual.shape != shape or not residual.is_contiguous():
                raise ValueError("TokenRoutedMLP: residual must be a contiguous tensor shaped like the input")
            r2d = residual.view(-1, H)
        out = moe_swiglu(x2d, route, w_gu, w_down, self.expert_intermediate_size, self.use_shared_expert,
                         residual=r2d)
        return out.view(shape)

    def _forward_all_experts(self, x2d: torch.Tensor) -> torch.Tensor:
        """token_ids=None: mean over all experts plus the shared expert
        (token_routed_mlp.py:180-194).  Computed as one dense SwiGLU of width (E+1)*P
        whose routed down-projection rows are scaled by 1/E."""
        key = ("all",) + tuple((p.data_ptr(), p._version) for p in self.parameters())
        if getattr(self, "_all_key", None) != key:
            E = self.num_experts
            sh = (self.shared_gate.weight, self.shared_up.weight, self.shared_down.weight) \
                if self.use_shared_expert else None
            with torch.no_grad():
                gate = torch.cat(([sh[0].t()] if sh else []) + [self.gate_proj_w[e] for e in range(E)], 1)
                up = torch.cat(([sh[1].t()] if sh else []) + [self.up_proj_w[e] for e in range(E)], 1)
                down = torch.cat(([sh[2].t()] if sh else []) + [self.down_proj_w[e] / E for e in range(E)], 0)
                self._all_packed = pack_moe_weights(gate.unsqueeze(0), up.unsqueeze(0), down.unsqueeze(0),
                                                    None, None, None)
            self._all_width = gate.shape[1]
            self._all_key = key
        T = x2d.shape[0]
        plan = RoutePlan(expert_id=torch.zeros(T, dtype=torch.int32, device=x2d.device),
                         perm=torch.arange(T, dtype=torch.int32, device=x2d.device),
                         inv_perm=torch.arange(T, dtype=torch.int32, device=x2d.device),
                         counts=torch.tensor([T], dtype=torch.int32, device=x2d.device),
                         offsets=torch.tensor([0, T], dtype=torch.int32, device=x2d.device),
                         num_experts=1)
        w_gu, w_down = self._all_packed
        return moe_swiglu(x2d, plan, w_gu, w_down, self._all_width, False)
