"""Token-ID-routed MoE with the shared lexical expert on the gfx950 kernels (piece 1).

Interfaces follow the reference:
  TokenRoutedMLP              core/token_routed_mlp.py:28-194 (same constructor,
                              parameters, buffer and state_dict keys)
  sort_tokens_by_expert       cuda/triton_token_routed.py:37-61
  sort_tokens_by_expert_fast  cuda/persistent_cggr.py:318-352
  cggr_grouped_gemm           cuda/triton_token_routed.py:197-231 (also under the
                              names grouped_gemm_pytorch, :64-86, and
                              persistent_cggr_gemm, cuda/persistent_cggr.py:355-410)
  persistent_swiglu_cggr      cuda/persistent_cggr.py:479-530
  fused_swiglu_triton         cuda/triton_token_routed.py:234-257
  fused_swiglu_simple         cuda/persistent_cggr.py:450-476

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


def _aligned_rows(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned base (the kernels' DMA needs both)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def permute_rows(x: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """out[i] = x[perm[i]] for a 2-D tensor (cdx_permute_rows)."""
    x = _aligned_rows(x)
    out = torch.empty_like(x)
    rb = x.shape[1] * x.element_size()
    with nat.launch_region("permute_rows", x.device, T=x.shape[0], row_bytes=rb):
        nat.check(nat.lib().cdx_permute_rows(x.data_ptr(), perm.data_ptr(), x.shape[0], rb, out.data_ptr(),
                                             nat.stream_of(x)), "cdx_permute_rows")
    return out


def unpermute_rows(x: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """out[perm[i]] = x[i] for a 2-D tensor (cdx_unpermute_rows)."""
    x = _aligned_rows(x)
    out = torch.empty_like(x)
    rb = x.shape[1] * x.element_size()
    with nat.launch_region("unpermute_rows", x.device, T=x.shape[0], row_bytes=rb):
        nat.check(nat.lib().cdx_unpermute_rows(x.data_ptr(), perm.data_ptr(), x.shape[0], rb, out.data_ptr(),
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


def sort_tokens_by_expert_fast(token_ids: torch.Tensor, expert_mapping: torch.Tensor, num_experts: int
                               ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(sorted_indices, expert_offsets [E+1], expert_counts [E]), all int64, of the token
    ids routed through ``expert_mapping`` (ids clamped to the vocabulary);
    cuda/persistent_cggr.py:318-352.  One cdx_route_plan; the order inside an expert
    is the original token order."""
    plan = route_plan(token_ids, expert_mapping, num_experts)
    return plan.perm.to(torch.int64), plan.offsets.to(torch.int64), plan.counts.to(torch.int64)


def _offsets_i32(expert_offsets: torch.Tensor, E: int, device: torch.device) -> torch.Tensor:
    offs = torch.as_tensor(expert_offsets)
    if offs.dim() != 1 or offs.numel() != E + 1:
        raise ValueError(f"expert_offsets must have num_experts + 1 = {E + 1} entries, got {tuple(offs.shape)}")
    # Values are not inspected on the host (that would synchronise): the kernels read
    # them clamped to [0, rows], and rows outside [offsets[0], offsets[E]) stay zero.
    return offs.to(device=device, dtype=torch.int32).contiguous()


def cggr_grouped_gemm(sorted_tokens: torch.Tensor, expert_weights: torch.Tensor,
                      expert_offsets: torch.Tensor) -> torch.Tensor:
    """out[o_e:o_{e+1}] = sorted_tokens[o_e:o_{e+1}] @ expert_weights[e], zero elsewhere;
    cuda/triton_token_routed.py:197-231.  expert_weights is [E, in, out] (bf16)."""
    forward_only("cggr_grouped_gemm", sorted_tokens, expert_weights)
    nat.require_device(sorted_tokens, expert_weights, what="cggr_grouped_gemm")
    T, K = sorted_tokens.shape
    E, K2, N = expert_weights.shape
    if K2 != K:
        raise ValueError(f"cggr_grouped_gemm: in_dim mismatch {K} vs {K2}")
    a = _aligned_rows(sorted_tokens)
    w_t = expert_weights.transpose(1, 2).contiguous()  # [E, N, K], K-contiguous
    offs = _offsets_i32(expert_offsets, E, a.device)
    out = torch.zeros(T, N, dtype=a.dtype, device=a.device)
    with nat.launch_region("grouped_gemm", a.device, T=T, K=K, N=N, E=E):
        nat.check(nat.lib().cdx_grouped_gemm_fwd(a.data_ptr(), T, K, N, E, offs.data_ptr(), w_t.data_ptr(),
                                                 out.data_ptr(), nat.stream_of(a)), "cdx_grouped_gemm_fwd")
    return out


cggr_grouped_gemm_triton = cggr_grouped_gemm
grouped_gemm = cggr_grouped_gemm


def grouped_gemm_pytorch(sorted_tokens: torch.Tensor, expert_weights: torch.Tensor, expert_offsets: torch.Tensor,
                         expert_counts: Optional[torch.Tensor] = None) -> torch.Tensor:
    """cuda/triton_token_routed.py:64-86 (the counts argument is not needed: the segments
    are expert_offsets).  Runs on cdx_grouped_gemm_fwd like cggr_grouped_gemm."""
    return cggr_grouped_gemm(sorted_tokens, expert_weights, expert_offsets)


def persistent_cggr_gemm(sorted_tokens: torch.Tensor, expert_weights: torch.Tensor, expert_offsets: torch.Tensor,
                         num_sms: int = 80) -> torch.Tensor:
    """cuda/persistent_cggr.py:355-410.  ``num_sms`` is accepted for API compatibility:
    the grid here is sized by the kernel from the tile count and the chip's XCDs."""
    return cggr_grouped_gemm(sorted_tokens, expert_weights, expert_offsets)


_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _swiglu(gate: torch.Tensor, up: torch.Tensor, round_silu: bool, what: str) -> torch.Tensor:
    nat.require_device(gate, up, dtype=None, what=what)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError(f"{what}: gate {tuple(gate.shape)} {gate.dtype} and up {tuple(up.shape)} {up.dtype} differ")
    code = _DTYPE_CODE.get(gate.dtype)
    if code is None:
        raise ValueError(f"{what}: dtype {gate.dtype} not supported (bf16, fp16, fp32)")
    g, u = _aligned_rows(gate), _aligned_rows(up)
    out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    with nat.launch_region("swiglu", gate.device, n=g.numel(), elt=g.element_size()):
        nat.check(nat.lib().cdx_swiglu_fwd(g.data_ptr(), u.data_ptr(), g.numel(), code, int(round_silu),
                                           out.data_ptr(), nat.stream_of(g)), "cdx_swiglu_fwd")
    return out


def fused_swiglu_triton(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up with silu rounded to the dtype first (cdx_swiglu_fwd, round_silu=1);
    cuda/triton_token_routed.py:234-257.  Non-contiguous inputs (the halves of a fused
    gate/up output) are made contiguous, as there."""
    forward_only("fused_swiglu_triton", gate, up)
    return _swiglu(gate, up, True, "fused_swiglu_triton")


def fused_swiglu_simple(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up in fp32, rounded once (cdx_swiglu_fwd, round_silu=0);
    cuda/persistent_cggr.py:450-476."""
    forward_only("fused_swiglu_simple", gate, up)
    return _swiglu(gate, up, False, "fused_swiglu_simple")


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
    return _moe_swiglu(x2d, plan.perm, plan.offsets, plan.num_experts, w_gu, w_down, ie, has_shared, residual)


def _moe_swiglu(x2d: torch.Tensor, perm: torch.Tensor, offsets: torch.Tensor, E: int, w_gu: torch.Tensor,
                w_down: torch.Tensor, ie: int, has_shared: bool, residual: Optional[torch.Tensor] = None
                ) -> torch.Tensor:
    T, H = x2d.shape
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
        nat.check(fn(x2d.data_ptr(), T, H, ie, E, int(has_shared), perm.data_ptr(), offsets.data_ptr(),
                     w_gu.data_ptr(), w_down.data_ptr(), inter.data_ptr(), out.data_ptr(), nat.stream_of(x2d)),
                  fname)
    return out


def persistent_swiglu_cggr(sorted_tokens: torch.Tensor, gate_weights: torch.Tensor, up_weights: torch.Tensor,
                           down_weights: torch.Tensor, expert_offsets: torch.Tensor, num_sms: int = 80
                           ) -> torch.Tensor:
    """SwiGLU experts over tokens already sorted by expert; cuda/persistent_cggr.py:479-530.

    out[o_e:o_{e+1}] = (silu(t @ gate[e]) * (t @ up[e])) @ down[e] for t the rows of
    segment e, zero outside [offsets[0], offsets[E]).  gate/up [E, H, I] and down
    [E, I, H] ([in, out], bf16).  Both GEMMs run on cdx_moe_swiglu_fwd with an
    identity permutation and no shared block; the gate/up products stay fp32 into
    the SwiGLU, which is rounded once (the reference rounds the two products to bf16
    first).  The weights are packed on every call, as the operator holds no state.
    ``num_sms`` is accepted for API compatibility."""
    forward_only("persistent_swiglu_cggr", sorted_tokens, gate_weights, up_weights, down_weights)
    nat.require_device(sorted_tokens, gate_weights, up_weights, down_weights, what="persistent_swiglu_cggr")
    if sorted_tokens.dim() != 2:
        raise ValueError("persistent_swiglu_cggr: sorted_tokens must be [tokens, hidden]")
    T, H = sorted_tokens.shape
    E, H2, ie = gate_weights.shape
    if H2 != H or up_weights.shape != gate_weights.shape or down_weights.shape != (E, ie, H):
        raise ValueError("persistent_swiglu_cggr: weight shapes must be gate/up [E, H, I] and down [E, I, H]")
    x = _aligned_rows(sorted_tokens)
    w_gu, w_down = pack_moe_weights(gate_weights, up_weights, down_weights, None, None, None)
    offs = _offsets_i32(expert_offsets, E, x.device)
    ident = torch.arange(T, dtype=torch.int32, device=x.device)
    # Rows are added into zeros (one exact add): rows that no segment covers stay zero.
    out = torch.zeros(T, H, dtype=x.dtype, device=x.device)
    return _moe_swiglu(x, ident, offs, E, w_gu, w_down, ie, False, residual=out)


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

    def refresh_packed_weights(self) -> None:
        """Drop the kernel-layout copies, so the next forward packs the parameters anew.

        In-place writes to a parameter bump its version and are picked up without this;
        writes through ``.data`` (``p.data.zero_()``) bump no version counter and need
        this call."""
        self._pack_key = None
        self._packed = None
        self._all_key = None

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
        ident = torch.arange(T, dtype=torch.int32, device=x2d.device)
        offsets = torch.arange(2, dtype=torch.int32, device=x2d.device) * T
        w_gu, w_down = self._all_packed
        return _moe_swiglu(x2d, ident, offsets, 1, w_gu, w_down, self._all_width, False)
