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
expert's columns are part of every token's product, so one fp32 accumulator sums
shared + routed before the single bf16 rounding.  The module's weights are views of
the two operands the kernels read (MLPOperands), so the kernels always see the live
weights.  No host synchronisation happens anywhere in the forward.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

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


def route_plans(ids: torch.Tensor, token_maps: Sequence[torch.Tensor], num_experts: int) -> List[RoutePlan]:
    """One bit-exact routing plan per map over the same ids (cdx_route_plans): plan y
    routes through token_maps[y], all of them in the same two launches.  Every map is
    int64 [V] with one V for all; ids as in route_plan.  Plan y's tensors are rows of
    [L, ...] buffers and equal route_plan(ids, token_maps[y], num_experts)."""
    L = len(token_maps)
    if L == 0:
        return []
    nat.require_device(ids, *token_maps, dtype=None, what="route_plans")
    V = token_maps[0].shape[0]
    maps = []
    for m in token_maps:
        if m.dim() != 1 or m.shape[0] != V:
            raise ValueError(f"route_plans: every map must be [{V}], got {tuple(m.shape)}")
        m = m if m.dtype == torch.int64 else m.to(torch.int64)
        maps.append(m if m.is_contiguous() else m.contiguous())
    ids = ids.reshape(-1)
    ids = ids if ids.dtype == torch.int64 else ids.to(torch.int64)
    ids = ids if ids.is_contiguous() else ids.contiguous()
    T = ids.shape[0]
    dev = ids.device
    i32 = dict(dtype=torch.int32, device=dev)
    expert_id = torch.empty(L, T, **i32)
    perm = torch.empty(L, T, **i32)
    inv_perm = torch.empty(L, T, **i32)
    counts = torch.empty(L, num_experts, **i32)
    offsets = torch.empty(L, num_experts + 1, **i32)
    lib = nat.lib()
    ws_bytes = lib.cdx_route_plans_workspace_bytes(T, num_experts, L)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    table = (ctypes.c_void_p * L)(*[m.data_ptr() for m in maps])
    with nat.launch_region("route_plan", dev, T=T, E=num_experts, V=V, L=L):
        nat.check(lib.cdx_route_plans(ids.data_ptr(), T, ctypes.cast(table, ctypes.c_void_p), L, V, num_experts,
                                      expert_id.data_ptr(), perm.data_ptr(), inv_perm.data_ptr(),
                                      counts.data_ptr(), offsets.data_ptr(), ws.data_ptr(), ws_bytes,
                                      nat.stream_of(ids)), "cdx_route_plans")
    return [RoutePlan(expert_id[y], perm[y], inv_perm[y], counts[y], offsets[y], num_experts) for y in range(L)]


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
# weight operands (layouts documented in include/cdx.h, cdx_moe_swiglu_fwd)
# ---------------------------------------------------------------------------

def padded_width(ie: int) -> int:
    return (ie + 63) // 64 * 64


def operand_views(w_gu: torch.Tensor, w_down: torch.Tensor, ie: int, has_shared: bool) -> dict:
    """The parameter-shaped views of the kernel operands w_gu [NB, 2, P, H] and
    w_down [NB, H, P] (block 0 the shared expert when has_shared):
      gate / up   [E, H, Ie]  routed gate_proj_w / up_proj_w ([in, out])
      down        [E, Ie, H]  routed down_proj_w ([in, out])
      lin_gate / lin_up [Ie, H], lin_down [H, Ie]   block 0 as nn.Linear weights
                              ([out, in]): the shared expert's, or the dense SwiGLU's
      shared_gate / shared_up / shared_down         the lin_* views, when has_shared"""
    s0 = 1 if has_shared else 0
    v = {"gate": w_gu[s0:, 0, :ie, :].transpose(1, 2), "up": w_gu[s0:, 1, :ie, :].transpose(1, 2),
         "down": w_down[s0:, :, :ie].transpose(1, 2),
         "lin_gate": w_gu[0, 0, :ie, :], "lin_up": w_gu[0, 1, :ie, :], "lin_down": w_down[0, :, :ie]}
    if has_shared:
        v.update(shared_gate=v["lin_gate"], shared_up=v["lin_up"], shared_down=v["lin_down"])
    return v


def new_operands(E: int, H: int, ie: int, has_shared: bool, dtype, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Zeroed kernel operands (w_gu [NB, 2, P, H], w_down [NB, H, P]) for E experts."""
    P = padded_width(ie)
    nb = E + (1 if has_shared else 0)
    return (torch.zeros(nb, 2, P, H, dtype=dtype, device=device),
            torch.zeros(nb, H, P, dtype=dtype, device=device))


def pack_moe_weights(gate_w: torch.Tensor, up_w: torch.Tensor, down_w: torch.Tensor,
                     shared_gate: Optional[torch.Tensor], shared_up: Optional[torch.Tensor],
                     shared_down: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fresh (w_gu, w_down) operands holding copies of the given weights: gate_w/up_w
    [E, H, Ie] and down_w [E, Ie, H] are [in, out]; shared_* are nn.Linear weights
    [out, in] (or None).  One strided copy per weight."""
    E, H, ie = gate_w.shape
    has_shared = shared_gate is not None
    w_gu, w_down = new_operands(E, H, ie, has_shared, gate_w.dtype, gate_w.device)
    views = operand_views(w_gu, w_down, ie, has_shared)
    with torch.no_grad():
        views["gate"].copy_(gate_w)
        views["up"].copy_(up_w)
        views["down"].copy_(down_w)
        if has_shared:
            views["shared_gate"].copy_(shared_gate)
            views["shared_up"].copy_(shared_up)
            views["shared_down"].copy_(shared_down)
    return w_gu, w_down


class MLPOperands:
    """The MoE kernel operands of one MLP module, w_gu [NB, 2, P, H] and
    w_down [NB, H, P], whose slices the module's weight Parameters are views of.

    Every write to a weight (in place, through ``.data``, by load_state_dict) therefore
    lands in the operand the kernel reads, and nothing is cached that could go stale.
    When a weight is no longer its view (the module was moved or cast, a Parameter was
    replaced or given new ``.data``), ``get`` copies the current weights into new
    operands and re-points the Parameters at them.  The operands are made outside
    inference mode, so that the weights stay writable after a forward run under
    torch.inference_mode()."""

    def __init__(self):
        self.bufs: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
        self.ptrs = None

    def get(self, params: dict, E: int, H: int, ie: int, has_shared: bool) -> Tuple[torch.Tensor, torch.Tensor]:
        """params maps the operand_views names to the module's Parameters."""
        ws = list(params.values())
        if self.bufs is None or [w.data_ptr() for w in ws] != self.ptrs:
            dt, dev = ws[0].dtype, ws[0].device
            if any(w.dtype != dt or w.device != dev for w in ws):
                raise ValueError("MLP weights must share one dtype and device")
            with torch.inference_mode(False), torch.no_grad():
                bufs = new_operands(E, H, ie, has_shared, dt, dev)
                views = operand_views(*bufs, ie, has_shared)
                for name, w in params.items():
                    if views[name].shape != w.shape:
                        raise ValueError(f"MLP weight {name}: shape {tuple(w.shape)}, expected "
                                         f"{tuple(views[name].shape)}")
                    views[name].copy_(w)
                    w.data = views[name]
            self.bufs = bufs
            self.ptrs = [w.data_ptr() for w in ws]
        return self.bufs


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
    nb = E + (1 if has_shared else 0)
    nat.require_device(x2d, w_gu, w_down, what="moe_swiglu")
    if w_gu.shape != (nb, 2, P, H) or w_down.shape != (nb, H, P) or not (w_gu.is_contiguous()
                                                                       and w_down.is_contiguous()):
        raise ValueError("moe_swiglu: weight operands must be contiguous [NB, 2, P, H] and [NB, H, P] "
                         f"for NB={nb}, P={P}, H={H}")
    S = 2 if has_shared else 1
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
    [E, I, H] ([in, out], bf16 only).  Both GEMMs run on cdx_moe_swiglu_fwd with an
    identity permutation and no shared block; the gate/up products stay fp32 into
    the SwiGLU, which is rounded once (the reference rounds the two products to bf16
    first).  The operator holds no state, so the weights are copied into the kernel
    layout on every call (three strided copies, about as many bytes as the GEMMs read;
    a cache would miss writes made through ``.data``).  ``num_sms`` is accepted for
    API compatibility."""
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
    core/token_routed_mlp.py:43-81.  From the first forward on, the six weight
    Parameters are views of the kernel operands (MLPOperands): strided, not
    contiguous, and read by the kernels on every call."""

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
        self._operands = MLPOperands()

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

    def _weights(self) -> dict:
        w = {"gate": self.gate_proj_w, "up": self.up_proj_w, "down": self.down_proj_w}
        if self.use_shared_expert:
            w.update(shared_gate=self.shared_gate.weight, shared_up=self.shared_up.weight,
                     shared_down=self.shared_down.weight)
        return w

    def kernel_weights(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(w_gu, w_down): the operands the kernels read, of which the weights are views."""
        return self._operands.get(self._weights(), self.num_experts, self.hidden_size,
                                  self.expert_intermediate_size, self.use_shared_expert)

    def plan(self, token_ids: torch.Tensor) -> RoutePlan:
        return route_plan(token_ids, self.token_to_expert, self.num_experts)

    def forward(self, hidden_states: torch.Tensor, token_ids: Optional[torch.Tensor] = None,
                route: Optional[RoutePlan] = None, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """[B, S, H] -> [B, S, H] = SharedMLP(x) + Expert_{map[token_id]}(x).

        ``route`` lets the caller pass the plan of this layer's map computed ahead
        (ComplexityModel computes every layer's in one call).  ``residual`` (same
        shape, contiguous) receives residual + MLP(x) in place and is returned: the
        block's residual add (core/layer.py:183) fused into the down pass."""
        forward_only("TokenRoutedMLP", hidden_states, residual, module=self)
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
        w_gu, w_down = self.kernel_weights()
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
        (token_routed_mlp.py:180-194).  Computed as one dense SwiGLU of width (E+1)*Ie
        whose routed down-projection rows are scaled by 1/E; its operands are built
        from the current weights on every call (this path is not the model's)."""
        E = self.num_experts
        sh = (self.shared_gate.weight, self.shared_up.weight, self.shared_down.weight) \
            if self.use_shared_expert else None
        with torch.no_grad():
            gate = torch.cat(([sh[0].t()] if sh else []) + [self.gate_proj_w[e] for e in range(E)], 1)
            up = torch.cat(([sh[1].t()] if sh else []) + [self.up_proj_w[e] for e in range(E)], 1)
            down = torch.cat(([sh[2].t()] if sh else []) + [self.down_proj_w[e] / E for e in range(E)], 0)
            w_gu, w_down = pack_moe_weights(gate.unsqueeze(0), up.unsqueeze(0), down.unsqueeze(0), None, None, None)
        T = x2d.shape[0]
        ident = torch.arange(T, dtype=torch.int32, device=x2d.device)
        offsets = torch.arange(2, dtype=torch.int32, device=x2d.device) * T
        return _moe_swiglu(x2d, ident, offsets, 1, w_gu, w_down, gate.shape[1], False)
