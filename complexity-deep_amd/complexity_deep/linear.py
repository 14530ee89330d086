"""The model's two ends on the gfx950 kernels: the token-embedding gather and the
tied LM head (models/modeling.py:74,101-103,177,206).

``embedding(ids, table)`` is nn.Embedding's lookup through cdx_embedding_fwd (an
exact row copy).  An id outside [0, vocab) gives a row of NaNs where nn.Embedding
raises: raising would need a host round trip, and the NaNs make every logit that
depends on the token NaN instead of a plausible number.
``linear(x, w)`` is a bias-free nn.Linear (x @ w^T, w stored [out, in]) through the
MFMA tile engine (cdx_linear_fwd; fp32 accumulation, one bf16 rounding).
``linear_residual_(x, w, residual)`` adds such a product to ``residual`` in place, with
the rounding of a separate bf16 add (cdx_linear_residual_fwd): the attention block's
o_proj and residual add (core/attention.py:71,181, core/layer.py:174) as an operator;
ComplexityModel keeps hipBLASLt's GEMM with beta = 1 for it, which ran the 1B forward
0.8% faster.
"""

from __future__ import annotations

import torch

from . import _native as nat


def embedding(ids: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """table[ids] for int64 ids of any shape; returns [*ids.shape, H]."""
    nat.require_device(table, what="embedding")
    nat.require_device(ids, table, dtype=None, what="embedding")
    if table.dim() != 2:
        raise ValueError("embedding: table must be [vocab, hidden]")
    V, H = table.shape
    flat = ids.reshape(-1)
    flat = flat if flat.dtype == torch.int64 else flat.to(torch.int64)
    flat = flat if flat.is_contiguous() else flat.contiguous()
    table = table if table.is_contiguous() else table.contiguous()
    out = torch.empty(flat.shape[0], H, dtype=table.dtype, device=table.device)
    with nat.launch_region("embedding", table.device, T=flat.shape[0], H=H):
        nat.check(nat.lib().cdx_embedding_fwd(flat.data_ptr(), flat.shape[0], table.data_ptr(), V, H,
                                              out.data_ptr(), nat.stream_of(table)), "cdx_embedding_fwd")
    return out.view(*ids.shape, H)


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x @ w^T for x [..., K], w [N, K] (nn.Linear weight layout), bf16; K a multiple of 64.

    For N not a multiple of 8 the result is a view of the first N columns of a
    [rows, round_up(N, 8)] buffer (the kernel stores whole 16-byte pieces); its leading
    dimensions still merge (``.view(-1, N)`` works)."""
    nat.require_device(x, w, what="linear")
    N, K = w.shape
    if x.shape[-1] != K:
        raise ValueError(f"linear: x has {x.shape[-1]} features, weight expects {K}")
    if K % 64 != 0:
        raise ValueError(f"linear: in_features={K} must be a multiple of 64 (cdx_linear_fwd)")
    x2 = x.reshape(-1, K)
    x2 = x2 if x2.is_contiguous() else x2.contiguous()
    w = w if w.is_contiguous() else w.contiguous()
    n8 = (N + 7) // 8 * 8
    out = torch.empty(x2.shape[0], n8, dtype=x.dtype, device=x.device)
    with nat.launch_region("lm_head", x.device, M=x2.shape[0], K=K, N=N):
        nat.check(nat.lib().cdx_linear_fwd(x2.data_ptr(), K, w.data_ptr(), K, x2.shape[0], K, N, out.data_ptr(), n8,
                                           nat.stream_of(x)), "cdx_linear_fwd")
    if n8 != N:
        out = out[:, :N]
    return out.view(*x.shape[:-1], N)


def linear_residual_(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """residual += x @ w^T in place (the product rounded to bf16, then the add), for
    x [..., K], w [N, K], residual [..., N] contiguous; K % 64 == 0, N % 8 == 0."""
    nat.require_device(x, w, residual, what="linear_residual_")
    N, K = w.shape
    if x.shape[-1] != K:
        raise ValueError(f"linear_residual_: x has {x.shape[-1]} features, weight expects {K}")
    if residual.shape[:-1] != x.shape[:-1] or residual.shape[-1] != N:
        raise ValueError(f"linear_residual_: residual shape {tuple(residual.shape)} does not match "
                         f"{tuple(x.shape[:-1]) + (N,)}")
    if not residual.is_contiguous():
        raise ValueError("linear_residual_: residual must be contiguous (it is updated in place)")
    x2 = x if x.is_contiguous() else x.contiguous()  # rows base + r * K
    M = x2.numel() // K if K else 0
    w = w if w.is_contiguous() else w.contiguous()
    with nat.launch_region("o_proj", x.device, M=M, K=K, N=N):
        nat.check(nat.lib().cdx_linear_residual_fwd(x2.data_ptr(), K, w.data_ptr(), K, M, K, N,
                                                    residual.data_ptr(), N, nat.stream_of(x)),
                  "cdx_linear_residual_fwd")
    return residual
