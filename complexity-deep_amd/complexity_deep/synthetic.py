"""Synthetic workloads of the benchmark configurations (no datasets are available).

* Token ids: truncated Zipf(s) over the vocabulary, P(id = k) proportional to
  (k + 1)^-s, so id 0 is the most frequent; sampled with torch.multinomial from a
  seeded CPU generator.
* Expert map: the reference's greedy bin-packing of that pmf
  (TokenRoutedMLP._build_token_mapping with token_frequencies = pmf), installed into
  every layer's ``token_to_expert`` buffer because ComplexityModel itself never
  passes frequencies (models/modeling.py:77-95).
* Routing stress stream (configuration 5): exactly round(0.90 T) ids from the heavy
  expert's vocabulary, round(0.01 T) from each other expert's, the rest id 0
  (padding), then a seeded shuffle.
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from .token_routed_mlp import TokenRoutedMLP


def zipf_pmf(vocab_size: int, s: float = 1.1) -> torch.Tensor:
    """float32 [V] pmf, computed in float64 and rounded once."""
    k = np.arange(1, vocab_size + 1, dtype=np.float64)
    w = k ** (-s)
    return torch.from_numpy((w / w.sum()).astype(np.float32))


def zipf_token_ids(batch: int, seq: int, vocab_size: int, s: float = 1.1, seed: int = 0) -> torch.Tensor:
    """int64 [batch, seq] ids drawn from zipf_pmf with a seeded CPU generator."""
    g = torch.Generator().manual_seed(seed)
    p = zipf_pmf(vocab_size, s).double()
    return torch.multinomial(p, batch * seq, replacement=True, generator=g).view(batch, seq)


def binpacked_map(vocab_size: int, num_experts: int, s: float = 1.1) -> torch.Tensor:
    return TokenRoutedMLP._build_token_mapping(vocab_size, num_experts, zipf_pmf(vocab_size, s))


def install_expert_map(model, token_map: torch.Tensor) -> None:
    """Copy one map into every layer's token_to_expert buffer."""
    with torch.no_grad():
        for layer in model.layers:
            if getattr(layer, "use_token_routed_mlp", False):
                buf = layer.mlp.token_to_expert
                buf.copy_(token_map.to(buf.device, buf.dtype))


def routing_stress_ids(T: int, token_map: torch.Tensor, num_experts: int, heavy: int = 1,
                       heavy_frac: float = 0.90, other_frac: float = 0.01, pad_id: int = 0,
                       seed: int = 0) -> torch.Tensor:
    """Configuration 5 stream: heavy_frac of ids from expert `heavy`'s vocabulary,
    other_frac from each other expert's, the remainder `pad_id`, shuffled (int64 [T])."""
    g = torch.Generator().manual_seed(seed)
    tmap = token_map.to("cpu", torch.int64)
    parts = []
    for e in range(num_experts):
        n = round(heavy_frac * T) if e == heavy else round(other_frac * T)
        vocab_e = (tmap == e).nonzero(as_tuple=True)[0]
        vocab_e = vocab_e[vocab_e != pad_id] if vocab_e.numel() > 1 else vocab_e
        if n > 0:
            parts.append(vocab_e[torch.randint(vocab_e.numel(), (n,), generator=g)])
    ids = torch.cat(parts) if parts else torch.empty(0, dtype=torch.int64)
    if ids.numel() > T:
        ids = ids[:T]
    ids = torch.cat([ids, torch.full((T - ids.numel(),), pad_id, dtype=torch.int64)])
    return ids[torch.randperm(T, generator=g)]


def normal_bf16(shape, seed: int, device: Optional[torch.device] = None) -> torch.Tensor:
    """N(0, 1) drawn in fp32 from a seeded CPU generator, cast to bf16."""
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g).to(torch.bfloat16)
    return t.to(device) if device is not None else t
