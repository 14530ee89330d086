"""Model, configuration and helpers; interfaces of models/config.py, models/modeling.py
and models/utils.py.

``ComplexityConfig`` is field-for-field the reference dataclass (config.py:13-109);
``ComplexityModel`` registers the same modules in the same order, so that
``torch.manual_seed(s); ComplexityModel(cfg)`` draws identical weights and the
state_dict keys and shapes match (modeling.py:69-149).

The forward (modeling.py:155-219) runs the hot path on the gfx950 kernels:
  * every routed layer gets its own routing plan through its own expert map, all of
    them computed by one call (cdx_route_plans) at the top of the forward;
  * both residual adds of every block run inside the kernels that produce the
    branch outputs (o_proj as hipBLASLt's GEMM with beta = 1, the MoE down pass's
    scatter epilogue), and every norm (each layer's two, the final one) is a
    plain RMSNorm of h;
  * the mu-QKV projection carries QK-norm and RoPE in its epilogue and feeds the
    causal GQA attention kernel (no mask, no KV cache);
  * mu guidance is one kernel that also applies the [-2, 2] clamp between layers;
  * the last layer's mu, which the reference computes and discards, is skipped;
  * the embedding gather and the tied LM head run on their own kernels
    (cdx_embedding_fwd, cdx_linear_fwd, for any vocabulary size).
o_proj runs as a PyTorch-ROCm op, as does attention with a mask or a KV cache
(generation).
"""

from __future__ import annotations

import inspect
import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Dict, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from ._grad import forward_only
from .layer import TransformerBlock
from .linear import embedding, linear
from .normalization import RMSNorm, rms_norm
from .token_routed_mlp import RoutePlan, TokenRoutedMLP, route_plans


@dataclass
class ComplexityConfig:
    vocab_size: int = 100_000
    hidden_size: int = 768
    intermediate_size: int = 2048
    num_hidden_layers: int = 12
    num_attention_heads: int = 12
    num_key_value_heads: int = 4
    max_position_embeddings: int = 2048
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-6
    attention_dropout: float = 0.0
    hidden_act: str = "silu"
    tie_word_embeddings: bool = True
    initializer_range: float = 0.02
    pad_token_id: int = 1
    bos_token_id: int = 2
    eos_token_id: int = 0
    use_token_routed_mlp: bool = True
    num_experts: int = 4
    shared_expert: bool = True
    use_mu_guidance: bool = True
    use_qk_norm: bool = True

    @classmethod
    def complexity_tiny(cls) -> "ComplexityConfig":
        return cls(hidden_size=256, intermediate_size=704, num_hidden_layers=6,
                   num_attention_heads=4, num_key_value_heads=2)

    @classmethod
    def complexity_20m(cls) -> "ComplexityConfig":
        return cls(hidden_size=320, intermediate_size=896, num_hidden_layers=8,
                   num_attention_heads=8, num_key_value_heads=4)

    @classmethod
    def complexity_small(cls) -> "ComplexityConfig":
        return cls(hidden_size=512, intermediate_size=1408, num_hidden_layers=8,
                   num_attention_heads=8, num_key_value_heads=4)

    @classmethod
    def complexity_150m(cls) -> "ComplexityConfig":
        return cls(hidden_size=768, intermediate_size=2048, num_hidden_layers=12,
                   num_attention_heads=12, num_key_value_heads=4)

    @classmethod
    def complexity_350m(cls) -> "ComplexityConfig":
        return cls(hidden_size=1280, intermediate_size=3456, num_hidden_layers=20,
                   num_attention_heads=16, num_key_value_heads=4)

    @classmethod
    def complexity_1b(cls) -> "ComplexityConfig":
        return cls(hidden_size=2048, intermediate_size=5632, num_hidden_layers=24,
                   num_attention_heads=16, num_key_value_heads=8, num_experts=8)

    def to_dict(self) -> dict:
        return {k: v for k, v in self.__dict__.items() if not k.startswith("_")}

    @classmethod
    def from_dict(cls, d: dict) -> "ComplexityConfig":
        known = set(inspect.signature(cls).parameters)
        return cls(**{k: v for k, v in d.items() if k in known})


@dataclass
class ModelOutput:
    logits: Optional[torch.Tensor] = None
    last_hidden_state: Optional[torch.Tensor] = None
    past_key_values: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None


@dataclass
class CausalLMOutput:
    loss: Optional[torch.Tensor] = None
    logits: Optional[torch.Tensor] = None
    past_key_values: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None


class ComplexityModel(nn.Module):
    """Decoder-only Complexity transformer (embed -> L blocks -> norm -> tied lm_head)."""

    def __init__(self, config: ComplexityConfig):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([
            TransformerBlock(
                hidden_size=config.hidden_size, intermediate_size=config.intermediate_size,
                num_attention_heads=config.num_attention_heads,
                num_key_value_heads=config.num_key_value_heads,
                max_position_embeddings=config.max_position_embeddings,
                rms_norm_eps=config.rms_norm_eps, rope_theta=config.rope_theta,
                attention_dropout=config.attention_dropout,
                use_token_routed_mlp=config.use_token_routed_mlp, num_experts=config.num_experts,
                vocab_size=config.vocab_size, shared_expert=config.shared_expert,
                use_qk_norm=config.use_qk_norm, use_mu_guidance=config.use_mu_guidance)
            for _ in range(config.num_hidden_layers)
        ])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight
        if config.use_mu_guidance:
            self.mu_init = nn.Parameter(torch.zeros(1, 1, config.hidden_size))
        self.apply(self._init_weights)
        self._init_residual_scaling()

    # ---- initialisation (modeling.py:117-149) --------------------------------
    def _init_weights(self, module: nn.Module) -> None:
        std = self.config.initializer_range
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=std)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=std)

    def _init_residual_scaling(self) -> None:
        std = self.config.initializer_range / (2 * self.config.num_hidden_layers) ** 0.5
        for layer in self.layers:
            nn.init.normal_(layer.self_attn.o_proj.weight, mean=0.0, std=std)
            mlp = layer.mlp
            if isinstance(getattr(mlp, "down_proj_w", None), nn.Parameter):
                nn.init.normal_(mlp.down_proj_w, mean=0.0, std=std)
            elif isinstance(getattr(mlp, "down_proj", None), nn.Linear):
                nn.init.normal_(mlp.down_proj.weight, mean=0.0, std=std)
            if isinstance(getattr(mlp, "shared_down", None), nn.Linear):
                nn.init.normal_(mlp.shared_down.weight, mean=0.0, std=std)

    # ---- routing plans ---------------------------------------------------------
    def routing_maps(self) -> List[Tuple[int, torch.Tensor]]:
        """(layer index, that layer's own token_to_expert buffer) for every routed layer:
        the maps the forward routes through, looked up afresh on every call as the
        reference does per layer (core/token_routed_mlp.py:149-150), so a write to any
        one layer's map, however made, takes effect at the next forward."""
        return [(i, layer.mlp.token_to_expert) for i, layer in enumerate(self.layers)
                if layer.use_token_routed_mlp]

    def set_token_frequencies(self, token_frequencies: torch.Tensor) -> torch.Tensor:
        """Build the greedy bin-packing map of ``token_frequencies`` ([vocab] corpus
        frequencies) once, with the native builder, and install it in every routed
        layer's ``token_to_expert`` buffer (saved in the state_dict as before).  The
        reference builds it per layer when TokenRoutedMLP is given frequencies
        (core/token_routed_mlp.py:80-116); ComplexityModel never passes any, so this
        is how a model gets the bin-packed map.  Returns the map."""
        mlps = [layer.mlp for layer in self.layers if getattr(layer, "use_token_routed_mlp", False)]
        if not mlps:
            raise ValueError("set_token_frequencies: the model has no token-routed MLP")
        tmap = TokenRoutedMLP._build_token_mapping(self.config.vocab_size, self.config.num_experts,
                                                   token_frequencies)
        with torch.no_grad():
            for mlp in mlps:
                mlp.token_to_expert.copy_(tmap.to(mlp.token_to_expert.device))
        return tmap

    def route_plans(self, input_ids: torch.Tensor) -> List[Optional[RoutePlan]]:
        """One routing plan per routed layer, each through the layer's own map: every
        plan of the forward in one cdx_route_plans call (two launches), with no host
        synchronisation.  Layers whose MLPs differ in expert count or vocabulary get
        a call per kind."""
        out: List[Optional[RoutePlan]] = [None] * len(self.layers)
        kinds: Dict[Tuple[int, int], List[Tuple[int, torch.Tensor]]] = {}
        for i, m in self.routing_maps():
            kinds.setdefault((self.layers[i].mlp.num_experts, m.shape[0]), []).append((i, m))
        for (E, _), entries in kinds.items():
            for (i, _), plan in zip(entries, route_plans(input_ids, [m for _, m in entries], E)):
                out[i] = plan
        return out

    # ---- forward (modeling.py:155-219) --------------------------------------------
    def forward(self, input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                labels: Optional[torch.Tensor] = None,
                past_key_values: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None,
                use_cache: bool = False) -> CausalLMOutput:
        forward_only("ComplexityModel", module=self)
        B, S = input_ids.shape
        h = embedding(input_ids, self.embed_tokens.weight)
        mu_prev = self.mu_init.expand(B, S, -1) if self.config.use_mu_guidance else None
        plans = self.route_plans(input_ids)
        new_kvs = [] if use_cache else None
        n_layers = len(self.layers)
        normed = rms_norm(h, self.layers[0].input_layernorm.weight, self.layers[0].input_layernorm.eps) \
            if n_layers else rms_norm(h, self.norm.weight, self.norm.eps)
        # Layers 1.. read their normalised input and mu side by side from one [B, S, 2H]
        # buffer, written by the layer before (one K = 2H operand for the projection).
        pair = torch.empty(B, S, 2 * h.shape[-1], dtype=h.dtype, device=h.device) \
            if self.config.use_mu_guidance and n_layers > 1 else None
        for i, layer in enumerate(self.layers):
            last = i + 1 == n_layers
            next_norm = self.norm if last else self.layers[i + 1].input_layernorm
            h, normed, new_kv, mu = layer.forward_fused(
                h, normed, next_norm, attention_mask=attention_mask,
                past_key_value=past_key_values[i] if past_key_values is not None else None,
                use_cache=use_cache, token_ids=input_ids, mu_prev=mu_prev, route=plans[i],
                want_mu=not last, pair=None if last else pair)
            if mu is not None:
                mu_prev = mu  # clamped to [-2, 2] inside the mu-guidance kernel
            if use_cache:
                new_kvs.append(new_kv)
        logits = linear(normed, self.lm_head.weight)
        loss = None
        if labels is not None:
            loss = F.cross_entropy(logits[..., :-1, :].contiguous().view(-1, self.config.vocab_size),
                                   labels[..., 1:].contiguous().view(-1), ignore_index=-100)
        return CausalLMOutput(loss=loss, logits=logits, past_key_values=new_kvs)

    def capture_forward(self, batch_size: int, seq_len: int) -> "GraphedForward":
        """This model's forward for [batch_size, seq_len] ids as a replayable HIP graph
        (GraphedForward); no counterpart in the reference."""
        return GraphedForward(self, batch_size, seq_len)

    # ---- generation (modeling.py:225-290) ---------------------------------------
    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 100, temperature: float = 1.0,
                 top_k: int = 50, top_p: float = 0.9, do_sample: bool = True,
                 eos_token_id: Optional[int] = None) -> torch.Tensor:
        if eos_token_id is None:
            eos_token_id = self.config.eos_token_id
        past = None
        for _ in range(max_new_tokens):
            step_ids = input_ids[:, -1:] if past is not None else input_ids
            out = self.forward(step_ids, past_key_values=past, use_cache=True)
            past = out.past_key_values
            logits = out.logits[:, -1, :] / temperature
            if top_k > 0:
                kth = torch.topk(logits, top_k)[0][..., -1, None]
                logits[logits < kth] = float("-inf")
            if top_p < 1.0:
                srt, idx = torch.sort(logits, descending=True)
                cum = torch.cumsum(F.softmax(srt, dim=-1), dim=-1)
                drop = cum > top_p
                drop[..., 1:] = drop[..., :-1].clone()
                drop[..., 0] = False
                logits[drop.scatter(1, idx, drop)] = float("-inf")
            if do_sample:
                nxt = torch.multinomial(F.softmax(logits, dim=-1), num_samples=1)
            else:
                nxt = logits.argmax(dim=-1, keepdim=True)
            input_ids = torch.cat([input_ids, nxt], dim=-1)
            if (nxt == eos_token_id).all():
                break
        return input_ids

    # ---- utilities (modeling.py:296-318) --------------------------------------------
    def num_parameters(self, trainable_only: bool = True) -> int:
        return sum(p.numel() for p in self.parameters() if p.requires_grad or not trainable_only)

    def save_pretrained(self, path: str) -> None:
        p = Path(path)
        p.mkdir(parents=True, exist_ok=True)
        with open(p / "config.json", "w") as f:
            json.dump(self.config.to_dict(), f, indent=2)
        torch.save(self.state_dict(), p / "model.pt")

    @classmethod
    def from_pretrained(cls, path: str, device: str = "cpu") -> "ComplexityModel":
        p = Path(path)
        with open(p / "config.json") as f:
            config = ComplexityConfig.from_dict(json.load(f))
        model = cls(config)
        weights = torch.load(p / "model.pt", map_location=device, weights_only=True)
        model.load_state_dict(weights, strict=False)
        return model.to(device)


SIZE_PRESETS = {
    "tiny": ComplexityConfig.complexity_tiny,
    "20m": ComplexityConfig.complexity_20m,
    "small": ComplexityConfig.complexity_small,
    "150m": ComplexityConfig.complexity_150m,
    "350m": ComplexityConfig.complexity_350m,
    "1b": ComplexityConfig.complexity_1b,
}


class GraphedForward:
    """ComplexityModel's forward for one fixed input shape, recorded once as a HIP
    graph and replayed on each call.

    A forward issues about fourteen launches per layer, and for small batches the
    Python that issues them is slower than the kernels (the 4 x 512 README model takes
    about 3.6 ms of host time per forward against about 2.2 ms of device time).  A
    replay issues the same kernels, in the same order and on the same buffers, from
    the device's queue, so results are the same bits as the eager forward.

    The graph reads every weight and expert map where it was at capture.  Values
    written there later (in place, through ``.data``, by load_state_dict) are seen by
    the next replay, since the kernels read the Parameters' own storage.  Storage that
    moves (a cast or a move of the model, a Parameter, buffer or submodule replaced, a
    Parameter given new ``.data``) is not: each call checks that every parameter and
    buffer still has the address it had at capture and every submodule is still in its
    place, and raises otherwise (capture again then).  The
    graph holds references to everything it reads, so nothing it replays from can be
    freed while it lives.  Each call copies ``input_ids`` into the graph's input
    buffer, replays, and returns the graph's logits tensor, which the next call
    overwrites.  Inference only (no labels, mask or KV cache)."""

    def __init__(self, model: "ComplexityModel", batch_size: int, seq_len: int, warmup: int = 2):
        if model.training:
            raise ValueError("GraphedForward: the model must be in eval mode")
        dev = next(model.parameters()).device
        if dev.type != "cuda":
            raise ValueError(f"GraphedForward: needs a GPU model, got {dev}")
        if batch_size <= 0 or seq_len <= 0:
            raise ValueError(f"GraphedForward: bad input shape ({batch_size}, {seq_len})")
        self.model = model
        self.shape = (int(batch_size), int(seq_len))
        self.input_ids = torch.zeros(self.shape, dtype=torch.long, device=dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.device(dev), torch.inference_mode():
            # Warm-up on a side stream (packs the weights, builds the RoPE tables), then
            # record one forward.
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                for _ in range(max(1, warmup)):
                    model(self.input_ids)
            torch.cuda.current_stream(dev).wait_stream(side)
            with torch.cuda.graph(self.graph):
                self.logits = model(self.input_ids).logits
        # What the replays read: the parameters and buffers (the kernel operands are
        # their storage), the MoE operands and the RoPE tables.  Each parameter and
        # buffer slot (module dict, name) is looked up afresh per call, so a replaced
        # Parameter is seen too; the dict lookups keep the check near 0.2 us per tensor.
        self._slots = [(d, n) for m in model.modules() for d in (m._parameters, m._buffers)
                       for n, t in d.items() if t is not None]
        self._ptrs = [d[n].data_ptr() for d, n in self._slots]
        # and every submodule slot, so that a replaced submodule is seen as well
        self._children = [(m._modules, n, c) for m in model.modules() for n, c in m._modules.items()]
        self._keep = [d[n] for d, n in self._slots] + \
                     [m._operands.bufs for m in model.modules() if hasattr(m, "_operands")] + \
                     [m._cs_table for m in model.modules() if getattr(m, "_cs_table", None) is not None] + \
                     [m._qkv_w.buf for m in model.modules() if getattr(m, "_qkv_w", None) is not None]

    def __call__(self, input_ids: torch.Tensor) -> torch.Tensor:
        if tuple(input_ids.shape) != self.shape:
            raise ValueError(f"GraphedForward: captured for input shape {self.shape}, got {tuple(input_ids.shape)}")
        try:
            moved = [d[n].data_ptr() for d, n in self._slots] != self._ptrs or \
                not all(d.get(n) is c for d, n, c in self._children)
        except (KeyError, AttributeError):
            moved = True  # a parameter or buffer was removed (or set to None)
        if moved:
            raise RuntimeError("GraphedForward: a parameter or buffer of the model has moved since capture "
                               "(cast, moved, replaced or re-bound); capture the forward again")
        self.input_ids.copy_(input_ids)
        with torch.cuda.device(self.input_ids.device):
            self.graph.replay()
        return self.logits


def create_complexity_model(size: str = "150m", vocab_size: int = 100_000, **overrides) -> ComplexityModel:
    """Preset config + overrides -> ComplexityModel; models/utils.py:19-44."""
    if size not in SIZE_PRESETS:
        raise ValueError(f"Unknown size '{size}'. Choose from {list(SIZE_PRESETS)}")
    config = SIZE_PRESETS[size]()
    config.vocab_size = vocab_size
    for k, v in overrides.items():
        if hasattr(config, k):
            setattr(config, k, v)
    return ComplexityModel(config)


def count_parameters(config: ComplexityConfig) -> dict:
    """Analytic parameter counts; models/utils.py:47-98."""
    H, I, V, L = config.hidden_size, config.intermediate_size, config.vocab_size, config.num_hidden_layers
    nq, nkv = config.num_attention_heads, config.num_key_value_heads
    D = H // nq
    E = config.num_experts if config.use_token_routed_mlp else 1
    ie = I // E
    qkv = nq * D * H + 2 * nkv * D * H
    attn = qkv + H * H + (qkv if config.use_mu_guidance else 0) + (2 * D if config.use_qk_norm else 0)
    if config.use_token_routed_mlp:
        mlp = E * 3 * H * ie + (3 * H * ie if config.shared_expert else 0)
    else:
        mlp = 3 * H * I
    mu = H + H * H if config.use_mu_guidance else 0
    per_layer = attn + mlp + 2 * H + mu
    total = V * H + L * per_layer + H
    return {"total": total, "embedding": V * H, "per_layer": per_layer, "attention_per_layer": attn,
            "mlp_per_layer": mlp, "mu_per_layer": mu, "num_layers": L,
            "memory_bf16_gb": total * 2 / (1024 ** 3)}
