"""CPU oracle for the complexity-deep hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker / the timed CPU
baseline.  The product (``complexity-deep_amd/``) never imports it and has no CPU
fallback.

What it restates (reference file:line it follows):

* integer routing, in C (``route_oracle.c``, loaded through ctypes):
  ``binpack_map``      core/token_routed_mlp.py:105-116
  ``modulo_map``       core/token_routed_mlp.py:118-119
  ``route_plan``       core/token_routed_mlp.py:149-150,166-170;
                       cuda/triton_token_routed.py:37-61
* floating point, in fp32 PyTorch on the CPU:
  ``rms_norm``         core/normalization.py:29-32
  ``add_rms_norm``     core/layer.py:173-178 / cuda/fused_residual.py:363-371
  ``mu_qkv``           core/attention.py:120-131
  ``token_routed_mlp`` core/token_routed_mlp.py:142-178
  ``grouped_gemm``     cuda/triton_token_routed.py:64-86
  ``attention``        core/attention.py:115-181, core/rotary.py:30-86
  ``causal_attention`` core/attention.py:162-181 (the attention core)
  ``attention_half``   core/layer.py:165-174 (norm, attention, residual add)
  ``mlp_half``         core/layer.py:176-183 (norm, MLP, residual add)
  ``mu_out``           core/layer.py:54-61, models/modeling.py:199-200
  ``layer``            core/layer.py:141-190 (the two halves, then mu)
  ``forward``          models/modeling.py:176-206, core/layer.py:54-61,141-190

``forward`` is nothing but the embedding lookup, ``layer`` per block (itself
``attention_half``, ``mlp_half`` and ``mu_out``) and the final norm and head, so the
golden logits that pin ``forward`` pin those four pieces too: a dropped term or a
wrong index in any of them moves the logits of every configuration the golden test
holds.

How each function is pinned (independently of its own formula) is listed in the
tests: tests/test_oracle_routing.py, tests/test_oracle_float.py and
tests/test_oracle_golden.py.
"""

from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path
from typing import Dict, Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    """Compile liboracle.so with gcc (make)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        c_i64p = ctypes.POINTER(ctypes.c_int64)
        c_i32p = ctypes.POINTER(ctypes.c_int32)
        lib.oracle_binpack_map.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_int64, ctypes.c_int32, c_i64p]
        lib.oracle_binpack_map.restype = ctypes.c_int
        lib.oracle_modulo_map.argtypes = [ctypes.c_int64, ctypes.c_int32, c_i64p]
        lib.oracle_modulo_map.restype = None
        lib.oracle_route_plan.argtypes = [c_i64p, ctypes.c_int64, c_i64p, ctypes.c_int64, ctypes.c_int32,
                                          c_i32p, c_i32p, c_i32p, c_i64p, c_i64p]
        lib.oracle_route_plan.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


# ---------------------------------------------------------------------------
# integer routing (C)
# ---------------------------------------------------------------------------

def binpack_map(freq, num_experts: int) -> np.ndarray:
    """Greedy Zipf bin-packing map (int64 [V]); token_routed_mlp.py:105-116."""
    f = np.ascontiguousarray(np.asarray(freq, dtype=np.float32))
    out = np.empty(f.shape[0], dtype=np.int64)
    rc = _load().oracle_binpack_map(_ptr(f, ctypes.c_float), f.shape[0], num_experts, _ptr(out, ctypes.c_int64))
    if rc != 0:
        raise ValueError("oracle_binpack_map failed")
    return out


def binpack_map_py(freq, num_experts: int) -> np.ndarray:
    """Pure-Python statement of the same greedy rule, for small cross-checks."""
    f = [float(v) for v in np.asarray(freq, dtype=np.float32)]
    order = sorted(range(len(f)), key=lambda i: (-f[i], i))
    loads = [0.0] * num_experts
    out = np.empty(len(f), dtype=np.int64)
    for tid in order:
        best = min(range(num_experts), key=lambda e: loads[e])
        out[tid] = best
        loads[best] += f[tid]
    return out


def modulo_map(vocab_size: int, num_experts: int) -> np.ndarray:
    out = np.empty(vocab_size, dtype=np.int64)
    _load().oracle_modulo_map(vocab_size, num_experts, _ptr(out, ctypes.c_int64))
    return out


def route_plan(ids, token_map: Optional[np.ndarray], num_experts: int, vocab_size: Optional[int] = None) -> Dict[str, np.ndarray]:
    """Stable counting-sort routing plan (C).  Returns int32 expert_id/perm/inv_perm
    and int64 counts/offsets."""
    ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int64).reshape(-1))
    T = ids.shape[0]
    if token_map is not None:
        token_map = np.ascontiguousarray(np.asarray(token_map, dtype=np.int64))
        V = token_map.shape[0] if vocab_size is None else vocab_size
        mp = _ptr(token_map, ctypes.c_int64)
    else:
        V = 0
        mp = None
    expert_id = np.empty(T, dtype=np.int32)
    perm = np.empty(T, dtype=np.int32)
    inv_perm = np.empty(T, dtype=np.int32)
    counts = np.empty(num_experts, dtype=np.int64)
    offsets = np.empty(num_experts + 1, dtype=np.int64)
    rc = _load().oracle_route_plan(_ptr(ids, ctypes.c_int64), T, mp, V, num_experts,
                                   _ptr(expert_id, ctypes.c_int32), _ptr(perm, ctypes.c_int32),
                                   _ptr(inv_perm, ctypes.c_int32), _ptr(counts, ctypes.c_int64),
                                   _ptr(offsets, ctypes.c_int64))
    if rc != 0:
        raise ValueError("oracle_route_plan failed")
    return {"expert_id": expert_id, "perm": perm, "inv_perm": inv_perm, "counts": counts, "offsets": offsets}


# ---------------------------------------------------------------------------
# floating point (fp32 torch on the CPU)
# ---------------------------------------------------------------------------

def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(device="cpu", dtype=torch.float32)


def rms_norm(x, weight, eps: float = 1e-6) -> torch.Tensor:
    """weight * x * rsqrt(mean(x^2) + eps) over the last dim; normalization.py:29-32."""
    x = _f32(x)
    ms = x.pow(2).mean(-1, keepdim=True)
    return _f32(weight) * (x * torch.rsqrt(ms + eps))


def add_rms_norm(x, residual, weight, eps: float = 1e-6):
    """(rms_norm(x + residual), x + residual); layer.py:173-178 / fused_residual.py:363-371."""
    h = _f32(x) + _f32(residual)
    return rms_norm(h, weight, eps), h


def mu_qkv(x, mu, wq, wk, wv, wmq, wmk, wmv):
    """q, k, v = cat([x, mu]) @ cat([W, W_mu], 1)^T for W in (q, k, v); attention.py:120-131.
    Weights are nn.Linear layout [out, in].  mu=None drops the mu term."""
    x = _f32(x)
    if mu is None:
        return tuple(x @ _f32(w).t() for w in (wq, wk, wv))
    xm = torch.cat([x, _f32(mu).expand_as(x)], dim=-1)
    return tuple(xm @ torch.cat([_f32(w), _f32(wm)], dim=1).t() for w, wm in ((wq, wmq), (wk, wmk), (wv, wmv)))


def swiglu_rows(x, w_gate_in_out, w_up_in_out, w_down_in_out):
    """silu(x @ Wg) * (x @ Wu) @ Wd with weights in [in, out] layout."""
    return (F.silu(x @ w_gate_in_out) * (x @ w_up_in_out)) @ w_down_in_out


def token_routed_mlp(hidden, token_ids, token_map, gate_w, up_w, down_w,
                     shared_gate=None, shared_up=None, shared_down=None):
    """Token-routed MLP; token_routed_mlp.py:142-178.

    gate_w/up_w [E, H, Ie], down_w [E, Ie, H] ([in, out]); shared_* are nn.Linear
    weights ([out, in]) or None.  token_ids=None is the average-all-experts path
    (token_routed_mlp.py:180-194)."""
    hidden = _f32(hidden)
    shape = hidden.shape
    H = shape[-1]
    x = hidden.reshape(-1, H)
    gate_w, up_w, down_w = _f32(gate_w), _f32(up_w), _f32(down_w)
    E = gate_w.shape[0]
    shared = 0.0
    if shared_gate is not None:
        shared = swiglu_rows(x, _f32(shared_gate).t(), _f32(shared_up).t(), _f32(shared_down).t())
    if token_ids is None:
        out = torch.zeros_like(x)
        for e in range(E):
            out = out + swiglu_rows(x, gate_w[e], up_w[e], down_w[e])
        return (out / E + shared).reshape(shape)
    tmap = torch.as_tensor(np.asarray(token_map), dtype=torch.int64)
    ids = torch.as_tensor(token_ids).reshape(-1).to(torch.int64).clamp(0, tmap.shape[0] - 1)
    eid = tmap[ids]
    routed = torch.zeros_like(x)
    for e in range(E):
        rows = (eid == e).nonzero(as_tuple=True)[0]
        if rows.numel():
            routed[rows] = swiglu_rows(x[rows], gate_w[e], up_w[e], down_w[e])
    return (routed + shared).reshape(shape)


def grouped_gemm(sorted_tokens, expert_weights, offsets):
    """out[o_e:o_{e+1}] = A[o_e:o_{e+1}] @ W[e]; triton_token_routed.py:64-86."""
    a = _f32(sorted_tokens)
    w = _f32(expert_weights)
    offs = [int(v) for v in np.asarray(offsets)]
    out = torch.zeros(a.shape[0], w.shape[2])
    for e in range(w.shape[0]):
        if offs[e + 1] > offs[e]:
            out[offs[e]:offs[e + 1]] = a[offs[e]:offs[e + 1]] @ w[e]
    return out


def rope_inv_freq(head_dim: int, theta: float = 10000.0) -> torch.Tensor:
    """fp32 theta^(-2i/D); rotary.py:35-36, evaluated on the CPU as at construction."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))


def rope_tables(inv_freq, seq_len: int):
    """cos/sin [S, D] with emb = cat(freqs, freqs); rotary.py:40-47."""
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, _f32(inv_freq))
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def _rotate_half(x):
    d = x.shape[-1] // 2
    return torch.cat([-x[..., d:], x[..., :d]], dim=-1)


def attention(x, mu, sd: Dict[str, torch.Tensor], prefix: str, cfg: dict):
    """GQA attention with mu-guided QKV, QK-RMSNorm, RoPE and causal softmax
    (no cache, no mask); attention.py:115-181."""
    B, S, H = x.shape
    nq, nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = H // nq
    g = lambda k: sd[prefix + k]
    q, k, v = mu_qkv(x, mu, g("q_proj.weight"), g("k_proj.weight"), g("v_proj.weight"),
                     g("mu_to_q.weight") if mu is not None else None,
                     g("mu_to_k.weight") if mu is not None else None,
                     g("mu_to_v.weight") if mu is not None else None)
    q = q.view(B, S, nq, D).transpose(1, 2)
    k = k.view(B, S, nkv, D).transpose(1, 2)
    v = v.view(B, S, nkv, D).transpose(1, 2)
    if cfg.get("use_qk_norm", True):
        q = rms_norm(q, g("q_norm.weight"), 1e-6)
        k = rms_norm(k, g("k_norm.weight"), 1e-6)
    # The reference builds its cos/sin cache in the constructor (rotary.py:38,40-47),
    # from the fp32 inv_freq, before any cast of the model: the tables are therefore
    # computed from (head_dim, rope_theta), not from the state_dict's inv_freq (which a
    # bf16 state_dict holds rounded).
    cos, sin = rope_tables(rope_inv_freq(D, cfg.get("rope_theta", 10000.0)), S)
    q = q * cos + _rotate_half(q) * sin
    k = k * cos + _rotate_half(k) * sin
    o = causal_attention(q, k, v)
    return o @ _f32(g("o_proj.weight")).t()


def causal_attention(q, k, v):
    """softmax(q k^T / sqrt(D), top-left causal) v with key/value heads repeated over
    query-head groups, merged to [B, S, nq * D]; attention.py:162-181 (SDPA with
    is_causal=True, then transpose + view).  q [B, nq, S, D], k/v [B, nkv, Skv, D]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, nq, S, D = q.shape
    rep = nq // k.shape[1]
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
    scores = (q @ k.transpose(-2, -1)) / math.sqrt(D)
    causal = torch.ones(S, k.shape[2], dtype=torch.bool).triu(1)
    scores = scores.masked_fill(causal, float("-inf"))
    o = torch.softmax(scores, dim=-1) @ v
    return o.transpose(1, 2).reshape(B, S, nq * D)


def attention_half(sd: Dict[str, torch.Tensor], cfg: dict, i: int, h: torch.Tensor,
                   mu_prev: Optional[torch.Tensor]) -> torch.Tensor:
    """First half of decoder block i in fp32: h + attention(input_layernorm(h), mu_prev);
    core/layer.py:165-174."""
    p = f"layers.{i}."
    sd = {k: _f32(v) for k, v in sd.items() if k.startswith(p)}
    h = _f32(h)
    n = rms_norm(h, sd[p + "input_layernorm.weight"], cfg.get("rms_norm_eps", 1e-6))
    return h + attention(n, None if mu_prev is None else _f32(mu_prev), sd, p + "self_attn.", cfg)


def mlp_half(sd: Dict[str, torch.Tensor], cfg: dict, i: int, h: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """Second half of decoder block i in fp32: h + mlp(post_attention_layernorm(h));
    core/layer.py:176-183."""
    p = f"layers.{i}."
    sd = {k: _f32(v) for k, v in sd.items() if k.startswith(p)}
    ids = torch.as_tensor(ids).to(torch.int64)
    h = _f32(h)
    n = rms_norm(h, sd[p + "post_attention_layernorm.weight"], cfg.get("rms_norm_eps", 1e-6))
    mp = p + "mlp."
    if cfg.get("use_token_routed_mlp", True):
        shared = cfg.get("shared_expert", True)
        m = token_routed_mlp(n, ids, sd[mp + "token_to_expert"].to(torch.int64).numpy(),
                             sd[mp + "gate_proj_w"], sd[mp + "up_proj_w"], sd[mp + "down_proj_w"],
                             sd[mp + "shared_gate.weight"] if shared else None,
                             sd[mp + "shared_up.weight"] if shared else None,
                             sd[mp + "shared_down.weight"] if shared else None)
    else:
        m = swiglu_rows(n, sd[mp + "gate_proj.weight"].t(), sd[mp + "up_proj.weight"].t(),
                        sd[mp + "down_proj.weight"].t())
    return h + m


def mu_out(sd: Dict[str, torch.Tensor], i: int, h: torch.Tensor) -> torch.Tensor:
    """mu of decoder block i from its output h, clamped to [-2, 2] as the model does
    between layers; core/layer.py:54-61, models/modeling.py:199-200."""
    p = f"layers.{i}.mu_guidance."
    mu = torch.clamp(_f32(sd[p + "mu"]), 0.0, 2.0) + _f32(h) @ _f32(sd[p + "mu_proj.weight"]).t()
    return torch.clamp(mu, -2.0, 2.0)


def layer(sd: Dict[str, torch.Tensor], cfg: dict, i: int, h: torch.Tensor, mu_prev: Optional[torch.Tensor],
          ids: torch.Tensor) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Decoder block i in fp32: (h_out, mu clamped to [-2, 2] or None) from the block
    input h and the previous mu; core/layer.py:141-190 with the model's clamp of
    models/modeling.py:199-200."""
    h = mlp_half(sd, cfg, i, attention_half(sd, cfg, i, h, mu_prev), ids)
    return h, (mu_out(sd, i, h) if cfg.get("use_mu_guidance", True) else None)


def forward(sd: Dict[str, torch.Tensor], cfg: dict, input_ids: torch.Tensor) -> torch.Tensor:
    """Full ComplexityModel forward in fp32 -> logits [B, S, V]; modeling.py:176-206.

    ``sd`` is a state_dict (any dtype/device; converted to fp32 CPU on use), ``cfg`` a
    ComplexityConfig.to_dict()-style dict.  Token-routed MLP with shared expert, mu
    guidance and QK norm follow the config flags."""
    sd = {k: _f32(v) for k, v in sd.items()}
    ids = torch.as_tensor(input_ids).to(torch.int64)
    B, S = ids.shape
    H = cfg["hidden_size"]
    eps = cfg.get("rms_norm_eps", 1e-6)
    use_mu = cfg.get("use_mu_guidance", True)
    h = sd["embed_tokens.weight"][ids]
    mu_prev = sd["mu_init"].expand(B, S, H) if use_mu else None
    for i in range(cfg["num_hidden_layers"]):
        h, mu_prev = layer(sd, cfg, i, h, mu_prev, ids)
    h = rms_norm(h, sd["norm.weight"], eps)
    lm = sd["lm_head.weight"] if "lm_head.weight" in sd else sd["embed_tokens.weight"]
    return h @ lm.t()
