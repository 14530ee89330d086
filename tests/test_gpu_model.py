"""End-to-end GPU forward of ComplexityModel in bf16.

The tiny golden configurations (weights drawn with the reference's seeded init, the
same expert maps and ids) run through every hot-path kernel and are compared with
the reference's own fp32 logits from tests/golden/model_golden.npz.  A whole
forward stacks many bf16 roundings (embedding, attention, o_proj, mu, lm_head are
bf16 PyTorch ops, as in the reference's bf16 run).  Against the reference's fp32
logits, whose weights are not rounded to bf16, the bound is normwise max rel err
<= 2e-2 and relative RMS <= 2e-2 (the weight rounding alone moves the mean abs error
to about 1e-3 on these logits).  Against the oracle run on the model's own bf16
weights, the whole north_star bound holds: max rel err <= 2e-2 and mean abs err
<= 1e-3 (on top of the bf16 output rounding, tests/_metrics.py).

Also checked: the unfused TransformerBlock.forward API against the oracle, the
generate() loop with a KV cache, and that one routing call per forward gives every
layer the plan of its own map.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from _metrics import errors

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "model_golden.npz"
MODEL_MAX_REL = 2e-2
MODEL_MEAN_ABS = 1e-3
MODEL_REL_RMS = 2e-2


def _entries():
    z = np.load(GOLDEN, allow_pickle=False)
    return z, json.loads(bytes(z["meta_json"]).decode())


def _model(cdx, entry, tmap):
    torch.manual_seed(entry["seed"])
    m = cdx.ComplexityModel(cdx.ComplexityConfig.from_dict(entry["cfg"]))
    if tmap.size:
        from complexity_deep.synthetic import install_expert_map
        install_expert_map(m, torch.from_numpy(tmap))
    return m.to(torch.bfloat16).cuda().eval()


@pytest.mark.parametrize("name", [m["name"] for m in _entries()[1]])
def test_forward_matches_reference_logits(cdx, oracle, name):
    print(f"model forward {name}", flush=True)
    z, meta = _entries()
    entry = next(m for m in meta if m["name"] == name)
    m = _model(cdx, entry, z[f"{name}/map"])
    ids = torch.from_numpy(z[f"{name}/ids"]).cuda()
    with torch.no_grad():
        logits = m(ids).logits
    e = errors(logits, torch.from_numpy(z[f"{name}/logits"]))
    print(name, "vs reference fp32 logits", e, flush=True)
    assert e["max_rel"] <= MODEL_MAX_REL and e["rel_rms"] <= MODEL_REL_RMS, e
    sd = {k: v.detach().float().cpu() for k, v in m.state_dict().items()}
    e = errors(logits, oracle.forward(sd, entry["cfg"], ids.cpu()))
    print(name, "vs oracle on the bf16 weights", e, flush=True)
    assert e["max_rel"] <= MODEL_MAX_REL and e["mean_abs_kernel"] <= MODEL_MEAN_ABS \
        and e["rel_rms"] <= MODEL_REL_RMS, e


def test_block_api_matches_oracle(cdx, oracle):
    print("TransformerBlock.forward", flush=True)
    z, meta = _entries()
    entry = meta[0]
    m = _model(cdx, entry, z[f"{entry['name']}/map"])
    layer = m.layers[0]
    ids = torch.from_numpy(z[f"{entry['name']}/ids"]).cuda()
    B, S = ids.shape
    H = entry["cfg"]["hidden_size"]
    h = torch.randn(B, S, H, device="cuda").to(torch.bfloat16)
    mu = torch.randn(B, S, H, device="cuda").clamp(-2, 2).to(torch.bfloat16)
    h_in = h.clone()
    with torch.no_grad():
        h_out, kv, mu_out = layer(h, token_ids=ids, mu_prev=mu)
    assert torch.equal(h, h_in), "the block API must not modify its input"
    sd = {k[len("layers.0."):]: v.float().cpu() for k, v in m.state_dict().items() if k.startswith("layers.0.")}
    cfg = entry["cfg"]
    n = oracle.rms_norm(h.float().cpu(), sd["input_layernorm.weight"])
    full = {("self_attn." + k[len("self_attn."):]): v for k, v in sd.items() if k.startswith("self_attn.")}
    a = oracle.attention(n, mu.float().cpu(), full, "self_attn.", cfg)
    h1 = h.float().cpu() + a
    n2 = oracle.rms_norm(h1, sd["post_attention_layernorm.weight"])
    mo = oracle.token_routed_mlp(n2, ids.cpu(), sd["mlp.token_to_expert"].long().numpy(), sd["mlp.gate_proj_w"],
                                 sd["mlp.up_proj_w"], sd["mlp.down_proj_w"], sd["mlp.shared_gate.weight"],
                                 sd["mlp.shared_up.weight"], sd["mlp.shared_down.weight"])
    h2 = h1 + mo
    e = errors(h_out, h2)
    assert e["max_rel"] <= MODEL_MAX_REL and e["rel_rms"] <= MODEL_REL_RMS, e
    mu_ref = torch.clamp(sd["mu_guidance.mu"], 0, 2) + h2 @ sd["mu_guidance.mu_proj.weight"].t()
    e = errors(mu_out, mu_ref)
    assert e["max_rel"] <= MODEL_MAX_REL, e


def oracle_plan(ids, tmap, E):
    from oracle import oracle as orc
    return orc.route_plan(ids.cpu().numpy(), tmap.cpu().numpy(), E)


def test_generate_and_plan_reuse(cdx, monkeypatch):
    print("generate + plan reuse", flush=True)
    z, meta = _entries()
    entry = meta[0]
    m = _model(cdx, entry, z[f"{entry['name']}/map"])
    import complexity_deep.modeling as modeling
    calls = []
    real = modeling.route_plans
    monkeypatch.setattr(modeling, "route_plans", lambda *a, **k: calls.append(len(a[1])) or real(*a, **k))
    ids = torch.from_numpy(z[f"{entry['name']}/ids"]).cuda()
    with torch.no_grad():
        m(ids)
    routed = sum(1 for layer in m.layers if layer.use_token_routed_mlp)
    assert calls == [routed], "one routing call per forward, one plan per routed layer"
    plans = m.route_plans(ids)
    for layer, plan in zip(m.layers, plans):
        if plan is None:
            continue
        ref = oracle_plan(ids, layer.mlp.token_to_expert, layer.mlp.num_experts)
        assert plan.perm.tolist() == ref["perm"].tolist() and plan.offsets.tolist() == ref["offsets"].tolist()
    out = m.generate(ids[:, :4], max_new_tokens=5, do_sample=False)
    assert out.shape == (2, 9)
    assert torch.equal(out[:, :4], ids[:, :4])
