"""End-to-end GPU forwards of the benchmark models, against the fp32 oracle.

* Configuration 1, the reference README's model (README.md:66-84): hidden 768, 18
  layers, 12 Q / 4 KV heads, intermediate 2048, 4 routed experts + shared expert, mu
  guidance, vocab 32000, seed 0; batch 4 x seq 512 Zipf(1.1) ids with the greedy
  bin-packed map.  The whole batch is compared.
* Configuration 4, the 1B preset (hidden 2048, 24 layers, 16 / 8 heads, intermediate
  5632, 8 experts + shared), seed 1; the full 8 x 2048 batch runs on the GPU and its
  first and last sequences are compared (the fp32 oracle takes a few seconds per
  2048 tokens on the host).
* Configuration 5, the routing stress: the same 1B model over 32 x 2048 ids of which
  90% fall in one expert's vocabulary; sequences 0 and 31 are compared.

The oracle receives the GPU model's own bf16 weights in fp32.  north_star bounds
layer outputs: max rel err <= 2e-2 and mean abs err <= 1e-3 against an fp32
reference.  Every kernel piece of every layer of configurations 1 and 4 is held to
exactly that, teacher forced (the oracle gets the GPU's own inputs to the piece; see
_check_layers).  The logits at the
end of the 18- or 24-layer stack carry every layer's bf16 roundings: they are held to
normwise max rel err <= 2e-2 and relative RMS <= 2e-2 (their mean abs error, about
0.8% of their RMS at configuration 1, is not a per-layer figure).  For
configurations 4 and 5 the first and the last sequence are compared: the last one's
rows land in the last M tiles of every persistent launch.

Also here: the reference's ablation pattern (run_ablations.py:45-78, mu_to_q/k/v
weights zeroed and restored through ``.data``) replayed after a forward; no host
synchronisation inside a warm forward (the forward is stream-ordered end to end;
checked with torch's sync debug mode); and a bf16-cast attention layer at S = 2048 against the oracle,
which pins the RoPE angles at long positions.
"""

from __future__ import annotations

import pytest
import torch

from _metrics import errors

pytestmark = pytest.mark.gpu
MODEL_MAX_REL = 2e-2
MODEL_REL_RMS = 2e-2


def _build(cdx, cfg, seed, device=None):
    from complexity_deep import synthetic as syn
    torch.manual_seed(seed)
    if device is not None:
        with torch.device(device):
            m = cdx.ComplexityModel(cfg)
    else:
        m = cdx.ComplexityModel(cfg)
    syn.install_expert_map(m, syn.binpacked_map(cfg.vocab_size, cfg.num_experts))
    return m.to("cuda", torch.bfloat16).eval()


def _fp32_state(m):
    return {k: v.detach().float().cpu() for k, v in m.state_dict().items()}


def _check(logits, ref, what):
    e = errors(logits, ref)
    print(f"{what}: {e}", flush=True)
    assert e["max_rel"] <= MODEL_MAX_REL and e["rel_rms"] <= MODEL_REL_RMS, (what, e)


def _piece_records(m, ids):
    """The model's forward run piece by piece (the steps of ComplexityModel.forward and
    TransformerBlock.forward_fused, with mu computed for the last block too); per block
    (h_in, mu_in, h_mid, h_out, mu_out) on the host in fp32, h_mid being h after the
    attention half's residual add."""
    from complexity_deep.linear import embedding
    from complexity_deep.normalization import rms_norm
    B, S = ids.shape
    recs = []
    with torch.no_grad():
        h = embedding(ids, m.embed_tokens.weight)
        mu_prev = m.mu_init.expand(B, S, -1)
        plans = m.route_plans(ids)
        for i, layer in enumerate(m.layers):
            h_in, mu_in = h.float().cpu(), mu_prev.float().cpu()
            ln1, ln2 = layer.input_layernorm, layer.post_attention_layernorm
            layer.self_attn(rms_norm(h, ln1.weight, ln1.eps), mu_prev=mu_prev, residual=h)
            h_mid = h.float().cpu()
            layer.mlp(rms_norm(h, ln2.weight, ln2.eps), token_ids=ids, route=plans[i], residual=h)
            mu = layer.mu_guidance.fused(h, -2.0, 2.0)
            recs.append((h_in, mu_in, h_mid, h.float().cpu(), mu.float().cpu()))
            mu_prev = mu
    return recs


def _check_layers(m, cfg, ids, oracle, what):
    """north_star's output bound (tests/_metrics.py) on every kernel piece of every
    block, each given the GPU's own input: the attention half (mu-QKV, attention,
    o_proj + residual add) against the oracle's from (h_in, mu_in); the MLP half
    (RMSNorm, routing, MoE + residual add) from h_mid; mu guidance from h_out.  Each
    output is bf16, rounded once where the comparison allows for it; chaining two
    halves instead would add the bf16 rounding of h between them, which at the 1B
    model's deep layers (|h| ~ 2) is alone the size of the mean abs bound."""
    from _metrics import assert_close_bf16
    sd = _fp32_state(m)
    c = cfg.to_dict()
    for i, (h_in, mu_in, h_mid, h_out, mu_o) in enumerate(_piece_records(m, ids)):
        with torch.no_grad():
            assert_close_bf16(h_mid, oracle.attention_half(sd, c, i, h_in, mu_in), f"{what} layer {i} attention")
            assert_close_bf16(h_out, oracle.mlp_half(sd, c, i, h_mid, ids.cpu()), f"{what} layer {i} mlp")
            assert_close_bf16(mu_o, oracle.mu_out(sd, i, h_out), f"{what} layer {i} mu")


def readme_config(cdx):
    return cdx.ComplexityConfig(vocab_size=32000, hidden_size=768, intermediate_size=2048, num_hidden_layers=18,
                                num_attention_heads=12, num_key_value_heads=4, num_experts=4, shared_expert=True,
                                use_mu_guidance=True)


def test_cfg1_readme_model_forward(cdx, oracle):
    from complexity_deep import synthetic as syn
    print("cfg1 README model, 4 x 512", flush=True)
    cfg = readme_config(cdx)
    m = _build(cdx, cfg, seed=0)
    ids = syn.zipf_token_ids(4, 512, cfg.vocab_size, seed=0)
    with torch.no_grad():
        logits = m(ids.cuda()).logits.float().cpu()
    assert logits.shape == (4, 512, cfg.vocab_size)
    with torch.no_grad():
        ref = oracle.forward(_fp32_state(m), cfg.to_dict(), ids)
    _check(logits, ref, "cfg1 logits")
    _check_layers(m, cfg, ids.cuda(), oracle, "cfg1")


@pytest.mark.parametrize("B,S", [(3, 333), (1, 1000), (5, 17)])
def test_ragged_readme_model_forward(cdx, oracle, B, S):
    """The README model on token counts that fill no tile: sequences that are not a
    multiple of 16, 64 or 128 tokens (waves whose rows span two sequences, the
    element-wise V^T stores, partial key tiles, partial M tiles of every GEMM and
    expert segments of any length), logits and every block's pieces against the
    oracle at the north-star bound."""
    from complexity_deep import synthetic as syn
    print(f"README model ragged B={B} S={S}", flush=True)
    cfg = readme_config(cdx)
    m = _build(cdx, cfg, seed=2)
    ids = syn.zipf_token_ids(B, S, cfg.vocab_size, seed=B * 1000 + S)
    with torch.no_grad():
        logits = m(ids.cuda()).logits.float().cpu()
        ref = oracle.forward(_fp32_state(m), cfg.to_dict(), ids)
    assert logits.shape == (B, S, cfg.vocab_size)
    _check(logits, ref, f"ragged {B}x{S} logits")
    _check_layers(m, cfg, ids.cuda(), oracle, f"ragged {B}x{S}")


def test_cfg4_1b_forward(cdx, oracle):
    from complexity_deep import synthetic as syn
    print("cfg4 1B model, 8 x 2048 (sequences 0 and 7 checked)", flush=True)
    cfg = cdx.ComplexityConfig.complexity_1b()
    cfg.vocab_size = 32000
    m = _build(cdx, cfg, seed=1, device="cuda")
    ids = syn.zipf_token_ids(8, 2048, cfg.vocab_size, seed=1)
    with torch.no_grad():
        logits = m(ids.cuda()).logits
    assert logits.shape == (8, 2048, cfg.vocab_size)
    # The same forward replayed from a recorded HIP graph gives the same bits.
    graphed = m.capture_forward(8, 2048)
    with torch.inference_mode():
        assert torch.equal(graphed(ids.cuda()), logits), "graph replay differs from the eager 1B forward"
    del graphed
    # Every block against the oracle block, teacher forced, on sequence 0 (the blocks'
    # rows are independent of the batch around them).
    _check_layers(m, cfg, ids[:1].cuda(), oracle, "cfg4 sequence 0")
    seqs = logits[[0, -1]].float().cpu()
    assert torch.isfinite(logits).all()
    sd = _fp32_state(m)
    del logits, m
    torch.cuda.empty_cache()
    with torch.no_grad():
        for j, b in enumerate((0, ids.shape[0] - 1)):
            ref = oracle.forward(sd, cfg.to_dict(), ids[b:b + 1])
            _check(seqs[j:j + 1], ref, f"cfg4 logits, sequence {b}")


def test_cfg5_route_stress_forward(cdx, oracle):
    """Configuration 5 through the whole 1B model: 65536 tokens (32 x 2048) with 90% of
    the ids in expert 1's vocabulary, 1% in each other expert's and the rest padding id 0,
    so one routed segment holds most of the batch.  Token rows are independent in the
    MoE and attention stays inside a sequence, so sequences 0 and 31 are each checked
    against the oracle on their own."""
    from complexity_deep import synthetic as syn
    print("cfg5 1B model, 32 x 2048 routing-stress ids (sequences 0 and 31 checked)", flush=True)
    cfg = cdx.ComplexityConfig.complexity_1b()
    cfg.vocab_size = 32000
    m = _build(cdx, cfg, seed=1, device="cuda")
    tmap = m.layers[0].mlp.token_to_expert.cpu()
    ids = syn.routing_stress_ids(32 * 2048, tmap, cfg.num_experts, heavy=1, seed=0).view(32, 2048)
    counts = torch.bincount(tmap[ids.view(-1)], minlength=cfg.num_experts)
    assert int(counts[1]) == round(0.9 * ids.numel()), counts  # the heavy expert
    with torch.no_grad():
        logits = m(ids.cuda()).logits
    assert logits.shape == (32, 2048, cfg.vocab_size)
    assert torch.isfinite(logits).all()
    seqs = logits[[0, -1]].float().cpu()
    sd = _fp32_state(m)
    del logits, m
    torch.cuda.empty_cache()
    with torch.no_grad():
        for j, b in enumerate((0, ids.shape[0] - 1)):
            ref = oracle.forward(sd, cfg.to_dict(), ids[b:b + 1])
            _check(seqs[j:j + 1], ref, f"cfg5 logits, sequence {b}")


@pytest.mark.parametrize("B,S", [(4, 512), (3, 333)])
def test_side_by_side_forward_equals_separate_operands(cdx, monkeypatch, B, S):
    """The model's forward writes each next layer's normalised input and mu into the two
    halves of one [B, S, 2H] buffer, so that the projection reads one operand.  With that
    buffer switched off (x and mu as separate tensors, the two-source projection) the
    logits must be the same bits: the re-layout changes no sum and no rounding."""
    from complexity_deep import layer as L
    from complexity_deep import synthetic as syn
    print(f"side-by-side forward vs separate operands, README model {B} x {S}", flush=True)
    cfg = readme_config(cdx)
    m = _build(cdx, cfg, seed=3)
    with torch.no_grad():
        m.mu_init.normal_(0, 0.5)  # a non-zero layer-0 mu, folded in both runs
    ids = syn.zipf_token_ids(B, S, cfg.vocab_size, seed=3).cuda()
    with torch.no_grad():
        side = m(ids).logits.clone()
        orig = L.TransformerBlock.forward_fused
        monkeypatch.setattr(L.TransformerBlock, "forward_fused",
                            lambda self, *a, **kw: orig(self, *a, **{**kw, "pair": None}))
        apart = m(ids).logits.clone()
    assert torch.equal(side, apart)


def _small(cdx):
    return cdx.ComplexityConfig(vocab_size=2048, hidden_size=256, intermediate_size=704, num_hidden_layers=3,
                                num_attention_heads=4, num_key_value_heads=2, num_experts=4)


def test_mu_ablation_replay_after_forward(cdx, oracle):
    """run_ablations.py:45-78: weights zeroed with .data.zero_() after a forward and
    restored with .data.copy_(); the forward must follow both writes."""
    from complexity_deep import synthetic as syn
    print("mu ablation replay", flush=True)
    cfg = _small(cdx)
    m = _build(cdx, cfg, seed=3)
    ids = syn.zipf_token_ids(2, 128, cfg.vocab_size, seed=3).cuda()
    with torch.inference_mode():
        base = m(ids).logits.clone()
    saved = {}
    for name, mod in m.named_modules():
        for attr in ("mu_to_k", "mu_to_q", "mu_to_v"):
            if hasattr(mod, attr):
                saved[(name, attr)] = getattr(mod, attr).weight.data.clone()
                getattr(mod, attr).weight.data.zero_()
    assert saved
    with torch.inference_mode():
        ablated = m(ids).logits.clone()
    ref = oracle.forward(_fp32_state(m), cfg.to_dict(), ids.cpu())  # the zeroed weights
    _check(ablated.float().cpu(), ref, "ablated logits")
    assert not torch.equal(ablated, base), "zeroing the mu weights must change the output"
    for (name, attr), w in saved.items():
        getattr(m.get_submodule(name), attr).weight.data.copy_(w)
    with torch.inference_mode():
        restored = m(ids).logits
    assert torch.equal(restored, base), "restoring the weights must give the first output bit for bit"


def test_per_layer_map_and_weight_writes(cdx, oracle):
    """Each layer routes through its own map, and the MLP weights the kernels read are
    the live Parameters: after writes through ``.data`` (which bump no version
    counter) to one layer's token_to_expert and to routed and shared MoE weights of
    other layers, the forward matches the oracle run on the edited state dict and
    differs from the forward before the edits (core/token_routed_mlp.py:149-174,
    run_ablations.py:81-97)."""
    from complexity_deep import synthetic as syn
    print("per-layer map and MoE weight .data writes", flush=True)
    cfg = _small(cdx)
    m = _build(cdx, cfg, seed=7)
    ids = syn.zipf_token_ids(2, 128, cfg.vocab_size, seed=7).cuda()
    with torch.inference_mode():
        base = m(ids).logits.clone()
    # layer 1 alone sends every token to expert 3
    m.layers[1].mlp.token_to_expert.data.fill_(3)
    plans = m.route_plans(ids)
    want = oracle.route_plan(ids.cpu().numpy(), m.layers[1].mlp.token_to_expert.cpu().numpy(), cfg.num_experts)
    assert plans[1].counts.tolist() == want["counts"].tolist() == [0, 0, 0, ids.numel()]
    assert not torch.equal(plans[0].counts, plans[1].counts)
    with torch.inference_mode():
        routed = m(ids).logits.clone()
    assert not torch.equal(routed, base), "layer 1's new map must change the output"
    _check(routed.float().cpu(), oracle.forward(_fp32_state(m), cfg.to_dict(), ids.cpu()), "layer-1 map edit")
    # routed and shared MoE weights of layers 0 and 2
    m.layers[0].mlp.gate_proj_w.data[2].mul_(-1.5)
    m.layers[2].mlp.shared_down.weight.data.mul_(4.0)
    m.layers[2].mlp.down_proj_w.data[0].zero_()
    with torch.inference_mode():
        edited = m(ids).logits.clone()
    assert not torch.equal(edited, routed), "the MoE weight writes must change the output"
    _check(edited.float().cpu(), oracle.forward(_fp32_state(m), cfg.to_dict(), ids.cpu()), "MoE weight edits")


def test_graphed_forward_sees_writes_and_refuses_moved_weights(cdx):
    """A replay reads the weights where they live: a ``.data`` write after capture shows
    in the next replay (equal to the eager forward), and a cast that moves the weights
    makes the replay raise instead of reading freed memory."""
    from complexity_deep import synthetic as syn
    print("GraphedForward after writes and a cast", flush=True)
    cfg = _small(cdx)
    m = _build(cdx, cfg, seed=8)
    ids = syn.zipf_token_ids(2, 64, cfg.vocab_size, seed=8).cuda()
    graphed = m.capture_forward(2, 64)
    with torch.inference_mode():
        first = graphed(ids).clone()
        assert torch.equal(first, m(ids).logits)
    m.layers[0].mlp.up_proj_w.data.mul_(2.0)
    m.layers[1].mlp.token_to_expert.data.fill_(0)
    m.layers[2].mu_guidance.mu.data.fill_(0.25)
    with torch.inference_mode():
        eager = m(ids).logits.clone()
        replay = graphed(ids).clone()
    assert not torch.equal(eager, first)
    assert torch.equal(replay, eager), "the replay must read the written weights"
    m.float()
    m.to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="moved since capture"):
        graphed(ids)
    # a replaced submodule is refused as well (capture again, and it replays)
    graphed = m.capture_forward(2, 64)
    with torch.inference_mode():
        assert torch.equal(graphed(ids), m(ids).logits)
    m.layers[1].mlp = type(m.layers[1].mlp)(cfg.hidden_size, cfg.intermediate_size, num_experts=cfg.num_experts,
                                              vocab_size=cfg.vocab_size).to("cuda", torch.bfloat16)
    with pytest.raises(RuntimeError, match="moved since capture"):
        graphed(ids)


def test_forward_has_no_host_sync(cdx):
    from complexity_deep import synthetic as syn
    print("no host sync in a warm forward", flush=True)
    cfg = _small(cdx)
    m = _build(cdx, cfg, seed=4)
    ids = syn.zipf_token_ids(2, 256, cfg.vocab_size, seed=4).cuda()
    with torch.inference_mode():
        m(ids)  # first call: weight bindings, map grouping, RoPE tables
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            out = m(ids).logits
        finally:
            torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()


def test_bf16_attention_long_positions(cdx, oracle):
    """A bf16-cast attention layer at S = 2048 (cast rounds the inv_freq buffer; the
    RoPE tables must still follow the fp32 constructor angles) against the oracle."""
    print("bf16 attention S=2048", flush=True)
    B, S, H, nq, nkv = 1, 2048, 1024, 8, 4
    torch.manual_seed(5)
    attn = cdx.ComplexityAttention(H, nq, nkv, max_position_embeddings=2048)
    with torch.no_grad():
        for n in ("q_norm", "k_norm"):
            getattr(attn, n).weight.uniform_(0.5, 1.5)
    attn = attn.to("cuda", torch.bfloat16).eval()
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    mu = torch.randn(B, S, H, generator=g).clamp(-2, 2).to(torch.bfloat16)
    with torch.no_grad():
        out, _ = attn(x.cuda(), mu_prev=mu.cuda())
    sd = {"a." + k: v.float().cpu() for k, v in attn.state_dict().items()}
    cfg = {"num_attention_heads": nq, "num_key_value_heads": nkv, "use_qk_norm": True, "rope_theta": 10000.0}
    ref = oracle.attention(x.float(), mu.float(), sd, "a.", cfg)
    e = errors(out, ref)
    print(f"bf16 attention S=2048: {e}", flush=True)
    assert e["max_rel"] <= 2e-2 and e["rel_rms"] <= 1e-2, e
