"""GPU parity of the fused mu-QKV + QK RMSNorm + RoPE kernel (cdx_mu_qkv_rope_fwd).

The reference chain is the fp32 oracle on the CPU, step by step as
core/attention.py:120-155 orders it: oracle.mu_qkv (the projection), the head split,
oracle.rms_norm over head_dim with the q_norm / k_norm weights, then RoPE with
oracle.rope_tables.  The kernel's q, k, v (head-major [B, heads, S, D]) are compared
with that chain at bf16 tolerance (tests/_metrics.py).

Covered:
* head dims 128 (the 1B and configuration-3 heads), 64 (README size) and 32;
* mu given per token, broadcast from one row (layer 0's mu_init), and absent;
* a KV-cache position offset (pos0 > 0, decode-style S = 1 included);
* no QK norm (use_qk_norm=False);
* token counts that are not tile multiples;
* configuration 4's full layer shape (8 x 2048 tokens), on 2 sequences sampled
  for the CPU chain, since the kernel treats every row independently.

The model path (ComplexityAttention.forward) is checked against the unfused
projection + PyTorch ops path of the same module, and a cached decode step against the
behaviour of the reference's SDPA call (top-left causal alignment: the new token sees
key 0 only).
"""

from __future__ import annotations

import pytest
import torch

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu
bf16 = torch.bfloat16


def _rope_ref(oracle, z, inv_freq, pos0):
    """z [B, h, S, D] fp32 -> RoPE at positions pos0 .. pos0+S-1 (rotary.py:57-86)."""
    S = z.shape[2]
    cos, sin = oracle.rope_tables(inv_freq, pos0 + S)
    cos, sin = cos[pos0:], sin[pos0:]
    half = z.shape[-1] // 2
    rot = torch.cat([-z[..., half:], z[..., :half]], dim=-1)
    return z * cos + rot * sin


def _reference(oracle, x, mu, ws, nq, nkv, D, qn, kn, inv_freq, pos0):
    B, S, H = x.shape
    q, k, v = oracle.mu_qkv(x.reshape(-1, H), None if mu is None else mu.reshape(-1, H).expand(B * S, H),
                            *ws[:3], *(ws[3:] if mu is not None else (None, None, None)))
    q = q.view(B, S, nq, D).transpose(1, 2)
    k = k.view(B, S, nkv, D).transpose(1, 2)
    v = v.view(B, S, nkv, D).transpose(1, 2)
    if qn is not None:
        q = oracle.rms_norm(q, qn, 1e-6)
        k = oracle.rms_norm(k, kn, 1e-6)
    return _rope_ref(oracle, q, inv_freq, pos0), _rope_ref(oracle, k, inv_freq, pos0), v


def _case(cdx, oracle, B, S, H, nq, nkv, mu_mode, pos0, qk_norm, seed):
    from complexity_deep.attention import mu_qkv_rope
    from complexity_deep.rotary import RotaryEmbedding
    D = H // nq
    print(f"qkv_rope B={B} S={S} H={H} heads={nq}/{nkv} D={D} mu={mu_mode} pos0={pos0} qk_norm={qk_norm}",
          flush=True)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, H, generator=g).to(bf16)
    if mu_mode == "full":
        mu = torch.randn(B, S, H, generator=g).clamp(-2, 2).to(bf16)
    elif mu_mode == "broadcast":
        mu = (torch.randn(1, 1, H, generator=g) * 0.5).to(bf16).expand(B, S, H)
    else:
        mu = None
    ws = [(torch.randn(d, H, generator=g) * 0.02).to(bf16) for d in (nq * D, nkv * D, nkv * D) * 2]
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16) if qk_norm else None
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16) if qk_norm else None
    rot = RotaryEmbedding(D, max_seq_len=64).cuda()
    table = rot.cos_sin_table(pos0 + S, torch.device("cuda"))
    wx = torch.cat(ws[:3], 0)
    w_pack = torch.cat([wx, torch.cat(ws[3:], 0)], 1).contiguous() if mu is not None else wx.contiguous()
    mu_dev = None if mu is None else (mu.cuda() if mu_mode == "full" else mu[:1, :1].cuda().expand(B, S, H))
    q, k, v = mu_qkv_rope(x.cuda(), mu_dev, w_pack.cuda(), H, nq, nkv, D,
                          None if qn is None else qn.cuda(), None if kn is None else kn.cuda(), 1e-6, table, pos0)
    torch.cuda.synchronize()
    rq, rk, rv = _reference(oracle, x, mu, ws, nq, nkv, D, qn, kn, rot.inv_freq.cpu(), pos0)
    assert q.shape == rq.shape and k.shape == rk.shape and v.shape == rv.shape
    assert_close_bf16(q, rq, "q")
    assert_close_bf16(k, rk, "k")
    assert_close_bf16(v, rv, "v")


@pytest.mark.parametrize("B,S,H,nq,nkv,mu_mode,pos0,qk_norm", [
    (2, 512, 2048, 16, 8, "full", 0, True),        # configuration 3/4 heads (D = 128)
    (2, 256, 768, 12, 4, "broadcast", 0, True),    # README size (D = 64), layer 0's mu
    (3, 77, 128, 4, 2, "full", 0, True),           # D = 32, ragged token count
    (1, 100, 256, 2, 1, None, 0, True),            # no mu (K = H), D = 128
    (2, 33, 512, 8, 2, "full", 40, True),          # KV-cache offset
    (4, 1, 512, 8, 8, "full", 511, True),          # decode step
    (2, 130, 512, 4, 4, "full", 0, False),         # no QK norm
])
def test_qkv_rope_matches_oracle(cdx, oracle, B, S, H, nq, nkv, mu_mode, pos0, qk_norm):
    _case(cdx, oracle, B, S, H, nq, nkv, mu_mode, pos0, qk_norm, seed=B * 1000 + S + H)


def test_qkv_rope_cfg4_layer_sampled(cdx, oracle):
    """8 x 2048 tokens, hidden 2048, 16/8 heads: the kernel runs on the whole batch,
    two whole sequences (first and last) are checked against the CPU chain."""
    from complexity_deep.attention import mu_qkv_rope
    from complexity_deep.rotary import RotaryEmbedding
    B, S, H, nq, nkv = 8, 2048, 2048, 16, 8
    D = H // nq
    print("qkv_rope cfg4 full layer", flush=True)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, S, H, generator=g).to(bf16)
    mu = torch.randn(B, S, H, generator=g).clamp(-2, 2).to(bf16)
    ws = [(torch.randn(d, H, generator=g) * 0.02).to(bf16) for d in (nq * D, nkv * D, nkv * D) * 2]
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16)
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16)
    rot = RotaryEmbedding(D).cuda()
    table = rot.cos_sin_table(S, torch.device("cuda"))
    w_pack = torch.cat([torch.cat(ws[:3], 0), torch.cat(ws[3:], 0)], 1).contiguous()
    q, k, v = mu_qkv_rope(x.cuda(), mu.cuda(), w_pack.cuda(), H, nq, nkv, D, qn.cuda(), kn.cuda(), 1e-6, table, 0)
    torch.cuda.synchronize()
    for b in (0, B - 1):
        rq, rk, rv = _reference(oracle, x[b:b + 1], mu[b:b + 1], ws, nq, nkv, D, qn, kn, rot.inv_freq.cpu(), 0)
        assert_close_bf16(q[b:b + 1], rq, f"q[{b}]")
        assert_close_bf16(k[b:b + 1], rk, f"k[{b}]")
        assert_close_bf16(v[b:b + 1], rv, f"v[{b}]")


@pytest.mark.parametrize("H,nq,nkv,with_cache", [(256, 4, 2, False), (768, 12, 4, True)])
def test_attention_fused_matches_unfused_path(cdx, monkeypatch, H, nq, nkv, with_cache):
    """ComplexityAttention.forward with the fused prologue against the same module
    forced through the projection kernel + PyTorch QK-norm / RoPE (the reference's op
    order), including a KV-cache continuation."""
    print(f"attention fused vs unfused H={H} cache={with_cache}", flush=True)
    torch.manual_seed(H)
    attn = cdx.ComplexityAttention(H, nq, nkv).to(bf16).cuda().eval()
    with torch.no_grad():
        attn.q_norm.weight.normal_(1, 0.1)
        attn.k_norm.weight.normal_(1, 0.1)
    x = torch.randn(2, 40, H, device="cuda").to(bf16)
    mu = torch.randn(2, 40, H, device="cuda").clamp(-2, 2).to(bf16)
    assert attn.fused_prologue

    def run(fused):
        monkeypatch.setattr(type(attn), "fused_prologue", property(lambda self: fused))
        with torch.no_grad():
            out, kv = attn(x, mu_prev=mu, use_cache=with_cache)
            if with_cache:
                out2, _ = attn(x[:, :3], mu_prev=mu[:, :3], past_key_value=kv, use_cache=True)
                return torch.cat([out, out2], 1)
            return out
    fused = run(True)
    unfused = run(False)
    d = (fused.float() - unfused.float()).abs().max() / unfused.float().abs().max()
    print("max rel fused vs unfused", float(d), flush=True)
    assert float(d) < 3e-2


def test_cached_decode_step_keeps_the_reference_sdpa_alignment(cdx):
    """A decode step with the KV cache calls SDPA as the reference does
    (core/attention.py:168-175: is_causal=(attention_mask is None)) with one query
    against all cached keys.  SDPA aligns a non-square causal mask at the top left, so
    that query sees key 0 only (the reference's generate() inherits this); the module
    keeps the call, so with o_proj the identity its output is, per query head, the
    first value row of that head's KV head, exactly."""
    H, nq, nkv, D = 256, 4, 2, 64
    print(f"cached decode step H={H} heads={nq}/{nkv}", flush=True)
    torch.manual_seed(5)
    attn = cdx.ComplexityAttention(H, nq, nkv).to(bf16).cuda().eval()
    with torch.no_grad():
        attn.o_proj.weight.copy_(torch.eye(H, dtype=bf16))
        x = torch.randn(2, 9, H, device="cuda").to(bf16)
        mu = torch.randn(2, 9, H, device="cuda").clamp(-2, 2).to(bf16)
        _, kv = attn(x[:, :8], mu_prev=mu[:, :8], use_cache=True)
        out, kv2 = attn(x[:, 8:], mu_prev=mu[:, 8:], past_key_value=kv, use_cache=True)
    v0 = kv2[1][:, :, 0, :]                                    # [B, nkv, D]
    expect = v0.repeat_interleave(nq // nkv, dim=1).reshape(2, 1, nq * D)
    assert kv2[1].shape == (2, nkv, 9, D)
    assert torch.equal(out, expect)


@pytest.mark.parametrize("B,S,H,nq,nkv,mu_mode,pos0,qk_norm", [
    (8, 2048, 2048, 16, 8, "full", 0, True),       # the 1B layer: D = 128, 64 x 16 tiles
    (16, 1024, 768, 12, 4, "broadcast", 0, True),  # D = 64: 64 x 5 tiles
    (64, 512, 512, 16, 4, None, 0, True),          # D = 32, no mu (K = H = 512): 128 x 3 tiles
    (32, 520, 1024, 8, 4, "full", 3, True),        # D = 128, S % 16 != 0: waves span two sequences
    (32, 384, 1024, 8, 2, "broadcast", 5, True),   # D = 128, 48 x 6 tiles, M tiles span sequences
    (24, 512, 1024, 8, 4, "full", 0, False),       # D = 128 without QK norm, 48 x 8 tiles
])
def test_qkv_rope_many_tiles(cdx, oracle, B, S, H, nq, nkv, mu_mode, pos0, qk_norm):
    """More tiles than CUs at each head dim, V stored plain and transposed (the
    transposed V must equal the plain V moved into that layout bit for bit, and q and
    k must not depend on V's layout), and sequences that do not split into whole
    128-row waves: rows of two sequences in one wave take the per-row token division
    and the element-wise V^T stores.  At head dim 128 with whole 128-token runs the
    transposed-V call runs the persistent form of the kernel and the plain-V call the
    one-tile-per-block form, so the equalities compare the two bit for bit."""
    from complexity_deep.attention import mu_qkv_rope, to_vt_layout
    from complexity_deep.rotary import RotaryEmbedding
    D = H // nq
    print(f"qkv_rope many tiles B={B} S={S} H={H} heads={nq}/{nkv} D={D} mu={mu_mode} pos0={pos0} "
          f"qk_norm={qk_norm}", flush=True)
    g = torch.Generator().manual_seed(B * S + H)
    x = torch.randn(B, S, H, generator=g).to(bf16)
    if mu_mode == "full":
        mu = torch.randn(B, S, H, generator=g).clamp(-2, 2).to(bf16)
    elif mu_mode == "broadcast":
        mu = (torch.randn(1, 1, H, generator=g) * 0.5).to(bf16).expand(B, S, H)
    else:
        mu = None
    ws = [(torch.randn(d, H, generator=g) * 0.02).to(bf16) for d in (nq * D, nkv * D, nkv * D) * 2]
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16)
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16)
    if not qk_norm:
        qn = kn = None
    rot = RotaryEmbedding(D).cuda()
    table = rot.cos_sin_table(pos0 + S, torch.device("cuda"))
    wx = torch.cat(ws[:3], 0)
    w_pack = (torch.cat([wx, torch.cat(ws[3:], 0)], 1) if mu is not None else wx).contiguous().cuda()
    xd = x.cuda()
    mud = None if mu is None else (mu.cuda() if mu_mode == "full" else mu[:1, :1].cuda().expand(B, S, H))
    args = (xd, mud, w_pack, H, nq, nkv, D, None if qn is None else qn.cuda(), None if kn is None else kn.cuda(),
            1e-6, table, pos0)
    q, k, v = mu_qkv_rope(*args)
    q2, k2, vt = mu_qkv_rope(*args, v_transposed=True)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(k, k2)
    assert torch.equal(vt, to_vt_layout(v)), "transposed V differs from the plain V"
    for b in (0, B - 1):
        rq, rk, rv = _reference(oracle, x[b:b + 1], None if mu is None else mu[b:b + 1], ws, nq, nkv, D, qn, kn,
                                rot.inv_freq.cpu(), pos0)
        assert_close_bf16(q[b:b + 1], rq, f"q[{b}]")
        assert_close_bf16(k[b:b + 1], rk, f"k[{b}]")
        assert_close_bf16(v[b:b + 1], rv, f"v[{b}]")


@pytest.mark.parametrize("B,S,H,nq,nkv", [(32, 512, 768, 12, 4),    # D = 64: 128 x 128 tiles vs 256 x 256
                                          (16, 1024, 2048, 16, 8)])  # D = 128: 256 x 256 vs persistent
def test_qkv_rope_sequences_independent_of_batch(cdx, B, S, H, nq, nkv):
    """A sequence's q, k and V^T do not depend on the rest of the batch: the first two
    sequences alone (few tiles: the 128-row tiles at head dim 64, one 256 x 256 tile per
    block at 128) and inside a batch of B (256-row tiles, the persistent form at head dim
    128) give the same bits.  Every tile form accumulates an element over K in the same
    order and runs the same QK-norm + RoPE arithmetic."""
    from complexity_deep.attention import mu_qkv_rope
    from complexity_deep.rotary import RotaryEmbedding
    D = H // nq
    print(f"qkv_rope sequences independent of batch B={B} S={S} H={H} D={D}", flush=True)
    g = torch.Generator().manual_seed(B + S + H)
    x = torch.randn(B, S, H, generator=g).to(bf16).cuda()
    mu = torch.randn(B, S, H, generator=g).clamp(-2, 2).to(bf16).cuda()
    N = (nq + 2 * nkv) * D
    w_pack = (torch.randn(N, 2 * H, generator=g) * 0.02).to(bf16).cuda()
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16).cuda()
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16).cuda()
    table = RotaryEmbedding(D).cuda().cos_sin_table(S, torch.device("cuda"))
    q, k, vt = mu_qkv_rope(x, mu, w_pack, H, nq, nkv, D, qn, kn, 1e-6, table, 0, v_transposed=True)
    q2, k2, vt2 = mu_qkv_rope(x[:2].contiguous(), mu[:2].contiguous(), w_pack, H, nq, nkv, D, qn, kn, 1e-6, table,
                              0, v_transposed=True)
    torch.cuda.synchronize()
    assert torch.equal(q2, q[:2]) and torch.equal(k2, k[:2])
    assert torch.equal(vt2[..., :S], vt[:2, ..., :S])
