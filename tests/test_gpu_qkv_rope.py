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
    (2, 1, 512, 8, 4, "broadcast", 100, True),     # layer 0's decode step (folded broadcast mu)
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
    (16, 1024, 1024, 8, 4, None, 0, True),         # D = 128 without mu: the persistent form with dense A
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


def _rope_unfolded(x, mu_row, w_pack, H, nq, nkv, D, qn, kn, table, vt):
    """cdx_mu_qkv_rope_fwd called directly with the broadcast row (ldmu = 0): the full
    K = 2H contraction that the fold replaces."""
    from complexity_deep import _native as nat
    from complexity_deep.attention import vt_ld_for
    B, S, _ = x.shape
    q = torch.empty(B, nq, S, D, dtype=bf16, device="cuda")
    k = torch.empty(B, nkv, S, D, dtype=bf16, device="cuda")
    vt_ld = vt_ld_for(S) if vt else 0
    v = torch.zeros(B, nkv, D, vt_ld, dtype=bf16, device="cuda") if vt else torch.empty(B, nkv, S, D, dtype=bf16,
                                                                                         device="cuda")
    nat.check(nat.lib().cdx_mu_qkv_rope_fwd(
        x.data_ptr(), H, mu_row.data_ptr(), 0, w_pack.data_ptr(), w_pack.data_ptr() + 2 * H, 2 * H, B, S, H, nq,
        nkv, D, qn.data_ptr(), kn.data_ptr(), 1e-6, table.data_ptr(), table.shape[0], 0, q.data_ptr(),
        k.data_ptr(), v.data_ptr(), vt_ld, nat.stream_of(x)), "cdx_mu_qkv_rope_fwd")
    return q, k, v


@pytest.mark.parametrize("B,S,H,nq,nkv,vt", [
    (8, 1024, 2048, 16, 8, True),   # 1B layer 0 heads, 512 tiles: the persistent form, K = 2112
    (2, 256, 768, 12, 4, False),    # README size, D = 64
    (1, 77, 128, 4, 2, False),      # D = 32, ragged, K = 192 against 256
])
def test_broadcast_mu_fold(cdx, oracle, B, S, H, nq, nkv, vt):
    """Layer 0's broadcast mu row through cdx_mu_qkv_rope_bcast_fwd (its W_mu product
    folded into one 64-column K block) against the unfolded K = 2H contraction of the
    same entry point family:
    * mu = 0: the fold adds exact zeros, so q, k, v equal the no-mu (K = H) kernel's bits;
    * mu one-hot at column j: the bias is W_mu[:, j] exactly (lo = 0) and the unfolded
      contraction adds exactly that product to the same fp32 sums, so the bits agree;
      a fold row or column taken from the wrong place fails here;
    * random mu: both within 1 bf16 ulp of each other, plus 2^-14 of the tensor's
      largest magnitude for outputs that RoPE's subtraction brings near zero (the
      bias's fp32 sum order differs, by a few fp32 ulps of the pre-norm values), and at
      the bf16 tolerance of the fp32 oracle chain."""
    from complexity_deep.attention import mu_qkv_rope
    from complexity_deep.rotary import RotaryEmbedding
    D = H // nq
    print(f"broadcast mu fold B={B} S={S} H={H} heads={nq}/{nkv} D={D} vt={vt}", flush=True)
    g = torch.Generator().manual_seed(B * S + H)
    x = torch.randn(B, S, H, generator=g).to(bf16)
    ws = [(torch.randn(d, H, generator=g) * 0.02).to(bf16) for d in (nq * D, nkv * D, nkv * D) * 2]
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16).cuda()
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16).cuda()
    rot = RotaryEmbedding(D).cuda()
    table = rot.cos_sin_table(S, torch.device("cuda"))
    w_pack = torch.cat([torch.cat(ws[:3], 0), torch.cat(ws[3:], 0)], 1).contiguous().cuda()
    xd = x.cuda()

    def folded(mu_row):
        return mu_qkv_rope(xd, mu_row.expand(B, S, H), w_pack, H, nq, nkv, D, qn, kn, 1e-6, table, 0,
                           v_transposed=vt)

    zero = torch.zeros(1, 1, H, dtype=bf16, device="cuda")
    no_mu = mu_qkv_rope(xd, None, w_pack, H, nq, nkv, D, qn, kn, 1e-6, table, 0, v_transposed=vt)
    for a, b, what in zip(folded(zero), no_mu, "qkv"):
        assert torch.equal(a, b), f"mu = 0: {what} differs from the no-mu kernel"

    j = H // 3
    one_hot = torch.zeros(1, 1, H, dtype=bf16, device="cuda")
    one_hot[..., j] = 1.0
    for a, b, what in zip(folded(one_hot), _rope_unfolded(xd, one_hot, w_pack, H, nq, nkv, D, qn, kn, table, vt),
                          "qkv"):
        if vt:
            a, b = a[..., :S], b[..., :S]
        assert torch.equal(a, b), f"one-hot mu: {what} differs from the unfolded contraction"

    mu_row = (torch.randn(1, 1, H, generator=g) * 0.5).to(bf16)
    got = folded(mu_row.cuda())
    ref = _rope_unfolded(xd, mu_row.cuda(), w_pack, H, nq, nkv, D, qn, kn, table, vt)
    torch.cuda.synchronize()
    for a, b, what in zip(got, ref, "qkv"):
        if vt:
            a, b = a[..., :S], b[..., :S]
        a, b = a.float(), b.float()
        ulp = torch.where(b == 0, torch.zeros_like(b), 2.0 ** (torch.floor(torch.log2(b.abs())) - 7))
        excess = float(((a - b).abs() - ulp - 2.0 ** -14 * b.abs().max()).max())
        assert excess <= 0, f"random mu: {what} off the unfolded contraction by {excess:.3g} beyond the bound"
        assert float((a != b).float().mean()) < 0.01, f"random mu: {what} differs in too many elements"
    if vt:
        from complexity_deep.attention import vt_columns
        got = (got[0], got[1], got[2][..., vt_columns(S, got[2].device)].transpose(-1, -2))
    rq, rk, rv = _reference(oracle, x[:1], mu_row.expand(1, S, H), ws, nq, nkv, D, qn.cpu(), kn.cpu(),
                            rot.inv_freq.cpu(), 0)
    assert_close_bf16(got[0][:1], rq, "q")
    assert_close_bf16(got[1][:1], rk, "k")
    assert_close_bf16(got[2][:1], rv, "v")


@pytest.mark.parametrize("B,S,H,nq,nkv,vt", [
    (8, 1024, 2048, 16, 8, True),   # 1B heads, 512 tiles: the persistent form
    (2, 256, 768, 12, 4, False),    # README size, D = 64
    (1, 77, 256, 4, 2, True),       # D = 64, ragged
])
def test_side_by_side_operands(cdx, B, S, H, nq, nkv, vt):
    """x and mu as the two halves of one [B, S, 2H] buffer (how the model lays them out)
    and the module's [N, 2H] weights: the projection then runs as one dense K = 2H
    contraction, which must give the bits of the two-source form on separate tensors."""
    from complexity_deep.attention import mu_qkv_rope
    from complexity_deep.rotary import RotaryEmbedding
    D = H // nq
    N = (nq + 2 * nkv) * D
    print(f"side-by-side operands B={B} S={S} H={H} heads={nq}/{nkv} D={D} vt={vt}", flush=True)
    g = torch.Generator().manual_seed(B + S + H)
    pair = torch.randn(B, S, 2 * H, generator=g).clamp(-2, 2).to(bf16).cuda()
    w = (torch.randn(N, 2 * H, generator=g) * 0.02).to(bf16).cuda()
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16).cuda()
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16).cuda()
    table = RotaryEmbedding(D).cuda().cos_sin_table(S, torch.device("cuda"))
    side = mu_qkv_rope(pair[..., :H], pair[..., H:], w[:, :H], H, nq, nkv, D, qn, kn, 1e-6, table, 0,
                       v_transposed=vt, w_mu=w[:, H:])
    apart = mu_qkv_rope(pair[..., :H].contiguous(), pair[..., H:].contiguous(), w[:, :H].contiguous(), H, nq,
                        nkv, D, qn, kn, 1e-6, table, 0, v_transposed=vt, w_mu=w[:, H:].contiguous())
    torch.cuda.synchronize()
    for a, b, what in zip(side, apart, "qkv"):
        assert torch.equal(a, b), f"{what} differs between the dense and the two-source form"
