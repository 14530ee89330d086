"""GPU parity of the causal GQA attention kernel (cdx_attention_fwd).

Reference: oracle.causal_attention (fp32, CPU), the attention core of
core/attention.py:162-181 (repeat_interleave + SDPA is_causal=True + head merge),
itself pinned by torch's SDPA and by the reference's golden logits.  The kernel gets
the same bf16 q, k, v (V through to_vt_layout) and its [B, S, nq*D] output is
compared at bf16 tolerance.

Covers head dims 128 / 64 / 32; GQA group sizes 1, 2 and 4; sequence lengths that
are and are not multiples of the 64-key tile and the 128-query block (1, 63, 77,
130, 200, 2048); the 1B shape (two full 2048-token sequences, 16/8 heads); the
transposed-V layout written by the projection kernel itself (mu_qkv_rope with
v_transposed=True) against the head-major V it writes otherwise.
"""

from __future__ import annotations

import pytest
import torch

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu
bf16 = torch.bfloat16


def _inputs(B, nq, nkv, S, D, seed):
    g = torch.Generator().manual_seed(seed)
    # unit-variance q / k rows (as after QK RMSNorm) so that softmax is not flat
    q = torch.randn(B, nq, S, D, generator=g).to(bf16)
    k = torch.randn(B, nkv, S, D, generator=g).to(bf16)
    v = torch.randn(B, nkv, S, D, generator=g).to(bf16)
    return q, k, v


@pytest.mark.parametrize("B,nq,nkv,S,D", [
    (2, 16, 8, 2048, 128),   # configuration 4's attention (two of the eight sequences)
    (1, 12, 4, 512, 64),     # README size
    (3, 4, 2, 77, 32),
    (2, 8, 2, 130, 128),     # group size 4, partial tiles
    (1, 4, 4, 200, 64),      # no grouping
    (2, 2, 1, 1, 64),        # a single token
    (1, 2, 2, 63, 32),
])
def test_attention_matches_oracle(cdx, oracle, B, nq, nkv, S, D):
    from complexity_deep.attention import causal_attention, to_vt_layout
    print(f"attention B={B} heads={nq}/{nkv} S={S} D={D}", flush=True)
    q, k, v = _inputs(B, nq, nkv, S, D, seed=S * 7 + D)
    out = causal_attention(q.cuda(), k.cuda(), to_vt_layout(v.cuda()))
    torch.cuda.synchronize()
    ref = oracle.causal_attention(q, k, v)
    assert out.shape == ref.shape == (B, S, nq * D)
    assert_close_bf16(out, ref, f"attention S={S} D={D}")


def test_projection_writes_the_transposed_v(cdx):
    """mu_qkv_rope(v_transposed=True) writes exactly to_vt_layout of the V it returns
    with v_transposed=False (bit for bit: the same accumulators, one rounding)."""
    from complexity_deep.attention import mu_qkv_rope, to_vt_layout
    from complexity_deep.rotary import RotaryEmbedding
    B, S, H, nq, nkv = 2, 200, 512, 4, 2
    D = H // nq
    print("projection transposed V", flush=True)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, S, H, generator=g).to(bf16).cuda()
    mu = torch.randn(B, S, H, generator=g).clamp(-2, 2).to(bf16).cuda()
    w = (torch.randn((nq + 2 * nkv) * D, 2 * H, generator=g) * 0.02).to(bf16).cuda()
    table = RotaryEmbedding(D).cuda().cos_sin_table(S, torch.device("cuda"))
    q1, k1, v1 = mu_qkv_rope(x, mu, w, H, nq, nkv, D, None, None, 0.0, table, 0, v_transposed=False)
    q2, k2, vt = mu_qkv_rope(x, mu, w, H, nq, nkv, D, None, None, 0.0, table, 0, v_transposed=True)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(k1, k2)
    assert torch.equal(vt, to_vt_layout(v1))


@pytest.mark.parametrize("H,nq,nkv,S", [(2048, 16, 8, 256), (768, 12, 4, 256), (512, 8, 4, 77)])
def test_attention_module_matches_sdpa_path(cdx, monkeypatch, H, nq, nkv, S):
    """ComplexityAttention.forward on the kernel path (no mask, no cache) against the
    same module through PyTorch's SDPA on the unfused projection (the reference's ops).
    S = 77 leaves a partial 16-key group, whose unwritten V columns must be cleared."""
    print(f"attention module H={H}", flush=True)
    torch.manual_seed(H)
    attn = cdx.ComplexityAttention(H, nq, nkv).to(bf16).cuda().eval()
    with torch.no_grad():
        attn.q_norm.weight.normal_(1, 0.1)
        attn.k_norm.weight.normal_(1, 0.1)
        for lin in (attn.q_proj, attn.k_proj, attn.v_proj, attn.mu_to_q, attn.mu_to_k, attn.mu_to_v, attn.o_proj):
            lin.weight.normal_(0, 0.02)
    x = torch.randn(2, S, H, device="cuda").to(bf16)
    mu = torch.randn(2, S, H, device="cuda").clamp(-2, 2).to(bf16)
    with torch.no_grad():
        fused, kv = attn(x, mu_prev=mu)
        assert torch.isfinite(fused).all()
        assert kv is None
        monkeypatch.setattr(type(attn), "fused_prologue", property(lambda self: False))
        ref, _ = attn(x, mu_prev=mu)
    d = (fused.float() - ref.float()).abs().max() / ref.float().abs().max()
    print("max rel kernel vs SDPA path", float(d), flush=True)
    assert float(d) < 3e-2


def test_attention_residual_out_projection(cdx):
    """ComplexityAttention with ``residual``: o_proj and the block's residual add
    (core/layer.py:174) as one GEMM with beta = 1, written into the residual, against
    o_proj followed by the bf16 add (one rounding fewer, so bf16 tolerance)."""
    print("attention residual o_proj", flush=True)
    torch.manual_seed(11)
    H, nq, nkv, S = 1024, 8, 4, 130
    attn = cdx.ComplexityAttention(H, nq, nkv).to(bf16).cuda().eval()
    with torch.no_grad():
        for lin in (attn.q_proj, attn.k_proj, attn.v_proj, attn.mu_to_q, attn.mu_to_k, attn.mu_to_v, attn.o_proj):
            lin.weight.normal_(0, 0.02)
    x = torch.randn(2, S, H, device="cuda").to(bf16)
    mu = torch.randn(2, S, H, device="cuda").clamp(-2, 2).to(bf16)
    h = torch.randn(2, S, H, device="cuda").to(bf16)
    with torch.no_grad():
        out, _ = attn(x, mu_prev=mu)
        expect = h + out
        got = h.clone()
        ret, kv = attn(x, mu_prev=mu, residual=got)
    torch.cuda.synchronize()
    assert ret.data_ptr() == got.data_ptr() and kv is None
    assert_close_bf16(got, expect.float(), "attention + residual")
