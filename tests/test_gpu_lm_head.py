"""GPU parity of the model's two ends: the embedding gather (cdx_embedding_fwd) and the
tied LM head GEMM (cdx_linear_fwd).

References: the embedding is an exact row copy, so it is checked bit for bit against
torch indexing of the same table (models/modeling.py:177), including ids outside
[0, vocab), which give NaN rows (nn.Embedding raises there).  The LM head is checked against the fp32 product
x.float() @ w.float().T (models/modeling.py:206) at the bf16 tolerance of
tests/_metrics.py, on configuration 4's shape (16384 tokens, hidden 2048, vocab
32000: the head of every 1B forward) and on ragged shapes; the model path is covered
by the golden-logit test.
"""

from __future__ import annotations

import pytest
import torch

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu
bf16 = torch.bfloat16


@pytest.mark.parametrize("T,V,H", [(16384, 32000, 2048), (77, 1000, 768), (1, 50, 64), (300, 257, 8)])
def test_embedding_is_an_exact_gather(cdx, T, V, H):
    from complexity_deep.linear import embedding
    print(f"embedding T={T} V={V} H={H}", flush=True)
    g = torch.Generator().manual_seed(T + V)
    table = torch.randn(V, H, generator=g).to(bf16).cuda()
    ids = torch.randint(0, V, (T,), generator=g).cuda()
    out = embedding(ids, table)
    torch.cuda.synchronize()
    assert out.shape == (T, H)
    assert torch.equal(out, table[ids])


def test_embedding_batched_ids_and_out_of_range(cdx):
    from complexity_deep.linear import embedding
    V, H = 100, 256
    table = torch.randn(V, H).to(bf16).cuda()
    ids = torch.tensor([[0, 99, -1, 100], [5, 1 << 40, 7, -(1 << 40)]], device="cuda")
    out = embedding(ids, table)
    torch.cuda.synchronize()
    assert out.shape == (2, 4, H)
    ok = (ids >= 0) & (ids < V)
    assert torch.equal(out[ok], table[ids[ok]])
    assert bool(torch.isnan(out[~ok]).all())


def test_model_out_of_range_id_poisons_only_what_depends_on_it(cdx):
    """nn.Embedding raises on an id outside [0, vocab); the forward cannot without a host
    round trip, so the bad token's row is NaN.  Every logit that depends on it (its own
    position and the later positions of its sequence) must be NaN.  The other sequence and
    the positions of earlier 128-query attention blocks never read the row and must be
    bit-identical to the forward with the id clamped (the routing lookup clamps it too).
    Positions of the bad token's own query block before it are not pinned: their PV
    product multiplies its NaN V row by a zero probability, as SDPA's would."""
    torch.manual_seed(0)
    cfg = cdx.ComplexityConfig(vocab_size=1000, hidden_size=256, intermediate_size=512,
                               num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                               num_experts=4, max_position_embeddings=256)
    m = cdx.ComplexityModel(cfg).cuda().to(bf16).eval()
    B, S, p = 2, 256, 200
    ids = torch.randint(0, cfg.vocab_size, (B, S), device="cuda")
    bad = ids.clone()
    bad[1, p] = cfg.vocab_size + 5
    with torch.no_grad():
        got = m(bad).logits.float()
        ref = m(bad.clamp(0, cfg.vocab_size - 1)).logits.float()
    torch.cuda.synchronize()
    assert bool(torch.isnan(got[1, p:]).all())
    assert torch.equal(got[1, :128], ref[1, :128])
    assert torch.equal(got[0], ref[0])
    assert not bool(torch.isnan(ref).any())


@pytest.mark.parametrize("M,K,N", [(16384, 2048, 32000), (300, 768, 1000), (1, 64, 8), (513, 128, 264)])
def test_linear_matches_fp32(cdx, M, K, N):
    from complexity_deep.linear import linear
    print(f"linear M={M} K={K} N={N}", flush=True)
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).to(bf16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(bf16)
    out = linear(x.cuda(), w.cuda())
    torch.cuda.synchronize()
    # fp32 reference on the GPU for the big case (16384 x 32000 x 2048 in fp32 on the
    # CPU would take minutes), on the CPU otherwise
    if M * N * K > 1 << 32:
        ref = (x.cuda().float() @ w.cuda().float().t())
    else:
        ref = x.float() @ w.float().t()
    assert_close_bf16(out, ref, f"linear {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(77, 128, 30), (300, 64, 1001), (1, 64, 1), (2, 256, 32003)])
def test_linear_any_out_features(cdx, M, K, N):
    """N not a multiple of 8 runs on the kernel too (the model's head for any
    vocabulary): a view of the first N columns of a padded buffer, whose leading
    dimensions still merge."""
    from complexity_deep.linear import linear
    print(f"linear odd N M={M} K={K} N={N}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(2, M, K, generator=g).to(bf16)
    w = (torch.randn(N, K, generator=g) * 0.05).to(bf16)
    out = linear(x.cuda(), w.cuda())
    torch.cuda.synchronize()
    assert out.shape == (2, M, N)
    assert_close_bf16(out.view(-1, N), x.float().view(-1, K) @ w.float().t(), f"linear {M}x{K}x{N}")


def test_linear_rejects_unsupported_shapes(cdx):
    from complexity_deep.linear import linear
    with pytest.raises(ValueError, match="multiple of 64"):
        linear(torch.randn(4, 100, device="cuda").to(bf16), torch.randn(64, 100, device="cuda").to(bf16))


def test_model_head_odd_vocab_runs_the_kernel(cdx, monkeypatch):
    """A vocabulary that is not a multiple of 8 takes the same kernel as any other
    (no nn.Linear path): the head call goes through cdx_linear_fwd, and the logits
    match the model run with the head in fp32."""
    import complexity_deep.modeling as modeling
    print("odd vocab model head", flush=True)
    cfg = cdx.ComplexityConfig(vocab_size=1001, hidden_size=128, intermediate_size=256, num_hidden_layers=1,
                               num_attention_heads=2, num_key_value_heads=1, num_experts=2)
    torch.manual_seed(3)
    m = cdx.ComplexityModel(cfg).to("cuda", bf16).eval()
    calls = []
    real = modeling.linear
    monkeypatch.setattr(modeling, "linear", lambda *a, **k: calls.append(a[1].shape) or real(*a, **k))
    monkeypatch.setattr(m.lm_head, "forward", lambda *a, **k: (_ for _ in ()).throw(AssertionError("nn.Linear")))
    ids = torch.randint(0, 1001, (2, 24)).cuda()
    with torch.no_grad():
        logits = m(ids).logits
    assert calls == [(1001, 128)]
    assert logits.shape == (2, 24, 1001)
    assert torch.isfinite(logits.float()).all()


@pytest.mark.parametrize("M,K,N", [(16384, 2048, 2048), (2048, 768, 768), (300, 128, 264), (513, 64, 8),
                                   (4096, 1024, 3072)])
def test_linear_residual_is_the_product_then_a_bf16_add(cdx, M, K, N):
    """o_proj + the block's residual add (core/attention.py:181, core/layer.py:174): the
    product rounded to bf16, then added to the residual with a bf16 add.  The product
    is the tile engine's (the same accumulation as cdx_linear_fwd, whatever the tile
    shape), so the result is checked bit for bit against linear() plus torch's bf16 add,
    and the product against the fp32 one at the bf16 tolerance."""
    from complexity_deep.linear import linear, linear_residual_
    print(f"linear_residual M={M} K={K} N={N}", flush=True)
    g = torch.Generator().manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(bf16).cuda()
    w = (torch.randn(N, K, generator=g) * 0.02).to(bf16).cuda()
    r0 = torch.randn(M, N, generator=g).to(bf16).cuda()
    res = r0.clone()
    out = linear_residual_(x, w, res)
    prod = linear(x, w)
    torch.cuda.synchronize()
    assert out.data_ptr() == res.data_ptr()
    assert torch.equal(res, r0 + prod)
    ref = x.float() @ w.float().t()
    assert_close_bf16(prod.float(), ref, f"linear_residual product {M}x{K}x{N}")
