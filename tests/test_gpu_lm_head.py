"""GPU parity of the model's two ends: the embedding gather (cdx_embedding_fwd) and the
tied LM head GEMM (cdx_linear_fwd).

References: the embedding is an exact row copy, so it is checked bit for bit against
torch indexing of the same table (models/modeling.py:177), including ids outside
[0, vocab), which give zero rows.  The LM head is checked against the fp32 product
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
    assert torch.count_nonzero(out[~ok]) == 0


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


def test_linear_rejects_unsupported_shapes(cdx):
    from complexity_deep.linear import linear, linear_supported
    assert not linear_supported(100, 64) and not linear_supported(64, 30)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        linear(torch.randn(4, 64, device="cuda").to(bf16), torch.randn(30, 64, device="cuda").to(bf16))
