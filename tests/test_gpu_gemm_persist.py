"""The persistent form of the MFMA tile engine against fp32 products.

Products whose M and N are whole 256 x 256 tiles and which have more tiles than the
GPU has CUs run on gemm_persist_kernel: one block per CU walks its XCD's tiles, a
tile's second-to-last K step fetches the next tile's first step, and the results are
staged through the LDS in two halves.  The shapes here are picked for that path and
its edges: the shortest K loop (two 64-wide K steps, so a tile's first refill is
already the next tile's), uneven tile counts per block, an M-tile count that leaves
a short last group in the tile order, the broadcast mu row (row stride 0) and a
strided weight view.  The three tile forms (256 x 128 tiles for small products, one
256 x 256 tile per block, persistent) must also agree bit for bit on the same rows.
Bound: the bf16 tolerance of the north star (max rel err
<= 2e-2 normwise, mean abs err <= 1e-3 relative to the fp32 scale), checked by
``assert_close_bf16``.
"""

from __future__ import annotations

import pytest
import torch

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu
bf16 = torch.bfloat16


@pytest.mark.parametrize("M,K,N", [(4096, 128, 8192),     # 512 tiles, two K steps each
                                   (2304, 192, 7936),     # 9 x 31 tiles: 1-2 per block, last group of 1
                                   (8192, 2048, 32000)])  # 125 N tiles, 15-16 per block
def test_persistent_linear(cdx, M, K, N):
    from complexity_deep.linear import linear
    print(f"persistent linear M={M} K={K} N={N}", flush=True)
    g = torch.Generator().manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(bf16).cuda()
    w = (torch.randn(N, K, generator=g) * 0.05).to(bf16).cuda()
    out = linear(x, w)
    ref = x.float() @ w.float().t()
    assert_close_bf16(out, ref, f"linear {M}x{K}x{N}")
    # a second call on the same buffers gives the same bits (no state kept across calls)
    assert torch.equal(linear(x, w), out)


def test_persistent_mu_qkv_broadcast_and_strided(cdx):
    from complexity_deep.attention import mu_qkv_project
    print("persistent mu_qkv: broadcast mu row, strided weights", flush=True)
    B, S, H, N = 8, 2048, 512, 2048  # 64 x 8 tiles, K = 2H = 1024
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, S, H, generator=g).to(bf16).cuda()
    mu_row = torch.randn(1, 1, H, generator=g).clamp(-2, 2).to(bf16).cuda()
    w = (torch.randn(N, 2 * H, generator=g) * 0.03).to(bf16).cuda()
    out = mu_qkv_project(x, mu_row.expand(B, S, H), w, H)
    xf = x.float().view(-1, H)
    ref = xf @ w[:, :H].float().t() + mu_row.float().view(1, H) @ w[:, H:].float().t()
    assert_close_bf16(out.view(-1, N), ref, "broadcast mu")
    # no mu: the x half of the packed weight, a view with row stride 2H
    out0 = mu_qkv_project(x, None, w[:, :H], H)
    assert_close_bf16(out0.view(-1, N), xf @ w[:, :H].float().t(), "mu=None, strided weight")


def test_persistent_mu_guidance_many_tiles(cdx):
    from complexity_deep.layer import mu_guidance
    print("persistent mu_guidance T=32768 H=1024", flush=True)
    T, H = 32768, 1024  # 128 x 4 tiles
    g = torch.Generator().manual_seed(12)
    h = torch.randn(T, H, generator=g).to(bf16).cuda()
    w = (torch.randn(H, H, generator=g) / H ** 0.5).to(bf16).cuda()
    bias = torch.linspace(0.0, 2.0, H).to(bf16).cuda()
    out = mu_guidance(h, w, bias, 0.0, 2.0, -2.0, 2.0)
    ref = torch.clamp(bias.float() + h.float() @ w.float().t(), -2.0, 2.0)
    assert_close_bf16(out, ref, "mu_guidance")


@pytest.mark.parametrize("K,N", [(768, 768), (2048, 2048), (1536, 1280)])
def test_tile_forms_agree_bit_for_bit(cdx, K, N):
    """The engine picks its tile form from the tile count: 128-row tiles (128 x 128, or
    128 x 64 for plain epilogues) when all of them are resident at once, else 256 x 64
    tiles (plain epilogues) when even 256 x 128 tiles number at most half the CUs,
    256 x 128 tiles when at most half as many 256 x 256 tiles as CUs, one 256 x 256 tile
    per block up to one per CU, the persistent form beyond.  Every form accumulates an
    output element over K in the same order, so rows are independent of the form: the
    first rows of a large product (persistent) equal the product of those rows alone
    (128-row tiles), of about 96 tiles' worth and of a middling batch (one tile per
    block), bit for bit.  Checked for the plain product, the product added to a
    residual (o_proj), the mu-QKV contraction (two K sources) and mu guidance (bias +
    clamp)."""
    from complexity_deep.attention import mu_qkv_project
    from complexity_deep.layer import mu_guidance
    from complexity_deep.linear import linear
    print(f"tile forms K={K} N={N}", flush=True)
    g = torch.Generator().manual_seed(K * 7 + N)
    nt = (N + 255) // 256
    big = 65536 if N <= 1280 else 32768  # far more 256 x 256 tiles than CUs: persistent
    mid = 256 * (192 // nt)              # about 192 tiles (256 CUs): one tile per block
    nar = 256 * -(-96 // nt)             # about 96 tiles: 256 x 128 tiles
    x = torch.randn(big, K, generator=g).to(bf16).cuda()
    w = (torch.randn(N, K, generator=g) * 0.05).to(bf16).cuda()
    full = linear(x, w)
    for rows in (256, nar, mid):
        assert torch.equal(linear(x[:rows].contiguous(), w), full[:rows]), f"linear rows={rows}"
    if K % 64 == 0 and N % 8 == 0:
        from complexity_deep.linear import linear_residual_
        r0 = torch.randn(big, N, generator=g).to(bf16).cuda()
        fr = linear_residual_(x, w, r0.clone())
        for rows in (256, nar, mid):
            part = linear_residual_(x[:rows].contiguous(), w, r0[:rows].clone())
            assert torch.equal(part, fr[:rows]), f"linear_residual rows={rows}"
    H = K // 2
    mu = torch.randn(big, H, generator=g).clamp(-2, 2).to(bf16).cuda()
    wq = (torch.randn(N, 2 * H, generator=g) * 0.05).to(bf16).cuda()
    fq = mu_qkv_project(x[:, :H].contiguous().view(1, big, H), mu.view(1, big, H), wq, H)
    for rows in (256, nar, mid):
        part = mu_qkv_project(x[:rows, :H].contiguous().view(1, rows, H), mu[:rows].contiguous().view(1, rows, H),
                              wq, H)
        assert torch.equal(part, fq[:, :rows]), f"mu_qkv rows={rows}"
    if N == K:
        wm = (torch.randn(N, K, generator=g) * 0.02).to(bf16).cuda()
        bias = torch.linspace(0.0, 2.0, N, device="cuda").to(bf16)
        fm = mu_guidance(x, wm, bias, 0.0, 2.0, -2.0, 2.0)
        for rows in (256, nar, mid):
            assert torch.equal(mu_guidance(x[:rows].contiguous(), wm, bias, 0.0, 2.0, -2.0, 2.0), fm[:rows]), \
                f"mu_guidance rows={rows}"
