"""GPU parity of the mu-guided QKV contraction (cdx_mu_qkv_fwd).

Against the fp32 oracle on the CPU (configuration 1's shape and ragged shapes) and,
at configuration 3's full size (32768 x [2048 | 2048] -> 4096), against a torch
fp32 GPU matmul of the same bf16 operands (a plain fp32 reference of the same op).
Covers mu = None, the broadcast mu row of layer 0 (row stride 0), M and N that are
not tile multiples, and the module / operator APIs.
"""

from __future__ import annotations

import pytest
import torch

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu
bf16 = torch.bfloat16


def _weights(H, qd, kvd, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(d, H, generator=g) * std).to(bf16) for d in (qd, kvd, kvd, qd, kvd, kvd)]


def _pack(ws, H, with_mu=True):
    wx = torch.cat(ws[:3], 0)
    return torch.cat([wx, torch.cat(ws[3:], 0)], 1).contiguous() if with_mu else wx.contiguous()


@pytest.mark.parametrize("M,H,qd,kvd", [(2048, 768, 768, 256), (77, 128, 128, 64), (1, 64, 64, 32),
                                        (300, 256, 256, 128), (513, 512, 256, 132)])
def test_mu_qkv_matches_oracle(cdx, oracle, M, H, qd, kvd):
    from complexity_deep.attention import mu_qkv_project
    print(f"mu_qkv M={M} H={H} q={qd} kv={kvd}", flush=True)
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, H, generator=g).to(bf16)
    mu = torch.randn(M, H, generator=g).clamp(-2, 2).to(bf16)
    ws = _weights(H, qd, kvd, M + 1)
    out = mu_qkv_project(x.cuda(), mu.cuda(), _pack(ws, H).cuda(), H)
    q, k, v = oracle.mu_qkv(x.float(), mu.float(), *[w.float() for w in ws])
    ref = torch.cat([q, k, v], 1)
    assert_close_bf16(out, ref, f"mu_qkv M={M}")
    # no mu: only the x half of the packed weight (row stride 2H)
    w_full = _pack(ws, H).cuda()
    out0 = mu_qkv_project(x.cuda(), None, w_full[:, :H], H)
    q0, k0, v0 = oracle.mu_qkv(x.float(), None, *[w.float() for w in ws[:3]], None, None, None)
    ref0 = torch.cat([q0, k0, v0], 1)
    assert_close_bf16(out0, ref0, "mu_qkv mu=None")


def test_mu_qkv_broadcast_mu_row(cdx, oracle):
    from complexity_deep.attention import mu_qkv_project
    B, S, H = 2, 100, 256
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, S, H, generator=g).to(bf16)
    mu_init = torch.randn(1, 1, H, generator=g).to(bf16)
    ws = _weights(H, 256, 128, 4)
    out = mu_qkv_project(x.cuda(), mu_init.cuda().expand(B, S, H), _pack(ws, H).cuda(), H)
    q, k, v = oracle.mu_qkv(x.float().view(-1, H), mu_init.float().view(1, H), *[w.float() for w in ws])
    ref = torch.cat([q, k, v], 1).view(B, S, -1)
    assert_close_bf16(out, ref, "broadcast mu")


def test_mu_qkv_cfg3_full_size(cdx):
    from complexity_deep.attention import mu_qkv_project
    print("mu_qkv cfg3 32768x4096x4096", flush=True)
    M, H, qd, kvd = 32768, 2048, 2048, 1024
    x = torch.randn(M, H, device="cuda").to(bf16)
    mu = torch.randn(M, H, device="cuda").to(bf16)
    w = (torch.randn(qd + 2 * kvd, 2 * H, device="cuda") * 0.02).to(bf16)
    out = mu_qkv_project(x, mu, w, H)
    ref = torch.cat([x, mu], 1).float() @ w.float().t()
    assert_close_bf16(out, ref, "mu_qkv cfg3")


def test_attention_projection_and_operator_api(cdx, oracle):
    print("ComplexityAttention.project_qkv / fused_mu_qkv_projection", flush=True)
    torch.manual_seed(0)
    attn = cdx.ComplexityAttention(256, 4, 2).to(bf16).cuda()
    B, S, H = 2, 64, 256
    x = torch.randn(B, S, H, device="cuda").to(bf16)
    mu = torch.randn(B, S, H, device="cuda").to(bf16)
    with torch.no_grad():
        packed = attn.project_qkv(x, mu)
        q, k, v = cdx.fused_mu_qkv_projection(
            x, mu, attn.q_proj.weight.t(), attn.k_proj.weight.t(), attn.v_proj.weight.t(),
            attn.mu_to_q.weight.t(), attn.mu_to_k.weight.t(), attn.mu_to_v.weight.t())
    assert torch.equal(torch.cat([q, k, v], -1), packed)
    ws = [getattr(attn, n).weight.float().cpu() for n in ("q_proj", "k_proj", "v_proj", "mu_to_q", "mu_to_k", "mu_to_v")]
    rq, rk, rv = oracle.mu_qkv(x.float().cpu(), mu.float().cpu(), *ws)
    ref = torch.cat([rq, rk, rv], -1)
    assert_close_bf16(packed, ref, "attention projection")


def test_mu_qkv_split_weight_buffers(cdx):
    """x and mu weights in two separate [N, H] buffers (the layout ComplexityAttention
    keeps, its Linear weights being views of them) give the same bits as the packed
    [N, 2H] form, for cdx_mu_qkv_fwd and cdx_mu_qkv_rope_fwd."""
    from complexity_deep.attention import mu_qkv_project, mu_qkv_rope
    from complexity_deep.rotary import RotaryEmbedding
    print("mu_qkv split weights", flush=True)
    B, S, H, nq, nkv, D = 2, 300, 512, 4, 2, 128
    g = torch.Generator().manual_seed(21)
    x = torch.randn(B, S, H, generator=g).to(bf16).cuda()
    mu = torch.randn(B, S, H, generator=g).clamp(-2, 2).to(bf16).cuda()
    ws = _weights(H, nq * D, nkv * D, 22)
    packed = _pack(ws, H).cuda()
    w_x = torch.cat(ws[:3], 0).cuda()
    w_mu = torch.cat(ws[3:], 0).cuda()
    assert torch.equal(mu_qkv_project(x, mu, w_x, H, w_mu=w_mu), mu_qkv_project(x, mu, packed, H))
    table = RotaryEmbedding(D).cos_sin_table(S, torch.device("cuda"))
    qn = torch.ones(D, dtype=bf16, device="cuda")
    a = mu_qkv_rope(x, mu, w_x, H, nq, nkv, D, qn, qn, 1e-6, table, 0, v_transposed=True, w_mu=w_mu)
    b = mu_qkv_rope(x, mu, packed, H, nq, nkv, D, qn, qn, 1e-6, table, 0, v_transposed=True)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
