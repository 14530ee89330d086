"""Seeded random shapes through the kernels' entry points.

Every case draws its shape from a fixed seed (its index), so a failure names a case
that reruns the same way.  Sizes are log-uniform, and every few cases are drawn large
with whole 256 x 256 tiles, so that the draws straddle the thresholds at which the GEMM
engine changes tile form (128-row tiles, 256 x 64, 256 x 128, one 256 x 256 tile per
block, persistent tiles) as well as partial tiles in every dimension; the MoE draws
cover its layouts (empty experts, single tokens, ragged segments, per-expert and
segmented down-pass tiles, with and without the shared expert).

References, on the same bf16 inputs:
  * the plain products (linear, linear + residual, mu-QKV, mu guidance): fp32 products
    in torch on the GPU;
  * the MoE: oracle.token_routed_mlp (fp32, pinned by a per-token brute force);
  * attention: oracle.causal_attention (fp32, pinned by SDPA);
  * the add + RMSNorm: oracle.add_rms_norm, and the bf16 add bit for bit.
Bound: the bf16 tolerance of the north star (max rel err <= 2e-2 normwise, mean abs err
<= 1e-3 against the fp32 reference rounded to bf16), checked by ``assert_close_bf16``.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu
bf16 = torch.bfloat16


def _log_int(rng: random.Random, lo: int, hi: int) -> int:
    """An integer in [lo, hi], log-uniform (small and large sizes alike)."""
    return min(hi, max(lo, int(math.exp(rng.uniform(math.log(lo), math.log(hi + 1))))))


def _data(seed: int, *shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(bf16).cuda()


@pytest.mark.parametrize("case", range(24))
def test_random_linear_and_residual(cdx, case):
    from complexity_deep.linear import linear, linear_residual_
    rng = random.Random(1000 + case)
    K = 64 * _log_int(rng, 1, 64)
    if case % 4 == 0:    # whole tiles, more of them than CUs: the persistent form
        M, N = 256 * rng.randint(16, 78), 256 * rng.randint(8, 32)
    elif case % 4 == 1:  # large, ragged
        M, N = _log_int(rng, 4096, 20000), 8 * _log_int(rng, 256, 1024)
    else:
        M, N = _log_int(rng, 1, 20000), 8 * _log_int(rng, 1, 1024)
    print(f"linear case {case}: M={M} K={K} N={N}", flush=True)
    x = _data(case, M, K)
    w = _data(case + 1, N, K, scale=K ** -0.5)
    ref = x.float() @ w.float().t()
    prod = linear(x, w)
    assert_close_bf16(prod, ref, f"linear {M}x{K}x{N}")
    r = _data(case + 2, M, N)
    got = linear_residual_(x, w, r.clone())
    # the engine's product (the same accumulation whatever the tile form) rounded to
    # bf16, then the bf16 add: the reference's two roundings
    assert torch.equal(got, r + prod), f"linear_residual {M}x{K}x{N}"


@pytest.mark.parametrize("case", range(12))
def test_random_mu_qkv(cdx, case):
    from complexity_deep.attention import mu_qkv_project
    rng = random.Random(2000 + case)
    H = 64 * _log_int(rng, 1, 32)
    if case % 3 == 0:
        M, N = 256 * rng.randint(16, 64), 256 * rng.randint(4, 24)
    else:
        M, N = _log_int(rng, 1, 16384), 8 * _log_int(rng, 1, 768)
    broadcast = rng.random() < 0.3
    print(f"mu_qkv case {case}: M={M} H={H} N={N} broadcast_mu={broadcast}", flush=True)
    x = _data(case, 1, M, H)
    mu = _data(case + 1, 1, 1 if broadcast else M, H).clamp(-2, 2)
    w = _data(case + 2, N, 2 * H, scale=(2 * H) ** -0.5)
    got = mu_qkv_project(x, mu.expand(1, M, H), w, H)
    ref = x.float().view(M, H) @ w[:, :H].float().t() + mu.float().view(-1, H) @ w[:, H:].float().t()
    assert_close_bf16(got.view(M, N), ref, f"mu_qkv {M}x{2 * H}x{N}")


@pytest.mark.parametrize("case", range(10))
def test_random_mu_guidance(cdx, case):
    from complexity_deep.layer import mu_guidance
    rng = random.Random(3000 + case)
    if case % 3 == 0:
        T, H = 256 * rng.randint(16, 80), 256 * rng.randint(1, 8)
    else:
        T, H = _log_int(rng, 1, 20000), 64 * _log_int(rng, 1, 32)
    print(f"mu_guidance case {case}: T={T} H={H}", flush=True)
    h = _data(case, T, H)
    w = _data(case + 1, H, H, scale=H ** -0.5)
    mu = _data(case + 2, H)
    got = mu_guidance(h, w, mu, 0.0, 2.0, -2.0, 2.0)
    ref = torch.clamp(h.float() @ w.float().t() + mu.float().clamp(0.0, 2.0), -2.0, 2.0)
    assert_close_bf16(got, ref, f"mu_guidance {T}x{H}")


@pytest.mark.parametrize("case", range(12))
def test_random_moe(cdx, oracle, case):
    rng = random.Random(4000 + case)
    E = rng.choice([1, 2, 3, 4, 8, 16])
    H = 64 * _log_int(rng, 1, 16)
    if case % 3 == 0:  # many tiles, 2 P a multiple of 256 (P = Ie padded to 64): persistent gate/up
        T, Ie = rng.randint(8192, 16384), 128 * rng.randint(2, 8) - rng.randrange(0, 64, 8)
    else:
        T, Ie = _log_int(rng, 1, 8192), 8 * _log_int(rng, 8, 128)
    V = _log_int(rng, max(E, 2), 1000)
    shared = rng.random() < 0.7
    print(f"moe case {case}: T={T} H={H} Ie={Ie} E={E} V={V} shared={shared}", flush=True)
    torch.manual_seed(case)
    m = cdx.TokenRoutedMLP(H, Ie * E, num_experts=E, vocab_size=V, shared_expert=shared)
    g = torch.Generator().manual_seed(case)
    tmap = torch.randint(0, E, (V,), generator=g)
    if E > 2:
        tmap[tmap == rng.randrange(E)] = 0  # an expert without tokens
    with torch.no_grad():
        m.token_to_expert.copy_(tmap)
        m.down_proj_w.normal_(0, 0.02, generator=g)
        if shared:
            for lin in (m.shared_gate, m.shared_up, m.shared_down):
                lin.weight.normal_(0, 0.02, generator=g)
    m = m.to(bf16).cuda()
    ids = torch.randint(0, V, (1, T), generator=g)
    x = torch.randn(1, T, H, generator=g).to(bf16)
    with torch.no_grad():
        got = m(x.cuda(), token_ids=ids.cuda())
    ref = oracle.token_routed_mlp(
        x.float(), ids, m.token_to_expert.cpu().numpy(), m.gate_proj_w.float().cpu(), m.up_proj_w.float().cpu(),
        m.down_proj_w.float().cpu(), m.shared_gate.weight.float().cpu() if shared else None,
        m.shared_up.weight.float().cpu() if shared else None, m.shared_down.weight.float().cpu() if shared else None)
    assert_close_bf16(got, ref, f"moe T={T} H={H} Ie={Ie} E={E}")


@pytest.mark.parametrize("case", range(10))
def test_random_attention(cdx, oracle, case):
    from complexity_deep.attention import causal_attention, to_vt_layout
    rng = random.Random(5000 + case)
    B = rng.randint(1, 4)
    D = rng.choice([32, 64, 128])
    nkv = rng.choice([1, 2, 4, 8])
    nq = nkv * rng.choice([1, 2, 4])
    S = _log_int(rng, 1, 1500)
    print(f"attention case {case}: B={B} heads={nq}/{nkv} S={S} D={D}", flush=True)
    g = torch.Generator().manual_seed(case)
    q = torch.randn(B, nq, S, D, generator=g).to(bf16)
    k = torch.randn(B, nkv, S, D, generator=g).to(bf16)
    v = torch.randn(B, nkv, S, D, generator=g).to(bf16)
    got = causal_attention(q.cuda(), k.cuda(), to_vt_layout(v.cuda()))
    ref = oracle.causal_attention(q, k, v)
    assert_close_bf16(got, ref, f"attention B={B} {nq}/{nkv} S={S} D={D}")


@pytest.mark.parametrize("case", range(8))
def test_random_add_rmsnorm(cdx, oracle, case):
    from complexity_deep.normalization import add_rms_norm
    rng = random.Random(6000 + case)
    T = _log_int(rng, 1, 20000)
    H = 8 * _log_int(rng, 1, 1024)
    print(f"add_rmsnorm case {case}: T={T} H={H}", flush=True)
    g = torch.Generator().manual_seed(case)
    x = torch.randn(T, H, generator=g).to(bf16)
    r = torch.randn(T, H, generator=g).to(bf16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(bf16)
    y, h = add_rms_norm(x.cuda(), r.cuda(), w.cuda(), 1e-6)
    h_ref = x + r  # the reference's bf16 add
    assert torch.equal(h.cpu(), h_ref), f"bf16 add T={T} H={H}"
    y_ref, _ = oracle.add_rms_norm(h_ref.float(), torch.zeros(T, H), w.float(), 1e-6)
    assert_close_bf16(y, y_ref, f"add_rmsnorm T={T} H={H}")
