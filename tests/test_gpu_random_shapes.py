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
  * the add + RMSNorm: oracle.add_rms_norm, and the bf16 add bit for bit;
  * layer 0's folded projection (a broadcast mu row): the unfolded K = 2H contraction;
  * the norm and mu guidance writing into the halves of a [T, 2H] buffer: their
    contiguous outputs, bit for bit.
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


def _rope_unfolded(x, mu_row, w_pack, H, nq, nkv, D, qn, kn, table, pos0, vt):
    """cdx_mu_qkv_rope_fwd with the broadcast row at ldmu = 0: the K = 2H contraction."""
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
        nkv, D, nat.ptr(qn), nat.ptr(kn), 1e-6, table.data_ptr(), table.shape[0], pos0, q.data_ptr(),
        k.data_ptr(), v.data_ptr(), vt_ld, nat.stream_of(x)), "cdx_mu_qkv_rope_fwd")
    return q, k, v


@pytest.mark.parametrize("case", range(8))
def test_random_broadcast_mu_fold(cdx, case):
    """Layer 0's folded projection (cdx_mu_qkv_rope_bcast_fwd, through mu_qkv_rope with a
    broadcast row) against the unfolded K = 2H contraction on random shapes: bit for bit
    for a one-hot mu row (the bias is then one column of W_mu exactly), within 1 bf16
    ulp plus 2^-14 of the largest output for a random row (the bias's fp32 summation
    order differs)."""
    from complexity_deep.attention import mu_qkv_rope
    from complexity_deep.rotary import RotaryEmbedding
    rng = random.Random(7000 + case)
    D = rng.choice([32, 64, 128])
    nkv = rng.choice([1, 2, 4])
    nq = nkv * rng.choice([1, 2, 4])
    while nq * D <= 64 or (nq * D) % 64:
        nq *= 2
    H = nq * D
    B = rng.randint(1, 4)
    S = _log_int(rng, 1, 600)
    pos0 = rng.choice([0, 0, rng.randint(1, 50)])
    vt = pos0 == 0 and rng.random() < 0.5
    qk_norm = rng.random() < 0.8
    print(f"broadcast fold case {case}: B={B} S={S} H={H} heads={nq}/{nkv} D={D} pos0={pos0} vt={vt} "
          f"qk_norm={qk_norm}", flush=True)
    g = torch.Generator().manual_seed(case)
    x = torch.randn(B, S, H, generator=g).to(bf16).cuda()
    N = (nq + 2 * nkv) * D
    w_pack = (torch.randn(N, 2 * H, generator=g) * H ** -0.5).to(bf16).cuda()
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16).cuda() if qk_norm else None
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(bf16).cuda() if qk_norm else None
    table = RotaryEmbedding(D).cuda().cos_sin_table(pos0 + S, torch.device("cuda"))

    def both(mu_row):
        a = mu_qkv_rope(x, mu_row.expand(B, S, H), w_pack, H, nq, nkv, D, qn, kn, 1e-6, table, pos0, v_transposed=vt)
        b = _rope_unfolded(x, mu_row, w_pack, H, nq, nkv, D, qn, kn, table, pos0, vt)
        # (V^T buffers: both hold zeros in every column no token maps to)
        return list(zip(a, b))

    one_hot = torch.zeros(1, 1, H, dtype=bf16, device="cuda")
    one_hot[..., rng.randrange(H)] = rng.choice([1.0, -2.0, 0.5])
    for (a, b), what in zip(both(one_hot), "qkv"):
        assert torch.equal(a, b), f"one-hot mu: {what} differs from the unfolded contraction"
    mu_row = torch.randn(1, 1, H, generator=g).clamp(-2, 2).to(bf16).cuda()
    for (a, b), what in zip(both(mu_row), "qkv"):
        a, b = a.float(), b.float()
        ulp = torch.where(b == 0, torch.zeros_like(b), 2.0 ** (torch.floor(torch.log2(b.abs())) - 7))
        excess = float(((a - b).abs() - ulp - 2.0 ** -14 * b.abs().max()).max())
        assert excess <= 0, f"random mu: {what} off the unfolded contraction by {excess:.3g} beyond the bound"


@pytest.mark.parametrize("case", range(6))
def test_random_norm_and_mu_guidance_into_a_pair(cdx, case):
    """The model's side-by-side writers on random shapes: the plain norm into the left
    half and mu guidance into the right half of a [T, 2H] buffer (rows at stride 2H)
    give the bits of their contiguous outputs and leave the other half alone."""
    from complexity_deep.layer import mu_guidance
    from complexity_deep.normalization import rms_norm
    rng = random.Random(8000 + case)
    T = _log_int(rng, 1, 20000)
    H = 64 * _log_int(rng, 1, 64)
    print(f"pair writers case {case}: T={T} H={H}", flush=True)
    g = torch.Generator().manual_seed(case)
    h = torch.randn(T, H, generator=g).to(bf16).cuda()
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(bf16).cuda()
    w = (torch.randn(H, H, generator=g) * H ** -0.5).to(bf16).cuda()
    mu_param = (torch.rand(H, generator=g) * 3 - 0.5).to(bf16).cuda()
    pair = torch.full((T, 2 * H), -3.0, dtype=bf16, device="cuda")
    rms_norm(h, nw, 1e-6, out=pair[:, :H])
    mu_guidance(h, w, mu_param, 0.0, 2.0, -2.0, 2.0, out=pair[:, H:])
    x_ref = rms_norm(h, nw, 1e-6)
    mu_ref = mu_guidance(h, w, mu_param, 0.0, 2.0, -2.0, 2.0)
    torch.cuda.synchronize()
    assert torch.equal(pair[:, :H], x_ref), f"norm into a pair T={T} H={H}"
    assert torch.equal(pair[:, H:], mu_ref), f"mu guidance into a pair T={T} H={H}"
