"""Pins the fp32 oracle (oracle/oracle.py) against independent statements.

rms_norm / add_rms_norm   torch.nn.functional.rms_norm (library routine); a constant
                          row normalises to +-weight; residual 0 reduces to the plain
                          norm; the residual sum is returned unnormalised.
mu_qkv                    separate fp64 F.linear terms x Wq^T + mu Wmu_q^T (the
                          concatenated contraction must equal the sum form);
                          mu = 0 reduces to the plain projection; operands are not
                          transposed or swapped (asymmetric shapes).
token_routed_mlp          per-token fp64 brute force with the token's own expert;
                          permutation invariance over tokens; clamping of ids; the
                          token_ids=None average-all path against its closed form.
grouped_gemm              per-row brute force.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F


def test_rms_norm_vs_library(oracle):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(37, 96, generator=g)
    w = torch.randn(96, generator=g)
    ref = F.rms_norm(x, (96,), w, eps=1e-6)
    torch.testing.assert_close(oracle.rms_norm(x, w, 1e-6), ref, rtol=1e-6, atol=1e-6)
    # larger eps matters and is added inside the sqrt
    torch.testing.assert_close(oracle.rms_norm(x * 1e-3, w, 1e-2), F.rms_norm(x * 1e-3, (96,), w, eps=1e-2),
                               rtol=1e-6, atol=1e-7)


def test_rms_norm_special_cases(oracle):
    w = torch.linspace(-2, 2, 64)
    for c in (3.0, -0.5):
        y = oracle.rms_norm(torch.full((2, 64), c), w, 0.0)
        torch.testing.assert_close(y, (w * np.sign(c)).expand(2, 64), rtol=1e-6, atol=1e-6)
    x = torch.randn(5, 64)
    y, h = oracle.add_rms_norm(x, torch.zeros_like(x), w)
    torch.testing.assert_close(y, oracle.rms_norm(x, w))
    r = torch.randn(5, 64)
    y, h = oracle.add_rms_norm(x, r, w)
    torch.testing.assert_close(h, x + r)
    torch.testing.assert_close(y, F.rms_norm(x + r, (64,), w, eps=1e-6), rtol=1e-6, atol=1e-6)


def test_mu_qkv_vs_sum_form(oracle):
    g = torch.Generator().manual_seed(1)
    T, H, qd, kvd = 11, 32, 48, 16
    x, mu = torch.randn(T, H, generator=g), torch.randn(T, H, generator=g)
    ws = [torch.randn(d, H, generator=g) for d in (qd, kvd, kvd, qd, kvd, kvd)]
    q, k, v = oracle.mu_qkv(x, mu, *ws)
    d = torch.float64
    for out, w, wm in ((q, ws[0], ws[3]), (k, ws[1], ws[4]), (v, ws[2], ws[5])):
        ref = F.linear(x.to(d), w.to(d)) + F.linear(mu.to(d), wm.to(d))
        torch.testing.assert_close(out.to(d), ref, rtol=1e-5, atol=1e-5)
    q0, k0, v0 = oracle.mu_qkv(x, torch.zeros_like(mu), *ws)
    torch.testing.assert_close(q0, x @ ws[0].t(), rtol=1e-6, atol=1e-5)
    qn, _, _ = oracle.mu_qkv(x, None, *ws[:3], None, None, None)
    torch.testing.assert_close(qn, x @ ws[0].t())
    # broadcast mu row (layer 0's mu_init.expand)
    qb, _, _ = oracle.mu_qkv(x, mu[:1], *ws)
    torch.testing.assert_close(qb, x @ ws[0].t() + mu[:1] @ ws[3].t(), rtol=1e-5, atol=1e-5)


def _brute_moe(x, ids, tmap, gw, uw, dw, sg, su, sd, V):
    x = x.double()
    out = torch.zeros_like(x)
    for t in range(x.shape[0]):
        e = int(tmap[min(max(int(ids[t]), 0), V - 1)])
        a = F.silu(x[t] @ gw[e].double()) * (x[t] @ uw[e].double())
        y = a @ dw[e].double()
        if sg is not None:
            s = F.silu(sg.double() @ x[t]) * (su.double() @ x[t])
            y = y + sd.double() @ s
        out[t] = y
    return out


@pytest.mark.parametrize("shared", [True, False])
def test_token_routed_mlp_brute_force(oracle, shared):
    g = torch.Generator().manual_seed(2)
    T, H, ie, E, V = 40, 24, 12, 3, 50
    x = torch.randn(T, H, generator=g)
    ids = torch.randint(-3, V + 3, (T,), generator=g)
    tmap = torch.randint(0, E, (V,), generator=g)
    gw, uw = torch.randn(E, H, ie, generator=g), torch.randn(E, H, ie, generator=g)
    dw = torch.randn(E, ie, H, generator=g)
    sg, su, sd = (torch.randn(ie, H, generator=g), torch.randn(ie, H, generator=g),
                  torch.randn(H, ie, generator=g)) if shared else (None, None, None)
    out = oracle.token_routed_mlp(x, ids, tmap.numpy(), gw, uw, dw, sg, su, sd)
    ref = _brute_moe(x, ids, tmap, gw, uw, dw, sg, su, sd, V)
    torch.testing.assert_close(out.double(), ref, rtol=1e-5, atol=1e-4)
    # permutation invariance over tokens
    p = torch.randperm(T, generator=g)
    outp = oracle.token_routed_mlp(x[p], ids[p], tmap.numpy(), gw, uw, dw, sg, su, sd)
    torch.testing.assert_close(outp, out[p], rtol=1e-5, atol=1e-5)


def test_token_routed_mlp_average_all(oracle):
    g = torch.Generator().manual_seed(3)
    T, H, ie, E = 9, 16, 8, 4
    x = torch.randn(T, H, generator=g)
    gw, uw, dw = torch.randn(E, H, ie, generator=g), torch.randn(E, H, ie, generator=g), torch.randn(E, ie, H, generator=g)
    sg, su, sd = torch.randn(ie, H, generator=g), torch.randn(ie, H, generator=g), torch.randn(H, ie, generator=g)
    out = oracle.token_routed_mlp(x, None, None, gw, uw, dw, sg, su, sd)
    xd = x.double()
    ref = sum((F.silu(xd @ gw[e].double()) * (xd @ uw[e].double())) @ dw[e].double() for e in range(E)) / E
    ref = ref + (F.silu(xd @ sg.double().t()) * (xd @ su.double().t())) @ sd.double().t()
    torch.testing.assert_close(out.double(), ref, rtol=1e-5, atol=1e-4)


def test_grouped_gemm_brute_force(oracle):
    g = torch.Generator().manual_seed(4)
    offs = np.array([0, 3, 3, 10, 16])
    a = torch.randn(16, 8, generator=g)
    w = torch.randn(4, 8, 5, generator=g)
    out = oracle.grouped_gemm(a, w, offs)
    for r in range(16):
        e = int(np.searchsorted(offs, r, side="right") - 1)
        torch.testing.assert_close(out[r], a[r] @ w[e], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("nq,nkv,S,D", [(4, 2, 37, 16), (6, 6, 20, 8), (8, 2, 64, 32)])
def test_causal_attention_vs_library_sdpa(oracle, nq, nkv, S, D):
    """The attention core against torch's scaled_dot_product_attention(is_causal=True)
    (a library routine) on repeated K/V heads, and the causal property: the output for
    query s does not change when keys/values after s are perturbed."""
    g = torch.Generator().manual_seed(S)
    q = torch.randn(2, nq, S, D, generator=g, dtype=torch.float64)
    k = torch.randn(2, nkv, S, D, generator=g, dtype=torch.float64)
    v = torch.randn(2, nkv, S, D, generator=g, dtype=torch.float64)
    out = oracle.causal_attention(q, k, v)
    rep = nq // nkv
    lib = torch.nn.functional.scaled_dot_product_attention(
        q, k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1), is_causal=True)
    lib = lib.transpose(1, 2).reshape(2, S, nq * D).float()
    assert torch.allclose(out, lib, atol=1e-5, rtol=1e-5)
    s = S // 2
    k2, v2 = k.clone(), v.clone()
    k2[:, :, s + 1:] += 3.0
    v2[:, :, s + 1:] -= 5.0
    out2 = oracle.causal_attention(q, k2, v2)
    assert torch.allclose(out[:, : s + 1], out2[:, : s + 1], atol=1e-6)
    assert not torch.allclose(out[:, s + 1:], out2[:, s + 1:])
