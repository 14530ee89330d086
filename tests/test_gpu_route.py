"""GPU routing plan (cdx_route_plan) and row permutes: bit-exact against the C oracle.

Covers the token streams of configurations 1, 2, 4 and 5 (Zipf(1.1) ids with the
bin-packed map; the 90%-skew stress stream), block boundaries (1023/1024/1025
tokens), T = 0 and 1, E = 1 and 64, out-of-range ids (clamped) and expert ids given
directly (map = NULL, the sort_tokens_by_expert path).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _check(plan, ref):
    for k in ("expert_id", "perm", "inv_perm", "counts", "offsets"):
        got = getattr(plan, k).cpu().numpy().astype(np.int64)
        np.testing.assert_array_equal(got, ref[k].astype(np.int64), err_msg=k)


def _zipf_case(cfg):
    from complexity_deep import synthetic as syn
    name, B, S, E, seed = cfg
    ids = syn.zipf_token_ids(B, S, 32000, seed=seed)
    tmap = syn.binpacked_map(32000, E)
    return ids, tmap


@pytest.mark.parametrize("cfg", [("cfg1", 4, 512, 4, 0), ("cfg2", 1, 16384, 4, 0), ("cfg4", 8, 2048, 8, 1)])
def test_plan_zipf_configs(cdx, oracle, cfg):
    print(f"route plan {cfg}", flush=True)
    ids, tmap = _zipf_case(cfg)
    E = cfg[3]
    plan = cdx.route_plan(ids.cuda(), tmap.cuda(), E)
    _check(plan, oracle.route_plan(ids.numpy(), tmap.numpy(), E))


def test_plan_stress_cfg5(cdx, oracle):
    from complexity_deep import synthetic as syn
    print("route plan cfg5 stress", flush=True)
    tmap = syn.binpacked_map(32000, 8)
    ids = syn.routing_stress_ids(65536, tmap, 8, heavy=1, seed=0)
    plan = cdx.route_plan(ids.cuda(), tmap.cuda(), 8)
    ref = oracle.route_plan(ids.numpy(), tmap.numpy(), 8)
    _check(plan, ref)
    assert int(plan.counts[1]) == round(0.9 * 65536)


@pytest.mark.parametrize("T,V,E,seed", [(0, 10, 4, 0), (1, 10, 4, 1), (1023, 300, 4, 2), (1024, 300, 4, 3),
                                        (1025, 300, 8, 4), (4097, 50, 1, 5), (3000, 5000, 64, 6),
                                        (100000, 32000, 8, 7)])
def test_plan_edge_cases(cdx, oracle, T, V, E, seed):
    print(f"route plan T={T} V={V} E={E}", flush=True)
    rng = np.random.default_rng(seed)
    ids = rng.integers(-7, V + 7, size=T).astype(np.int64)
    tmap = rng.integers(0, E, size=V).astype(np.int64)
    plan = cdx.route_plan(torch.from_numpy(ids).cuda(), torch.from_numpy(tmap).cuda(), E)
    _check(plan, oracle.route_plan(ids, tmap, E))


def test_plan_direct_expert_ids(cdx, oracle):
    rng = np.random.default_rng(8)
    eids = rng.integers(0, 5, size=7777).astype(np.int64)
    plan = cdx.route_plan(torch.from_numpy(eids).cuda(), None, 5)
    _check(plan, oracle.route_plan(eids, None, 5))


def test_permute_roundtrip_and_sort_api(cdx, oracle):
    from complexity_deep.token_routed_mlp import permute_rows, unpermute_rows
    print("permute/unpermute + sort_tokens_by_expert", flush=True)
    rng = np.random.default_rng(9)
    T, H, E = 5000, 2048, 8
    eids = rng.integers(0, E, size=T).astype(np.int64)
    x = torch.randn(T, H).to(torch.bfloat16).cuda()
    e_dev = torch.from_numpy(eids).cuda()
    sorted_x, sorted_idx, offs, counts = cdx.sort_tokens_by_expert(x, e_dev, E)
    ref = oracle.route_plan(eids, None, E)
    assert sorted_idx.dtype == torch.int64 and offs.dtype == torch.int64 and counts.dtype == torch.int64
    np.testing.assert_array_equal(sorted_idx.cpu().numpy(), ref["perm"])
    np.testing.assert_array_equal(offs.cpu().numpy(), ref["offsets"])
    np.testing.assert_array_equal(counts.cpu().numpy(), ref["counts"])
    assert torch.equal(sorted_x, x[sorted_idx])
    perm = sorted_idx.to(torch.int32)
    back = unpermute_rows(sorted_x, perm)
    assert torch.equal(back, x)
    assert torch.equal(permute_rows(x, perm), sorted_x)


@pytest.mark.parametrize("T,E", [(256 * 1024, 64), (256 * 1024 + 1, 8), (300_000, 64), (1_000_003, 5)])
def test_plan_large_token_counts(cdx, oracle, T, E):
    """Token counts at and past 256 blocks of 1024, where each block walks several
    rounds of 1024 tokens; random ids over a 32000 map, E up to 64."""
    print(f"route plan large T={T} E={E}", flush=True)
    g = torch.Generator().manual_seed(T)
    ids = torch.randint(0, 32000, (T,), generator=g)
    tmap = torch.randint(0, E, (32000,), generator=g)
    plan = cdx.route_plan(ids.cuda(), tmap.cuda(), E)
    _check(plan, oracle.route_plan(ids.numpy(), tmap.numpy(), E))


@pytest.mark.parametrize("T,L,E,V", [(16384, 24, 8, 32000), (2048, 18, 4, 32000), (1025, 130, 8, 500),
                                     (0, 3, 4, 100), (777, 1, 64, 1000)])
def test_route_plans_each_map(cdx, oracle, T, L, E, V):
    """cdx_route_plans: plan y of one call equals the oracle's plan of map y over the
    same ids, for L maps (L = 130 crosses the 128-plans-per-launch chunk), with maps
    that are equal, permuted, degenerate (one expert) and random."""
    print(f"route plans T={T} L={L} E={E} V={V}", flush=True)
    g = torch.Generator().manual_seed(T + L)
    ids = torch.randint(-3, V + 3, (T,), generator=g)
    base = torch.randint(0, E, (V,), generator=g)
    maps = []
    for y in range(L):
        kind = y % 4
        if kind == 0:
            m = base.clone()
        elif kind == 1:
            m = (base + y) % E
        elif kind == 2:
            m = torch.full((V,), y % E, dtype=torch.long)
        else:
            m = torch.randint(0, E, (V,), generator=g)
        maps.append(m)
    plans = cdx.route_plans(ids.cuda(), [m.cuda() for m in maps], E)
    assert len(plans) == L
    for y, (plan, m) in enumerate(zip(plans, maps)):
        _check(plan, oracle.route_plan(ids.numpy(), m.numpy(), E))


@pytest.mark.parametrize("W,dtype,offset", [(3, torch.bfloat16, 0), (5, torch.float32, 0), (7, torch.uint8, 1),
                                             (12, torch.int16, 1), (2048, torch.bfloat16, 1)])
def test_permute_rows_any_width(cdx, W, dtype, offset):
    """Rows that are not whole 16-byte vectors, or whose base is not 16-byte aligned
    (a slice one element in), gather and scatter exactly, as tokens[sorted_indices]
    does for any token matrix (cuda/triton_token_routed.py:55)."""
    from complexity_deep.token_routed_mlp import permute_rows, unpermute_rows
    print(f"permute rows W={W} {dtype} offset={offset}", flush=True)
    T = 3001
    g = torch.Generator().manual_seed(W)
    if dtype.is_floating_point:
        full = torch.randn(T * W + offset, generator=g).to(dtype)
    else:
        full = torch.randint(0, 100, (T * W + offset,), generator=g).to(dtype)
    x = full[offset:].view(T, W).cuda() if offset == 0 else full.cuda()[offset:].view(T, W)
    perm = torch.randperm(T, generator=g).to(torch.int32).cuda()
    out = permute_rows(x, perm)
    assert torch.equal(out, x[perm.long()])
    assert torch.equal(unpermute_rows(out, perm), x)
    eids = torch.randint(0, 5, (T,), generator=g).cuda()
    sorted_x, idx, _, _ = cdx.sort_tokens_by_expert(x.reshape(T, W), eids, 5)
    assert torch.equal(sorted_x, x[idx])
