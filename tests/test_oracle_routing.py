"""Pins the integer oracle (oracle/route_oracle.c) without retyping its formulas.

* bin-packing (token_routed_mlp.py:105-116): the C argmin loop against a
  pure-Python statement and against the product's native builder (cdx_binpack_map,
  a stable sort plus a (load, expert) min-heap: three independent implementations
  of the same greedy rule), plus the load-balance
  facts the Zipf(1.1) pmf fixes at V=32000: E=4 splits the mass exactly in four;
  E=8 leaves token 0 (14.2% of the mass) alone in expert 0; map[0..9] values.
* routing plan (token_routed_mlp.py:149-170, triton_token_routed.py:37-61): against
  numpy's stable argsort / bincount / cumsum and the invariants of a stable
  partition, including clamping and edge cases.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch


def zipf(V, s=1.1):
    k = np.arange(1, V + 1, dtype=np.float64)
    w = k ** (-s)
    return (w / w.sum()).astype(np.float32)


@pytest.mark.parametrize("V,E", [(1000, 2), (2000, 3), (3000, 4), (1500, 8), (64, 64)])
def test_binpack_c_matches_python_and_heap(oracle, V, E):
    from complexity_deep.token_routed_mlp import TokenRoutedMLP
    f = zipf(V)
    c = oracle.binpack_map(f, E)
    py = oracle.binpack_map_py(f, E)
    heap = TokenRoutedMLP._build_token_mapping(V, E, torch.from_numpy(f)).numpy()
    np.testing.assert_array_equal(c, py)
    np.testing.assert_array_equal(c, heap)


def test_binpack_with_ties_and_random_freqs(oracle):
    from complexity_deep.token_routed_mlp import TokenRoutedMLP
    rng = np.random.default_rng(3)
    f = rng.integers(0, 5, size=500).astype(np.float32)  # many ties
    for E in (2, 5, 7):
        c = oracle.binpack_map(f, E)
        np.testing.assert_array_equal(c, oracle.binpack_map_py(f, E))
        np.testing.assert_array_equal(c, TokenRoutedMLP._build_token_mapping(500, E, torch.from_numpy(f)).numpy())


@pytest.mark.parametrize("E", [8, 64])
def test_binpack_native_zipf_32000(oracle, E):
    """The 1B configuration's map (and a 64-expert one) from the native builder."""
    from complexity_deep.token_routed_mlp import TokenRoutedMLP
    f = zipf(32000)
    np.testing.assert_array_equal(oracle.binpack_map(f, E),
                                  TokenRoutedMLP._build_token_mapping(32000, E, torch.from_numpy(f)).numpy())


def test_binpack_native_negative_and_nan(oracle):
    from complexity_deep.token_routed_mlp import TokenRoutedMLP
    rng = np.random.default_rng(5)
    f = rng.normal(size=700).astype(np.float32)  # negative loads are legal arithmetic
    np.testing.assert_array_equal(oracle.binpack_map(f, 6), TokenRoutedMLP._build_token_mapping(700, 6, torch.from_numpy(f)).numpy())
    f[10] = np.nan
    with pytest.raises(RuntimeError, match="NaN"):
        TokenRoutedMLP._build_token_mapping(700, 6, torch.from_numpy(f))


def _loads(f, m, E):
    return np.array([f[m == e].astype(np.float64).sum() for e in range(E)])


def test_binpack_zipf_32000_facts(oracle):
    f = zipf(32000)
    m4 = oracle.binpack_map(f, 4)
    l4 = _loads(f, m4, 4)
    assert np.max(l4) / np.mean(l4) < 1.0001
    assert m4[:10].tolist() == [0, 1, 2, 3, 3, 2, 3, 2, 1, 3]
    m8 = oracle.binpack_map(f, 8)
    l8 = _loads(f, m8, 8)
    assert np.flatnonzero(m8 == 0).tolist() == [0]  # token 0 alone in expert 0
    assert abs(l8[0] - 0.1420) < 5e-4
    assert np.allclose(l8[1:], (1 - l8[0]) / 7, rtol=1e-3)
    assert m8[:10].tolist() == [0, 1, 2, 3, 4, 5, 6, 7, 7, 6]
    # modulo routing is what the reference falls back to without frequencies
    mm = oracle.modulo_map(32000, 4)
    np.testing.assert_array_equal(mm, np.arange(32000) % 4)
    lm = _loads(f, mm, 4)
    assert 1.32 < np.max(lm) / np.mean(lm) < 1.34


def _numpy_plan(ids, tmap, E, V):
    ids = np.asarray(ids, dtype=np.int64)
    if tmap is not None:
        e = tmap[np.clip(ids, 0, V - 1)]
    else:
        e = ids
    e = np.clip(e, 0, E - 1)
    perm = np.argsort(e, kind="stable")
    counts = np.bincount(e, minlength=E)
    offs = np.concatenate([[0], np.cumsum(counts)])
    return e, perm, counts, offs


def _check_plan(plan, ids, tmap, E, V):
    e, perm, counts, offs = _numpy_plan(ids, tmap, E, V)
    T = len(ids)
    np.testing.assert_array_equal(plan["expert_id"], e)
    np.testing.assert_array_equal(plan["perm"], perm)
    np.testing.assert_array_equal(plan["counts"], counts)
    np.testing.assert_array_equal(plan["offsets"], offs)
    inv = plan["inv_perm"]
    np.testing.assert_array_equal(inv[plan["perm"]], np.arange(T))
    # invariants of a stable partition
    assert plan["counts"].sum() == T
    srt = plan["expert_id"][plan["perm"]]
    assert np.all(np.diff(srt) >= 0)
    for x in range(E):
        seg = plan["perm"][offs[x]:offs[x + 1]]
        assert np.all(np.diff(seg) > 0)


@pytest.mark.parametrize("T,V,E,seed", [(0, 10, 4, 0), (1, 10, 4, 0), (1023, 500, 4, 1), (1025, 500, 8, 2),
                                        (5000, 32000, 8, 3), (4096, 100, 1, 4), (3000, 1000, 64, 5)])
def test_route_plan_matches_numpy(oracle, T, V, E, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(-5, V + 5, size=T)  # includes out-of-range ids (clamped)
    tmap = rng.integers(0, E, size=V).astype(np.int64)
    plan = oracle.route_plan(ids, tmap, E)
    _check_plan(plan, ids, tmap, E, V)


def test_route_plan_expert_ids_direct(oracle):
    rng = np.random.default_rng(7)
    eids = rng.integers(0, 6, size=2000)
    plan = oracle.route_plan(eids, None, 6)
    _check_plan(plan, eids, None, 6, 0)


def test_route_plan_skewed_stress(oracle):
    f = zipf(32000)
    tmap = oracle.binpack_map(f, 8)
    from complexity_deep.synthetic import routing_stress_ids
    ids = routing_stress_ids(65536, torch.from_numpy(tmap), 8, heavy=1, seed=0).numpy()
    plan = oracle.route_plan(ids, tmap, 8)
    _check_plan(plan, ids, tmap, 8, 32000)
    c = plan["counts"]
    assert c[1] == round(0.9 * 65536)
    assert all(c[e] == round(0.01 * 65536) for e in range(2, 8))
    assert c[0] == 65536 - c[1:].sum()  # expert 0 owns only the padding id 0


def test_model_set_token_frequencies(oracle):
    """ComplexityModel.set_token_frequencies installs the oracle's bin-packed map in
    every routed layer (and the map is what the state_dict saves)."""
    import complexity_deep as cd
    cfg = cd.ComplexityConfig.complexity_tiny()
    cfg.vocab_size = 1000
    torch.manual_seed(0)
    model = cd.ComplexityModel(cfg)
    f = zipf(cfg.vocab_size)
    tmap = model.set_token_frequencies(torch.from_numpy(f))
    want = oracle.binpack_map(f, cfg.num_experts)
    np.testing.assert_array_equal(tmap.numpy(), want)
    sd = model.state_dict()
    keys = [k for k in sd if k.endswith("mlp.token_to_expert")]
    assert keys and all(np.array_equal(sd[k].numpy(), want) for k in keys)
