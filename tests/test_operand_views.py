"""CPU checks of what the forward hands the kernels (no GPU needed):

* every routed layer routes through its own ``token_to_expert`` buffer, looked up at
  each call, so a write to one layer's map (through ``.data`` too) reaches that
  layer's plan and no other (reference: core/token_routed_mlp.py:149-150, called per
  layer from core/layer.py:180; the ablation pattern of run_ablations.py:81-97);
* the MLP weights are views of the kernel operands in the layout include/cdx.h
  documents for cdx_moe_swiglu_fwd (w_gu [NB, 2, P, H], w_down [NB, H, P], block 0
  the shared expert, padding zero), so any write to a weight is a write to the
  operand, and a moved or cast module is re-bound with its values intact.
"""

from __future__ import annotations

import torch

import complexity_deep as cdx
from complexity_deep import modeling
from complexity_deep.token_routed_mlp import padded_width


def _small(layers=3, E=4, V=512, H=128, I=352, shared=True):
    cfg = cdx.ComplexityConfig(vocab_size=V, hidden_size=H, intermediate_size=I, num_hidden_layers=layers,
                               num_attention_heads=2, num_key_value_heads=1, num_experts=E, shared_expert=shared)
    torch.manual_seed(0)
    return cdx.ComplexityModel(cfg)


def test_each_layer_routes_through_its_own_map(monkeypatch):
    m = _small()
    seen = []
    monkeypatch.setattr(modeling, "route_plans", lambda ids, maps, E: seen.append((list(maps), E)) or [None] * len(maps))
    ids = torch.zeros(1, 4, dtype=torch.long)
    m.route_plans(ids)
    (maps, E), = seen
    assert E == 4 and len(maps) == 3
    for layer, mp in zip(m.layers, maps):
        assert mp is layer.mlp.token_to_expert
    # The verdict's demonstration: equal maps, then layer 1's zeroed through .data.
    assert all(torch.equal(maps[0], mp) for mp in maps)
    m.layers[1].mlp.token_to_expert.data.zero_()
    seen.clear()
    m.route_plans(ids)
    (maps, _), = seen
    assert maps[1] is m.layers[1].mlp.token_to_expert and int(maps[1].abs().sum()) == 0
    assert not torch.equal(maps[0], maps[1]) and torch.equal(maps[0], maps[2])
    # A map replaced outright is picked up too.
    new = torch.arange(512) % 2
    m.layers[2].mlp.token_to_expert = new
    seen.clear()
    m.route_plans(ids)
    assert seen[0][0][2] is new


def test_moe_weights_are_views_of_the_operands():
    torch.manual_seed(1)
    E, H, I = 3, 128, 3 * 176  # Ie = 176 -> P = 192: padding columns
    mlp = cdx.TokenRoutedMLP(H, I, num_experts=E, vocab_size=64, shared_expert=True)
    before = {k: v.clone() for k, v in mlp.state_dict().items()}
    w_gu, w_down = mlp.kernel_weights()
    P, ie = padded_width(176), 176
    assert w_gu.shape == (E + 1, 2, P, H) and w_down.shape == (E + 1, H, P)
    # Values kept, layout as documented.
    for k, v in mlp.state_dict().items():
        assert torch.equal(v, before[k]), k
    for e in range(E):
        assert torch.equal(w_gu[1 + e, 0, :ie], mlp.gate_proj_w[e].t())
        assert torch.equal(w_gu[1 + e, 1, :ie], mlp.up_proj_w[e].t())
        assert torch.equal(w_down[1 + e, :, :ie], mlp.down_proj_w[e].t())
    assert torch.equal(w_gu[0, 0, :ie], mlp.shared_gate.weight)
    assert torch.equal(w_gu[0, 1, :ie], mlp.shared_up.weight)
    assert torch.equal(w_down[0, :, :ie], mlp.shared_down.weight)
    assert int(torch.count_nonzero(w_gu[:, :, ie:])) == 0 and int(torch.count_nonzero(w_down[:, :, ie:])) == 0
    # Writes through .data (no version bump) land in the operands.
    mlp.gate_proj_w.data[2, 5, 7] = 3.0
    mlp.down_proj_w.data[0].zero_()
    mlp.shared_down.weight.data[9, 11] = -2.0
    assert float(w_gu[3, 0, 7, 5]) == 3.0
    assert int(torch.count_nonzero(w_down[1, :, :ie])) == 0
    assert float(w_down[0, 9, 11]) == -2.0
    assert mlp.kernel_weights()[0] is w_gu  # nothing re-bound
    # A cast re-binds into new operands with the same values.
    snap = {k: v.clone() for k, v in mlp.state_dict().items()}
    mlp = mlp.double()
    g2, d2 = mlp.kernel_weights()
    assert g2.dtype == torch.float64 and g2.data_ptr() != w_gu.data_ptr()
    for k, v in mlp.state_dict().items():
        assert torch.equal(v, snap[k].double()), k
    assert mlp.gate_proj_w.data_ptr() == g2[1, 0].data_ptr()


def test_dense_swiglu_weights_are_views():
    torch.manual_seed(2)
    mlp = cdx.SwiGLU(128, 200)
    w_gu, w_down = mlp.kernel_weights()
    assert w_gu.shape == (1, 2, 256, 128) and w_down.shape == (1, 128, 256)
    assert torch.equal(w_gu[0, 0, :200], mlp.gate_proj.weight)
    assert torch.equal(w_gu[0, 1, :200], mlp.up_proj.weight)
    assert torch.equal(w_down[0, :, :200], mlp.down_proj.weight)
    mlp.up_proj.weight.data.fill_(0.5)
    assert torch.all(w_gu[0, 1, :200] == 0.5) and int(torch.count_nonzero(w_gu[0, 1, 200:])) == 0


def test_state_dict_round_trip_of_bound_weights(tmp_path):
    m = _small(layers=2)
    for layer in m.layers:
        layer.mlp.kernel_weights()
    sd = {k: v.clone() for k, v in m.state_dict().items()}
    m.save_pretrained(str(tmp_path))
    m2 = cdx.ComplexityModel.from_pretrained(str(tmp_path))
    for k, v in m2.state_dict().items():
        assert torch.equal(v, sd[k]), k
    # loading into a bound model writes through the views
    m3 = _small(layers=2)
    for layer in m3.layers:
        layer.mlp.kernel_weights()
    g = m3.layers[1].mlp._operands.bufs[0]
    m3.load_state_dict(sd)
    assert m3.layers[1].mlp._operands.bufs[0] is g
    assert torch.equal(g[1, 0, :88], sd["layers.1.mlp.gate_proj_w"][0].t())
