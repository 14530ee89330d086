"""Golden vectors written from the reference package by tests/golden/make_golden.py.

* The product's CPU-side model construction (modeling.py / layer.py / ...) draws
  bit-identical weights to the reference for the same seed: every state_dict
  tensor's SHA-256 matches.  This pins init order, parameter shapes and keys.
* The oracle's fp32 forward, fed those weights and the same expert map, reproduces
  the reference's fp32 logits (pins the forward composition: norm placement, mu
  flow and clamps, QK-norm before RoPE, GQA, tied head).
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "model_golden.npz"


def _load():
    z = np.load(GOLDEN, allow_pickle=False)
    meta = json.loads(bytes(z["meta_json"]).decode())
    return z, meta


def _digest(t):
    return hashlib.sha256(t.detach().cpu().contiguous().numpy().tobytes()).hexdigest()


def _build(entry):
    from complexity_deep import ComplexityConfig, ComplexityModel
    torch.manual_seed(entry["seed"])
    return ComplexityModel(ComplexityConfig.from_dict(entry["cfg"]))


def _variants():
    _, meta = _load()
    return [m["name"] for m in meta]


@pytest.mark.parametrize("name", _variants())
def test_seeded_init_matches_reference(name):
    _, meta = _load()
    entry = next(m for m in meta if m["name"] == name)
    model = _build(entry)
    sd = model.state_dict()
    assert set(sd) == set(entry["hashes"]), "state_dict keys differ from the reference"
    bad = [k for k, t in sd.items() if _digest(t) != entry["hashes"][k]]
    assert not bad, f"tensors differing from the reference init: {bad[:5]}"


@pytest.mark.parametrize("name", _variants())
def test_oracle_forward_matches_reference_logits(oracle, name):
    z, meta = _load()
    entry = next(m for m in meta if m["name"] == name)
    model = _build(entry)
    sd = dict(model.state_dict())
    tmap = z[f"{name}/map"]
    if tmap.size:
        for i in range(entry["cfg"]["num_hidden_layers"]):
            sd[f"layers.{i}.mlp.token_to_expert"] = torch.from_numpy(tmap)
    ids = torch.from_numpy(z[f"{name}/ids"])
    logits = oracle.forward(sd, entry["cfg"], ids)
    ref = torch.from_numpy(z[f"{name}/logits"])
    torch.testing.assert_close(logits, ref, rtol=1e-4, atol=2e-5)
