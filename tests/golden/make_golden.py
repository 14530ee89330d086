"""Write tests/golden/model_golden.npz from the reference package.

Run in the build container only (the reference is not present on the GPU box):

    python tests/golden/make_golden.py

What it pins, for three tiny configurations that cover the config branches
(token-routed + shared + mu; routed without shared expert under modulo routing;
dense SwiGLU without mu guidance):

  * seeded initialisation: SHA-256 of every state_dict tensor after
    ``torch.manual_seed(seed); ComplexityModel(cfg)`` (models/modeling.py:69-149,
    the RNG consumption order nothing else fixes);
  * the end-to-end fp32 CPU forward: logits for a fixed token batch with a fixed
    expert map installed in every layer (models/modeling.py:155-219).

Only data is written (ids, maps, logits, hashes, configs).  This script is the only
place the reference is imported.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "model_golden.npz"

VARIANTS = [
    {"name": "routed_shared_mu", "seed": 0, "map": "binpack",
     "cfg": dict(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                 num_attention_heads=4, num_key_value_heads=2, num_experts=4)},
    {"name": "routed_noshared_modulo", "seed": 1, "map": "modulo",
     "cfg": dict(vocab_size=200, hidden_size=128, intermediate_size=384, num_hidden_layers=2,
                 num_attention_heads=2, num_key_value_heads=1, num_experts=2, shared_expert=False)},
    {"name": "dense_nomu", "seed": 2, "map": None,
     "cfg": dict(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                 num_attention_heads=2, num_key_value_heads=2, use_token_routed_mlp=False,
                 use_mu_guidance=False)},
]
BATCH, SEQ = 2, 16


def tensor_digest(t: torch.Tensor) -> str:
    a = t.detach().cpu().contiguous()
    return hashlib.sha256(a.numpy().tobytes()).hexdigest()


def zipf_pmf(V: int, s: float = 1.1) -> torch.Tensor:
    k = np.arange(1, V + 1, dtype=np.float64)
    w = k ** (-s)
    return torch.from_numpy((w / w.sum()).astype(np.float32))


def main() -> None:
    sys.path.insert(0, str(REF))
    from complexity_deep import ComplexityConfig, ComplexityModel, TokenRoutedMLP  # the reference

    arrays = {}
    meta = []
    for v in VARIANTS:
        cfg = ComplexityConfig(**v["cfg"])
        torch.manual_seed(v["seed"])
        model = ComplexityModel(cfg).eval()
        sd = model.state_dict()
        hashes = {k: tensor_digest(t) for k, t in sd.items()}
        E = cfg.num_experts
        if v["map"] == "binpack":
            tmap = TokenRoutedMLP._build_token_mapping(cfg.vocab_size, E, zipf_pmf(cfg.vocab_size))
        elif v["map"] == "modulo":
            tmap = torch.arange(cfg.vocab_size, dtype=torch.long) % E
        else:
            tmap = None
        if tmap is not None:
            with torch.no_grad():
                for layer in model.layers:
                    layer.mlp.token_to_expert.copy_(tmap)
        g = torch.Generator().manual_seed(100 + v["seed"])
        ids = torch.multinomial(zipf_pmf(cfg.vocab_size).double(), BATCH * SEQ, replacement=True,
                                generator=g).view(BATCH, SEQ)
        with torch.no_grad():
            logits = model(ids).logits
        n = v["name"]
        arrays[f"{n}/ids"] = ids.numpy()
        arrays[f"{n}/map"] = (tmap if tmap is not None else torch.zeros(0, dtype=torch.long)).numpy()
        arrays[f"{n}/logits"] = logits.numpy().astype(np.float32)
        meta.append({"name": n, "seed": v["seed"], "cfg": cfg.to_dict(), "hashes": hashes,
                     "map": v["map"]})
    arrays["meta_json"] = np.frombuffer(json.dumps(meta, sort_keys=True).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
