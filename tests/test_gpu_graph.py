"""ComplexityModel's forward replayed from a HIP graph (GraphedForward) gives the same
bits as the eager forward.

The graph is replayed several times, on different ids, with eager forwards and
synchronisations between the replays, and every replay is compared with the eager
result of the same ids (a replay that reused stale buffers, or a node that does
not replay like its eager launch, shows up as a difference)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shared,mu,B,S", [(True, True, 4, 512), (False, True, 2, 300), (True, False, 1, 77)])
def test_graphed_forward_matches_eager(cdx, shared, mu, B, S):
    from complexity_deep import synthetic as syn
    cfg = cdx.ComplexityConfig(vocab_size=32000, hidden_size=768, intermediate_size=2048, num_hidden_layers=4,
                               num_attention_heads=12, num_key_value_heads=4, num_experts=4, shared_expert=shared,
                               use_mu_guidance=mu)
    torch.manual_seed(0)
    m = cdx.ComplexityModel(cfg)
    syn.install_expert_map(m, syn.binpacked_map(cfg.vocab_size, cfg.num_experts))
    m = m.to("cuda", torch.bfloat16).eval()
    print(f"graphed forward: README model with 4 layers, shared={shared} mu={mu}, {B} x {S}", flush=True)
    graphed = m.capture_forward(B, S)
    with torch.inference_mode():
        for seed in (0, 1, 2, 0):
            ids = syn.zipf_token_ids(B, S, cfg.vocab_size, seed=seed).cuda()
            got = graphed(ids).clone()
            torch.cuda.synchronize()
            expect = m(ids).logits
            torch.cuda.synchronize()
            assert torch.equal(got, expect), f"replay on ids of seed {seed} differs from the eager forward"
        with pytest.raises(ValueError, match="captured for input shape"):
            graphed(torch.zeros(B, S + 1, dtype=torch.long, device="cuda"))
