"""GPU parity of the mu-guidance kernel (cdx_mu_guidance_fwd).

Reference (core/layer.py:54-61, models/modeling.py:199-200), restated in fp32 on the
CPU: mu = clamp(mu_param, 0, 2) + h @ W_mu^T, then the model's clamp to [-2, 2].
Checked at configuration 4's shape (16384 x 2048) with and without the outer clamp,
at ragged token counts, with a parameter that needs its own clamp (applied by the
kernel's epilogue), through the MuGuidance module, and after a write to the parameter
through ``.data`` (read on every call: nothing cached).
"""

from __future__ import annotations

import math

import pytest
import torch

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu
bf16 = torch.bfloat16


@pytest.mark.parametrize("T,H,lo,hi", [(16384, 2048, -2.0, 2.0), (16384, 2048, -math.inf, math.inf),
                                       (77, 256, -2.0, 2.0), (1, 64, -2.0, 2.0), (300, 768, -0.5, 0.5)])
def test_mu_guidance_matches_reference(cdx, T, H, lo, hi):
    from complexity_deep.layer import mu_guidance
    print(f"mu_guidance T={T} H={H} clamp=({lo}, {hi})", flush=True)
    g = torch.Generator().manual_seed(T + H)
    h = torch.randn(T, H, generator=g).to(bf16)
    # unit-size projections around a bias in [0, 2]: the clamp to [-2, 2] bites on about
    # a sixth of the values, and the bf16 output floor stays at the N(0, 1) level
    w = (torch.randn(H, H, generator=g) / math.sqrt(H)).to(bf16)
    mu_param = torch.linspace(-1.0, 3.0, H).to(bf16)                        # below 0 and above 2: clamped first
    bias = torch.clamp(mu_param.float(), 0.0, 2.0)
    out = mu_guidance(h.cuda(), w.cuda(), mu_param.cuda(), 0.0, 2.0, lo, hi)
    ref = torch.clamp(bias + h.float() @ w.float().t(), lo, hi)
    assert_close_bf16(out, ref, "mu_guidance")
    if math.isfinite(lo):
        assert float(out.float().min()) >= lo and float(out.float().max()) <= hi


def test_mu_guidance_module(cdx):
    print("MuGuidance module", flush=True)
    torch.manual_seed(0)
    m = cdx.MuGuidance(512)
    with torch.no_grad():
        m.mu.copy_(torch.linspace(-1, 3, 512))
        m.mu_proj.weight.normal_(0, 0.1)
    m = m.to(bf16).cuda()
    h = torch.randn(2, 40, 512).to(bf16)
    with torch.no_grad():
        out = m(h.cuda())
        out_clamped = m.fused(h.cuda(), -2.0, 2.0)
    ref = torch.clamp(m.mu.float().cpu(), 0, 2) + h.float() @ m.mu_proj.weight.float().cpu().t()
    assert_close_bf16(out, ref, "module (unclamped, as the reference returns it)")
    assert_close_bf16(out_clamped, torch.clamp(ref, -2, 2), "module fused clamp")


def test_mu_guidance_follows_data_writes(cdx):
    """A write through ``.data`` (which bumps no version counter) to either parameter
    shows in the next call: the kernel reads both on every call."""
    print("MuGuidance .data writes", flush=True)
    torch.manual_seed(1)
    m = cdx.MuGuidance(256)
    with torch.no_grad():
        m.mu_proj.weight.normal_(0, 0.02)
    m = m.to(bf16).cuda()
    h = torch.randn(3, 17, 256).to(bf16).cuda()
    with torch.no_grad():
        before = m(h)
        m.mu.data.fill_(1.5)
        m.mu_proj.weight.data.mul_(2.0)
        after = m(h)
    with torch.no_grad():
        ref = 1.5 + h.float().cpu() @ m.mu_proj.weight.float().cpu().t()
    assert not torch.equal(before, after)
    assert_close_bf16(after, ref, "after .data writes")


@pytest.mark.parametrize("T,H", [(16384, 2048), (300, 768), (5, 64)])
def test_mu_guidance_into_the_right_half_of_a_pair(cdx, T, H):
    """Written into the right half of a [T, 2H] buffer (output rows at stride 2H, as the
    model places mu beside the next layer's x): the same bits as the contiguous output,
    and the left half untouched."""
    from complexity_deep.layer import mu_guidance
    print(f"mu_guidance into a pair T={T} H={H}", flush=True)
    g = torch.Generator().manual_seed(T * 3 + H)
    h = torch.randn(T, H, generator=g).to(bf16).cuda()
    w = (torch.randn(H, H, generator=g) / math.sqrt(H)).to(bf16).cuda()
    mu_param = torch.linspace(-1.0, 3.0, H).to(bf16).cuda()
    ref = mu_guidance(h, w, mu_param, 0.0, 2.0, -2.0, 2.0)
    pair = torch.full((T, 2 * H), 7.0, dtype=bf16, device="cuda")
    out = mu_guidance(h, w, mu_param, 0.0, 2.0, -2.0, 2.0, out=pair[:, H:])
    torch.cuda.synchronize()
    assert out.data_ptr() == pair[:, H:].data_ptr()
    assert torch.equal(pair[:, H:], ref)
    assert bool((pair[:, :H] == 7.0).all()), "the left half was written"
