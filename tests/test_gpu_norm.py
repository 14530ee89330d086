"""GPU parity of the add+RMSNorm kernel (cdx_add_rmsnorm_fwd) against the oracle.

* h = x + residual must be bit-identical to torch's bf16 add (the reference's
  residual add, core/layer.py:174,183).
* The normalised output meets the bf16 bar of tests/_metrics.py against the fp32
  oracle evaluated on the same bf16 inputs.
Shapes cover configuration 3 at full size (32768 x 2048), configuration 1's H=768,
single rows, partial blocks, H not a multiple of 64, the largest H (8192) and the
in-place form.
"""

from __future__ import annotations

import pytest
import torch

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu

bf16 = torch.bfloat16


def _data(T, H, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(bf16)
    r = torch.randn(T, H, generator=g).to(bf16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(bf16)
    return x, r, w


@pytest.mark.parametrize("T,H", [(1, 8), (3, 768), (257, 2048), (32768, 2048), (64, 8192), (5, 1000), (4096, 768)])
def test_add_rmsnorm_matches_oracle(cdx, oracle, T, H):
    from complexity_deep.normalization import add_rms_norm
    print(f"add_rmsnorm T={T} H={H}", flush=True)
    x, r, w = _data(T, H, T + H)
    y, h = add_rms_norm(x.cuda(), r.cuda(), w.cuda(), 1e-6)
    torch.cuda.synchronize()
    h_ref = x + r  # bf16 add on the CPU, rounded once like the reference
    assert torch.equal(h.cpu(), h_ref)
    y_ref, _ = oracle.add_rms_norm(h_ref.float(), torch.zeros(T, H), w.float(), 1e-6)
    assert_close_bf16(y, y_ref, f"add_rmsnorm T={T} H={H}")


@pytest.mark.parametrize("T,H", [(7, 64), (2048, 768), (1000, 2048)])
def test_plain_rmsnorm_matches_oracle(cdx, oracle, T, H):
    print(f"rmsnorm T={T} H={H}", flush=True)
    x, _, w = _data(T, H, 11)
    norm = cdx.RMSNorm(H).cuda().to(bf16)
    with torch.no_grad():
        norm.weight.copy_(w)
        y = norm(x.cuda().view(1, T, H))
    assert y.shape == (1, T, H)
    assert_close_bf16(y.view(T, H), oracle.rms_norm(x.float(), w.float(), 1e-6), "rmsnorm")


@pytest.mark.parametrize("T,H", [(16384, 2048), (2048, 768), (5, 1000), (3, 8)])
def test_rmsnorm_into_the_left_half_of_a_pair(cdx, T, H):
    """cdx_rmsnorm_ld_fwd: output rows at stride 2H (the left half of a [T, 2H] buffer, as
    the model places the next layer's x beside its mu) hold the same bits as the
    contiguous plain norm, and the right half is untouched."""
    from complexity_deep.normalization import rms_norm
    print(f"rmsnorm into a pair T={T} H={H}", flush=True)
    x, _, w = _data(T, H, 23)
    x, w = x.cuda(), w.cuda()
    ref = rms_norm(x, w, 1e-6)
    pair = torch.full((T, 2 * H), 7.0, dtype=bf16, device="cuda")
    out = rms_norm(x.view(1, T, H), w, 1e-6, out=pair[:, :H].view(1, T, H))
    torch.cuda.synchronize()
    assert out.data_ptr() == pair.data_ptr()
    assert torch.equal(pair[:, :H], ref)
    assert bool((pair[:, H:] == 7.0).all()), "the right half was written"


def test_empty_and_large_eps(cdx, oracle):
    from complexity_deep.normalization import add_rms_norm
    e = torch.empty(0, 64, dtype=bf16, device="cuda")
    y, h = add_rms_norm(e, e, torch.ones(64, dtype=bf16, device="cuda"))
    assert y.shape == (0, 64) and h.shape == (0, 64)
    x, r, w = _data(16, 256, 3)
    xs = x * 0.01
    y, _ = add_rms_norm(xs.cuda(), None, w.cuda(), eps=1e-2)
    assert_close_bf16(y, oracle.rms_norm(xs.float(), w.float(), 1e-2), "eps")


def test_reference_operator_api(cdx, oracle):
    print("fused_residual_rmsnorm API", flush=True)
    x, r, w = _data(4 * 128, 512, 5)
    x3, r3 = x.view(4, 128, 512).cuda(), r.view(4, 128, 512).cuda()
    out, res = cdx.fused_residual_rmsnorm(x3, r3, w.cuda(), eps=1e-6, store_residual=True)
    assert out.shape == (4, 128, 512) and res.shape == (4, 128, 512)
    assert torch.equal(res.cpu().view(-1, 512), x + r)
    (out_only,) = cdx.fused_residual_rmsnorm(x3, r3, w.cuda(), eps=1e-6, store_residual=False)
    assert torch.equal(out_only, out)
    y_ref, _ = oracle.add_rms_norm((x + r).float(), torch.zeros(512, 512), w.float())
    assert_close_bf16(out.view(-1, 512), y_ref, "fused_residual_rmsnorm")
    # in-place variant: hidden += mlp_out
    hidden = r.cuda().clone()
    y2 = cdx.fused_add_rmsnorm_inplace(hidden, x.cuda(), w.cuda())
    assert torch.equal(hidden.cpu(), x + r)
    assert torch.equal(y2, out.view(-1, 512))
    m = cdx.FusedResidualRMSNorm(512).cuda().to(bf16)
    with torch.no_grad():
        m.weight.copy_(w)
        o3, r3b = m(x3, r3)
    assert torch.equal(o3, out) and torch.equal(r3b, res)


def test_out_buffers_are_checked(cdx):
    """Caller-provided out / residual_out must be contiguous bf16 tensors of x's shape
    on x's device: the kernel writes T * H values through their base pointers."""
    from complexity_deep.normalization import add_rms_norm
    x = torch.randn(8, 256, device="cuda").to(bf16)
    r = torch.randn(8, 256, device="cuda").to(bf16)
    w = torch.ones(256, device="cuda", dtype=bf16)
    bad = [torch.empty(8, 128, device="cuda", dtype=bf16),           # shape
           torch.empty(8, 256, device="cuda", dtype=torch.float32),  # dtype
           torch.empty(256, 8, device="cuda", dtype=bf16).t(),       # not contiguous
           torch.empty(8, 256, dtype=bf16)]                          # device
    for t in bad:
        with pytest.raises(ValueError, match="out must be"):
            add_rms_norm(x, r, w, out=t)
        with pytest.raises(ValueError, match="residual_out must be"):
            add_rms_norm(x, r, w, residual_out=t)
    y, h = add_rms_norm(x, r, w, out=torch.empty_like(x), residual_out=r)
    assert h.data_ptr() == r.data_ptr()
