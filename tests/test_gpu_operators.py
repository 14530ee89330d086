"""GPU parity of the reference's MoE operator API on the HIP kernels.

  persistent_swiglu_cggr      cuda/persistent_cggr.py:479-530
  fused_swiglu_triton         cuda/triton_token_routed.py:234-257
  fused_swiglu_simple         cuda/persistent_cggr.py:450-476
  grouped_gemm_pytorch        cuda/triton_token_routed.py:64-86
  persistent_cggr_gemm        cuda/persistent_cggr.py:355-410
  sort_tokens_by_expert_fast  cuda/persistent_cggr.py:318-352

The GEMM operators are compared with the fp32 oracle (oracle.grouped_gemm,
oracle.swiglu_rows) under the bf16 bound of tests/_metrics.py, including ragged
segments, empty experts and offsets that leave rows uncovered (those rows must be
exactly zero, as the reference's torch.zeros output leaves them).  The routing
operator is bit-exact against the C oracle.  The elementwise SwiGLU is compared
with a plain fp32 PyTorch statement of each variant's rounding (silu in fp32, then
either one rounding or a rounding of silu first); the kernel's exp may differ from
torch's in the last fp32 bit, so a result may sit one unit of the output dtype away.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from _metrics import assert_close_bf16

pytestmark = pytest.mark.gpu
bf16 = torch.bfloat16


def _ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[dtype]
    tiny = {torch.bfloat16: 2.0 ** -133, torch.float16: 2.0 ** -24, torch.float32: 2.0 ** -149}[dtype]
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-38)))
    return torch.maximum(torch.exp2(e - mant), torch.full_like(x, tiny))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n", [1, 7, 4096 * 3 + 5, 1 << 20])
def test_fused_swiglu_variants(cdx, dtype, n):
    print(f"swiglu {dtype} n={n}", flush=True)
    g = torch.Generator().manual_seed(n)
    gate = (torch.randn(n, generator=g) * 3).to(dtype)
    up = torch.randn(n, generator=g).to(dtype)
    s32 = F.silu(gate.float())
    refs = {
        "simple": (s32 * up.float()).to(dtype),
        "triton": (s32.to(dtype).float() * up.float()).to(dtype),
    }
    outs = {"simple": cdx.fused_swiglu_simple(gate.cuda(), up.cuda()).cpu(),
            "triton": cdx.fused_swiglu_triton(gate.cuda(), up.cuda()).cpu()}
    for k in refs:
        got, ref = outs[k].float(), refs[k].float()
        assert outs[k].dtype == dtype and outs[k].shape == gate.shape
        d = (got - ref).abs()
        if dtype == torch.float32:
            # exp and the division differ from torch's silu by a few fp32 ulps
            units = 8.0
        else:
            # one rounding: at most one unit off; the triton form rounds silu first, and a
            # one-unit change of silu moves the rounded product by up to two units
            units = 1.0 if k == "simple" else 2.0
        bad = d > _ulp(ref, dtype) * units * 1.0001
        assert not bool(bad.any()), f"{k}: {int(bad.sum())} of {n} off by more than {units} units"
        if dtype != torch.float32:
            assert float((d > 0).float().mean()) < 0.02, f"{k}: too many last-bit differences"


def test_fused_swiglu_noncontiguous_halves(cdx):
    """The halves of a fused gate/up output (non-contiguous views) and a 2-D shape."""
    g = torch.Generator().manual_seed(3)
    fused = torch.randn(300, 2 * 704, generator=g).to(bf16).cuda()
    gate, up = fused[:, :704], fused[:, 704:]
    out = cdx.fused_swiglu_triton(gate, up)
    ref = F.silu(gate.float()).to(bf16).float() * up.float()
    assert out.shape == (300, 704) and out.is_contiguous()
    assert float((out.float() - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -7


def _swiglu_segments_ref(oracle, x, gw, uw, dw, offs):
    out = torch.zeros(x.shape[0], dw.shape[2])
    for e in range(gw.shape[0]):
        s0, s1 = int(offs[e]), int(offs[e + 1])
        if s1 > s0:
            out[s0:s1] = oracle.swiglu_rows(x[s0:s1].float(), gw[e].float(), uw[e].float(), dw[e].float())
    return out


@pytest.mark.parametrize("H,I,offsets", [
    (512, 704, [0, 300, 300, 1300, 1377, 1377]),      # ragged, empty experts, full coverage
    (768, 512, [100, 400, 400, 900]),                  # rows outside [100, 900) uncovered
    (256, 176, [0, 5, 5, 5, 4000]),                    # Ie padded to 192, tiny and large segments
    (2048, 704, [0, 2048, 2560, 9000, 9001, 12000]),   # the 1B expert width
])
def test_persistent_swiglu_cggr(cdx, oracle, H, I, offsets):
    print(f"persistent_swiglu_cggr H={H} I={I} offs={offsets}", flush=True)
    E = len(offsets) - 1
    T = max(offsets[-1], 1000)
    g = torch.Generator().manual_seed(H + I)
    x = torch.randn(T, H, generator=g).to(bf16)
    gw = (torch.randn(E, H, I, generator=g) * 0.02).to(bf16)
    uw = (torch.randn(E, H, I, generator=g) * 0.02).to(bf16)
    dw = (torch.randn(E, I, H, generator=g) * 0.02).to(bf16)
    offs = torch.tensor(offsets, dtype=torch.int64)
    out = cdx.persistent_swiglu_cggr(x.cuda(), gw.cuda(), uw.cuda(), dw.cuda(), offs.cuda()).cpu()
    ref = _swiglu_segments_ref(oracle, x, gw, uw, dw, offsets)
    lo, hi = offsets[0], offsets[-1]
    assert torch.count_nonzero(out[:lo]) == 0 and torch.count_nonzero(out[hi:]) == 0, "uncovered rows must be 0"
    assert_close_bf16(out[lo:hi], ref[lo:hi], f"persistent_swiglu_cggr H={H}")


def test_grouped_gemm_aliases(cdx, oracle):
    print("grouped_gemm_pytorch / persistent_cggr_gemm", flush=True)
    g = torch.Generator().manual_seed(11)
    offsets = [64, 64, 900, 1001, 1800]
    T, K, N = 2000, 384, 256
    a = torch.randn(T, K, generator=g).to(bf16)
    w = (torch.randn(len(offsets) - 1, K, N, generator=g) * 0.05).to(bf16)
    offs = torch.tensor(offsets)
    counts = offs[1:] - offs[:-1]
    ref = oracle.grouped_gemm(a.float(), w.float(), offs.numpy())
    for out in (cdx.grouped_gemm_pytorch(a.cuda(), w.cuda(), offs.cuda(), counts.cuda()),
                cdx.persistent_cggr_gemm(a.cuda(), w.cuda(), offs.cuda(), num_sms=80)):
        out = out.cpu()
        assert torch.count_nonzero(out[:64]) == 0 and torch.count_nonzero(out[1800:]) == 0
        assert_close_bf16(out[64:1800], ref[64:1800], "grouped gemm alias")


@pytest.mark.parametrize("T,E", [(2048, 4), (16384, 8), (1, 3)])
def test_sort_tokens_by_expert_fast(cdx, oracle, T, E):
    from complexity_deep import synthetic as syn
    ids = syn.zipf_token_ids(1, T, 32000, seed=T).view(-1)
    ids[::97] = 40000  # out of range: clamped to the last id
    tmap = syn.binpacked_map(32000, E)
    idx, offs, counts = cdx.sort_tokens_by_expert_fast(ids.cuda(), tmap.cuda(), E)
    ref = oracle.route_plan(ids.numpy(), tmap.numpy(), E)
    assert idx.dtype == offs.dtype == counts.dtype == torch.int64
    np.testing.assert_array_equal(idx.cpu().numpy(), ref["perm"].astype(np.int64))
    np.testing.assert_array_equal(offs.cpu().numpy(), ref["offsets"].astype(np.int64))
    np.testing.assert_array_equal(counts.cpu().numpy(), ref["counts"].astype(np.int64))
