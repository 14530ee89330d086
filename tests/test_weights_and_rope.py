"""CPU tests of two host-side contracts of the attention module.

* RoPE tables: the reference builds its cos/sin cache in the constructor from the
  fp32 inverse frequencies (core/rotary.py:35-47), before any cast of the model.  The
  tables here must stay that accurate after ``model.to(torch.bfloat16)``, which rounds
  the ``inv_freq`` buffer.  Checked against float64 cos/sin of the exact angles; the
  bound (3e-4) covers the fp32 rounding of p * inv_freq at p < 2048, while angles
  from a bf16-rounded inv_freq are off by whole radians there.
* Projection weights: q/k/v_proj and mu_to_q/k/v weights are views of the column
  halves of the [N, 2H] buffer the kernel reads (QKVWeights), so writes through ``.data`` (the
  pattern of the reference's run_ablations.py:45-78) reach the kernel operand; the
  views survive load_state_dict and are re-established after a cast or move.
"""

from __future__ import annotations

import math

import pytest
import torch


def _exact_cos_sin(n: int, dim: int, theta: float = 10000.0):
    j = torch.arange(0, dim, 2, dtype=torch.float64)
    inv = 1.0 / theta ** (j / dim)
    ang = torch.outer(torch.arange(n, dtype=torch.float64), inv)
    return ang.cos(), ang.sin()


@pytest.mark.parametrize("dim", [32, 64, 128])
def test_rope_table_survives_bf16_cast(dim):
    from complexity_deep.rotary import RotaryEmbedding
    rot = RotaryEmbedding(dim, max_seq_len=2048).to(torch.bfloat16)
    assert rot.inv_freq.dtype == torch.bfloat16
    table = rot.cos_sin_table(2048, torch.device("cpu"))
    assert table.dtype == torch.float32 and table.shape[:2] >= (2048, dim // 2)
    c, s = _exact_cos_sin(2048, dim)
    err = max(float((table[:2048, :, 0].double() - c).abs().max()),
              float((table[:2048, :, 1].double() - s).abs().max()))
    assert err < 3e-4, err
    # Past the construction length the table keeps growing from exact angles.
    big = rot.cos_sin_table(5000, torch.device("cpu"))
    c, s = _exact_cos_sin(5000, dim)
    assert float((big[:5000, :, 0].double() - c).abs().max()) < 8e-4


def test_rope_cached_tables_cast_like_the_reference():
    """cos_cached of a bf16 module = bf16 of the fp32 table (the reference casts its
    constructor-built buffers); a grown cache is built from exact angles too."""
    from complexity_deep.rotary import RotaryEmbedding
    rot = RotaryEmbedding(128, max_seq_len=256).to(torch.bfloat16)
    c, s = _exact_cos_sin(256, 128)
    cos_ref = torch.cat([c, c], dim=-1)
    assert rot.cos_cached.dtype == torch.bfloat16
    assert float((rot.cos_cached.double() - cos_ref).abs().max()) <= 2 ** -8
    cos, sin = rot(1024)  # grows the cache past max_seq_len
    c, s = _exact_cos_sin(1024, 128)
    assert cos.dtype == torch.bfloat16
    assert float((cos.double() - torch.cat([c, c], -1)).abs().max()) <= 2 ** -8
    assert float((sin.double() - torch.cat([s, s], -1)).abs().max()) <= 2 ** -8


def _attn():
    from complexity_deep import ComplexityAttention
    torch.manual_seed(0)
    return ComplexityAttention(256, 4, 2)


def test_qkv_weights_are_views_of_the_kernel_operand():
    a = _attn()
    sd0 = {k: v.clone() for k, v in a.state_dict().items()}
    w_x, w_mu = a.qkv_weights()
    assert w_x.shape == (256 + 2 * 128, 256) and w_mu.shape == w_x.shape
    # side by side: row n of one [N, 2H] buffer is [W_x[n] | W_mu[n]]
    assert w_x.stride() == (512, 1) and w_mu.data_ptr() == w_x.data_ptr() + 256 * w_x.element_size()
    assert torch.equal(w_x, torch.cat([sd0["q_proj.weight"], sd0["k_proj.weight"], sd0["v_proj.weight"]]))
    assert torch.equal(w_mu, torch.cat([sd0["mu_to_q.weight"], sd0["mu_to_k.weight"], sd0["mu_to_v.weight"]]))
    # Binding changes neither keys nor values.
    sd1 = a.state_dict()
    assert list(sd1) == list(sd0) and all(torch.equal(sd0[k], sd1[k]) for k in sd0)
    # A .data write (no version bump) lands in the operand.
    a.mu_to_k.weight.data.zero_()
    assert torch.count_nonzero(w_mu[256:384]) == 0 and torch.count_nonzero(w_mu[:256]) > 0
    w_x2, w_mu2 = a.qkv_weights()
    assert w_mu2.data_ptr() == w_mu.data_ptr(), "an intact binding must not be rebuilt"
    # Restore through .data.copy_, as the reference's ablation context does.
    a.mu_to_k.weight.data.copy_(sd0["mu_to_k.weight"])
    assert torch.equal(w_mu[256:384], sd0["mu_to_k.weight"])
    # load_state_dict copies into the views.
    sd2 = {k: v * 2 if v.is_floating_point() else v for k, v in sd0.items()}
    a.load_state_dict(sd2)
    assert torch.equal(w_x[:256], sd2["q_proj.weight"])
    assert a.qkv_weights()[0].data_ptr() == w_x.data_ptr()


def test_qkv_weights_rebind_after_cast_and_replacement():
    a = _attn()
    w_x, _ = a.qkv_weights()
    ref = w_x.clone()
    a = a.to(torch.bfloat16)
    w_xb, w_mub = a.qkv_weights()
    assert w_xb.dtype == torch.bfloat16 and w_xb.data_ptr() != w_x.data_ptr()
    assert torch.equal(w_xb, ref.to(torch.bfloat16))
    a.v_proj.weight.data.fill_(1.0)
    assert torch.all(w_xb[384:] == 1.0)
    # A replaced Parameter is copied in at the next call.
    a.q_proj.weight = torch.nn.Parameter(torch.full((256, 256), 3.0, dtype=torch.bfloat16))
    w_x3, _ = a.qkv_weights()
    assert torch.all(w_x3[:256] == 3.0) and torch.all(w_x3[384:] == 1.0)
    assert a.q_proj.weight.data_ptr() == w_x3.data_ptr()


def test_qkv_weights_bound_in_inference_mode_stay_writable():
    a = _attn()
    with torch.inference_mode():
        w_x, w_mu = a.qkv_weights()
    assert not w_x.is_inference()
    a.mu_to_q.weight.data.zero_()  # raises for an inference tensor outside inference mode
    assert torch.count_nonzero(w_mu[:256]) == 0


def test_oracle_rope_frequencies_are_the_constructor_ones(oracle):
    """The oracle's tables come from (head_dim, theta) like the reference's constructor;
    for an fp32 state_dict that is exactly the inv_freq buffer."""
    from complexity_deep.rotary import RotaryEmbedding
    for dim, theta in ((64, 10000.0), (128, 10000.0), (128, 500000.0)):
        rot = RotaryEmbedding(dim, theta=theta)
        assert torch.equal(oracle.rope_inv_freq(dim, theta), rot.inv_freq)
    assert math.isclose(float(oracle.rope_inv_freq(128)[1]), 10000.0 ** (-2 / 128), rel_tol=1e-6)


def test_graphed_forward_needs_gpu_eval_model():
    """GraphedForward refuses a model in training mode and a model on the host."""
    import complexity_deep as cdx
    cfg = cdx.ComplexityConfig(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                               num_attention_heads=2, num_key_value_heads=1, num_experts=2)
    m = cdx.ComplexityModel(cfg)
    with pytest.raises(ValueError, match="eval mode"):
        cdx.GraphedForward(m.train(), 1, 8)
    with pytest.raises(ValueError, match="needs a GPU model"):
        cdx.GraphedForward(m.eval(), 1, 8)
