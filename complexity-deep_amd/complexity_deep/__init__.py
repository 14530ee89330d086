"""complexity_deep on MI355X: the reference's Python API over gfx950 HIP kernels.

Drop-in names (same constructors, parameters and state_dict keys as the reference
package ``complexity_deep``): ComplexityConfig, ComplexityModel, CausalLMOutput,
ModelOutput, create_complexity_model, count_parameters, TransformerBlock,
MuGuidance, ComplexityAttention (alias MuGuidedAttention), TokenRoutedMLP, SwiGLU,
RMSNorm, RotaryEmbedding, apply_rotary_pos_emb; and the operator functions
fused_residual_rmsnorm, fused_add_rmsnorm_inplace, fused_rmsnorm,
sort_tokens_by_expert, sort_tokens_by_expert_fast, cggr_grouped_gemm (also as
grouped_gemm_pytorch and persistent_cggr_gemm), persistent_swiglu_cggr,
fused_swiglu_triton, fused_swiglu_simple, fused_mu_qkv_projection.

The hot path (routing, MoE grouped SwiGLU GEMM, mu-QKV GEMM, add+RMSNorm) runs only
on the kernels in libcdx.so; the forward is inference-only (no backward).
"""

from .attention import ComplexityAttention, FusedMuQKVProjection, MuGuidedAttention, fused_mu_qkv_projection
from .layer import MuGuidance, TransformerBlock
from .mlp import SwiGLU
from .modeling import (CausalLMOutput, ComplexityConfig, ComplexityModel, GraphedForward, ModelOutput, SIZE_PRESETS,
                       count_parameters, create_complexity_model)
from .normalization import (FusedResidualRMSNorm, RMSNorm, fused_add_rmsnorm_inplace, fused_residual_rmsnorm,
                            fused_rmsnorm)
from .rotary import RotaryEmbedding, apply_rotary_pos_emb
from .token_routed_mlp import (RoutePlan, TokenRoutedMLP, cggr_grouped_gemm, cggr_grouped_gemm_triton,
                               fused_swiglu_simple, fused_swiglu_triton, grouped_gemm_pytorch,
                               persistent_cggr_gemm, persistent_swiglu_cggr, route_plan, route_plans, sort_tokens_by_expert,
                               sort_tokens_by_expert_fast)

__version__ = "1.0.0"

__all__ = [
    "RMSNorm", "RotaryEmbedding", "apply_rotary_pos_emb", "ComplexityAttention", "MuGuidedAttention",
    "SwiGLU", "TokenRoutedMLP", "TransformerBlock", "MuGuidance", "ComplexityConfig", "ComplexityModel",
    "CausalLMOutput", "ModelOutput", "GraphedForward", "create_complexity_model", "count_parameters", "SIZE_PRESETS",
    "fused_residual_rmsnorm", "fused_add_rmsnorm_inplace", "fused_rmsnorm", "FusedResidualRMSNorm",
    "sort_tokens_by_expert", "sort_tokens_by_expert_fast", "cggr_grouped_gemm", "cggr_grouped_gemm_triton",
    "grouped_gemm_pytorch", "persistent_cggr_gemm", "persistent_swiglu_cggr", "fused_swiglu_triton",
    "fused_swiglu_simple", "route_plan", "route_plans", "RoutePlan",
    "fused_mu_qkv_projection", "FusedMuQKVProjection",
]
