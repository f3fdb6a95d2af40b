"""gfx950 fused kernel layer with TrainScale's kernel API.

The exports mirror the hot-path names of TrainScale's ``kernels/__init__.py``
(data_pipeline/trainer/kernels/__init__.py:15-124): ``fast_rms_layernorm`` is
the layernorm_kernels variant there, as here.
"""
from .fused_kernels import (
    Fast_CrossEntropyLoss,
    Fast_RMS_LayerNorm,
    Fast_RoPE,
    Fast_SwiGLU,
    HipRMSNorm,
    TritonRMSNorm,
    fast_cross_entropy_loss,
    swiglu_forward,
)
from .layernorm_kernels import (
    FusedAddRMSLayerNormFunction,
    FusedRMSNorm,
    RMSLayerNormFunction,
    RMSNorm,
    fast_rms_layernorm,
    fused_add_rms_layernorm,
    rms_layernorm,
)
from .rope_kernels import (
    Fast_RoPE_Embedding,
    FusedRoPEQKFunction,
    RoPEConfig,
    RoPEFrequencyCache,
    RoPEFunction,
    RoPEScalingType,
    RotaryEmbedding,
    apply_rope,
    apply_rope_qk,
    apply_rope_theta,
    fast_rope_embedding,
    inplace_rope_embedding,
    precompute_freqs_cis,
)

__all__ = [
    "Fast_CrossEntropyLoss",
    "fast_cross_entropy_loss",
    "Fast_SwiGLU",
    "swiglu_forward",
    "Fast_RMS_LayerNorm",
    "HipRMSNorm",
    "TritonRMSNorm",
    "RMSLayerNormFunction",
    "RMSNorm",
    "rms_layernorm",
    "fast_rms_layernorm",
    "FusedAddRMSLayerNormFunction",
    "fused_add_rms_layernorm",
    "FusedRMSNorm",
    "Fast_RoPE",
    "Fast_RoPE_Embedding",
    "FusedRoPEQKFunction",
    "RoPEFunction",
    "RoPEConfig",
    "RoPEFrequencyCache",
    "RoPEScalingType",
    "RotaryEmbedding",
    "apply_rope",
    "apply_rope_qk",
    "apply_rope_theta",
    "fast_rope_embedding",
    "inplace_rope_embedding",
    "precompute_freqs_cis",
]
