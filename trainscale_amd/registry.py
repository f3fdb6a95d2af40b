"""RMSNorm, SwiGLU-MLP and rotary patch boundary with TrainScale's registry API.

Mirrors ``register_layer_patch``, ``LAYER_PATCHES``, ``auto_patch_layernorm``,
``auto_patch_mlp`` and the RMSNorm/MLP part of ``KernelPatcher``
(data_pipeline/trainer/registry/__init__.py:997-1091, :1194-1200, :1331-1418):
every module whose class name is registered gets its ``forward`` replaced, an
RMSNorm by ``fast_rms_layernorm`` and a gate/up/down MLP by
``down_proj(swiglu_forward(gate_proj(x), up_proj(x)))``, both on the gfx950
kernels. The patched forward keeps calling the module's original forward for
tensors that are not on a GPU (the module's own code, not a copy of the kernel
math).

Rotary modules (``auto_patch_rope``, registry/__init__.py:1209-1282): the
reference only records a RoPEConfig on the module. Here the patch also routes
the rotation itself: the ``apply_rotary_pos_emb`` function of the module's
transformers model file is replaced by ``hf_apply_rotary_pos_emb`` (the gfx950
kernel reading the model's own cos/sin per token), with the original kept for
CPU tensors and for layouts it does not cover.
"""
from __future__ import annotations

from typing import Callable, Dict, List, Tuple

import torch
import torch.nn as nn

import sys

from .kernels.fused_kernels import fast_rms_layernorm, swiglu_forward
from .kernels.rope_kernels import RoPEConfig, RoPEScalingType, hf_apply_rotary_pos_emb

__all__ = ["LAYER_PATCHES", "NORMS_WITH_OTHER_MATH", "register_layer_patch", "auto_patch_layernorm", "auto_patch_mlp",
           "auto_patch_rope", "KernelPatcher", "patch_model"]

LAYER_PATCHES: Dict[str, Callable[[nn.Module], None]] = {}


def register_layer_patch(class_name: str, patch_fn: Callable[[nn.Module], None]) -> None:
    """Registers `patch_fn` for modules of class `class_name` (registry/__init__.py:997-1000)."""
    LAYER_PATCHES[class_name] = patch_fn


def auto_patch_layernorm(module: nn.Module) -> None:
    """Routes an RMSNorm module's forward to the gfx950 kernel (registry/__init__.py:1033-1054)."""
    original_forward = module.forward
    eps = getattr(module, "eps", getattr(module, "variance_epsilon", 1e-6))

    def patched_forward(hidden_states):
        weight = getattr(module, "weight", None)
        if (not isinstance(hidden_states, torch.Tensor) or weight is None
                or not isinstance(weight, torch.Tensor) or not hidden_states.is_cuda
                or not weight.is_cuda):
            return original_forward(hidden_states)
        return fast_rms_layernorm(hidden_states, weight, eps)

    module.forward = patched_forward
    module._trainscale_amd_patched = True


for _name in ("LlamaRMSNorm", "Qwen2RMSNorm", "Qwen3RMSNorm", "GemmaRMSNorm", "Gemma2RMSNorm",
              "MistralRMSNorm", "Phi3RMSNorm", "Phi4RMSNorm", "YiRMSNorm", "FalconRMSNorm",
              "FalconH1RMSNorm", "CohereLayerNorm", "GraniteRMSNorm", "StarcoderLayerNorm",
              "DeepseekRMSNorm", "DeepseekV2RMSNorm", "MixtralRMSNorm", "DbrxLayerNorm",
              "GrokRMSNorm", "InternVLRMSNorm"):
    register_layer_patch(_name, auto_patch_layernorm)

# Registered norm classes whose own forward is not x * rstd * w. The reference's
# table (registry/__init__.py:1058-1077) routes them to the plain RMSNorm kernel all
# the same, and so does KernelPatcher by default, to stay a drop-in: Gemma's norms
# compute x * rstd * (1 + w) with w initialised to zeros (a patched Gemma model
# normalises with weight 0 where its own forward uses 1); Cohere's, StarCoder's and
# DBRX's LayerNorms subtract the row mean (and may add a bias).
# KernelPatcher(skip_inexact_norms=True) leaves these modules on their own forward.
NORMS_WITH_OTHER_MATH: Dict[str, str] = {
    "GemmaRMSNorm": "x * rstd * (1 + w)",
    "Gemma2RMSNorm": "x * rstd * (1 + w)",
    "CohereLayerNorm": "LayerNorm: subtracts the mean",
    "StarcoderLayerNorm": "LayerNorm: subtracts the mean, adds a bias",
    "DbrxLayerNorm": "LayerNorm: subtracts the mean",
}


def auto_patch_mlp(module: nn.Module) -> None:
    """Routes a gate/up/down MLP through the gfx950 SwiGLU kernel (registry/__init__.py:1080-1091)."""
    if not (hasattr(module, "gate_proj") and hasattr(module, "up_proj")
            and hasattr(module, "down_proj")):
        return
    original_forward = module.forward

    def patched_forward(x):
        if not isinstance(x, torch.Tensor) or not x.is_cuda:
            return original_forward(x)
        return module.down_proj(swiglu_forward(module.gate_proj(x), module.up_proj(x)))

    module.forward = patched_forward
    module._trainscale_amd_patched = True


for _name in ("LlamaMLP", "Qwen2MLP", "Qwen3MLP", "MistralMLP", "MixtralBlockSparseTop2MLP",
              "Phi3MLP", "Phi4MLP"):
    register_layer_patch(_name, auto_patch_mlp)


_ROPE_TYPES = {"linear": RoPEScalingType.LINEAR, "ntk": RoPEScalingType.NTK,
               "yarn": RoPEScalingType.YARN, "dynamic": RoPEScalingType.DYNAMIC_NTK,
               "longrope": RoPEScalingType.LONGROPE}


def _routed_apply(original):
    """apply_rotary_pos_emb that runs the gfx950 kernel where it covers the call."""

    def apply_rotary_pos_emb(q, k, cos, sin, *args, **kwargs):
        unsqueeze_dim = kwargs.get("unsqueeze_dim", args[0] if args else 1)
        ok = (set(kwargs) <= {"unsqueeze_dim"} and len(args) <= 1
              and isinstance(unsqueeze_dim, int) and unsqueeze_dim in (1, 2)
              and isinstance(q, torch.Tensor) and q.is_cuda and k.is_cuda and cos.is_cuda
              and q.dim() == 4 and k.dim() == 4 and cos.dim() == 3
              and q.shape[-1] == cos.shape[-1] == k.shape[-1] and q.shape[-1] % 2 == 0
              and q.dtype == k.dtype and sin.shape == cos.shape)
        if ok:
            # the table rows the kernel reads: cos/sin [1 or B, S, D] against q and k of
            # [B, H, S, D] (unsqueeze_dim 1) or [B, S, H, D] (2); other layouts, which
            # broadcasting might still accept, go to the original function
            s_dim = 2 if unsqueeze_dim == 1 else 1
            B, S = q.shape[0], q.shape[s_dim]
            ok = (k.shape[0] == B and k.shape[s_dim] == S and cos.shape[0] in (1, B)
                  and cos.shape[1] == S)
        if not ok:
            return original(q, k, cos, sin, *args, **kwargs)
        return hf_apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim)

    apply_rotary_pos_emb._trainscale_amd_original = original
    return apply_rotary_pos_emb


def auto_patch_rope(module: nn.Module) -> None:
    """Records the module's RoPEConfig (registry/__init__.py:1209-1265) and routes its model
    file's apply_rotary_pos_emb to the gfx950 kernel."""
    dim = getattr(module, "dim", getattr(module, "head_dim", 64))
    base = getattr(module, "base", getattr(module, "rope_theta", 10000.0))
    max_seq = getattr(module, "max_position_embeddings", getattr(module, "max_seq_len_cached", 8192))
    scaling_type, factor = RoPEScalingType.NONE, 1.0
    rope_scaling = getattr(module, "rope_scaling", None)
    if isinstance(rope_scaling, dict):
        scaling_type = _ROPE_TYPES.get(str(rope_scaling.get("type", "none")).lower(),
                                       RoPEScalingType.NONE)
        factor = rope_scaling.get("factor", 1.0)
    module._rope_config = RoPEConfig(dim=dim, max_seq_len=max_seq, base=base,
                                     scaling_type=scaling_type, scaling_factor=factor)
    module._uses_triton_rope = True
    model_file = sys.modules.get(module.__class__.__module__)
    fn = getattr(model_file, "apply_rotary_pos_emb", None) if model_file is not None else None
    if callable(fn) and not hasattr(fn, "_trainscale_amd_original"):
        setattr(model_file, "apply_rotary_pos_emb", _routed_apply(fn))
    module._trainscale_amd_patched = True


for _name in ("LlamaRotaryEmbedding", "LlamaLinearScalingRotaryEmbedding",
              "LlamaDynamicNTKScalingRotaryEmbedding", "Qwen2RotaryEmbedding",
              "Qwen3RotaryEmbedding", "MistralRotaryEmbedding", "GemmaRotaryEmbedding",
              "Gemma2RotaryEmbedding", "Phi3RotaryEmbedding", "Phi4RotaryEmbedding",
              "FalconRotaryEmbedding", "YiRotaryEmbedding"):
    register_layer_patch(_name, auto_patch_rope)


class KernelPatcher:
    """Applies the registered layer patches to a model (registry/__init__.py:1331-1418).

    ``patch_attention`` and ``patch_fp8`` are accepted for signature
    compatibility; this layer registers no attention or FP8 patches, so they
    select nothing. ``skip_inexact_norms`` (not in the reference) leaves the
    classes of NORMS_WITH_OTHER_MATH unpatched; by default they are patched, as
    the reference patches them.
    """

    def __init__(self, patch_layernorm: bool = True, patch_mlp: bool = True,
                 patch_attention: bool = True, patch_rope: bool = True, patch_fp8: bool = False,
                 verbose: bool = False, skip_inexact_norms: bool = False):
        self.skip_inexact_norms = skip_inexact_norms
        self.patch_layernorm = patch_layernorm
        self.patch_mlp = patch_mlp
        self.patch_attention = patch_attention
        self.patch_rope = patch_rope
        self.patch_fp8 = patch_fp8
        self.verbose = verbose
        self.patched_layers: List[Tuple[str, str]] = []

    def patch(self, model: nn.Module) -> nn.Module:
        for name, module in model.named_modules():
            cls = module.__class__.__name__
            fn = LAYER_PATCHES.get(cls)
            if fn is None or getattr(module, "_trainscale_amd_patched", False):
                continue
            if cls.endswith(("RMSNorm", "LayerNorm")):
                if not self.patch_layernorm:
                    continue
                if self.skip_inexact_norms and cls in NORMS_WITH_OTHER_MATH:
                    continue
            elif cls.endswith("MLP"):
                if not self.patch_mlp:
                    continue
            elif "Rotary" in cls:
                if not self.patch_rope:
                    continue
            fn(module)
            if getattr(module, "_trainscale_amd_patched", False):
                self.patched_layers.append((name, cls))
        if self.verbose and self.patched_layers:
            print(f"patched {len(self.patched_layers)} layers")
        return model


def patch_model(model: nn.Module) -> nn.Module:
    return KernelPatcher().patch(model)
