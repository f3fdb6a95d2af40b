"""Drop-in counterparts of TrainScale's ``kernels/rope_kernels.py``.

Reference (``data_pipeline/trainer/``):

* frequency tables: ``RoPEConfig``, ``RoPEScalingType``, ``compute_rope_frequencies``,
  ``precompute_freqs_cis`` (kernels/rope_kernels.py:37-78, :146-375) — host-side
  table math, restated here op for op;
* ``RoPEFunction`` / ``apply_rope(x, cos, sin, position_ids, position_offset,
  interleaved, inplace)`` (:1031-1106, :1258-1285): single tensor, optional
  explicit ``position_ids`` (packed sequences), in place by default;
* ``FusedRoPEQKFunction`` / ``apply_rope_qk`` / ``inplace_rope_embedding``
  (:1109-1198, :1288-1350): Q and K together, in place, ``position_offset``;
* ``Fast_RoPE_Embedding`` / ``fast_rope_embedding`` (:1202-1251, :1316-1322);
* ``RotaryEmbedding`` (:1357-1492).

All rotations run in one gfx950 kernel (``ts_rope_apply``): fp32 arithmetic,
one rounding to the data dtype. Backward is the transpose rotation written to a
new gradient tensor in one pass (the reference clones the gradient and then
rotates it in place: two passes).

Semantics kept from the reference: in-place forwards return the input tensor
object modified in place. One difference: 1-D ``position_ids`` of length S are
applied to every sequence of the batch (the reference's Triton path indexed a
1-D tensor by the batch index instead).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from enum import Enum, auto
from typing import Dict, List, Optional, Tuple, Union

import torch
import torch.nn as nn
from torch import Tensor

from .. import ops

__all__ = [
    "RoPEConfig",
    "RoPEScalingType",
    "precompute_freqs_cis",
    "compute_rope_frequencies",
    "compute_inv_freq",
    "RoPEFrequencyCache",
    "RoPEFunction",
    "FusedRoPEQKFunction",
    "Fast_RoPE_Embedding",
    "apply_rope",
    "apply_rope_qk",
    "fast_rope_embedding",
    "inplace_rope_embedding",
    "apply_rope_theta",
    "RotaryEmbedding",
    "hf_apply_rotary_pos_emb",
    "position_ids_from_cu_seqlens",
    "ROPE_GROUP_SIZE",
]

ROPE_GROUP_SIZE = 4  # kept for API compatibility; the gfx950 kernel needs no head grouping


class RoPEScalingType(Enum):
    NONE = auto()
    LINEAR = auto()
    NTK = auto()
    YARN = auto()
    DYNAMIC_NTK = auto()
    LONGROPE = auto()


@dataclass
class RoPEConfig:
    """RoPE configuration (reference: kernels/rope_kernels.py:47-78)."""
    dim: int
    max_seq_len: int = 8192
    base: float = 10000.0
    scaling_type: RoPEScalingType = RoPEScalingType.NONE
    scaling_factor: float = 1.0
    yarn_beta_fast: float = 32.0
    yarn_beta_slow: float = 1.0
    yarn_mscale: float = 1.0
    yarn_mscale_all_dim: float = 0.0
    ntk_alpha: Optional[float] = None
    longrope_short_factor: Optional[List[float]] = None
    longrope_long_factor: Optional[List[float]] = None
    use_fp32_precision: bool = True
    cache_freqs: bool = True
    block_size: int = 64
    num_warps: int = 4
    group_size: int = 4


_SCALING_NAMES = {
    "none": RoPEScalingType.NONE,
    "linear": RoPEScalingType.LINEAR,
    "pi": RoPEScalingType.LINEAR,
    "ntk": RoPEScalingType.NTK,
    "dynamic_ntk": RoPEScalingType.DYNAMIC_NTK,
    "yarn": RoPEScalingType.YARN,
    "longrope": RoPEScalingType.LONGROPE,
}


def _base_inv_freq(base: float, dim: int, device) -> Tensor:
    return 1.0 / (base ** (torch.arange(0, dim, 2, device=device, dtype=torch.float32) / dim))


def compute_inv_freq(config: RoPEConfig, device=None) -> Tensor:
    """Inverse frequencies per scaling type (reference: kernels/rope_kernels.py:198-314)."""
    dim = config.dim
    st = config.scaling_type
    if st == RoPEScalingType.NTK:
        base = config.base * (config.scaling_factor ** (dim / (dim - 2)))
        return _base_inv_freq(base, dim, device)
    if st == RoPEScalingType.DYNAMIC_NTK:
        base = config.base * ((config.scaling_factor * config.max_seq_len / config.max_seq_len)
                              - (config.scaling_factor - 1)) ** (dim / (dim - 2))
        return _base_inv_freq(base, dim, device)
    if st == RoPEScalingType.YARN:
        base_inv = _base_inv_freq(config.base, dim, device)
        wavelengths = 2 * math.pi / base_inv
        low_freq = wavelengths / config.yarn_beta_fast
        high_freq = wavelengths / config.yarn_beta_slow
        ramp = torch.clamp((wavelengths - low_freq) / (high_freq - low_freq), 0.0, 1.0)
        return base_inv * (1 - ramp) + (base_inv / config.scaling_factor) * ramp
    if st == RoPEScalingType.LONGROPE:
        base_inv = _base_inv_freq(config.base, dim, device)
        if config.longrope_long_factor is not None:
            factors = torch.tensor(config.longrope_long_factor, device=device,
                                   dtype=torch.float32)[: dim // 2]
            return base_inv / factors
        return base_inv
    return _base_inv_freq(config.base, dim, device)


def _yarn_mscale(config: RoPEConfig) -> float:
    if config.yarn_mscale_all_dim > 0:
        return config.yarn_mscale_all_dim
    if config.scaling_factor <= 1.0:
        return 1.0
    return 0.1 * math.log(config.scaling_factor) + 1.0


def compute_rope_frequencies(config: RoPEConfig, seq_len: int, device, dtype) -> Tuple[Tensor, Tensor]:
    """cos/sin [seq_len, dim//2] (reference: kernels/rope_kernels.py:146-195)."""
    inv_freq = compute_inv_freq(config, device)
    t = torch.arange(seq_len, device=device, dtype=torch.float32)
    if config.scaling_type == RoPEScalingType.LINEAR:
        t = t / config.scaling_factor
    freqs = torch.outer(t, inv_freq)
    if config.scaling_type == RoPEScalingType.YARN:
        freqs = freqs * _yarn_mscale(config)
    cos = torch.cos(freqs)
    sin = torch.sin(freqs)
    if dtype != torch.float32:
        cos = cos.to(dtype)
        sin = sin.to(dtype)
    return cos, sin


class RoPEFrequencyCache:
    """Memoised cos/sin tables (reference: kernels/rope_kernels.py:109-143)."""

    _cache: Dict[Tuple, Tuple[Tensor, Tensor]] = {}

    @classmethod
    def clear_cache(cls):
        cls._cache.clear()

    @classmethod
    def get_freqs(cls, config: RoPEConfig, seq_len: int, device, dtype) -> Tuple[Tensor, Tensor]:
        key = (config.dim, config.base, config.scaling_type, config.scaling_factor, seq_len,
               device, dtype)
        if key not in cls._cache or not config.cache_freqs:
            cos, sin = compute_rope_frequencies(config, seq_len, device, dtype)
            if config.cache_freqs:
                cls._cache[key] = (cos, sin)
            return cos, sin
        return cls._cache[key]


def precompute_freqs_cis(dim: int, max_seq_len: int, theta: float = 10000.0,
                         scaling_factor: float = 1.0, scaling_type: str = "none",
                         device: Union[str, torch.device] = "cuda",
                         dtype: torch.dtype = torch.float32, **kwargs) -> Tuple[Tensor, Tensor]:
    """cos/sin tables (reference: kernels/rope_kernels.py:317-375)."""
    config = RoPEConfig(
        dim=dim, max_seq_len=max_seq_len, base=theta,
        scaling_type=_SCALING_NAMES.get(scaling_type.lower(), RoPEScalingType.NONE),
        scaling_factor=scaling_factor,
        yarn_beta_fast=kwargs.get("yarn_beta_fast", 32.0),
        yarn_beta_slow=kwargs.get("yarn_beta_slow", 1.0),
        yarn_mscale=kwargs.get("yarn_mscale", 1.0),
        longrope_long_factor=kwargs.get("longrope_long_factor"),
        longrope_short_factor=kwargs.get("longrope_short_factor"),
    )
    if isinstance(device, str):
        device = torch.device(device)
    return compute_rope_frequencies(config, max_seq_len, device, dtype)


# ---------------------------------------------------------------------------
# Autograd functions
# ---------------------------------------------------------------------------

class RoPEFunction(torch.autograd.Function):
    """Single-tensor RoPE (reference: kernels/rope_kernels.py:1031-1106)."""

    @staticmethod
    def forward(ctx, x: Tensor, cos: Tensor, sin: Tensor, position_ids: Optional[Tensor],
                position_offset: int, interleaved: bool, inplace: bool) -> Tensor:
        ctx.save_for_backward(cos, sin, position_ids)
        ctx.position_offset = position_offset
        ctx.interleaved = interleaved
        ctx.shape = x.shape
        x = ops._bshd(x, "apply_rope x")
        out = x if inplace else torch.empty_like(x, memory_format=torch.contiguous_format)
        ops.rope_apply(x, out, None, None, cos=cos, sin=sin, position_ids=position_ids,
                       position_offset=position_offset, interleaved=interleaved)
        return out

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        cos, sin, position_ids = ctx.saved_tensors
        g = ops._bshd(grad_output, "apply_rope grad")
        grad_input = torch.empty_like(g, memory_format=torch.contiguous_format)
        ops.rope_apply(g, grad_input, None, None, cos=cos, sin=sin, position_ids=position_ids,
                       position_offset=ctx.position_offset, interleaved=ctx.interleaved,
                       backward=True)
        return grad_input, None, None, None, None, None, None


class FusedRoPEQKFunction(torch.autograd.Function):
    """Q and K in one launch, in place (reference: kernels/rope_kernels.py:1109-1198)."""

    @staticmethod
    def forward(ctx, Q: Tensor, K: Tensor, cos: Tensor, sin: Tensor, position_offset: int,
                interleaved: bool) -> Tuple[Tensor, Tensor]:
        ctx.save_for_backward(cos, sin)
        ctx.position_offset = position_offset
        ctx.interleaved = interleaved
        Q = ops._bshd(Q, "apply_rope_qk Q")
        K = ops._bshd(K, "apply_rope_qk K")
        ops.rope_apply(Q, Q, K, K, cos=cos, sin=sin, position_offset=position_offset,
                       interleaved=interleaved)
        return Q, K

    @staticmethod
    def backward(ctx, dQ: Optional[Tensor], dK: Optional[Tensor]):
        cos, sin = ctx.saved_tensors
        dq_out = dk_out = None
        if dQ is not None:
            dQ = ops._bshd(dQ, "apply_rope_qk dQ")
            dq_out = torch.empty_like(dQ, memory_format=torch.contiguous_format)
        if dK is not None:
            dK = ops._bshd(dK, "apply_rope_qk dK")
            dk_out = torch.empty_like(dK, memory_format=torch.contiguous_format)
        ops.rope_apply(dQ, dq_out, dK, dk_out, cos=cos, sin=sin,
                       position_offset=ctx.position_offset, interleaved=ctx.interleaved,
                       backward=True)
        return dq_out, dk_out, None, None, None, None


class Fast_RoPE_Embedding(torch.autograd.Function):
    """Legacy in-place single-tensor RoPE (reference: kernels/rope_kernels.py:1202-1251)."""

    @staticmethod
    def forward(ctx, Q: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
        cos = cos.squeeze()
        sin = sin.squeeze()
        ctx.save_for_backward(cos, sin)
        Q = ops._bshd(Q, "fast_rope_embedding Q")
        ops.rope_apply(Q, Q, None, None, cos=cos, sin=sin)
        return Q

    @staticmethod
    def backward(ctx, dQ: Tensor):
        cos, sin = ctx.saved_tensors
        dQ = ops._bshd(dQ, "fast_rope_embedding dQ")
        out = torch.empty_like(dQ, memory_format=torch.contiguous_format)
        ops.rope_apply(dQ, out, None, None, cos=cos, sin=sin, backward=True)
        return out, None, None


class _RoPEThetaFunction(torch.autograd.Function):
    """RoPE with sin/cos evaluated on the GPU from inv_freq (no tables)."""

    @staticmethod
    def forward(ctx, x: Tensor, inv_freq: Tensor, pos_div: float,
                position_ids: Optional[Tensor], position_offset: int, interleaved: bool,
                inplace: bool, angle_scale: float = 1.0) -> Tensor:
        ctx.save_for_backward(position_ids)
        ctx.inv_freq = inv_freq
        ctx.pos_div = pos_div
        ctx.angle_scale = angle_scale
        ctx.position_offset = position_offset
        ctx.interleaved = interleaved
        x = ops._bshd(x, "apply_rope_theta x")
        out = x if inplace else torch.empty_like(x, memory_format=torch.contiguous_format)
        ops.rope_apply(x, out, None, None, inv_freq=inv_freq, pos_div=pos_div,
                       angle_scale=angle_scale, position_ids=position_ids,
                       position_offset=position_offset, interleaved=interleaved)
        return out

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        (position_ids,) = ctx.saved_tensors
        g = ops._bshd(grad_output, "apply_rope_theta grad")
        grad_input = torch.empty_like(g, memory_format=torch.contiguous_format)
        ops.rope_apply(g, grad_input, None, None, inv_freq=ctx.inv_freq, pos_div=ctx.pos_div,
                       angle_scale=ctx.angle_scale, position_ids=position_ids,
                       position_offset=ctx.position_offset, interleaved=ctx.interleaved,
                       backward=True)
        return grad_input, None, None, None, None, None, None, None


# ---------------------------------------------------------------------------
# API functions
# ---------------------------------------------------------------------------

def apply_rope(x: Tensor, cos: Tensor, sin: Tensor, position_ids: Optional[Tensor] = None,
               position_offset: int = 0, interleaved: bool = False,
               inplace: bool = True) -> Tensor:
    """RoPE of x [B,S,H,D] (reference: kernels/rope_kernels.py:1258-1285)."""
    return RoPEFunction.apply(x, cos.contiguous(), sin.contiguous(), position_ids,
                              position_offset, interleaved, inplace)


def apply_rope_qk(Q: Tensor, K: Tensor, cos: Tensor, sin: Tensor, position_offset: int = 0,
                  interleaved: bool = False) -> Tuple[Tensor, Tensor]:
    """In-place RoPE of Q and K (reference: kernels/rope_kernels.py:1288-1313)."""
    return FusedRoPEQKFunction.apply(Q, K, cos.contiguous(), sin.contiguous(), position_offset,
                                     interleaved)


def fast_rope_embedding(Q: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Legacy interface (reference: kernels/rope_kernels.py:1316-1322)."""
    return Fast_RoPE_Embedding.apply(Q, cos, sin)


def inplace_rope_embedding(Q: Tensor, K: Tensor, cos: Tensor, sin: Tensor,
                           position_offset: int = 0) -> Tuple[Tensor, Tensor]:
    """In-place NeoX RoPE of Q and K (reference: kernels/rope_kernels.py:1325-1350)."""
    cos = cos.squeeze().contiguous()
    sin = sin.squeeze().contiguous()
    return apply_rope_qk(Q, K, cos, sin, position_offset, interleaved=False)


def apply_rope_theta(x: Tensor, theta: float = 10000.0, position_ids: Optional[Tensor] = None,
                     position_offset: int = 0, interleaved: bool = False, inplace: bool = True,
                     scaling_factor: float = 1.0, inv_freq: Optional[Tensor] = None,
                     angle_scale: float = 1.0) -> Tensor:
    """RoPE with in-register sin/cos: no cos/sin tables are read.

    The angle of pair i at position p is fp32(p / scaling_factor) * inv_freq[i],
    the fp32 product ``precompute_freqs_cis`` forms on the host, with
    inv_freq = 1/theta**(arange(0, D, 2)/D) unless given, then times angle_scale
    when that is not 1 (YaRN's mscale, rope_kernels.py:181-184).
    """
    if inv_freq is None:
        inv_freq = _base_inv_freq(theta, x.shape[-1], "cpu")
    return _RoPEThetaFunction.apply(x, inv_freq, float(scaling_factor), position_ids,
                                    position_offset, interleaved, inplace, float(angle_scale))


class _HFTableRoPEFunction(torch.autograd.Function):
    """Rotation of HF-layout Q and K with HF's per-token cos/sin.

    q, k: [B, S, H, D] views (any strides, unit last stride); cos, sin: [B or 1, S, D]
    with duplicated halves (cat(freqs, freqs), the NeoX layout). Token (b, s)
    uses row b * S + s of the flattened tables (row s when they are shared over
    the batch), reading its first D / 2 columns. Returns new [B, S, H, D] tensors.
    """

    @staticmethod
    def forward(ctx, q: Tensor, k: Tensor, cos: Tensor, sin: Tensor):
        B, S = q.shape[0], q.shape[1]
        if cos.shape[0] == 1:
            pos = torch.arange(S, device=q.device, dtype=torch.int64)
        else:
            pos = torch.arange(B * S, device=q.device, dtype=torch.int64).view(B, S)
        cos2 = cos.reshape(-1, cos.shape[-1])
        sin2 = sin.reshape(-1, sin.shape[-1])
        q_out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        k_out = torch.empty(k.shape, dtype=k.dtype, device=k.device)
        ops.rope_apply(q, q_out, k, k_out, cos=cos2, sin=sin2, position_ids=pos)
        ctx.save_for_backward(cos2, sin2, pos)
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq: Tensor, dk: Tensor):
        cos2, sin2, pos = ctx.saved_tensors
        dq_in, dk_in = torch.empty_like(dq), torch.empty_like(dk)
        ops.rope_apply(dq, dq_in, dk, dk_in, cos=cos2, sin=sin2, position_ids=pos, backward=True)
        return dq_in, dk_in, None, None


def hf_apply_rotary_pos_emb(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor,
                            unsqueeze_dim: int = 1) -> Tuple[Tensor, Tensor]:
    """Drop-in for transformers' ``apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim)``:
    q, k are [B, H, S, D] (unsqueeze_dim=1) or [B, S, H, D] (unsqueeze_dim=2), cos/sin
    [B, S, D] with duplicated halves. Computes q*cos + rotate_half(q)*sin in fp32 with
    one rounding (transformers' eager form rounds each product and the sum)."""
    if unsqueeze_dim == 1:
        qo, ko = _HFTableRoPEFunction.apply(q.transpose(1, 2), k.transpose(1, 2), cos, sin)
        return qo.transpose(1, 2), ko.transpose(1, 2)
    return _HFTableRoPEFunction.apply(q, k, cos, sin)


def position_ids_from_cu_seqlens(cu_seqlens, total: Optional[int] = None) -> Tensor:
    """Per-token positions of packed rows from their document boundaries.

    cu_seqlens: one int32/int64 tensor [n_docs + 1] (0 = cu[0] < ... < cu[-1] = real
    tokens of the row) or a list of them, one per packed row: the format
    ``pack_sequences`` emits (data_pipeline/trainer/packing.py:98-194). Returns int64
    [rows, total] (total defaults to the longest row's cu[-1]) with positions 0..len-1
    inside each document and 0 on padding: the position_ids ``pack_sequences``
    builds, for ``apply_rope(..., position_ids=...)``. Runs on the tensors' device.
    """
    rows = list(cu_seqlens) if isinstance(cu_seqlens, (list, tuple)) else [cu_seqlens]
    rows = [c.to(torch.int64) for c in rows]
    n = int(max(int(c[-1].item()) for c in rows)) if total is None else int(total)
    out = torch.zeros((len(rows), n), dtype=torch.int64, device=rows[0].device)
    for i, cu in enumerate(rows):
        lens = cu[1:] - cu[:-1]
        starts = torch.repeat_interleave(cu[:-1], lens)
        real = starts.numel()
        if real > n:
            raise ValueError(f"position_ids_from_cu_seqlens: row {i} has {real} tokens > {n}")
        out[i, :real] = torch.arange(real, device=cu.device, dtype=torch.int64) - starts
    return out


class RotaryEmbedding(nn.Module):
    """RoPE module with cached tables (reference: kernels/rope_kernels.py:1357-1458).

    Like the reference, the tables are cast to the activation dtype before use.
    ``in_register=True`` evaluates sin/cos on the GPU in fp32 instead (more
    accurate than bf16 tables, no table reads), from the same fp32 angle as
    the tables, YaRN's mscale included.
    """

    def __init__(self, dim: int, max_seq_len: int = 8192, base: float = 10000.0,
                 scaling_type: str = "none", scaling_factor: float = 1.0,
                 interleaved: bool = False, in_register: bool = False, **kwargs):
        super().__init__()
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.base = base
        self.scaling_factor = scaling_factor
        self.interleaved = interleaved
        self.config = RoPEConfig(dim=dim, max_seq_len=max_seq_len, base=base,
                                 scaling_type=_SCALING_NAMES.get(scaling_type.lower(),
                                                                 RoPEScalingType.NONE),
                                 scaling_factor=scaling_factor, **kwargs)
        self.in_register = in_register
        cos, sin = compute_rope_frequencies(self.config, max_seq_len, torch.device("cpu"),
                                            torch.float32)
        self.register_buffer("cos_cached", cos, persistent=False)
        self.register_buffer("sin_cached", sin, persistent=False)
        self._seq_len_cached = max_seq_len
        self._inv_freq = compute_inv_freq(self.config, "cpu")

    def _update_cache(self, seq_len: int, device, dtype):
        if seq_len > self._seq_len_cached:
            cos, sin = compute_rope_frequencies(self.config, seq_len, device, dtype)
            self.cos_cached = cos
            self.sin_cached = sin
            self._seq_len_cached = seq_len
        elif self.cos_cached.device != device or self.cos_cached.dtype != dtype:
            self.cos_cached = self.cos_cached.to(device=device, dtype=dtype)
            self.sin_cached = self.sin_cached.to(device=device, dtype=dtype)

    def _pos_div(self) -> float:
        return self.config.scaling_factor if self.config.scaling_type == RoPEScalingType.LINEAR else 1.0

    def forward(self, x: Tensor, position_ids: Optional[Tensor] = None,
                position_offset: int = 0) -> Tensor:
        if self.in_register:
            mscale = (_yarn_mscale(self.config)
                      if self.config.scaling_type == RoPEScalingType.YARN else 1.0)
            return apply_rope_theta(x, position_ids=position_ids,
                                    position_offset=position_offset,
                                    interleaved=self.interleaved, inplace=True,
                                    scaling_factor=self._pos_div(), inv_freq=self._inv_freq,
                                    angle_scale=mscale)
        self._update_cache(x.shape[1] + position_offset, x.device, x.dtype)
        return apply_rope(x, self.cos_cached, self.sin_cached, position_ids=position_ids,
                          position_offset=position_offset, interleaved=self.interleaved,
                          inplace=True)

    def forward_qk(self, Q: Tensor, K: Tensor, position_ids: Optional[Tensor] = None,
                   position_offset: int = 0) -> Tuple[Tensor, Tensor]:
        # position_ids is accepted and ignored, as in the reference (:1460-1486).
        self._update_cache(Q.shape[1] + position_offset, Q.device, Q.dtype)
        return apply_rope_qk(Q, K, self.cos_cached, self.sin_cached,
                             position_offset=position_offset, interleaved=self.interleaved)

    def get_freqs(self, seq_len: int) -> Tuple[Tensor, Tensor]:
        return self.cos_cached[:seq_len], self.sin_cached[:seq_len]
