"""Host-side logic that needs no GPU: no silent CPU fallback, workload generators,
byte accounting, and the RMSNorm patch boundary."""
import pytest
import torch
import torch.nn as nn

from trainscale_amd import ops, registry, workloads as W
from trainscale_amd.kernels import (Fast_RoPE, apply_rope, fast_cross_entropy_loss,
                                    fast_rms_layernorm, rms_layernorm)
from trainscale_amd.loss import ChunkedCrossEntropyLoss


def test_cpu_tensors_raise_instead_of_falling_back():
    x = torch.randn(4, 64)
    w = torch.ones(64)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        fast_rms_layernorm(x, w)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        rms_layernorm(x, w)
    q = torch.randn(1, 4, 2, 16)
    cos = torch.ones(4, 8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        Fast_RoPE.apply(q, q.clone(), cos, cos, False)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        apply_rope(q, cos, cos)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        fast_cross_entropy_loss(torch.randn(4, 32), torch.zeros(4, dtype=torch.long))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ChunkedCrossEntropyLoss()(torch.randn(4, 32), torch.zeros(4, dtype=torch.long))


def test_as_rows_strides():
    t = torch.randn(3, 5, 16)
    t2, ld = ops.as_rows(t)
    assert t2.shape == (15, 16) and ld == 16
    big = torch.randn(10, 48)
    v, ld = ops.as_rows(big[:, 16:32])
    assert ld == 48 and v.data_ptr() == big[:, 16:32].data_ptr()
    e = torch.randn(1, 16).expand(4, 16)
    v, ld = ops.as_rows(e)
    assert ld == 16 and v.is_contiguous()


def test_config_byte_counts():
    # compulsory traffic quoted for the configs (fwd + bwd)
    b = W.rmsnorm_bytes(16384, 4096)
    assert b["fwd"] == 268_509_184 and b["fwd"] + b["bwd"] == 671_244_288
    b = W.rope_bytes(16384, 40, 128)
    assert b["fwd"] + b["bwd"] == 671_088_640
    b = W.rmsnorm_bytes(32768, 8192)
    assert b["fwd"] == 1_073_889_280 and b["bwd"] == 1_610_776_576
    b = W.rope_bytes(32768, 72, 128, pos_bytes=32768 * 8)
    assert b["fwd"] == 1_208_221_696
    assert W.linear_ce_flops(8192, 4096, 128256) == 25_821_343_383_552


def test_packed_lengths_and_position_ids():
    lens = W.packed_doc_lengths(32768, 64, 4096, 3)
    assert sum(lens) == 32768
    assert all(1 <= n <= 4096 for n in lens) and all(n >= 64 for n in lens[:-1])
    pos = W.packed_position_ids(lens)
    assert pos.shape == (1, 32768)
    starts = [0]
    for n in lens[:-1]:
        starts.append(starts[-1] + n)
    assert all(int(pos[0, s]) == 0 for s in starts)
    assert int(pos.max()) == max(lens) - 1


def test_workload_generators_are_seeded():
    a = W.ce_workload("cpu", scale=1 / 256, V=1000)
    b = W.ce_workload("cpu", scale=1 / 256, V=1000)
    assert torch.equal(a.tensors["logits"], b.tensors["logits"])
    labels = a.tensors["labels"]
    assert int((labels == -100).sum()) == round(0.1 * labels.numel())


class LlamaRMSNorm(nn.Module):
    def __init__(self, n, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(n))
        self.variance_epsilon = eps

    def forward(self, h):
        var = h.float().pow(2).mean(-1, keepdim=True)
        return self.weight * (h * torch.rsqrt(var + self.variance_epsilon)).to(h.dtype)


def test_patch_boundary_keeps_cpu_modules_on_their_own_forward():
    model = nn.Sequential(nn.Linear(8, 8), LlamaRMSNorm(8))
    x = torch.randn(3, 8)
    before = model(x)
    patcher = registry.KernelPatcher()
    patcher.patch(model)
    assert patcher.patched_layers == [("1", "LlamaRMSNorm")]
    assert torch.equal(model(x), before)  # CPU tensors: the module's original forward
    assert "LlamaRMSNorm" in registry.LAYER_PATCHES


class GemmaRMSNorm(nn.Module):
    """HF Gemma's norm: x * rstd * (1 + w), w initialised to zeros."""

    def __init__(self, n, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(n))
        self.eps = eps

    def forward(self, h):
        var = h.float().pow(2).mean(-1, keepdim=True)
        return (h.float() * torch.rsqrt(var + self.eps) * (1.0 + self.weight.float())).to(h.dtype)


def test_norms_with_other_math_are_patched_as_the_reference_does_unless_skipped():
    # registry/__init__.py:1058-1077 routes GemmaRMSNorm to the plain RMSNorm kernel;
    # KernelPatcher does too by default, and leaves it alone with skip_inexact_norms
    assert registry.LAYER_PATCHES["GemmaRMSNorm"] is registry.auto_patch_layernorm
    assert set(registry.NORMS_WITH_OTHER_MATH) <= set(registry.LAYER_PATCHES)
    m1 = nn.Sequential(GemmaRMSNorm(8), LlamaRMSNorm(8))
    p1 = registry.KernelPatcher()
    p1.patch(m1)
    assert p1.patched_layers == [("0", "GemmaRMSNorm"), ("1", "LlamaRMSNorm")]
    m2 = nn.Sequential(GemmaRMSNorm(8), LlamaRMSNorm(8))
    p2 = registry.KernelPatcher(skip_inexact_norms=True)
    p2.patch(m2)
    assert p2.patched_layers == [("1", "LlamaRMSNorm")]
    assert not getattr(m2[0], "_trainscale_amd_patched", False)


class LlamaMLP(nn.Module):
    def __init__(self, h, i):
        super().__init__()
        self.gate_proj = nn.Linear(h, i, bias=False)
        self.up_proj = nn.Linear(h, i, bias=False)
        self.down_proj = nn.Linear(i, h, bias=False)

    def forward(self, x):
        return self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


def test_patch_boundary_mlp_and_flags():
    model = nn.Sequential(LlamaMLP(8, 16), LlamaRMSNorm(8))
    x = torch.randn(3, 8)
    before = model(x)
    patcher = registry.KernelPatcher(patch_layernorm=False)
    patcher.patch(model)
    assert patcher.patched_layers == [("0", "LlamaMLP")]
    assert torch.equal(model(x), before)  # CPU tensors keep the original forward
    p2 = registry.KernelPatcher()
    p2.patch(model)  # idempotent for the MLP, patches the norm now
    assert p2.patched_layers == [("1", "LlamaRMSNorm")]
    assert "LlamaMLP" in registry.LAYER_PATCHES and "Qwen2MLP" in registry.LAYER_PATCHES


def test_position_ids_from_cu_seqlens_matches_pack_sequences_format():
    from trainscale_amd.kernels.rope_kernels import position_ids_from_cu_seqlens
    rows, cus = [], []
    for seed, total in ((1, 700), (2, 1024)):
        lens = W.packed_doc_lengths(total, 5, 200, seed)
        pos = W.packed_position_ids(lens)[0]
        pad = torch.zeros(1024 - pos.numel(), dtype=torch.int64)
        rows.append(torch.cat([pos, pad]))  # pack_sequences pads positions with 0
        cus.append(torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32))
    expect = torch.stack(rows)
    got = position_ids_from_cu_seqlens(cus, total=1024)
    assert torch.equal(got, expect)
    assert torch.equal(position_ids_from_cu_seqlens(cus[1]), expect[1:])


def test_rope_patch_routes_hf_apply_and_keeps_cpu_path():
    transformers = pytest.importorskip("transformers")
    from transformers.models.llama import modeling_llama as ml
    original = ml.apply_rotary_pos_emb
    cfg = transformers.LlamaConfig(hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                                   num_attention_heads=4, num_key_value_heads=2,
                                   vocab_size=100, max_position_embeddings=64)
    torch.manual_seed(0)
    model = transformers.LlamaModel(cfg).eval()
    ids = torch.randint(0, 100, (2, 9))
    with torch.no_grad():
        before = model(ids).last_hidden_state
    try:
        patcher = registry.KernelPatcher(patch_layernorm=False, patch_mlp=False)
        patcher.patch(model)
        assert ("rotary_emb", "LlamaRotaryEmbedding") in patcher.patched_layers
        assert ml.apply_rotary_pos_emb is not original
        assert ml.apply_rotary_pos_emb._trainscale_amd_original is original
        assert model.rotary_emb._rope_config.dim in (16, 64)
        with torch.no_grad():
            after = model(ids).last_hidden_state  # CPU tensors: the original function
        assert torch.equal(before, after)
    finally:
        ml.apply_rotary_pos_emb = original


def test_guard_bands_see_every_stray_write():
    """The guard-band check of tests/test_gpu_guard.py, on the CPU: a write one element
    before the tensor, one past it, or into the padding between its rows is seen, and
    so is a changed NaN payload; writes inside the tensor are not."""
    from helpers import Guarded, same
    for dtype in (torch.bfloat16, torch.float16, torch.float32, torch.uint8):
        vals = torch.arange(12).reshape(3, 4).to(dtype)
        g = Guarded(3, 4, 6, dtype, torch.device("cpu"), vals)
        assert g.intact() and torch.equal(g.t, vals)
        g.t.zero_()
        assert g.intact()  # inside the tensor
        base = g.t.storage_offset()
        for off in (-1, 4, 6 * 2 + 4, 6 * 3):  # before, row padding (two rows), past the end
            h = Guarded(3, 4, 6, dtype, torch.device("cpu"), vals)
            h.buf[base + off] = 1
            assert not h.intact(), (dtype, off)
    a = torch.tensor([float("nan")], dtype=torch.bfloat16)
    b = a.view(torch.int16).clone().add_(1).view(torch.bfloat16)  # another NaN payload
    assert same(a, a) and not same(a, b)
