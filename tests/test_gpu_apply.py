"""The drop-in load path on the GPU, end to end: a transformers Gemma decoder (PaliGemma-2B
layer shapes, eager attention) saved as a checkpoint under the policy's module path,
packed by ``pack_w4a4_prefix.pack_checkpoint`` (the reference's ``scripts/pack_w4a4_prefix.py``
format), installed by ``apply_w4a4_from_dir`` (apply.py:91-118) and run through
transformers' own ``GemmaModel.forward`` (its causal mask, rotary tables and KV cache).

Every W4A4 op of that forward is recorded and checked against the oracle on its actual
input (as in test_gpu_prefix_lm.py), the fused decoder layers must be the ones that ran,
and the KV cache must hold the prefix's key/value states.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from tests.test_gpu_prefix_lm import _check_call, _Recorder

pytestmark = pytest.mark.gpu

PREFIX = "paligemma_with_expert.paligemma.model.language_model"


class _Policy(nn.Module):
    """The module path of the PaliGemma language model inside the policy."""

    def __init__(self, lm: nn.Module):
        super().__init__()
        self.paligemma_with_expert = nn.Module()
        self.paligemma_with_expert.paligemma = nn.Module()
        self.paligemma_with_expert.paligemma.model = nn.Module()
        self.paligemma_with_expert.paligemma.model.language_model = lm


def _gemma(layers: int):
    from transformers.models.gemma.configuration_gemma import GemmaConfig
    from transformers.models.gemma.modeling_gemma import GemmaModel

    from pi05_fast.w4a4.prefix_lm import PALIGEMMA_2B_LM

    kw = dict(PALIGEMMA_2B_LM)
    kw.update(num_hidden_layers=layers, vocab_size=512)
    cfg = GemmaConfig(**kw)
    cfg._attn_implementation = "eager"
    torch.manual_seed(20260923)
    lm = GemmaModel(cfg)
    with torch.no_grad():
        for name, p in lm.named_parameters():
            if name.endswith("proj.weight"):
                p.normal_(0.0, 0.02)
            elif "norm" in name:
                p.normal_(0.0, 0.05)
    return lm


def _pack(tmp_path, layers: int):
    """A Gemma LM of PaliGemma-2B layer shapes, its checkpoint under the policy's module
    path and the W4A4 pack written from it."""
    from safetensors.torch import save_file

    from pi05_fast.w4a4.pack_w4a4_prefix import pack_checkpoint

    lm = _gemma(layers)
    ckpt = {f"model.{PREFIX}.{k}": v.contiguous() for k, v in lm.state_dict().items() if k.endswith("proj.weight")}
    save_file(ckpt, str(tmp_path / "model.safetensors"))
    meta = pack_checkpoint(tmp_path / "model.safetensors", tmp_path / "pack")
    assert len(meta["layers"]) == 7 * layers
    return lm


def _run_lm(lm, cuda, s=300):
    from transformers.cache_utils import DynamicCache

    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(1, s, 2048, generator=gen) / 2048**0.5).half().to(cuda)
    cache = DynamicCache()
    with torch.no_grad():
        out = lm(inputs_embeds=x, use_cache=True, past_key_values=cache)
    torch.cuda.synchronize()
    hidden = out.last_hidden_state
    assert hidden.shape == (1, s, 2048) and torch.isfinite(hidden).all()
    return hidden, cache


def _cast_floating_tensors(module, dtype) -> None:
    """The reference's prefix-LM cast after the pack is applied (rocm_pi05_optim.py:136-154):
    floating parameters and buffers are cast in place, the INT4 packed weights are left."""
    for t in list(module.parameters()) + list(module.buffers()):
        if t.is_floating_point() and t.dtype != dtype:
            t.data = t.data.to(dtype)


def _check_fused_forward(lm, cuda, monkeypatch, layers, s=300):
    rec = _Recorder(monkeypatch)
    _, cache = _run_lm(lm, cuda, s)
    kinds = [c[0] for c in rec.calls]
    assert kinds.count("rms_norm_int4_gemm3") == layers
    assert kinds.count("prefix_attention_o_proj") == layers
    assert kinds.count("rms_norm_int4_gemm2_gelu") == layers
    assert kinds.count("int4_gemm_residual") == layers
    for i, call in enumerate(rec.calls):
        _check_call(cuda, i, call)
    assert cache.get_seq_length(0) == s and cache.get_seq_length(layers - 1) == s
    # the cached key states are the RoPE'd keys the attention op returned
    att = [c for c in rec.calls if c[0] == "prefix_attention_o_proj"]
    assert torch.equal(cache.layers[0].keys, att[0][3][1])


def test_pack_apply_forward(cuda, tmp_path, monkeypatch):
    from pi05_fast.w4a4 import W4A4Linear
    from pi05_fast.w4a4.apply import apply_w4a4_from_dir
    from pi05_fast.w4a4.norm import FusedRMSNorm

    layers = 2
    lm = _pack(tmp_path, layers)
    policy = _Policy(lm.to(device=cuda, dtype=torch.float16)).eval()
    assert apply_w4a4_from_dir(policy, tmp_path / "pack") == 7 * layers
    for layer in lm.layers:
        assert hasattr(layer, "_w4a4_layer_forward"), "fused decoder layer not installed"
        assert isinstance(layer.input_layernorm, FusedRMSNorm)
        assert all(isinstance(getattr(layer.mlp, p), W4A4Linear) for p in ("gate_proj", "up_proj", "down_proj"))
    _check_fused_forward(lm, cuda, monkeypatch, layers)


def test_pack_applied_to_bf16_model_then_cast_to_fp16(cuda, tmp_path, monkeypatch):
    """The reference's order (rocm_pi05_optim.py:216-237): the policy is cast to bf16, the
    pack is applied, and only then is the prefix LM cast to fp16.  The fused norms and
    decoder layers are installed by structure, so after the cast the forward runs them."""
    from pi05_fast.w4a4.apply import apply_w4a4_from_dir
    from pi05_fast.w4a4.norm import FusedRMSNorm

    layers = 2
    lm = _pack(tmp_path, layers)
    policy = _Policy(lm.to(device=cuda, dtype=torch.bfloat16)).eval()
    assert apply_w4a4_from_dir(policy, tmp_path / "pack") == 7 * layers
    for layer in lm.layers:
        assert hasattr(layer, "_w4a4_layer_forward"), "fused decoder layer not installed on the bf16 model"
        assert isinstance(layer.input_layernorm, FusedRMSNorm)
        assert layer.input_layernorm.weight.dtype == torch.bfloat16
    _cast_floating_tensors(lm, torch.float16)
    assert lm.layers[0].input_layernorm.weight.dtype == torch.float16
    _check_fused_forward(lm, cuda, monkeypatch, layers)


def test_pack_apply_reference_layouts(cuda, tmp_path, monkeypatch):
    """PI05_W4A4_MFMA=0: the reference's load-time layouts are kept (q/k/v/o/down row-padded
    to K/8+8, gate/up WMMA-preshuffled to K/8+9, apply.py:45-88) and the reference's call
    routes run: int4_gemm3 for QKV, int4_gemm2_tiled + act_fn for gate/up, int4_gemm for o
    and down.  Every op matches the oracle, and each weight is repacked into the MFMA
    layout on its first call only (a second forward repacks nothing)."""
    from pi05_fast.w4a4 import extension as ext
    from pi05_fast.w4a4.apply import apply_w4a4_from_dir

    monkeypatch.setenv("PI05_W4A4_MFMA", "0")
    layers = 2
    lm = _pack(tmp_path, layers)
    policy = _Policy(lm.to(device=cuda, dtype=torch.float16)).eval()
    assert apply_w4a4_from_dir(policy, tmp_path / "pack") == 7 * layers
    mlp = lm.layers[0].mlp
    assert mlp.gate_proj.preshuffled and mlp.gate_proj.packed.shape[1] == 2048 // 8 + 9
    assert lm.layers[0].self_attn.o_proj.packed.shape[1] == 2048 // 8 + 8
    assert not mlp._w4a4_fuse_gelu
    assert not hasattr(lm.layers[0], "_w4a4_layer_forward")

    repacks = []
    real = ext.repack_weight

    def counting(*a, **kw):
        repacks.append(tuple(a[0].shape))
        return real(*a, **kw)

    monkeypatch.setattr(ext, "repack_weight", counting)
    rec = _Recorder(monkeypatch)
    y1, _ = _run_lm(lm, cuda)
    assert len(repacks) == 7 * layers
    kinds = [c[0] for c in rec.calls]
    assert kinds.count("int4_gemm3") == layers
    assert kinds.count("int4_gemm2_tiled") == layers
    assert kinds.count("int4_gemm") == 2 * layers
    for i, call in enumerate(rec.calls):
        _check_call(cuda, i, call)
    y2, _ = _run_lm(lm, cuda)
    assert len(repacks) == 7 * layers, "weights were repacked again on the second forward"
    assert torch.equal(y1, y2)
