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


def test_pack_apply_forward(cuda, tmp_path, monkeypatch):
    from safetensors.torch import save_file

    from pi05_fast.w4a4 import W4A4Linear
    from pi05_fast.w4a4.apply import apply_w4a4_from_dir
    from pi05_fast.w4a4.norm import FusedRMSNorm
    from pi05_fast.w4a4.pack_w4a4_prefix import pack_checkpoint
    from transformers.cache_utils import DynamicCache

    layers = 2
    lm = _gemma(layers)
    ckpt = {f"model.{PREFIX}.{k}": v.contiguous() for k, v in lm.state_dict().items() if k.endswith("proj.weight")}
    save_file(ckpt, str(tmp_path / "model.safetensors"))
    meta = pack_checkpoint(tmp_path / "model.safetensors", tmp_path / "pack")
    assert len(meta["layers"]) == 7 * layers

    policy = _Policy(lm.to(device=cuda, dtype=torch.float16)).eval()
    assert apply_w4a4_from_dir(policy, tmp_path / "pack") == 7 * layers
    for layer in lm.layers:
        assert hasattr(layer, "_w4a4_layer_forward"), "fused decoder layer not installed"
        assert isinstance(layer.input_layernorm, FusedRMSNorm)
        assert all(isinstance(getattr(layer.mlp, p), W4A4Linear) for p in ("gate_proj", "up_proj", "down_proj"))

    rec = _Recorder(monkeypatch)
    s = 300
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(1, s, 2048, generator=gen) / 2048**0.5).half().to(cuda)
    cache = DynamicCache()
    with torch.no_grad():
        out = lm(inputs_embeds=x, use_cache=True, past_key_values=cache)
    torch.cuda.synchronize()
    hidden = out.last_hidden_state
    assert hidden.shape == (1, s, 2048) and torch.isfinite(hidden).all()
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
