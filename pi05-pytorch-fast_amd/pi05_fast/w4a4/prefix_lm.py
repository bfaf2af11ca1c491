"""PaliGemma-2B-shaped prefix language model running every projection through W4A4.

The reference runs the PaliGemma Gemma-2B language model of LeRobot's PI05 policy with
all q/k/v/o/gate/up/down Linears replaced by W4A4 layers and the attention / MLP
forwards patched to the shared-quant fused versions (rocm_pi05_optim.py:204-237 ->
apply.py:91-213).  LeRobot is not available here, so this module assembles the same
stack from transformers' Gemma decoder layers: 18 layers, hidden 2048, 8 heads x 256,
1 KV head, intermediate 16384, RMSNorm (1 + w), RoPE, GELU-tanh, fp16, and installs the
same hooks (``apply.fuse_shared_activation_quant``); on the GPU the RMSNorms run as one
kernel each (``norm.fuse_rmsnorm``), RoPE + attention as the two kernels of
``extension.prefix_attention`` (``PI05_W4A4_FUSE_ATTN=0``: transformers' RoPE and the
fp16 eager attention below), and each decoder layer runs ``apply.fuse_decoder_layers``'
forward: norms fused into the activation quants, residual adds into the o/down GEMM
epilogues (``PI05_W4A4_FUSE_LAYER=0``: the per-module forwards).

Layers are constructed on the meta device (no fp32 weights are ever materialised); the
seven projections are W4A4Linear modules holding packed weights, the norms are real.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from pi05_fast.w4a4.apply import fuse_decoder_layers, fuse_shared_activation_quant, load_time_weight
from pi05_fast.w4a4.linear import W4A4Linear
from pi05_fast.w4a4.norm import fuse_rmsnorm

PALIGEMMA_2B_LM = dict(
    hidden_size=2048,
    num_hidden_layers=18,
    num_attention_heads=8,
    num_key_value_heads=1,
    head_dim=256,
    intermediate_size=16384,
    rms_norm_eps=1e-6,
    rope_theta=10000.0,
    hidden_act="gelu_pytorch_tanh",
    max_position_embeddings=8192,
    vocab_size=257152,
)

PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
ATTN_IMPL = "w4a4_eager"


def _eager_attention(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
    """fp16 eager attention with fp32 softmax (transformers' eager_attention_forward
    semantics: repeat_kv, scaled QK^T, additive mask, softmax(fp32) -> fp16, PV).  The
    transposed key is made contiguous before the batched product."""
    n_rep = query.shape[1] // key.shape[1]
    if n_rep > 1:
        b, h, s, d = key.shape
        key = key[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)
        value = value[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)
    scores = torch.matmul(query, key.transpose(2, 3).contiguous()) * scaling
    if attention_mask is not None:
        scores = scores + attention_mask[:, :, :, : key.shape[-2]]
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype)
    out = torch.matmul(probs, value.contiguous())
    return out.transpose(1, 2).contiguous(), probs


def _register_attention() -> None:
    from transformers.modeling_utils import AttentionInterface

    AttentionInterface.register(ATTN_IMPL, _eager_attention)


def gemma_config(num_layers: int | None = None, **overrides):
    from transformers.models.gemma.configuration_gemma import GemmaConfig

    kw = dict(PALIGEMMA_2B_LM)
    if num_layers is not None:
        kw["num_hidden_layers"] = num_layers
    kw.update(overrides)
    cfg = GemmaConfig(**kw)
    _register_attention()
    cfg._attn_implementation = ATTN_IMPL
    return cfg


def synthetic_packed_weight(n: int, k: int, device, gen: torch.Generator) -> torch.Tensor:
    """Packed int32 [N, K/8+1] of a synthetic rotated weight: codes ~ round(N(0, 2))
    clamped to [-7, 7] (the code statistics of a packed N(0, 0.02) weight) and scales
    0.01 * U[0.9, 1.1).  Generated on `device` (no CPU packing of 2B weights)."""
    codes = torch.randn((n, k), device=device, generator=gen).mul_(2.0).round_().clamp_(-7, 7)
    codes = codes.to(torch.int32).view(n, k // 8, 8) & 0xF
    word = torch.zeros((n, k // 8), dtype=torch.int32, device=device)
    for j in range(8):
        word |= codes[..., j] << (4 * j)
    scale = (torch.rand((n,), device=device, generator=gen) * 0.2 + 0.9) * 0.01
    return torch.cat([word, scale.view(torch.int32)[:, None]], dim=1)


class PrefixLM(nn.Module):
    """Gemma decoder stack over prefix embeddings: normalizer, N layers, final RMSNorm."""

    def __init__(self, config, layers: nn.ModuleList, norm: nn.Module, rotary: nn.Module):
        super().__init__()
        self.config = config
        self.layers = layers
        self.norm = norm
        self.rotary_emb = rotary
        self._pos_cache: dict = {}

    def _positions(self, hidden: torch.Tensor, b: int, s: int):
        """Position ids 0..s-1 and their rotary (cos, sin), which depend only on (b, s, dtype):
        computed once per shape instead of every forward (six small kernels)."""
        key = (b, s, hidden.dtype, hidden.device)
        hit = self._pos_cache.get(key)
        if hit is None:
            position_ids = torch.arange(s, device=hidden.device)[None].expand(b, s)
            hit = (position_ids, self.rotary_emb(hidden, position_ids))
            self._pos_cache[key] = hit
        return hit

    def forward(self, inputs_embeds: torch.Tensor, attention_mask: torch.Tensor | None = None) -> torch.Tensor:
        b, s, _ = inputs_embeds.shape
        hidden = inputs_embeds * torch.tensor(self.config.hidden_size**0.5, dtype=inputs_embeds.dtype)
        position_ids, pos = self._positions(hidden, b, s)
        for layer in self.layers:
            hidden = layer(hidden, attention_mask=attention_mask, position_ids=position_ids,
                           position_embeddings=pos)
        return self.norm(hidden)


def build_prefix_lm(
    device: torch.device | str = "cuda",
    num_layers: int = 18,
    seed: int = 20260923,
    packed: dict[str, torch.Tensor] | None = None,
    fuse: bool = True,
) -> tuple[PrefixLM, dict[str, torch.Tensor]]:
    """Build the W4A4 prefix LM.  Returns (model, packed row-major weights by module name).

    ``packed`` maps "layers.{i}.{self_attn|mlp}.{proj}" to int32 [N, K/8+1]; missing
    entries are synthesised on the device with ``synthetic_packed_weight``.
    """
    from transformers.models.gemma.modeling_gemma import (
        GemmaDecoderLayer,
        GemmaRMSNorm,
        GemmaRotaryEmbedding,
    )

    device = torch.device(device)
    cfg = gemma_config(num_layers)
    gen = torch.Generator(device=device).manual_seed(seed)
    cpu_gen = torch.Generator().manual_seed(seed)
    with torch.device("meta"):
        layers = nn.ModuleList([GemmaDecoderLayer(cfg, i) for i in range(num_layers)])
    weights: dict[str, torch.Tensor] = dict(packed or {})
    for i, layer in enumerate(layers):
        for parent_name in ("self_attn", "mlp"):
            parent = getattr(layer, parent_name)
            for proj in PROJECTIONS:
                lin = getattr(parent, proj, None)
                if lin is None:
                    continue
                name = f"layers.{i}.{parent_name}.{proj}"
                w = weights.get(name)
                if w is None:
                    w = synthetic_packed_weight(lin.out_features, lin.in_features, device, gen)
                    weights[name] = w
                w_rt, pre = load_time_weight(w, name, lin.in_features, lin.out_features, device)
                setattr(parent, proj, W4A4Linear(w_rt, in_features=lin.in_features, preshuffled=pre))
        for norm_name in ("input_layernorm", "post_attention_layernorm"):
            norm = getattr(layer, norm_name).to_empty(device=device)
            with torch.no_grad():
                norm.weight.copy_(torch.randn(norm.weight.shape, generator=cpu_gen) * 0.05)
    layers = layers.to(device=device, dtype=torch.float16)
    norm = GemmaRMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps).to(device=device, dtype=torch.float16)
    rotary = GemmaRotaryEmbedding(cfg).to(device)
    model = PrefixLM(cfg, layers, norm, rotary).eval()
    if fuse:
        fuse_shared_activation_quant(model)
        fuse_rmsnorm(model)
        fuse_decoder_layers(model)
    return model, weights


def prefix_inputs(batch: int, tokens: int, device, seed: int = 20260923) -> torch.Tensor:
    """Synthetic prefix embeddings fp16 [B, S, 2048] ~ N(0, 1/sqrt(2048)) (embedding scale)."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, tokens, PALIGEMMA_2B_LM["hidden_size"], generator=gen) / math.sqrt(
        PALIGEMMA_2B_LM["hidden_size"]
    )
    return x.to(device=device, dtype=torch.float16)


def prefix_ops(tokens: int, batch: int = 1, num_layers: int = 18) -> dict[str, float]:
    """Algorithmic int ops (2*M*N*K) per forward of each W4A4 GEMM class."""
    m = tokens * batch
    h, inter = PALIGEMMA_2B_LM["hidden_size"], PALIGEMMA_2B_LM["intermediate_size"]
    per = {
        "qkv": 2.0 * m * (2048 + 256 + 256) * h,
        "o": 2.0 * m * h * 2048,
        "gate_up": 2.0 * m * 2 * inter * h,
        "down": 2.0 * m * h * inter,
    }
    return {k: v * num_layers for k, v in per.items()}
