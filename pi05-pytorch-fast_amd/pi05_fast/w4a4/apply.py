"""Model integration: load packed weights, replace Linears, fuse shared activation quant.

Mirror of the reference's ``pi05_fast/w4a4/apply.py`` (lines 1-243) with one addition:
at load time every weight is repacked once on the device into the gfx950
MFMA-fragment-major layout (``PI05_W4A4_MFMA=1``, the default), so every projection --
not only gate/up -- runs the fast layout.  With ``PI05_W4A4_MFMA=0`` the reference's own
load-time layouts are kept (row padding ``PI05_W4A4_ROW_PAD_WORDS``, WMMA preshuffle of
gate/up ``PI05_W4A4_GATE_PRESHUFFLE``) and the ops convert them on every call.

``PI05_W4A4_FUSE_GELU`` (default 1) routes gate/up through ``int4_gemm2_gelu`` when the
MLP's activation is torch's GELU-tanh: the GEMM epilogue computes
``gelu(gate, approximate="tanh") * up`` with the same fp16 roundings as the reference's
eager ``act_fn(gate) * up`` (bit-identical outputs), without writing gate and up.
``PI05_W4A4_FUSE_GELU=0`` keeps the eager form.
"""

from __future__ import annotations

import functools
import json
import os
import types
import weakref
from pathlib import Path
from typing import Iterable

import torch
import torch.nn as nn

from pi05_fast.w4a4.extension import register_cache_clearer
from pi05_fast.w4a4.linear import W4A4Linear
from pi05_fast.w4a4.pack import MFMA_MARKER_WORDS, preshuffle_wmma_weight, should_rotate

# Prefix language-model GEMMs only (SigLIP / expert / embeddings stay floating point).
DEFAULT_NAME_PREFIXES = ("paligemma_with_expert.paligemma.model.language_model.layers.",)


def _set_module(root: nn.Module, name: str, new: nn.Module) -> None:
    parent = root
    *parts, leaf = name.split(".")
    for p in parts:
        parent = getattr(parent, p)
    setattr(parent, leaf, new)


def iter_packable_linears(
    model: nn.Module,
    name_prefixes: Iterable[str] = DEFAULT_NAME_PREFIXES,
) -> list[tuple[str, nn.Linear]]:
    """Linears under ``name_prefixes`` with in_features % 64 == 0 (apply.py:29-42)."""
    out = []
    for name, mod in model.named_modules():
        if not isinstance(mod, nn.Linear):
            continue
        if not any(name.startswith(p) for p in name_prefixes):
            continue
        if mod.in_features % 64 != 0:
            continue
        out.append((name, mod))
    return out


def _row_pad_words() -> int:
    pad = max(1, int(os.environ.get("PI05_W4A4_ROW_PAD_WORDS", "8")))
    if pad == MFMA_MARKER_WORDS:
        raise ValueError(
            f"PI05_W4A4_ROW_PAD_WORDS={pad} collides with the MFMA layout marker stride K/8+{pad}"
        )
    return pad


def load_time_weight(
    w: torch.Tensor, name: str, in_features: int, out_features: int, device: torch.device | None
) -> tuple[torch.Tensor, bool]:
    """The packed tensor a W4A4Linear keeps at runtime and whether it is WMMA-preshuffled."""
    use_mfma = os.environ.get("PI05_W4A4_MFMA", "1") != "0"
    on_gpu = device is not None and torch.device(device).type == "cuda"
    if use_mfma and on_gpu and out_features % 16 == 0:
        from pi05_fast.w4a4.extension import repack_weight, repack_weight_e3m2

        w_mfma = repack_weight(w.to(device), k=in_features, tiled=False)
        # The MLP's gate/up weights (K = 2048) take the E3M2 form of the same codes, which
        # the FP6-MFMA GEMM reads (PI05_W4A4_E3M2=0: the INT4 MFMA layout for all); the INT4
        # form stays registered as its twin for calls of few rows, which run faster on it.
        if (os.environ.get("PI05_W4A4_E3M2", "1") != "0" and name.endswith((".mlp.gate_proj", ".mlp.up_proj"))
                and in_features == 2048 and out_features % 32 == 0):
            from pi05_fast.w4a4.extension import register_int4_twin

            w_e3m2 = repack_weight_e3m2(w_mfma, k=in_features, tiled=False)
            register_int4_twin(w_e3m2, w_mfma, in_features)
            return w_e3m2, False
        return w_mfma, False
    gate_preshuffle = os.environ.get("PI05_W4A4_GATE_PRESHUFFLE", "1") != "0"
    row_pad_words = _row_pad_words()
    logical_words = in_features // 8
    preshuffled = (
        gate_preshuffle
        and name.endswith((".mlp.gate_proj", ".mlp.up_proj"))
        and in_features == 2048
        and out_features == 16384
    )
    if preshuffled:
        w = preshuffle_wmma_weight(w, in_features)
    elif row_pad_words > 1 and w.shape[1] == logical_words + 1:
        if in_features % 128 == 0 and row_pad_words == in_features // 16 + 16:
            raise ValueError(f"PI05_W4A4_ROW_PAD_WORDS={row_pad_words} collides with the E3M2 layout marker "
                             f"stride 3K/16+16 at K={in_features}")
        w = torch.nn.functional.pad(w, (0, row_pad_words - 1))
    if device is not None:
        w = w.to(device)
    return w, preshuffled


def replace_linears_from_packed(
    model: nn.Module,
    packed: dict[str, torch.Tensor],
    meta_layers: dict[str, dict],
    device: torch.device | None = None,
) -> int:
    """Swap each packed layer's nn.Linear for a W4A4Linear (apply.py:45-88)."""
    n = 0
    for name, spec in meta_layers.items():
        key = f"{name}.packed"
        if key not in packed:
            continue
        in_features = int(spec["in_features"])
        out_features = int(spec["out_features"])
        w, preshuffled = load_time_weight(packed[key], name, in_features, out_features, device)
        bias = packed.get(f"{name}.bias")
        if bias is not None and device is not None:
            bias = bias.to(device)
        _set_module(
            model,
            name,
            W4A4Linear(
                w,
                bias=bias,
                rotate=spec.get("rotate"),
                in_features=in_features,
                preshuffled=preshuffled,
            ),
        )
        n += 1
    return n


def apply_w4a4_from_dir(model: nn.Module, pack_dir: str | Path) -> int:
    """Load ``packed.safetensors`` + ``meta.json`` and install the W4A4 layers (apply.py:91-118)."""
    pack_dir = Path(pack_dir).expanduser()
    meta_path = pack_dir / "meta.json"
    st_path = pack_dir / "packed.safetensors"
    if not meta_path.is_file() or not st_path.is_file():
        raise FileNotFoundError(f"need {meta_path} and {st_path}")
    meta = json.loads(meta_path.read_text())
    from safetensors.torch import load_file

    packed = load_file(str(st_path))
    device = next(model.parameters()).device
    from pi05_fast.w4a4.extension import preload

    preload()
    n = replace_linears_from_packed(model, packed, meta["layers"], device=device)
    n_fuse = fuse_shared_activation_quant(model)
    from pi05_fast.w4a4.norm import fuse_rmsnorm

    n_norm = fuse_rmsnorm(model)
    n_layer = fuse_decoder_layers(model)
    n_mfma = sum(isinstance(m, W4A4Linear) and m.mfma for m in model.modules())
    n_pre = sum(isinstance(m, W4A4Linear) and m.preshuffled for m in model.modules())
    print(
        f"w4a4: replaced {n} Linear modules from {pack_dir}; "
        f"shared-quant fused {n_fuse} QKV/MLP groups; one-kernel RMSNorm {n_norm}; "
        f"fused decoder layers {n_layer}; "
        f"MFMA-fragment-major {n_mfma}; WMMA-preshuffled gate/up {n_pre}",
        flush=True,
    )
    return n


def _as_fp16_contig(x: torch.Tensor) -> torch.Tensor:
    xf = x if x.dtype == torch.float16 else x.to(dtype=torch.float16)
    return xf if xf.is_contiguous() else xf.contiguous()


def _fused_mlp_forward(self, x: torch.Tensor) -> torch.Tensor:
    """Gate/up with one shared activation quant, then down (apply.py:126-142)."""
    from pi05_fast.w4a4.extension import int4_gemm, int4_gemm2, int4_gemm2_gelu, int4_gemm2_tiled

    xf = _as_fp16_contig(x)
    if getattr(self, "_w4a4_fuse_gelu", False):
        h = int4_gemm2_gelu(xf, self.gate_proj.packed, self.up_proj.packed)
    else:
        if self.gate_proj.preshuffled and self.up_proj.preshuffled:
            gate, up = int4_gemm2_tiled(xf, self.gate_proj.packed, self.up_proj.packed)
        else:
            gate, up = int4_gemm2(xf, self.gate_proj.packed, self.up_proj.packed)
        h = self.act_fn(gate) * up
    if not h.is_contiguous():
        h = h.contiguous()
    y = int4_gemm(h, self.down_proj.packed)
    return y if y.dtype == x.dtype else y.to(dtype=x.dtype)


_EAGER_ATTENTION = ("eager", "w4a4_eager")


def _prefix_attention_fits(self, q: torch.Tensor, k: torch.Tensor, attention_mask, past_key_values) -> bool:
    """Whether RoPE + attention of this call can run as ``extension.prefix_attention``:
    an eager attention implementation (bidirectional unless the additive mask says
    otherwise), head_dim 256, fp16 on the GPU, at most 1024 tokens, no dropout, logit
    softcap or sliding window, an fp16 [B|1, 1, S, >=S] mask or none, and an empty cache
    (a prefix forward).  ``PI05_W4A4_FUSE_ATTN=0`` keeps transformers' path."""
    if q.dim() != 3:
        return False
    return _attention_call_fits(self, q.shape, int(k.size(-1)), q.dtype, q.is_cuda, attention_mask,
                                past_key_values)


def _attention_call_fits(self, q_shape, k_width: int, dtype, is_cuda: bool, attention_mask,
                         past_key_values) -> bool:
    if os.environ.get("PI05_W4A4_FUSE_ATTN", "1") == "0":
        return False
    cfg = self.config
    if getattr(cfg, "_attn_implementation", "eager") not in _EAGER_ATTENTION:
        return False
    if self.training and getattr(self, "attention_dropout", 0.0):
        return False
    if getattr(cfg, "attn_logit_softcapping", None) or getattr(self, "sliding_window", None):
        return False
    if self.head_dim != 256 or dtype != torch.float16 or not is_cuda or len(q_shape) != 3:
        return False
    b, s, q_width = int(q_shape[0]), int(q_shape[1]), int(q_shape[2])
    if s > 1024 or k_width % 256 or q_width % k_width:
        return False
    if attention_mask is not None:
        m = attention_mask
        if m.dtype != torch.float16 or m.dim() != 4 or m.size(1) != 1 or m.size(0) not in (1, b):
            return False
        if m.size(2) != s or m.size(3) < s:
            return False
    if past_key_values is not None and past_key_values.get_seq_length(self.layer_idx) != 0:
        return False
    return True


def _fused_attn_forward(
    self,
    hidden_states: torch.Tensor,
    position_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None,
    attention_mask: torch.Tensor | None = None,
    past_key_values=None,
    **kwargs,
):
    """Gemma attention with QKV from one int4_gemm3 call (apply.py:145-191).  When the call
    fits (``_prefix_attention_fits``), RoPE and the attention run as the two kernels of
    ``extension.prefix_attention``; otherwise transformers' RoPE and attention interface."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from transformers.models.gemma.modeling_gemma import apply_rotary_pos_emb, eager_attention_forward

    from pi05_fast.w4a4.extension import int4_gemm3

    input_shape = hidden_states.shape[:-1]
    hidden_shape = (*input_shape, -1, self.head_dim)
    q, k, v = int4_gemm3(
        _as_fp16_contig(hidden_states),
        self.q_proj.packed,
        self.k_proj.packed,
        self.v_proj.packed,
    )
    cos, sin = position_embeddings
    if (cos.dtype == torch.float16 and sin.dtype == torch.float16
            and _prefix_attention_fits(self, q, k, attention_mask, past_key_values)):
        from pi05_fast.w4a4.extension import prefix_attention

        out, key_states = prefix_attention(
            q, k, v, cos, sin, attention_mask, float(self.scaling),
            q.size(-1) // self.head_dim, k.size(-1) // self.head_dim,
        )
        if past_key_values is not None:
            value_states = v.view(hidden_shape).transpose(1, 2)
            past_key_values.update(key_states, value_states, self.layer_idx)
        return self.o_proj(out.reshape(*input_shape, -1)), None

    query_states = q.view(hidden_shape).transpose(1, 2)
    key_states = k.view(hidden_shape).transpose(1, 2)
    value_states = v.view(hidden_shape).transpose(1, 2)

    query_states, key_states = apply_rotary_pos_emb(query_states, key_states, cos, sin)

    if past_key_values is not None:
        key_states, value_states = past_key_values.update(key_states, value_states, self.layer_idx)

    attention_interface = ALL_ATTENTION_FUNCTIONS.get_interface(
        self.config._attn_implementation, eager_attention_forward
    )
    attn_output, attn_weights = attention_interface(
        self,
        query_states,
        key_states,
        value_states,
        attention_mask,
        dropout=0.0 if not self.training else self.attention_dropout,
        scaling=self.scaling,
        **kwargs,
    )
    attn_output = attn_output.reshape(*input_shape, -1).contiguous()
    attn_output = self.o_proj(attn_output)
    return attn_output, attn_weights


def _norm_parts(norm) -> tuple[torch.Tensor, float, bool] | None:
    """(weight, eps, unit_offset) of a Gemma RMSNorm module (transformers' GemmaRMSNorm
    or norm.FusedRMSNorm) with a 1-D weight, or None.  The weight's dtype and device are
    checked per call (``_norms_fit``)."""
    from pi05_fast.w4a4.norm import FusedRMSNorm

    w = getattr(norm, "weight", None)
    if not isinstance(w, torch.Tensor) or w.dim() != 1:
        return None
    if isinstance(norm, FusedRMSNorm):
        return w, norm.eps, norm.unit_offset
    if type(norm).__name__ == "GemmaRMSNorm":
        return w, float(norm.eps), True
    return None


def _norms_fit(parts, x: torch.Tensor) -> bool:
    """Whether the fused norm + quant kernels can take these norms for input x: fp16
    weights on x's device."""
    return all(p is not None and p[0].dtype == torch.float16 and p[0].device == x.device for p in parts)


def _decoder_layer_fits(layer) -> bool:
    """A Gemma decoder layer whose seven projections are bias-free MFMA-layout W4A4 layers,
    whose MLP uses the fused GELU-tanh*up epilogue and whose norms are Gemma RMSNorms over
    2048 features.  Structure only: dtypes are checked per call, so a model that is cast to
    fp16 after the pack is applied (rocm_pi05_optim.py:231-237) runs the fused layer."""
    attn, mlp = getattr(layer, "self_attn", None), getattr(layer, "mlp", None)
    if attn is None or mlp is None or not getattr(mlp, "_w4a4_fuse_gelu", False):
        return False
    projs = [getattr(attn, n, None) for n in ("q_proj", "k_proj", "v_proj", "o_proj")]
    projs += [getattr(mlp, n, None) for n in ("gate_proj", "up_proj", "down_proj")]
    if not all(isinstance(p, W4A4Linear) and p.mfma and p.bias is None for p in projs):
        return False
    norms = [_norm_parts(getattr(layer, n, None)) for n in ("input_layernorm", "post_attention_layernorm")]
    return all(n is not None and n[0].numel() == 2048 for n in norms) and projs[0].in_features == 2048


def _fused_decoder_layer_forward(
    self,
    hidden_states: torch.Tensor,
    attention_mask: torch.Tensor | None = None,
    position_ids=None,
    past_key_values=None,
    use_cache: bool | None = False,
    position_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None,
    **kwargs,
):
    """GemmaDecoderLayer.forward (modeling_gemma.py) with the edges of the W4A4 ops fused:
    input_layernorm into the QKV activation quant, RoPE + attention + o_proj as
    ``extension.prefix_attention_o_proj`` (the o-proj activation quant inside the attention
    kernel, the attention residual add in the o_proj epilogue),
    post_attention_layernorm into the gate/up activation quant (GELU-tanh*up epilogue) and
    the MLP residual add into the down_proj epilogue.  Calls that do not fit the fused
    attention run the layer's original forward."""
    from pi05_fast.w4a4 import extension as ext

    attn, mlp = self.self_attn, self.mlp
    x = hidden_states
    norms = (_norm_parts(self.input_layernorm), _norm_parts(self.post_attention_layernorm))
    if not (
        x.dtype == torch.float16
        and x.dim() == 3
        and x.is_contiguous()
        and position_embeddings is not None
        and all(t.dtype == torch.float16 for t in position_embeddings)
        and _norms_fit(norms, x)
        and _attention_call_fits(attn, (x.size(0), x.size(1), attn.q_proj.out_features),
                                 attn.k_proj.out_features, x.dtype, x.is_cuda, attention_mask, past_key_values)
    ):
        return self._w4a4_layer_forward(hidden_states, attention_mask=attention_mask, position_ids=position_ids,
                                        past_key_values=past_key_values, use_cache=use_cache,
                                        position_embeddings=position_embeddings, **kwargs)
    (w1, eps1, off1), (w2, eps2, off2) = norms
    cos, sin = position_embeddings
    hd = attn.head_dim
    # Cache warming (PI05_W4A4_CACHE_WARM=0: off): the attention launch's idle CUs read the
    # o-proj, gate and up weights into the Infinity Cache, and the down-proj input quant's
    # idle workgroup slots the down-proj weights.  The next layer's QKV weights were tried
    # as well: no gain, and the longer warming outlasts the attention.
    warming = os.environ.get("PI05_W4A4_CACHE_WARM", "1") != "0"
    # (the tail of the up weight is warmed by the gate/up op's own norm + quant launch)
    warm = None
    if warming:
        # the forms the gate/up GEMM reads for this many rows (INT4 twins at few rows, whose
        # own norm + quant launch warms nothing: the whole up weight then)
        rows = x.numel() // x.size(-1)
        wg, wu = ext.gemm_weights_for_rows([mlp.gate_proj.packed, mlp.up_proj.packed], mlp.gate_proj.in_features,
                                           rows)
        warm = [attn.o_proj.packed, wg, wu if wu is not mlp.up_proj.packed else ext.gate_up_warm_split(wu)[0]]
    wk_rope = _k_rope_weight(attn, x)
    if wk_rope is not None:
        # One KV head: RoPE and the attention's K/V layout in the QKV GEMM epilogue.
        q, key_states, v, kv = ext.rms_norm_int4_gemm3_rope(x, w1, eps1, attn.q_proj.packed, wk_rope,
                                                            attn.v_proj.packed, cos, sin, unit_offset=off1)
        x2, _ = ext.prefix_attention_o_proj_kv(q, v, kv, cos, sin, attention_mask, float(attn.scaling),
                                               q.size(-1) // hd, attn.o_proj.packed, x, warm=warm, return_out=False)
    else:
        q, k, v = ext.rms_norm_int4_gemm3(x, w1, eps1, attn.q_proj.packed, attn.k_proj.packed, attn.v_proj.packed,
                                          unit_offset=off1)
        x2, key_states, _ = ext.prefix_attention_o_proj(q, k, v, cos, sin, attention_mask, float(attn.scaling),
                                                        q.size(-1) // hd, k.size(-1) // hd, attn.o_proj.packed, x,
                                                        warm=warm, return_out=False)
    if past_key_values is not None:
        value_states = v.view(*v.shape[:-1], -1, hd).transpose(1, 2)
        past_key_values.update(key_states, value_states, attn.layer_idx)
    if os.environ.get("PI05_W4A4_FUSE_DOWN_QUANT", "0") == "1" and ext.is_mfma_layout(mlp.gate_proj.packed,
                                                                                   mlp.gate_proj.in_features):
        # The down projection's activation quant in the gate/up launch (one launch fewer).
        y, _ = ext.rms_norm_int4_mlp(x2, w2, eps2, mlp.gate_proj.packed, mlp.up_proj.packed, mlp.down_proj.packed,
                                     x2, warm=[mlp.down_proj.packed] if warming else None, unit_offset=off2)
        return y
    h = ext.rms_norm_int4_gemm2_gelu(x2, w2, eps2, mlp.gate_proj.packed, mlp.up_proj.packed, unit_offset=off2)
    return ext.int4_gemm_residual(h, mlp.down_proj.packed, x2, warm=[mlp.down_proj.packed] if warming else None)


def _k_rope_weight(attn: nn.Module, x: torch.Tensor):
    """The RoPE-pair-ordered copy of the K weight (``extension.rope_pair_weight``) when the
    QKV call can take the attention prep in its epilogue: one KV head of 256, MFMA-layout
    q/k/v weights, a token count that is a multiple of 8; else None.  The copy is kept on
    the module and rebuilt when the K weight tensor is replaced, modified in place through
    itself or given new storage (``.data = ...``), in eager calls; a compiled graph uses the
    copy an eager call built, else the separate prep.  A write through ``.data`` needs
    ``extension.clear_weight_caches()``.  ``PI05_W4A4_FUSE_KV=0`` keeps the separate K/V
    prep launch."""
    if os.environ.get("PI05_W4A4_FUSE_KV", "1") == "0" or int(x.size(1)) % 8:
        return None
    wk = attn.k_proj.packed
    kin = int(x.size(-1))
    if int(wk.size(0)) != 256 or attn.head_dim != 256 or int(attn.v_proj.packed.size(0)) != 256:
        return None
    if not all(w.dim() == 2 and w.size(1) == kin // 8 + MFMA_MARKER_WORDS
               for w in (attn.q_proj.packed, wk, attn.v_proj.packed)):
        return None
    hit = getattr(attn, "_w4a4_k_rope", None)
    if torch.compiler.is_compiling():
        # a traced graph uses the copy an eager call built; it builds none itself
        return hit[2] if hit is not None and hit[0] is wk else None
    if hit is not None and hit[0] is wk and hit[1] == wk._version and hit[3] == wk.data_ptr():
        return hit[2]
    if not wk.is_cuda:
        return None
    from pi05_fast.w4a4.extension import rope_pair_weight

    out = rope_pair_weight(wk)
    attn._w4a4_k_rope = (wk, wk._version, out, wk.data_ptr())
    _K_ROPE_HOLDERS.add(attn)
    return out


# Attention modules holding a RoPE-pair K copy, for extension.clear_weight_caches().
_K_ROPE_HOLDERS: weakref.WeakSet = weakref.WeakSet()


def _clear_k_rope_copies() -> None:
    for attn in list(_K_ROPE_HOLDERS):
        attn.__dict__.pop("_w4a4_k_rope", None)
    _K_ROPE_HOLDERS.clear()


register_cache_clearer(_clear_k_rope_copies)


def fuse_decoder_layers(model: nn.Module) -> int:
    """Install ``_fused_decoder_layer_forward`` on every decoder layer that fits
    (``_decoder_layer_fits``); the original forward stays reachable for calls that do not.
    ``PI05_W4A4_FUSE_LAYER=0`` keeps the per-module forwards.  Returns the layers fused."""
    if os.environ.get("PI05_W4A4_FUSE_LAYER", "1") == "0":
        return 0
    n = 0
    for mod in model.modules():
        if hasattr(mod, "input_layernorm") and hasattr(mod, "self_attn") and _decoder_layer_fits(mod):
            if not hasattr(mod, "_w4a4_layer_forward"):
                mod._w4a4_layer_forward = mod.forward
            mod.forward = types.MethodType(_fused_decoder_layer_forward, mod)
            n += 1
    return n


def _is_torch_gelu_tanh(act) -> bool:
    """True iff ``act`` evaluates ``torch.nn.functional.gelu(x, approximate="tanh")`` (the
    default of transformers' GELUTanh, Gemma's ``gelu_pytorch_tanh``): the function whose
    fp16 results the fused gate/up epilogue reproduces bit for bit."""
    fn = getattr(act, "act", act)
    return (
        isinstance(fn, functools.partial)
        and fn.func is torch.nn.functional.gelu
        and not fn.args
        and fn.keywords == {"approximate": "tanh"}
    )


def fuse_shared_activation_quant(model: nn.Module) -> int:
    """One activation quant for QKV and one for gate/up (apply.py:194-213)."""
    if os.environ.get("PI05_W4A4_FUSE_QUANT", "1") == "0":
        return 0
    fuse_gelu = os.environ.get("PI05_W4A4_FUSE_GELU", "1") == "1"
    n = 0
    for mod in model.modules():
        qkv = (getattr(mod, "q_proj", None), getattr(mod, "k_proj", None), getattr(mod, "v_proj", None))
        if all(isinstance(p, W4A4Linear) for p in qkv):
            mod.forward = types.MethodType(_fused_attn_forward, mod)
            n += 1
            continue
        gate_up = (
            getattr(mod, "gate_proj", None),
            getattr(mod, "up_proj", None),
            getattr(mod, "down_proj", None),
        )
        if all(isinstance(p, W4A4Linear) for p in gate_up) and hasattr(mod, "act_fn"):
            # The fused epilogue reads row-major or MFMA-layout weights; WMMA-preshuffled
            # gate/up weights (PI05_W4A4_MFMA=0 with the reference's gate preshuffle) take the
            # reference's int4_gemm2_tiled + act_fn route instead.
            mod._w4a4_fuse_gelu = (
                fuse_gelu
                and gate_up[0].packed.shape == gate_up[1].packed.shape
                and not (gate_up[0].preshuffled or gate_up[1].preshuffled)
                and _is_torch_gelu_tanh(mod.act_fn)
            )
            mod.forward = types.MethodType(_fused_mlp_forward, mod)
            n += 1
    return n


def maybe_apply_w4a4_from_env(model: nn.Module) -> int:
    """Apply the pack named by ``PI05_W4A4_PACK`` if set (apply.py:216-220)."""
    path = os.environ.get("PI05_W4A4_PACK", "").strip()
    if not path:
        return 0
    return apply_w4a4_from_dir(model, path)


def pack_model_linears(
    model: nn.Module,
    name_prefixes: Iterable[str] = DEFAULT_NAME_PREFIXES,
) -> tuple[dict[str, torch.Tensor], dict[str, dict]]:
    """Pack every eligible Linear to the on-disk format (apply.py:223-243)."""
    from pi05_fast.w4a4.pack import pack_linear_weight

    tensors: dict[str, torch.Tensor] = {}
    layers: dict[str, dict] = {}
    for name, lin in iter_packable_linears(model, name_prefixes):
        rotate = should_rotate(lin.in_features)
        packed = pack_linear_weight(lin.weight, rotate=rotate)
        tensors[f"{name}.packed"] = packed.contiguous()
        if lin.bias is not None:
            tensors[f"{name}.bias"] = lin.bias.detach().cpu().contiguous()
        layers[name] = {
            "in_features": lin.in_features,
            "out_features": lin.out_features,
            "rotate": rotate,
            "has_bias": lin.bias is not None,
        }
    return tensors, layers
