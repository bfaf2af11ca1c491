"""Prefix attention on the GPU (through the C ABI): RoPE + attention between int4_gemm3 and
o_proj of the fused attention forward (apply.py:167-188).

- Key states with RoPE must equal transformers' ``apply_rotary_pos_emb`` on the same fp16
  tensors bit for bit, and the MFMA-fragment-major K / V^T copies must hold exactly those
  keys and V (zero key padding) at the positions the C ABI header states.
- The attention output is floating point: it is checked against a float32 torch
  reference of the same op (RoPE'd q/k from torch, fp32 scores + mask, fp32 softmax, fp32
  PV) with rel-L2 <= 2e-3, next to transformers' eager fp16 path, whose own error
  against that reference is of the same size (fp16 scores, fp16 probabilities).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

D = 256
REL_L2 = 2e-3


@pytest.fixture(scope="module")
def ext(cuda):
    from pi05_fast.w4a4 import extension

    extension.preload()
    return extension


def _rotary(b: int, s: int, device, offset: int = 0):
    from pi05_fast.w4a4.prefix_lm import gemma_config
    from transformers.models.gemma.modeling_gemma import GemmaRotaryEmbedding

    cfg = gemma_config(1)
    rot = GemmaRotaryEmbedding(cfg).to(device)
    x = torch.zeros(1, dtype=torch.float16, device=device)
    pos = (torch.arange(s, device=device) + offset)[None].expand(b, s)
    return rot(x, pos)


def _inputs(b, s, h, kvh, device, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, s, h * D, generator=gen).to(torch.float16).to(device)
    k = torch.randn(b, s, kvh * D, generator=gen).to(torch.float16).to(device)
    v = torch.randn(b, s, kvh * D, generator=gen).to(torch.float16).to(device)
    cos, sin = _rotary(b, s, device, offset=seed % 7)
    return q, k, v, cos, sin


def _padding_causal_mask(b, s, lengths, device, broadcast=False):
    """Additive fp16 mask: query i sees keys j <= i that are inside the sequence's length."""
    neg = torch.finfo(torch.float16).min
    i = torch.arange(s)[:, None]
    j = torch.arange(s)[None, :]
    m = torch.zeros(1 if broadcast else b, 1, s, s)
    for bi in range(m.size(0)):
        m[bi, 0] = torch.where((j <= i) & (j < lengths[bi]), 0.0, neg)
    return m.to(torch.float16).to(device)


def _torch_rope(q, k, cos, sin, h, kvh):
    from transformers.models.gemma.modeling_gemma import apply_rotary_pos_emb

    b, s, _ = q.shape
    qs = q.view(b, s, h, D).transpose(1, 2)
    ks = k.view(b, s, kvh, D).transpose(1, 2)
    return apply_rotary_pos_emb(qs, ks, cos, sin)


def _reference(q, k, v, cos, sin, mask, scaling, h, kvh):
    """float32 attention on the torch-RoPE'd fp16 q/k, output [B, S, H*D] float32."""
    b, s, _ = q.shape
    qr, kr = _torch_rope(q, k, cos, sin, h, kvh)
    rep = h // kvh
    kf = kr.float().repeat_interleave(rep, dim=1)
    vf = v.view(b, s, kvh, D).transpose(1, 2).float().repeat_interleave(rep, dim=1)
    scores = torch.matmul(qr.float(), kf.transpose(2, 3).contiguous()) * scaling
    if mask is not None:
        scores = scores + mask[:, :, :, :s].float()
    p = torch.softmax(scores, dim=-1)
    o = torch.matmul(p, vf.contiguous())
    return o.transpose(1, 2).reshape(b, s, h * D)


def _eager(q, k, v, cos, sin, mask, scaling, h, kvh):
    from pi05_fast.w4a4.prefix_lm import _eager_attention

    b, s, _ = q.shape
    qr, kr = _torch_rope(q, k, cos, sin, h, kvh)
    vs = v.view(b, s, kvh, D).transpose(1, 2)
    out, _ = _eager_attention(None, qr, kr, vs, mask, scaling)
    return out.reshape(b, s, h * D)


def _rel_l2(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm())


def _fragments_k(kp: torch.Tensor) -> torch.Tensor:
    """[s_pad, 256] keys -> K fragments [s_pad/16, 8, 64, 8]: fragment (j, t), lane
    L = 16*(L/16) + L%16 holds K[16j + L%16][32t + 8(L/16) + 0..7]."""
    nj = kp.size(0) // 16
    return kp.view(nj, 16, 8, 4, 8).permute(0, 2, 3, 1, 4).reshape(nj, 8, 64, 8)


def _fragments_vt(vp: torch.Tensor) -> torch.Tensor:
    """[s_pad, 256] values -> V^T fragments [16, s_pad/32, 64, 8]: fragment (db, t), lane L
    holds V[32t + 8(L/16) + 0..7][16db + L%16]."""
    nst = vp.size(0) // 32
    return vp.view(nst, 4, 8, 16, 16).permute(3, 0, 1, 4, 2).reshape(16, nst, 64, 8)


@pytest.mark.parametrize("b,s,kvh", [(1, 776, 1), (2, 100, 1), (1, 1, 1), (1, 1024, 1), (1, 64, 2), (8, 776, 1)])
def test_key_rope_and_mfma_layouts(ext, cuda, b, s, kvh):
    h = 8
    q, k, v, cos, sin = _inputs(b, s, h, kvh, cuda, seed=s + b)
    lib = ext.load_int4_gemm()
    s_pad = (s + 63) // 64 * 64
    k_rope = torch.empty(b, kvh, s, D, dtype=torch.float16, device=cuda)
    kvm = torch.full((b, kvh, 2, s_pad * D), 7.0, dtype=torch.float16, device=cuda)
    assert lib.pi05w4a4_attn_kv_mfma_elems(b, s, kvh, D) == kvm.numel()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.pi05w4a4_attn_kv_prep(
        ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()), kvh * D,
        ctypes.c_void_p(cos.contiguous().data_ptr()), ctypes.c_void_p(sin.contiguous().data_ptr()),
        b, s, kvh, D, ctypes.c_void_p(k_rope.data_ptr()), ctypes.c_void_p(kvm.data_ptr()), stream)
    assert rc == 0, lib.pi05w4a4_last_error()
    torch.cuda.synchronize()
    _, k_want = _torch_rope(q, k, cos, sin, h, kvh)
    assert torch.equal(k_rope, k_want.contiguous())
    vs = v.view(b, s, kvh, D)
    for bi in range(b):
        for g in range(kvh):
            kp = torch.zeros(s_pad, D, dtype=torch.float16, device=cuda)
            kp[:s] = k_want[bi, g]
            vp = torch.zeros(s_pad, D, dtype=torch.float16, device=cuda)
            vp[:s] = vs[bi, :, g]
            assert torch.equal(kvm[bi, g, 0].view(s_pad // 16, 8, 64, 8), _fragments_k(kp))
            assert torch.equal(kvm[bi, g, 1].view(16, s_pad // 32, 64, 8), _fragments_vt(vp))


CASES = [
    # b, s, h, kvh, mask kind
    (1, 776, 8, 1, None),
    (1, 776, 8, 1, "zeros"),
    (2, 100, 8, 1, "padding"),
    (3, 33, 8, 1, "broadcast"),
    (1, 1, 8, 1, None),
    (1, 1024, 8, 1, "padding"),
    (1, 128, 4, 2, "padding"),
    (2, 77, 8, 1, "padding"),
    (8, 776, 8, 1, "zeros"),    # the batch-8 x 776 forward point
    (8, 776, 8, 1, "padding"),
]


@pytest.mark.parametrize("b,s,h,kvh,kind", CASES)
def test_prefix_attention_matches_fp32_reference(ext, cuda, b, s, h, kvh, kind):
    q, k, v, cos, sin = _inputs(b, s, h, kvh, cuda, seed=1000 + s * 3 + b)
    scaling = D**-0.5
    if kind is None:
        mask = None
    elif kind == "zeros":
        mask = torch.zeros(b, 1, s, s, dtype=torch.float16, device=cuda)
    elif kind == "broadcast":
        mask = _padding_causal_mask(b, s, [s - 5], cuda, broadcast=True)
    else:
        lengths = [max(1, s - 17 * i) for i in range(b)]
        mask = _padding_causal_mask(b, s, lengths, cuda)
    with torch.no_grad():
        got, k_rope = ext.prefix_attention(q, k, v, cos, sin, mask, scaling, h, kvh)
        want = _reference(q, k, v, cos, sin, mask, scaling, h, kvh)
        eager = _eager(q, k, v, cos, sin, mask, scaling, h, kvh)
    torch.cuda.synchronize()
    assert got.shape == (b, s, h * D) and k_rope.shape == (b, kvh, s, D)
    assert torch.isfinite(got).all()
    err, err_eager = _rel_l2(got, want), _rel_l2(eager, want)
    assert err <= REL_L2, f"rel-L2 {err:.2e} vs fp32 (eager fp16: {err_eager:.2e})"
    assert _rel_l2(got, eager) <= REL_L2


def test_prefix_attention_unaligned_mask_is_padded(ext, cuda):
    """A mask whose rows are not a multiple of 4 keys is copied into the kernel's form."""
    b, s, h, kvh = 1, 75, 8, 1
    q, k, v, cos, sin = _inputs(b, s, h, kvh, cuda, seed=5)
    mask = _padding_causal_mask(b, s, [70], cuda)
    assert mask.stride(2) % 4 != 0
    with torch.no_grad():
        got, _ = ext.prefix_attention(q, k, v, cos, sin, mask, D**-0.5, h, kvh)
        want = _reference(q, k, v, cos, sin, mask, D**-0.5, h, kvh)
    assert _rel_l2(got, want) <= REL_L2


def test_prefix_attention_op_errors(ext, cuda):
    q, k, v, cos, sin = _inputs(1, 8, 8, 1, cuda, seed=3)
    with pytest.raises(RuntimeError, match="float16"):
        ext.prefix_attention(q.float(), k, v, cos, sin, None, 0.0625, 8, 1)
    with pytest.raises(RuntimeError, match="do not match"):
        ext.prefix_attention(q, k, v, cos, sin, None, 0.0625, 4, 1)
    big = torch.zeros(1, 1025, 8 * D, dtype=torch.float16, device=cuda)
    kb = torch.zeros(1, 1025, D, dtype=torch.float16, device=cuda)
    cb = torch.zeros(1, 1025, D, dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="sequence length"):
        ext.prefix_attention(big, kb, kb, cb, cb, None, 0.0625, 8, 1)


def _attention_layer(cuda, fuse_attn: bool, monkeypatch):
    from pi05_fast.w4a4.prefix_lm import build_prefix_lm

    monkeypatch.setenv("PI05_W4A4_FUSE_ATTN", "1" if fuse_attn else "0")
    model, _ = build_prefix_lm(cuda, num_layers=1)
    return model


def test_decoder_attention_uses_kernel_and_fills_cache(ext, cuda, monkeypatch):
    """The fused attention forward routes through prefix_attention, stores the same key and
    value states in a KV cache as transformers' path, and gives an attention output close
    to it (the INT4 o_proj amplifies fp16-level differences, so the comparison is made on
    o_proj's input)."""
    from transformers.cache_utils import DynamicCache

    from pi05_fast.w4a4 import extension, linear
    from pi05_fast.w4a4.prefix_lm import prefix_inputs

    model = _attention_layer(cuda, True, monkeypatch)
    attn = model.layers[0].self_attn
    s = 776
    x = prefix_inputs(1, s, cuda)
    mask = torch.zeros(1, 1, s, s, dtype=torch.float16, device=cuda)
    pos = torch.arange(s, device=cuda)[None]
    emb = model.rotary_emb(x, pos)

    seen = {}
    real_attn, real_gemm = extension.prefix_attention, linear.int4_gemm

    def spy_attn(*a, **kw):
        seen["calls"] = seen.get("calls", 0) + 1
        return real_attn(*a, **kw)

    def spy_gemm(xin, w):
        seen.setdefault("o_in", []).append(xin.detach().clone())
        return real_gemm(xin, w)

    monkeypatch.setattr(extension, "prefix_attention", spy_attn)
    monkeypatch.setattr(linear, "int4_gemm", spy_gemm)
    with torch.no_grad():
        cache_f = DynamicCache()
        attn(x, position_embeddings=emb, attention_mask=mask, past_key_values=cache_f)
        monkeypatch.setenv("PI05_W4A4_FUSE_ATTN", "0")
        cache_e = DynamicCache()
        attn(x, position_embeddings=emb, attention_mask=mask, past_key_values=cache_e)
    torch.cuda.synchronize()
    assert seen["calls"] == 1
    kf, vf = cache_f.layers[0].keys, cache_f.layers[0].values
    ke, ve = cache_e.layers[0].keys, cache_e.layers[0].values
    assert torch.equal(kf, ke) and torch.equal(vf, ve)
    o_fused, o_eager = seen["o_in"][0], seen["o_in"][1]
    assert _rel_l2(o_fused, o_eager) <= REL_L2


@pytest.mark.parametrize("b,s,kind", [(1, 776, "zeros"), (2, 77, "padding"), (1, 5, None), (8, 776, "zeros")])
def test_attention_output_quant_matches_oracle(ext, cuda, b, s, kind):
    """With one KV head and 8 query heads the attention kernel quantizes its own output
    rows for the o projection: codes, scale bits and row corrections equal the oracle's
    K = 2048 activation quant of the fp16 output it also returns."""
    from oracle import w4a4_oracle as orc
    from pi05_fast.w4a4.pack import codes_from_fragment_major, qcorr_from_fragment_major

    h, kvh = 8, 1
    q, k, v, cos, sin = _inputs(b, s, h, kvh, cuda, seed=77 + s)
    mask = None if kind is None else (torch.zeros(b, 1, s, s, dtype=torch.float16, device=cuda) if kind == "zeros"
                                      else _padding_causal_mask(b, s, [max(1, s - 9 * i) for i in range(b)], cuda))
    with torch.no_grad():
        out, _, codes, scales = ext._prefix_attention_impl(q, k, v, cos, sin, mask, D**-0.5, h, kvh,
                                                           quantize_out=True)
    torch.cuda.synchronize()
    m = b * s
    q_ref, s_ref = orc.quant_activation(out.reshape(m, 2048).cpu().numpy())
    got = orc.unpack_nibbles(codes_from_fragment_major(codes.cpu(), m, 2048).numpy(), 2048)
    assert int(np.count_nonzero(got != q_ref)) == 0
    assert np.array_equal(scales.cpu().numpy().view(np.int32), s_ref.view(np.int32))
    qc = qcorr_from_fragment_major(codes.cpu(), m, 2048).numpy()
    assert np.array_equal(qc, -128 * q_ref[:, 1::2].astype(np.int64).sum(axis=1))


@pytest.mark.parametrize("b,s,h,kvh", [(1, 776, 8, 1), (2, 100, 8, 1), (2, 61, 8, 1), (1, 64, 4, 2), (8, 776, 8, 1)])
def test_prefix_attention_o_proj_matches_oracle(ext, cuda, b, s, h, kvh):
    """residual + o_proj(attention): the fp16 result equals the oracle's W4A4 o projection of
    the returned attention output plus the residual, bit for bit, through the fused quant
    (one KV head, 8 heads; at S = 61 the last workgroup's 4 tokens run past the sequence)
    and through the separate quantizer (other head counts)."""
    from oracle import w4a4_oracle as orc
    from tests import w4a4_inputs as inp

    q, k, v, cos, sin = _inputs(b, s, h, kvh, cuda, seed=300 + s)
    mask = _padding_causal_mask(b, s, [max(1, s - 13 * i) for i in range(b)], cuda)
    gen = inp.generator(h * D + s)
    w_o = inp.packed_weight(gen, 2048, h * D)
    res = (torch.randn(b, s, 2048, generator=gen) * 2.0).half().to(cuda)
    w_mfma = ext.repack_weight(w_o.to(cuda), k=h * D)
    with torch.no_grad():
        x2, key_states, out = ext.prefix_attention_o_proj(q, k, v, cos, sin, mask, D**-0.5, h, kvh, w_mfma, res)
        want_attn = _reference(q, k, v, cos, sin, mask, D**-0.5, h, kvh)
    torch.cuda.synchronize()
    assert _rel_l2(out, want_attn) <= REL_L2
    _, k_want = _torch_rope(q, k, cos, sin, h, kvh)
    assert torch.equal(key_states, k_want.contiguous())
    ref = orc.int4_gemm_ref(out.reshape(b * s, h * D).cpu().numpy(), w_o.numpy())
    want = (ref.astype(np.float32) + res.reshape(b * s, 2048).cpu().numpy().astype(np.float32)).astype(np.float16)
    got = x2.reshape(b * s, 2048).cpu().numpy()
    nbad = int(np.count_nonzero(got.view(np.int16) != want.view(np.int16)))
    assert nbad == 0, f"{nbad}/{got.size} outputs differ"


@pytest.mark.parametrize("b,s,h,kvh", [(1, 776, 8, 1), (2, 100, 8, 1), (8, 776, 8, 1)])
def test_prefix_attention_cache_warm_changes_nothing(ext, cuda, b, s, h, kvh):
    """The cache-warming variant (idle workgroups of the attention launch read further
    buffers: here the weights of an MLP, 48 MB) returns the same bits as the plain call,
    and leaves the buffers it read unchanged; at batch 8 the attention fills every CU and
    no workgroup warms."""
    from tests import w4a4_inputs as inp

    q, k, v, cos, sin = _inputs(b, s, h, kvh, cuda, seed=900 + s + b)
    mask = _padding_causal_mask(b, s, [max(1, s - 7 * i) for i in range(b)], cuda)
    gen = inp.generator(77 + s)
    w_o = ext.repack_weight(inp.packed_weight(gen, 2048, h * D).to(cuda), k=h * D)
    res = (torch.randn(b, s, 2048, generator=gen) * 2.0).half().to(cuda)
    big = [torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device=cuda) for n in (4 << 20, 4 << 20, 4 << 20)]
    keep = [t.clone() for t in big]
    with torch.no_grad():
        plain = ext.prefix_attention_o_proj(q, k, v, cos, sin, mask, D**-0.5, h, kvh, w_o, res)
        warm = ext.prefix_attention_o_proj(q, k, v, cos, sin, mask, D**-0.5, h, kvh, w_o, res, warm=big)
    torch.cuda.synchronize()
    for a, c in zip(plain, warm):
        assert torch.equal(a, c)
    for t, t0 in zip(big, keep):
        assert torch.equal(t, t0)
    # a caller that does not use the attention output: the kernel skips writing it
    with torch.no_grad():
        lean = ext.prefix_attention_o_proj(q, k, v, cos, sin, mask, D**-0.5, h, kvh, w_o, res, warm=big,
                                           return_out=False)
    torch.cuda.synchronize()
    assert torch.equal(lean[0], plain[0]) and torch.equal(lean[1], plain[1])
    assert lean[2].numel() == (0 if kvh == 1 and h == 8 else plain[2].numel())
