"""The W4A4 prefix LM on the GPU (through the C ABI): every W4A4 op of a real forward,
checked against the oracle on the very inputs it received.

A whole-model comparison with a CPU forward is not a usable bar for this model: per-token
INT4 activation quantization makes the forward chaotic (a perturbation that flips a few
codes changes a projection's output by a few percent, and the next layers amplify it).
Running the same decoder on the CPU with oracle projections in fp32 and in fp64 already
gives final hidden states 16% apart after two layers, and fp16 vs fp32 33%.  So the
forward is checked operation by operation instead: the GPU forward runs normally (fp16,
shared-quant fused QKV and gate/up forwards, fused GELU*up epilogue), every W4A4 op call
is recorded with its actual input, and each output must equal the oracle's W4A4 semantics
(`int4_gemm_ref`: FWHT + INT4 quant, exact integer matmul, `(acc*s_a)*s_w` to fp16) on
that input bit for bit.  The fused GELU*up output must equal torch's eager
`gelu(g, approximate="tanh") * u` of the oracle's g and u, bit for bit.  With the fused
decoder layers (the default) the recorded ops also carry the input norms (the oracle's
`rms_norm_lanes` of the recorded input is what gets quantized) and the residual adds
(fp16(y + residual)).  RoPE + attention run as ``prefix_attention``, checked against an
fp32 reference in test_gpu_attention.py; no reference test pins the decoder around the
W4A4 ops (parity unpinned there).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import w4a4_oracle as orc

pytestmark = pytest.mark.gpu


def _build(cuda, layers: int, fuse_gelu: bool, fuse_layer: bool = True):
    from pi05_fast.w4a4.prefix_lm import build_prefix_lm

    env = {"PI05_W4A4_FUSE_GELU": "1" if fuse_gelu else "0", "PI05_W4A4_FUSE_LAYER": "1" if fuse_layer else "0"}
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return build_prefix_lm(cuda, num_layers=layers)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


class _Recorder:
    """Wraps the extension ops (and the name linear.py imported) to record every call."""

    NAMES = ("int4_gemm", "int4_gemm_tiled", "int4_gemm2", "int4_gemm2_tiled", "int4_gemm3", "int4_gemm2_gelu",
             "rms_norm_int4_gemm3", "rms_norm_int4_gemm2_gelu", "int4_gemm_residual", "prefix_attention_o_proj",
             "rms_norm_int4_gemm3_rope", "prefix_attention_o_proj_kv", "rms_norm_int4_mlp")

    def __init__(self, monkeypatch):
        from pi05_fast.w4a4 import extension, linear

        self.calls = []
        for name in self.NAMES:
            fn = getattr(extension, name)
            wrapped = self._wrap(name, fn)
            monkeypatch.setattr(extension, name, wrapped)
            if hasattr(linear, name):
                monkeypatch.setattr(linear, name, wrapped)

    def _wrap(self, name, fn):
        def run(*args, **kwargs):
            out = fn(*args, **kwargs)
            outs = out if isinstance(out, tuple) else (out,)
            keep = [a.detach().clone() if isinstance(a, torch.Tensor) else a for a in args]
            self.calls.append((name, keep, dict(kwargs), [o.detach().clone() for o in outs]))
            return out

        return run


def _row_major(w: torch.Tensor, k: int) -> np.ndarray:
    """The L1 row-major [N, K/8+1] form of a weight in any layout the ops take: MFMA
    (K/8+16), E3M2 column pairs (3K/16+16), WMMA-tiled (K/8+9) or row-major / row-padded
    (scale at word K/8)."""
    from pi05_fast.w4a4 import pack

    if k % 128 == 0 and w.shape[1] == 3 * k // 16 + pack.E3M2_MARKER_WORDS:
        codes, scales = pack.codes_from_e3m2_weight(w.cpu(), k)
        return np.concatenate([orc.pack_nibbles(codes.numpy()).astype(np.int32),
                               scales.numpy().view(np.int32)[:, None]], axis=1)
    if w.shape[1] == k // 8 + pack.MFMA_MARKER_WORDS:
        return pack.unpack_mfma_weight(w.cpu(), k).numpy()
    if w.shape[1] == k // 8 + pack.WMMA_PRESHUFFLE_PAD_WORDS:
        return orc.unshuffle_wmma_weight(w.cpu().numpy(), k)
    return np.ascontiguousarray(w.cpu().numpy()[:, : k // 8 + 1])


def _oracle_h(x: np.ndarray, w: torch.Tensor, k: int) -> np.ndarray:
    """The oracle's W4A4 output for fp16 rows x [M, K] and an MFMA-layout weight."""
    return orc.int4_gemm_ref(x, _row_major(w, k))


# GEMM column gc of the RoPE-pair-ordered K weight is key dimension 16 P + 128 h + c
# (gc = 32 P + 16 h + c): extension.rope_pair_weight.
ROPE_PAIR_DIM = np.array([(gc // 32) * 16 + 128 * ((gc // 16) % 2) + gc % 16 for gc in range(256)])


def _check_qkv_rope(cuda, i, args, kwargs, outs) -> None:
    """rms_norm_int4_gemm3_rope: q and v against the oracle; the key states against
    transformers' apply_rotary_pos_emb of the oracle's k; the fragment-major K/V^T against
    the K/V prep kernel run on the oracle's k and v (that kernel's own test pins it)."""
    from transformers.models.gemma.modeling_gemma import apply_rotary_pos_emb

    from pi05_fast.w4a4 import extension as ext

    x, norm_w, eps, w_q, w_k, w_v, cos, sin = args[:8]
    b, s, k = x.shape
    xn = orc.rms_norm_lanes(x.reshape(-1, k).cpu().numpy(), norm_w.cpu().numpy(), eps,
                            unit_offset=kwargs.get("unit_offset", True))
    q_got, kr_got, v_got, kv_got = outs
    for nm, w, o in (("q", w_q, q_got), ("v", w_v, v_got)):
        want = _oracle_h(xn, w, k)
        nbad = int(np.count_nonzero(o.reshape(want.shape).cpu().numpy().view(np.int16) != want.view(np.int16)))
        assert nbad == 0, f"call {i} (rms_norm_int4_gemm3_rope {nm}): {nbad}/{want.size} fp16 outputs differ"
    kp = _oracle_h(xn, w_k, k)
    k_want = np.empty_like(kp)
    k_want[:, ROPE_PAIR_DIM] = kp
    kt = torch.from_numpy(k_want).to(cuda).view(b, s, 1, 256)
    vt = torch.from_numpy(_oracle_h(xn, w_v, k)).to(cuda).view(b, s, 1, 256)
    cs, sn = ext._rope_tables(cos, sin, b, s)
    _, kr_want = apply_rotary_pos_emb(kt.transpose(1, 2), kt.transpose(1, 2), cs, sn)
    assert torch.equal(kr_got, kr_want.contiguous()), f"call {i}: key states differ from apply_rotary_pos_emb"
    lib = ext.load_int4_gemm()
    kr_prep = torch.empty_like(kr_got)
    kv_prep = torch.empty_like(kv_got)
    ktc, vtc = kt.contiguous(), vt.contiguous()
    st = torch.cuda.current_stream().cuda_stream
    assert lib.pi05w4a4_attn_kv_prep(ktc.data_ptr(), vtc.data_ptr(), 256, cs.data_ptr(), sn.data_ptr(), b, s, 1, 256,
                                     kr_prep.data_ptr(), kv_prep.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert torch.equal(kv_got, kv_prep), f"call {i}: fragment-major K/V^T differ from the K/V prep kernel's"


def _check_mlp(cuda, i, args, kwargs, outs) -> None:
    """rms_norm_int4_mlp: h = eager gelu*up of the oracle's gate and up of the oracle's norm
    of x; y = fp16(oracle(h) @ down + residual), the oracle quantizing h itself."""
    x, norm_w, eps, w_gate, w_up, w_down, res = args[:7]
    k = x.shape[-1]
    xn = orc.rms_norm_lanes(x.reshape(-1, k).cpu().numpy(), norm_w.cpu().numpy(), eps,
                            unit_offset=kwargs.get("unit_offset", True))
    g = torch.from_numpy(_oracle_h(xn, w_gate, k)).to(cuda)
    u = torch.from_numpy(_oracle_h(xn, w_up, k)).to(cuda)
    h_want = (torch.nn.functional.gelu(g, approximate="tanh") * u).cpu().numpy()
    y_got, h_got = outs
    h_np = h_got.reshape(h_want.shape).cpu().numpy()
    nbad = int(np.count_nonzero(h_np.view(np.int16) != h_want.view(np.int16)))
    assert nbad == 0, f"call {i} (rms_norm_int4_mlp h): {nbad}/{h_want.size} fp16 outputs differ"
    n = h_want.shape[1]
    y_want = _oracle_h(h_np, w_down, n)
    y_want = (y_want.astype(np.float32) + res.reshape(y_want.shape).cpu().numpy().astype(np.float32)).astype(np.float16)
    got = y_got.reshape(y_want.shape).cpu().numpy()
    nbad = int(np.count_nonzero(got.view(np.int16) != y_want.view(np.int16)))
    assert nbad == 0, f"call {i} (rms_norm_int4_mlp y): {nbad}/{got.size} fp16 outputs differ from the oracle"


def _check_call(cuda, i, call) -> None:
    """One recorded W4A4 op against the oracle, bit for bit."""
    name, args, kwargs, outs = call
    if name == "rms_norm_int4_gemm3_rope":
        _check_qkv_rope(cuda, i, args, kwargs, outs)
        return
    if name == "rms_norm_int4_mlp":
        _check_mlp(cuda, i, args, kwargs, outs)
        return
    if name in ("prefix_attention_o_proj", "prefix_attention_o_proj_kv"):
        # the o projection of the attention output it returned (quantized inside the kernel)
        from pi05_fast.w4a4 import extension as ext

        if name == "prefix_attention_o_proj":
            w_o, res = args[9], args[10]
            x2, out = outs[0], outs[2]
            if out.numel() == 0:  # the fused layer drops the attention output: recompute it
                out = ext.prefix_attention(*args[:9])[0]
        else:
            q, v, kv, cos, sin, mask, scaling, heads, w_o, res = args[:10]
            x2, out = outs
            if out.numel() == 0:
                out = ext._prefix_attention_impl(q, v, v, cos, sin, mask, scaling, heads, 1, kv_mfma=kv)[0]
        k = out.shape[-1]
        want = _oracle_h(out.reshape(-1, k).cpu().numpy(), w_o, k)
        want = (want.astype(np.float32) + res.reshape(want.shape).cpu().numpy().astype(np.float32)).astype(np.float16)
        got = x2.reshape(want.shape).cpu().numpy()
        nbad = int(np.count_nonzero(got.view(np.int16) != want.view(np.int16)))
        assert nbad == 0, f"call {i} ({name}): {nbad}/{got.size} fp16 outputs differ from the oracle"
        return
    x = args[0]
    k = x.shape[-1]
    what = f"call {i} ({name}, K={k})"
    xn = x.reshape(-1, k).cpu().numpy()
    if name.startswith("rms_norm_"):
        norm_w, eps, ws = args[1], args[2], args[3:]
        xn = orc.rms_norm_lanes(xn, norm_w.cpu().numpy(), eps, unit_offset=kwargs.get("unit_offset", True))
    elif name == "int4_gemm_residual":
        ws = args[1:2]
    else:
        ws = args[1:]
    if name.endswith("gelu"):
        g = torch.from_numpy(_oracle_h(xn, ws[0], k)).to(cuda)
        u = torch.from_numpy(_oracle_h(xn, ws[1], k)).to(cuda)
        wants = [(torch.nn.functional.gelu(g, approximate="tanh") * u).cpu().numpy()]
    else:
        wants = [_oracle_h(xn, w, k) for w in ws]
        if name == "int4_gemm_residual":
            res = args[2].reshape(wants[0].shape).cpu().numpy()
            wants = [(wants[0].astype(np.float32) + res.astype(np.float32)).astype(np.float16)]
    for want, o in zip(wants, outs):
        got = o.reshape(want.shape).cpu().numpy()
        nbad = int(np.count_nonzero(got.view(np.int16) != want.view(np.int16)))
        assert nbad == 0, f"{what}: {nbad}/{got.size} fp16 outputs differ from the oracle"


# The benchmark's forward points: the headline forward itself (all 18 layers at 776
# tokens, every one of its 72 W4A4 calls checked; about a minute of oracle work on the
# host, hence its own time limit), 776 tokens over 2 layers in each fusion mode, 640 and
# 768 tokens, and the batch-8 x 776 throughput point (M = 6208: 56 row tiles, a
# 7168-workgroup gate/up grid, attention at batch 8), plus a deep short forward.
FORWARDS = [
    # layers, tokens, batch, fused decoder layer, RoPE + K/V layout in the QKV epilogue
    pytest.param(18, 776, 1, True, True, marks=pytest.mark.timeout(900)),
    (2, 776, 1, True, True), (2, 776, 1, True, False), (2, 776, 1, False, False), (18, 128, 1, True, True),
    (18, 128, 1, False, False), (2, 640, 1, True, True), (2, 768, 1, True, True), (1, 776, 8, True, True),
    (1, 776, 8, True, False), (1, 776, 8, False, False),
]


@pytest.mark.parametrize("layers,tokens,batch,fuse_layer,fuse_kv", FORWARDS)
def test_prefix_lm_forward_ops_match_oracle(cuda, monkeypatch, layers, tokens, batch, fuse_layer, fuse_kv):
    from pi05_fast.w4a4.prefix_lm import prefix_inputs

    print(f"prefix LM forward: {layers} layers x {tokens} tokens x batch {batch}, fused layer {fuse_layer}, "
          f"fused K/V prep {fuse_kv}", flush=True)
    monkeypatch.setenv("PI05_W4A4_FUSE_KV", "1" if fuse_kv else "0")
    model, _ = _build(cuda, layers, fuse_gelu=True, fuse_layer=fuse_layer)
    rec = _Recorder(monkeypatch)
    x = prefix_inputs(batch, tokens, cuda)
    mask = torch.zeros(batch, 1, tokens, tokens, dtype=torch.float16, device=cuda)
    with torch.no_grad():
        y = model(x, mask)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    from pi05_fast.w4a4.norm import FusedRMSNorm

    assert isinstance(model.layers[0].input_layernorm, FusedRMSNorm)
    kinds = [c[0] for c in rec.calls]
    if fuse_layer:
        qkv, attn = ("rms_norm_int4_gemm3_rope", "prefix_attention_o_proj_kv") if fuse_kv else \
            ("rms_norm_int4_gemm3", "prefix_attention_o_proj")
        assert kinds.count(qkv) == layers  # input norm + QKV (+ RoPE and the K/V layout)
        assert kinds.count("rms_norm_int4_gemm2_gelu") == layers  # post norm + gate/up + GELU*up
        assert kinds.count(attn) == layers  # attention, o + residual add
        assert kinds.count("int4_gemm_residual") == layers  # down + residual add
    else:
        assert kinds.count("int4_gemm3") == layers  # QKV
        assert kinds.count("int4_gemm2_gelu") == layers  # gate/up + GELU*up
        assert kinds.count("int4_gemm") == 2 * layers  # o and down
    assert len(kinds) == 4 * layers
    for i, call in enumerate(rec.calls):
        _check_call(cuda, i, call)
        rec.calls[i] = None  # release the recorded tensors as soon as they are checked


@pytest.mark.parametrize("layers,tokens,batch", [(2, 776, 1), (1, 776, 8), (2, 200, 1)])
def test_prefix_lm_fused_down_quant_ops_match_oracle(cuda, monkeypatch, layers, tokens, batch):
    """PI05_W4A4_FUSE_DOWN_QUANT=1: the MLP block runs as rms_norm_int4_mlp (the down
    projection's activation quant in the gate/up launch); every call against the oracle,
    and the forward equals the one without that fusion bit for bit."""
    from pi05_fast.w4a4.prefix_lm import prefix_inputs

    print(f"prefix LM forward, fused down quant: {layers} layers x {tokens} tokens x batch {batch}", flush=True)
    monkeypatch.setenv("PI05_W4A4_FUSE_DOWN_QUANT", "1")
    monkeypatch.setenv("PI05_W4A4_E3M2", "0")  # the down quant rides on the INT4 gate/up launch
    model, _ = _build(cuda, layers, fuse_gelu=True, fuse_layer=True)
    rec = _Recorder(monkeypatch)
    x = prefix_inputs(batch, tokens, cuda)
    mask = torch.zeros(batch, 1, tokens, tokens, dtype=torch.float16, device=cuda)
    with torch.no_grad():
        y = model(x, mask)
    torch.cuda.synchronize()
    kinds = [c[0] for c in rec.calls]
    assert kinds.count("rms_norm_int4_mlp") == layers and len(kinds) == 3 * layers
    for i, call in enumerate(rec.calls):
        _check_call(cuda, i, call)
        rec.calls[i] = None
    monkeypatch.setenv("PI05_W4A4_FUSE_DOWN_QUANT", "0")
    with torch.no_grad():
        y_unfused = model(x, mask)
    torch.cuda.synchronize()
    assert torch.equal(y, y_unfused)


def test_prefix_lm_fused_gelu_is_bit_exact(cuda):
    """The fused gate/up epilogue gives the same forward, bit for bit, as the eager
    act_fn(gate) * up between two fp16 GEMM outputs."""
    from pi05_fast.w4a4.prefix_lm import prefix_inputs

    fused, _ = _build(cuda, 2, fuse_gelu=True, fuse_layer=False)
    eager, _ = _build(cuda, 2, fuse_gelu=False, fuse_layer=False)
    assert fused.layers[0].mlp._w4a4_fuse_gelu and not eager.layers[0].mlp._w4a4_fuse_gelu
    x = prefix_inputs(1, 776, cuda)
    mask = torch.zeros(1, 1, 776, 776, dtype=torch.float16, device=cuda)
    with torch.no_grad():
        y_fused = fused(x, mask)
        y_eager = eager(x, mask)
    torch.cuda.synchronize()
    assert torch.equal(y_fused, y_eager)
