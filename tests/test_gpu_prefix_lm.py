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
`gelu(g, approximate="tanh") * u` of the oracle's g and u, bit for bit.  The decoder's
RMSNorms run as the one-kernel ``pi05_w4a4::rms_norm`` (checked against transformers'
module in test_gpu_parity.py); RoPE and attention are transformers' modules, which no
reference test pins (parity unpinned there).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import w4a4_oracle as orc

pytestmark = pytest.mark.gpu


def _build(cuda, layers: int, fuse_gelu: bool):
    from pi05_fast.w4a4.prefix_lm import build_prefix_lm

    old = os.environ.get("PI05_W4A4_FUSE_GELU")
    os.environ["PI05_W4A4_FUSE_GELU"] = "1" if fuse_gelu else "0"
    try:
        return build_prefix_lm(cuda, num_layers=layers)
    finally:
        if old is None:
            del os.environ["PI05_W4A4_FUSE_GELU"]
        else:
            os.environ["PI05_W4A4_FUSE_GELU"] = old


class _Recorder:
    """Wraps the extension ops (and the name linear.py imported) to record every call."""

    NAMES = ("int4_gemm", "int4_gemm2", "int4_gemm3", "int4_gemm2_gelu")

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
        def run(x, *ws):
            out = fn(x, *ws)
            outs = out if isinstance(out, tuple) else (out,)
            self.calls.append((name, x.detach().clone(), [w for w in ws], [o.detach().clone() for o in outs]))
            return out

        return run


def _row_major(w: torch.Tensor, k: int) -> np.ndarray:
    from pi05_fast.w4a4 import pack

    assert w.shape[1] == k // 8 + pack.MFMA_MARKER_WORDS, "forward weights are MFMA-layout"
    return pack.unpack_mfma_weight(w.cpu(), k).numpy()


def _oracle(x: torch.Tensor, w: torch.Tensor) -> np.ndarray:
    k = x.shape[-1]
    return orc.int4_gemm_ref(x.reshape(-1, k).cpu().numpy(), _row_major(w, k))


@pytest.mark.parametrize("layers,tokens", [(2, 776), (18, 128)])
def test_prefix_lm_forward_ops_match_oracle(cuda, monkeypatch, layers, tokens):
    from pi05_fast.w4a4.prefix_lm import prefix_inputs

    model, _ = _build(cuda, layers, fuse_gelu=True)
    rec = _Recorder(monkeypatch)
    x = prefix_inputs(1, tokens, cuda)
    mask = torch.zeros(1, 1, tokens, tokens, dtype=torch.float16, device=cuda)
    with torch.no_grad():
        y = model(x, mask)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    from pi05_fast.w4a4.norm import FusedRMSNorm

    assert isinstance(model.layers[0].input_layernorm, FusedRMSNorm)
    kinds = [c[0] for c in rec.calls]
    assert kinds.count("int4_gemm3") == layers  # QKV
    assert kinds.count("int4_gemm2_gelu") == layers  # gate/up + GELU*up
    assert kinds.count("int4_gemm") == 2 * layers  # o and down
    for i, (name, xin, ws, outs) in enumerate(rec.calls):
        what = f"call {i} ({name}, K={xin.shape[-1]})"
        if name == "int4_gemm2_gelu":
            g = torch.from_numpy(_oracle(xin, ws[0])).to(cuda)
            u = torch.from_numpy(_oracle(xin, ws[1])).to(cuda)
            want = (torch.nn.functional.gelu(g, approximate="tanh") * u).cpu().numpy()
            got = outs[0].reshape(want.shape).cpu().numpy()
            nbad = int(np.count_nonzero(got.view(np.int16) != want.view(np.int16)))
            assert nbad == 0, f"{what}: {nbad}/{got.size} fused GELU*up outputs differ"
            continue
        for w, o in zip(ws, outs):
            want = _oracle(xin, w)
            got = o.reshape(want.shape).cpu().numpy()
            nbad = int(np.count_nonzero(got.view(np.int16) != want.view(np.int16)))
            assert nbad == 0, f"{what}: {nbad}/{got.size} fp16 outputs differ from the oracle"


def test_prefix_lm_fused_gelu_is_bit_exact(cuda):
    """The fused gate/up epilogue gives the same forward, bit for bit, as the eager
    act_fn(gate) * up between two fp16 GEMM outputs."""
    from pi05_fast.w4a4.prefix_lm import prefix_inputs

    fused, _ = _build(cuda, 2, fuse_gelu=True)
    eager, _ = _build(cuda, 2, fuse_gelu=False)
    assert fused.layers[0].mlp._w4a4_fuse_gelu and not eager.layers[0].mlp._w4a4_fuse_gelu
    x = prefix_inputs(1, 776, cuda)
    mask = torch.zeros(1, 1, 776, 776, dtype=torch.float16, device=cuda)
    with torch.no_grad():
        y_fused = fused(x, mask)
        y_eager = eager(x, mask)
    torch.cuda.synchronize()
    assert torch.equal(y_fused, y_eager)
