"""torch.compile over the W4A4 ops on the GPU, as the reference deploys the policy
(rocm_pi05_optim.py:254-262: ``torch.compile(..., mode="max-autotune-no-cudagraphs",
fullgraph=True)`` with the W4A4 custom ops traced through their fake implementations,
extension.py:89-138).  A W4A4Linear, the shared-quant fused MLP (GELU-tanh*up epilogue)
and the fused decoder layer are compiled with fullgraph=True; each compiled module must
give the eager module's output bit for bit.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

MODE = "max-autotune-no-cudagraphs"


@pytest.fixture(scope="module")
def layer_and_inputs(cuda):
    from pi05_fast.w4a4.prefix_lm import build_prefix_lm, prefix_inputs

    model, _ = build_prefix_lm(cuda, num_layers=1)
    s = 776
    x = prefix_inputs(1, s, cuda) * 2048**0.5
    position_ids, pos = model._positions(x, 1, s)
    mask = torch.zeros(1, 1, s, s, dtype=torch.float16, device=cuda)
    return model.layers[0], x.contiguous(), position_ids, pos, mask


def _compiled(mod):
    torch._dynamo.reset()
    return torch.compile(mod, mode=MODE, fullgraph=True)


def test_compiled_w4a4_linear(layer_and_inputs):
    layer, x, *_ = layer_and_inputs
    lin = layer.self_attn.o_proj
    print("compile W4A4Linear", flush=True)
    with torch.no_grad():
        want = lin(x)
        got = _compiled(lin)(x)
        again = _compiled(lin)(x)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(again, want)


def test_compiled_fused_mlp(layer_and_inputs):
    layer, x, *_ = layer_and_inputs
    mlp = layer.mlp
    assert mlp._w4a4_fuse_gelu
    print("compile fused MLP", flush=True)
    with torch.no_grad():
        want = mlp(x)
        got = _compiled(mlp)(x)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_compiled_fused_decoder_layer(layer_and_inputs, monkeypatch):
    from pi05_fast.w4a4 import extension as ext

    layer, x, position_ids, pos, mask = layer_and_inputs
    assert hasattr(layer, "_w4a4_layer_forward"), "the fused decoder layer is installed"
    seen = []
    real = ext.int4_gemm_residual

    def spy(*a, **kw):
        seen.append(1)
        return real(*a, **kw)

    print("compile fused decoder layer", flush=True)
    with torch.no_grad():
        monkeypatch.setattr(ext, "int4_gemm_residual", spy)
        want = layer(x, attention_mask=mask, position_ids=position_ids, position_embeddings=pos)
        assert seen, "the eager call ran the fused layer"
        monkeypatch.setattr(ext, "int4_gemm_residual", real)
        got = _compiled(layer)(x, attention_mask=mask, position_ids=position_ids, position_embeddings=pos)
    torch.cuda.synchronize()
    want = want[0] if isinstance(want, tuple) else want
    got = got[0] if isinstance(got, tuple) else got
    assert torch.equal(got, want)
