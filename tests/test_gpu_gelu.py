"""The gate/up epilogue's GELU-tanh * up over its whole input domain.

The epilogue rounds the dequantized gate to fp16 before the GELU, so every fp16 bit
pattern (finite, inf and NaN) is a possible GELU input: evaluating all 2^16 of them
against torch's eager `gelu(g, approximate="tanh") * u` on the same GPU covers every
case the fused kernel can meet.  The elementwise entry point pi05w4a4_gelu_tanh_mul runs
the same device function as the GEMM epilogue.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext(cuda):
    from pi05_fast.w4a4 import extension

    extension.preload()
    return extension


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return (a.view(torch.int16) == b.view(torch.int16)) | (torch.isnan(a) & torch.isnan(b))


def test_gelu_tanh_mul_every_fp16_gate(ext, cuda):
    g = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(torch.float16).to(cuda)
    gen = torch.Generator().manual_seed(11)
    ups = [torch.ones_like(g), torch.randn(g.shape, generator=gen).half().to(cuda),
           (torch.rand(g.shape, generator=gen) * 60000 - 30000).half().to(cuda)]
    for i, u in enumerate(ups):
        y = ext.gelu_tanh_mul(g, u)
        want = torch.nn.functional.gelu(g, approximate="tanh") * u
        torch.cuda.synchronize()
        bad = ~_same_bits(y, want)
        nbad = int(bad.sum())
        if nbad:
            idx = torch.nonzero(bad).flatten()[:5].tolist()
            detail = [(float(g[j]), float(u[j]), float(y[j]), float(want[j])) for j in idx]
            pytest.fail(f"up set {i}: {nbad} of {g.numel()} outputs differ from eager, e.g. {detail}")


def test_gelu_tanh_mul_shapes_and_errors(ext, cuda):
    gen = torch.Generator().manual_seed(3)
    g = torch.randn(3, 1000, 7, generator=gen).half().to(cuda)
    u = torch.randn(3, 1000, 7, generator=gen).half().to(cuda)
    y = ext.gelu_tanh_mul(g, u)
    assert y.shape == g.shape
    assert bool(_same_bits(y, torch.nn.functional.gelu(g, approximate="tanh") * u).all())
    # strided inputs are made contiguous; empty inputs give empty outputs
    gt, ut = g.transpose(0, 2), u.transpose(0, 2)
    assert bool(_same_bits(ext.gelu_tanh_mul(gt, ut), torch.nn.functional.gelu(gt, approximate="tanh") * ut).all())
    assert ext.gelu_tanh_mul(g[:0], u[:0]).numel() == 0
    with pytest.raises(RuntimeError, match="shapes differ"):
        ext.gelu_tanh_mul(g, u[:1])
    with pytest.raises(RuntimeError, match="float16"):
        ext.gelu_tanh_mul(g.float(), u.float())
