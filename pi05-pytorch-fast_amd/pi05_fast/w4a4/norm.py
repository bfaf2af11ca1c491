"""RMSNorm of the decoder around the W4A4 projections, in one HIP kernel.

transformers' GemmaRMSNorm (modeling_gemma.py:64-78), which feeds every QKV and gate/up
activation quant of the prefix LM, runs eagerly as seven elementwise and reduction
kernels with fp32 intermediates in HBM.  ``FusedRMSNorm`` computes the same
``fp16((x * rsqrt(mean(x^2) + eps)) * (1 + w))`` in fp32, one wave per row, through
``pi05w4a4_rmsnorm``.  Only the order of the sum of squares differs from torch's
reduction, so an output can differ from the eager module's by one fp16 ulp.
"""

from __future__ import annotations

import os

import torch
import torch.nn as nn


class FusedRMSNorm(nn.Module):
    """Drop-in for GemmaRMSNorm on fp16 CUDA/HIP tensors (weight offset 1 when
    ``unit_offset``); raises on anything else rather than falling back."""

    def __init__(self, weight: torch.Tensor, eps: float, unit_offset: bool = True):
        super().__init__()
        self.weight = nn.Parameter(weight.detach().to(torch.float16), requires_grad=False)
        self.eps = float(eps)
        self.unit_offset = bool(unit_offset)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from pi05_fast.w4a4.extension import rms_norm

        return rms_norm(x, self.weight, self.eps, self.unit_offset)

    def extra_repr(self) -> str:
        return f"{tuple(self.weight.shape)}, eps={self.eps}, unit_offset={self.unit_offset}"


def fuse_rmsnorm(model: nn.Module) -> int:
    """Replace every fp16 CUDA/HIP GemmaRMSNorm of ``model`` by ``FusedRMSNorm``.
    ``PI05_W4A4_FUSE_NORM=0`` keeps the eager modules.  Returns the number replaced."""
    if os.environ.get("PI05_W4A4_FUSE_NORM", "1") == "0":
        return 0
    todo = []
    for name, mod in model.named_modules():
        for child_name, child in mod.named_children():
            w = getattr(child, "weight", None)
            if (
                type(child).__name__ == "GemmaRMSNorm"
                and isinstance(w, torch.Tensor)
                and w.dim() == 1
                and w.is_cuda
                and w.dtype == torch.float16
                and w.numel() % 8 == 0
            ):
                todo.append((mod, child_name, child))
    for parent, child_name, child in todo:
        setattr(parent, child_name, FusedRMSNorm(child.weight, child.eps, unit_offset=True))
    return len(todo)
