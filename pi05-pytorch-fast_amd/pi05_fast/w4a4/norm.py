"""RMSNorm of the decoder around the W4A4 projections, in one HIP kernel.

transformers' GemmaRMSNorm (modeling_gemma.py:64-78), which feeds every QKV and gate/up
activation quant of the prefix LM, runs eagerly as seven elementwise and reduction
kernels with fp32 intermediates in HBM.  ``FusedRMSNorm`` computes the same
``fp16((x * r) * (1 + w))``, r = 1/sqrt(mean(x^2) + eps), in fp32, one wave per row,
through ``pi05w4a4_rmsnorm``.  Only the order of the sum of squares and the rounding of
the reciprocal square root differ from torch's eager ops, so an output can differ from
the eager module's by one fp16 ulp.

The module is installed by structure (every GemmaRMSNorm), whatever the model's dtype at
that moment: the reference applies the W4A4 pack to a bf16 model and casts the prefix LM
to fp16 afterwards (rocm_pi05_optim.py:216-237).  The kernel runs on fp16 CUDA/HIP
inputs with an fp16 weight; any other call computes GemmaRMSNorm's own formula.
"""

from __future__ import annotations

import os

import torch
import torch.nn as nn


class FusedRMSNorm(nn.Module):
    """Drop-in for GemmaRMSNorm (weight offset 1 when ``unit_offset``): the one-kernel
    norm for fp16 CUDA/HIP tensors, GemmaRMSNorm's eager formula for any other dtype or
    device.  ``weight`` is the replaced module's parameter itself, so casts of the model
    apply to it."""

    def __init__(self, weight: torch.Tensor, eps: float, unit_offset: bool = True):
        super().__init__()
        self.weight = weight if isinstance(weight, nn.Parameter) else nn.Parameter(weight.detach(), requires_grad=False)
        self.eps = float(eps)
        self.unit_offset = bool(unit_offset)

    def kernel_fits(self, x: torch.Tensor) -> bool:
        w = self.weight
        return x.dtype == torch.float16 and w.dtype == torch.float16 and x.is_cuda and w.device == x.device

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.kernel_fits(x):
            from pi05_fast.w4a4.extension import rms_norm

            return rms_norm(x, self.weight, self.eps, self.unit_offset)
        # transformers' GemmaRMSNorm.forward (modeling_gemma.py:64-78)
        xf = x.float()
        out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        g = (1.0 + self.weight.float()) if self.unit_offset else self.weight.float()
        return (out * g).type_as(x)

    def extra_repr(self) -> str:
        return f"{tuple(self.weight.shape)}, eps={self.eps}, unit_offset={self.unit_offset}"


def fuse_rmsnorm(model: nn.Module) -> int:
    """Replace every GemmaRMSNorm of ``model`` (1-D weight, width a multiple of 8) by
    ``FusedRMSNorm``.  ``PI05_W4A4_FUSE_NORM=0`` keeps the eager modules.  Returns the
    number replaced."""
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
                and w.numel() % 8 == 0
            ):
                todo.append((mod, child_name, child))
    for parent, child_name, child in todo:
        setattr(parent, child_name, FusedRMSNorm(child.weight, child.eps, unit_offset=True))
    return len(todo)
