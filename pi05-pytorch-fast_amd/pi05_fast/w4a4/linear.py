"""Drop-in ``nn.Linear`` replacement running the W4A4 GEMM (mirror of the reference's
``pi05_fast/w4a4/linear.py:10-65``)."""

from __future__ import annotations

import torch
import torch.nn as nn

from pi05_fast.w4a4.extension import int4_gemm, int4_gemm_tiled
from pi05_fast.w4a4.pack import (
    E3M2_MARKER_WORDS,
    MFMA_MARKER_WORDS,
    WMMA_PRESHUFFLE_PAD_WORDS,
    pack_linear_weight,
    should_rotate,
)


class W4A4Linear(nn.Module):
    """Runtime INT4 activations x packed INT4 weights.

    ``packed`` is int32 ``[N, K/8 + 1]`` (row-major), ``[N, K/8 + P]`` (row-padded),
    ``[N, K/8 + 9]`` with ``preshuffled=True`` (WMMA-tiled) or ``[N, K/8 + 16]`` (gfx950
    MFMA-fragment-major, see ``extension.repack_weight``).
    """

    def __init__(
        self,
        packed: torch.Tensor,
        bias: torch.Tensor | None = None,
        rotate: bool | None = None,
        in_features: int | None = None,
        preshuffled: bool = False,
    ):
        super().__init__()
        if packed.dim() != 2:
            raise ValueError("packed weight must be [N, K/8+1]")
        self.out_features = packed.shape[0]
        self.in_features = in_features or (packed.shape[1] - 1) * 8
        if packed.shape[1] < self.in_features // 8 + 1:
            raise ValueError("packed weight row is too short for in_features")
        self.rotate = should_rotate(self.in_features, rotate)
        self.preshuffled = preshuffled
        if self.preshuffled and packed.shape[1] != self.in_features // 8 + WMMA_PRESHUFFLE_PAD_WORDS:
            raise ValueError("preshuffled weight must use the K/8+9 marker stride")
        self.register_buffer("packed", packed.to(torch.int32), persistent=True)
        # Callers read ``proj.weight.dtype``; keep a dtype marker, not real weights.
        self.register_buffer(
            "weight",
            torch.empty(0, dtype=torch.float16, device=packed.device),
            persistent=False,
        )
        if bias is not None:
            self.bias = nn.Parameter(bias.detach().clone(), requires_grad=False)
        else:
            self.register_parameter("bias", None)

    @property
    def mfma(self) -> bool:
        """True when ``packed`` is in a gfx950 MFMA operand layout: the INT4
        fragment-major layout or the E3M2 column pairs of the FP6-MFMA GEMM."""
        return not self.preshuffled and (
            (self.packed.shape[1] == self.in_features // 8 + MFMA_MARKER_WORDS and self.out_features % 16 == 0)
            or self.e3m2
        )

    @property
    def e3m2(self) -> bool:
        """True when ``packed`` holds the codes as E3M2 column pairs ``[N, 3K/16 + 16]``."""
        return (
            not self.preshuffled
            and self.in_features % 128 == 0
            and self.packed.shape[1] == 3 * self.in_features // 16 + E3M2_MARKER_WORDS
            and self.out_features % 32 == 0
        )

    @classmethod
    def from_linear(cls, linear: nn.Linear, rotate: bool | None = None) -> "W4A4Linear":
        packed = pack_linear_weight(linear.weight, rotate=rotate)
        bias = linear.bias.detach() if linear.bias is not None else None
        return cls(packed, bias=bias, rotate=rotate, in_features=linear.in_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x if x.dtype == torch.float16 else x.to(dtype=torch.float16)
        if not xf.is_contiguous():
            xf = xf.contiguous()
        y = int4_gemm_tiled(xf, self.packed) if self.preshuffled else int4_gemm(xf, self.packed)
        if y.dtype != x.dtype:
            y = y.to(dtype=x.dtype)
        if self.bias is not None:
            y = y + self.bias.to(dtype=y.dtype)
        return y

    def extra_repr(self) -> str:
        layout = "wmma" if self.preshuffled else ("e3m2" if self.e3m2 else ("mfma" if self.mfma else "row"))
        return (
            f"in={self.in_features}, out={self.out_features}, "
            f"rotate={self.rotate}, layout={layout}"
        )
