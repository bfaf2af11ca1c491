"""PyTorch-CPU restatement of the reference's W4A4 semantics -- TEST INFRASTRUCTURE ONLY.

The CPU baseline that ``bench.py`` reports next to the GPU figures: the reference's CPU
path ``int4_gemm_ref`` (``pi05_fast/w4a4/pack.py:134-145``) -- fp32 Sylvester FWHT, per-token
INT4 quant (``quant_activation_cpu``, pack.py:113-131), unpack of the packed weights
(pack.py:71-76, 104-110), exact integer matmul, ``(acc * s_a) * s_w`` to fp16 -- written with
torch CPU ops so that it runs at BLAS speed on the host cores.  The integer matmul has two
forms, both exact (|acc| <= 56 K < 2^24): the reference's fp32 ``a @ b.T`` (pack.py:143) and
``torch._int_mm`` on int8 codes.  Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg use
this module; ``tests/test_oracle.py`` pins it bit for bit against the numpy oracle
(``w4a4_oracle``), which is itself pinned to the reference's golden vectors.
"""

from __future__ import annotations

import math

import torch

ROTATE_K = frozenset({1024, 2048, 16384})  # pi05_fast/w4a4/pack.py:14


def fwht_unnormalized(x: torch.Tensor) -> torch.Tensor:
    """Unnormalised Sylvester FWHT along the last dim in fp32, stages h = 1, 2, 4, ...
    writing (a + b, a - b) (pack.py:18-31)."""
    x = x.float().contiguous()
    n = x.shape[-1]
    if n <= 0 or n & (n - 1):
        raise ValueError(f"FWHT length must be a power of 2, got {n}")
    lead = x.shape[:-1]
    h = 1
    while h < n:
        v = x.view(*lead, n // (2 * h), 2, h)
        a, b = v[..., 0, :], v[..., 1, :]
        x = torch.stack((a + b, a - b), dim=-2).reshape(*lead, n)
        h *= 2
    return x


def quant_activation(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x fp16 [M, K] -> (codes int8 [M, K], scale fp32 [M]) (pack.py:113-131): sdiv =
    amax/7 + 1e-12, codes = clamp(round_half_even(x'/sdiv), -7, 7), scale = sdiv * fp32(1/sqrt(K))
    when K is rotated."""
    k = x.shape[-1]
    xf = x.float()
    rot = k in ROTATE_K
    if rot:
        xf = fwht_unnormalized(xf)
    sdiv = xf.abs().amax(dim=-1) / 7.0 + 1e-12
    scale = sdiv * torch.tensor(1.0 / math.sqrt(k), dtype=torch.float32) if rot else sdiv
    q = torch.round(xf / sdiv.unsqueeze(-1)).clamp_(-7, 7).to(torch.int8)
    return q, scale


def unpack_weight(packed: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int32 [N, K/8+1] -> (codes int8 [N, K], scale fp32 [N]) (pack.py:71-76, 104-110):
    element 8p+j is nibble j of word p, nibbles >= 8 mean value - 16."""
    n, row = packed.shape
    k = (row - 1) * 8
    w = packed[:, :-1].contiguous()
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    nib = (w.unsqueeze(-1) >> shifts) & 0xF
    q = torch.where(nib >= 8, nib - 16, nib).reshape(n, k).to(torch.int8)
    scale = packed[:, -1].contiguous().view(torch.float32)
    return q, scale


def gemm_acc(q_a: torch.Tensor, q_w: torch.Tensor, method: str) -> torch.Tensor:
    """acc[m, n] = sum_k q_a[m, k] q_w[n, k] as int32, by the reference's fp32 product
    (``"fp32"``, pack.py:143) or ``torch._int_mm`` on int8 (``"int_mm"``); both exact."""
    if method == "fp32":
        return (q_a.float() @ q_w.float().T).to(torch.int32)
    if method == "int_mm":
        return torch._int_mm(q_a, q_w.T)
    raise ValueError(f"unknown matmul method {method!r}")


def int4_gemm_ref(x: torch.Tensor, packed_ws: list[torch.Tensor], method: str = "fp32") -> list[torch.Tensor]:
    """The reference's int4_gemm / int4_gemm2 / int4_gemm3 on the CPU: one activation quant
    shared by every weight (int4_gemm.cu:626-642 semantics), then per weight the exact
    integer matmul and fp16((acc * s_a) * s_w).  x fp16 [M, K]."""
    q_a, s_a = quant_activation(x)
    outs = []
    for packed in packed_ws:
        q_w, s_w = unpack_weight(packed)
        acc = gemm_acc(q_a, q_w, method)
        outs.append(((acc.float() * s_a.unsqueeze(-1)) * s_w.unsqueeze(0)).to(torch.float16))
    return outs
