"""Seeded synthetic inputs of the benchmark configurations (shared by tests and bench).

Activations: fp16 ~N(0,1) with floor(K/100) randomly chosen K-channels scaled x20.
Down-projection input: fp16(gelu_tanh(N(0,1)) * N(0,1)).
Weights: N(0, 0.02) packed by the oracle's pack_linear_weight, or random packed words
as in the reference's test fixture (tests/test_w4a4.py:12-21: all 16 nibble values,
including -8, scales U[0.01, 0.06)).
"""

from __future__ import annotations

import numpy as np
import torch

SEED = 20260923


def generator(offset: int = 0) -> torch.Generator:
    return torch.Generator().manual_seed(SEED + offset)


def activations(gen: torch.Generator, m: int, k: int) -> torch.Tensor:
    x = torch.randn(m, k, generator=gen, dtype=torch.float32)
    cols = torch.randperm(k, generator=gen)[: max(1, k // 100)]
    x[:, cols] *= 20.0
    return x.to(torch.float16)


def geglu_activations(gen: torch.Generator, m: int, k: int) -> torch.Tensor:
    g = torch.randn(m, k, generator=gen, dtype=torch.float32)
    u = torch.randn(m, k, generator=gen, dtype=torch.float32)
    return (torch.nn.functional.gelu(g, approximate="tanh") * u).to(torch.float16)


def random_packed(gen: torch.Generator, n: int, k: int) -> torch.Tensor:
    """int32 [N, K/8+1] with uniformly random payload words and scales in [0.01, 0.06)."""
    payload = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), generator=gen, dtype=torch.int32)
    scales = torch.rand(n, generator=gen, dtype=torch.float32) * 0.05 + 0.01
    return torch.cat((payload, scales.view(torch.int32).unsqueeze(1)), dim=1)


def packed_weight(gen: torch.Generator, n: int, k: int) -> torch.Tensor:
    """W ~ N(0, 0.02) packed to int32 [N, K/8+1] with the oracle's packer."""
    from oracle import w4a4_oracle as orc

    w = torch.randn(n, k, generator=gen, dtype=torch.float32) * 0.02
    return torch.from_numpy(orc.pack_linear_weight(w.numpy()))


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()
