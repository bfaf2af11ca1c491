#!/usr/bin/env python3
"""Write the golden fixtures that pin the oracle to the reference's CPU semantics.

Run in the development container only (the reference tree is not present on the GPU
machines):

    python tests/golden/make_golden.py [--ref /root/reference]

It loads the reference's ``pi05_fast/w4a4/pack.py`` by file path (that module imports
only ``torch``, ``math`` and ``typing``), runs its CPU functions on small seeded inputs
and stores inputs + outputs in ``tests/golden/w4a4_golden.npz``.  Nothing of the
reference is copied: the fixture holds arrays only.

Functions covered (reference file:line):
  * ``fwht_unnormalized``      pi05_fast/w4a4/pack.py:18-31
  * ``pack_nibbles``           pi05_fast/w4a4/pack.py:34-42
  * ``preshuffle_wmma_weight`` pi05_fast/w4a4/pack.py:45-68
  * ``unpack_nibbles``         pi05_fast/w4a4/pack.py:71-76
  * ``pack_linear_weight``     pi05_fast/w4a4/pack.py:85-101
  * ``quant_activation_cpu``   pi05_fast/w4a4/pack.py:113-131
  * ``int4_gemm_ref``          pi05_fast/w4a4/pack.py:134-145
"""

from __future__ import annotations

import argparse
import importlib.util
import math
from pathlib import Path

import numpy as np
import torch

SEED = 20260923  # seed used by the reference's GPU tests (tests/test_w4a4.py:52)


def _load_pack(ref_root: Path):
    path = ref_root / "pi05_fast" / "w4a4" / "pack.py"
    spec = importlib.util.spec_from_file_location("_ref_w4a4_pack", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _activations(gen: torch.Generator, m: int, k: int) -> torch.Tensor:
    """fp16 ~N(0,1) with floor(K/100) outlier channels scaled x20 (plus edge rows)."""
    x = torch.randn(m, k, generator=gen, dtype=torch.float32)
    n_out = max(1, k // 100)
    cols = torch.randperm(k, generator=gen)[:n_out]
    x[:, cols] *= 20.0
    x = x.to(torch.float16)
    # edge rows: all-zero row, one-hot row, constant row
    x[0].zero_()
    if m > 1:
        x[1].zero_()
        x[1, k // 3] = 3.0
    if m > 2:
        x[2].fill_(0.5)
    return x


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", type=Path, default=Path("/root/reference"))
    ap.add_argument("--out", type=Path, default=Path(__file__).resolve().parent / "w4a4_golden.npz")
    args = ap.parse_args()
    pack = _load_pack(args.ref)
    gen = torch.Generator().manual_seed(SEED)
    out: dict[str, np.ndarray] = {}

    # FWHT on random fp32 rows (several lengths)
    for n in (8, 64, 2048):
        x = torch.randn(3, n, generator=gen, dtype=torch.float32)
        out[f"fwht_in_{n}"] = x.numpy()
        out[f"fwht_out_{n}"] = pack.fwht_unnormalized(x).numpy()

    # nibble pack / unpack on all 16 codes
    codes = torch.arange(-8, 8, dtype=torch.int32).repeat(4).view(2, 32)
    out["nib_codes"] = codes.numpy()
    out["nib_packed"] = pack.pack_nibbles(codes).numpy()
    words = torch.randint(-(2**31), 2**31 - 1, (3, 5), generator=gen, dtype=torch.int32)
    out["nib_words"] = words.numpy()
    out["nib_unpacked"] = pack.unpack_nibbles(words, 40).numpy()

    # activation quant (rotated K in {1024,2048,16384}; unrotated K in {64,192,512})
    for m, k in ((6, 64), (5, 192), (6, 512), (6, 1024), (8, 2048), (4, 16384)):
        x = _activations(gen, m, k)
        q, s = pack.quant_activation_cpu(x)
        out[f"act_x_{k}"] = x.numpy()
        out[f"act_q_{k}"] = q.to(torch.int8).numpy()
        out[f"act_s_{k}"] = s.numpy()

    # weight pack
    for n, k in ((8, 64), (8, 192), (8, 1024), (16, 2048), (2, 16384)):
        w = torch.randn(n, k, generator=gen, dtype=torch.float32) * 0.02
        if n > 2:
            w[1].zero_()  # all-zero output channel: scale = 1e-12/7
        out[f"w_in_{n}x{k}"] = w.numpy()
        out[f"w_packed_{n}x{k}"] = pack.pack_linear_weight(w).numpy()

    # end-to-end CPU reference GEMM
    for m, n, k in ((6, 8, 64), (8, 16, 2048), (4, 2, 16384), (6, 8, 1024)):
        x = out[f"act_x_{k}"][:m]
        pw = out[f"w_packed_{n}x{k}"]
        y = pack.int4_gemm_ref(torch.from_numpy(x), torch.from_numpy(pw))
        out[f"gemm_y_{m}x{n}x{k}"] = y.numpy()

    # WMMA preshuffle (layout L3) of a random payload, as in the reference's own test
    pw = torch.randint(-(2**31), 2**31 - 1, (7, 64 // 8), generator=gen, dtype=torch.int32)
    sc = torch.rand(7, generator=gen, dtype=torch.float32) * 0.05 + 0.01
    packed = torch.cat((pw, sc.view(torch.int32).unsqueeze(1)), dim=1)
    out["pre_in"] = packed.numpy()
    out["pre_out"] = pack.preshuffle_wmma_weight(packed, 64).numpy()

    # constants
    out["inv_sqrt_k"] = np.array(
        [np.float32(1.0 / math.sqrt(k)) for k in (1024, 2048, 16384)], dtype=np.float32
    )
    out["seed"] = np.array([SEED], dtype=np.int64)
    np.savez_compressed(args.out, **out)
    total = sum(v.nbytes for v in out.values())
    print(f"wrote {args.out} ({len(out)} arrays, {total / 1e6:.2f} MB uncompressed)")


if __name__ == "__main__":
    main()
