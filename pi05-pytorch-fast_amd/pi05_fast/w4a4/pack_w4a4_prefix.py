#!/usr/bin/env python3
"""Pack PaliGemma language-model Linear weights for W4A4 (no full policy load).

Command-line counterpart of the reference's ``scripts/pack_w4a4_prefix.py`` (lines 14-81):
reads ``<model>/model.safetensors`` and writes ``packed.safetensors`` + ``meta.json``
(``"format": "embedl-int4-gemm-v1"``) with int32 ``[N, K/8+1]`` rows per projection.

    python -m pi05_fast.w4a4.pack_w4a4_prefix --model DIR --out DIR
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import torch

LM_PREFIX = "paligemma_with_expert.paligemma.model.language_model.layers."
PROJECTIONS = (".q_proj", ".k_proj", ".v_proj", ".o_proj", ".gate_proj", ".up_proj", ".down_proj")
FORMAT = "embedl-int4-gemm-v1"


def weight_to_module_name(key: str) -> str | None:
    """Checkpoint key -> module name of a packable LM projection, else None."""
    name = key[len("model."):] if key.startswith("model.") else key
    if not name.endswith(".weight"):
        return None
    name = name[: -len(".weight")]
    if name.startswith(LM_PREFIX) and name.endswith(PROJECTIONS):
        return name
    return None


def pack_checkpoint(st_path: Path, out_dir: Path, source: str | None = None) -> dict:
    """Pack every LM projection of one safetensors file; returns the meta dict."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    from pi05_fast.w4a4.pack import pack_linear_weight, should_rotate

    tensors: dict[str, torch.Tensor] = {}
    layers: dict[str, dict] = {}
    with safe_open(str(st_path), framework="pt") as f:
        keys = list(f.keys())
        for key in keys:
            mod = weight_to_module_name(key)
            if mod is None:
                continue
            w = f.get_tensor(key)
            n, k = w.shape
            if k % 64 != 0:
                print(f"skip {mod}: K={k} not multiple of 64")
                continue
            rotate = should_rotate(k)
            tensors[f"{mod}.packed"] = pack_linear_weight(w, rotate=rotate).contiguous()
            bias_key = key[: -len("weight")] + "bias"
            has_bias = bias_key in keys
            if has_bias:
                tensors[f"{mod}.bias"] = f.get_tensor(bias_key).contiguous()
            layers[mod] = {"in_features": k, "out_features": n, "rotate": rotate, "has_bias": has_bias}
            print(f"packed {mod}  [{n}, {k}] rotate={rotate}")
    out_dir.mkdir(parents=True, exist_ok=True)
    save_file(tensors, str(out_dir / "packed.safetensors"))
    meta = {"format": FORMAT, "source": source or str(st_path.parent), "layers": layers}
    (out_dir / "meta.json").write_text(json.dumps(meta, indent=2) + "\n")
    print(f"wrote {len(layers)} layers -> {out_dir}")
    return meta


def main(argv: list[str] | None = None) -> None:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--model", type=Path, default=Path.home() / "model_data" / "pi05_snapflow_1nfe")
    p.add_argument("--out", type=Path, default=Path("models/w4a4_prefix"))
    args = p.parse_args(argv)
    st = args.model.expanduser() / "model.safetensors"
    if not st.is_file():
        sys.exit(f"missing {st}")
    pack_checkpoint(st, args.out, source=str(args.model.expanduser()))


if __name__ == "__main__":
    main()
