#!/usr/bin/env python3
"""Build ``pi05_fast/w4a4/_lib/libpi05_w4a4.so`` with hipcc for gfx950 (in-tree).

    python pi05-pytorch-fast_amd/build_lib.py [--arch gfx950] [--verbose]

hipcc compiles each HIP translation unit under ``csrc/`` to a position-independent
object (in parallel, with per-unit flags) and links them into a shared library exporting
the C ABI of ``include/pi05_w4a4.h``.  The library links only the HIP runtime (no torch
headers or libraries).
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shlex
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
SOURCES = ["quant_rot.hip", "repack.hip", "gemm.hip", "rmsnorm.hip", "attention.hip", "capi.hip"]
OUT = PKG_ROOT / "pi05_fast" / "w4a4" / "_lib" / "libpi05_w4a4.so"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


# Per-unit flags.  quant_rot.hip's row quantizers are latency-bound single waves: the
# machine scheduler's max-ILP strategy interleaves their independent chains better
# (RMSNorm + quant at 776 x 2048: 5.61 -> 5.21 us); it makes the GEMMs slower.
UNIT_FLAGS = {"quant_rot.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]}


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    diag = "\n".join(l for l in (proc.stdout + proc.stderr).splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{diag}")
    if diag.strip() and verbose:
        print(diag, flush=True)


def build(arch: str = "gfx950", verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    common = [
        f"--offload-arch={arch}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Packed-fp32 instructions are kept out of the generated code on purpose.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
    ] + shlex.split(os.environ.get("PI05_W4A4_EXTRA_CFLAGS", ""))
    with tempfile.TemporaryDirectory(prefix="pi05w4a4_build_") as work:
        objs = [str(Path(work) / (Path(src).stem + ".o")) for src in SOURCES]
        # An explicit compilation-unit ID per unit (the default one hashes the command line,
        # which names the temporary object) keeps the library byte-identical between builds.
        cmds = [[hipcc()] + common + UNIT_FLAGS.get(src, [])
                + [f"-cuid=pi05w4a4_{Path(src).stem}", "-c", str(CSRC / src), "-o", obj]
                for src, obj in zip(SOURCES, objs)]
        workers = max(1, min(len(cmds), os.cpu_count() or 1))
        with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
            for fut in [pool.submit(_run, c, verbose) for c in cmds]:
                fut.result()
        _run([hipcc(), f"--offload-arch={arch}", "-shared", "-fPIC", "-o", str(tmp)] + objs, verbose)
    os.replace(tmp, OUT)
    return OUT


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--arch", default=os.environ.get("PYTORCH_ROCM_ARCH", "gfx950"))
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    out = build(args.arch, args.verbose)
    print(f"built {out}")


if __name__ == "__main__":
    sys.exit(main())
