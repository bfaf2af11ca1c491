#!/usr/bin/env python3
"""Build ``pi05_fast/w4a4/_lib/libpi05_w4a4.so`` with hipcc for gfx950 (in-tree).

    python pi05-pytorch-fast_amd/build_lib.py [--arch gfx950] [--verbose] [--out PATH]

hipcc compiles each HIP translation unit under ``csrc/`` to a position-independent
object (in parallel, with per-unit flags) and links them into a shared library exporting
the C ABI of ``include/pi05_w4a4.h``.  The library links only the HIP runtime (no torch
headers or libraries).  ``pi05_fast.w4a4.extension.load_int4_gemm()`` runs the same build
on first use when the library is absent, as the reference's loader JIT-builds its
extension (``pi05_fast/w4a4/extension.py:15-75``).

Knobs (the reference loader's, ``extension.py:37,60-64,73``):
  * target: ``--arch``, else ``PYTORCH_ROCM_ARCH``, else ``GPU_ARCHS``, else gfx950.  A
    list (``;``, ``,`` or blanks) gives one ``--offload-arch`` each.  The kernels use
    gfx950 instructions (CDNA4 int8 MFMA shapes, permlane swaps), so other targets fail to
    compile;
  * ``PI05_W4A4_VERBOSE=1`` (or ``--verbose``): print every hipcc command and its output;
  * ``PI05_W4A4_EXTRA_CFLAGS``: extra hipcc flags (shell-split), appended to every unit.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import re
import shlex
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
SOURCES = ["quant_rot.hip", "repack.hip", "gemm.hip", "rmsnorm.hip", "attention.hip", "capi.hip"]
OUT = PKG_ROOT / "pi05_fast" / "w4a4" / "_lib" / "libpi05_w4a4.so"
DEFAULT_ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def target_archs(arch: str | None = None) -> list[str]:
    """The offload targets: ``arch``, else PYTORCH_ROCM_ARCH, else GPU_ARCHS, else gfx950."""
    spec = arch or os.environ.get("PYTORCH_ROCM_ARCH") or os.environ.get("GPU_ARCHS") or DEFAULT_ARCH
    archs = [a for a in re.split(r"[;,\s]+", spec) if a]
    if not archs:
        raise ValueError(f"no offload target in {spec!r}")
    return archs


def verbose_from_env() -> bool:
    return os.environ.get("PI05_W4A4_VERBOSE", "0") == "1"


# Per-unit flags.  quant_rot.hip's row quantizers are latency-bound single waves: the
# machine scheduler's max-ILP strategy interleaves their independent chains better
# (RMSNorm + quant at 776 x 2048: 5.61 -> 5.21 us); it makes the GEMMs slower.
UNIT_FLAGS = {"quant_rot.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]}


def compile_commands(archs: list[str], work: Path) -> tuple[list[list[str]], list[str]]:
    """hipcc command lines of every unit (objects under ``work``) and the object paths."""
    common = [f"--offload-arch={a}" for a in archs] + [
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Packed-fp32 instructions are kept out of the generated code on purpose.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
    ] + shlex.split(os.environ.get("PI05_W4A4_EXTRA_CFLAGS", ""))
    objs = [str(work / (Path(src).stem + ".o")) for src in SOURCES]
    # An explicit compilation-unit ID per unit (the default one hashes the command line,
    # which names the temporary object) keeps the library byte-identical between builds.
    cmds = [[hipcc()] + common + UNIT_FLAGS.get(src, [])
            + [f"-cuid=pi05w4a4_{Path(src).stem}", "-c", str(CSRC / src), "-o", obj]
            for src, obj in zip(SOURCES, objs)]
    return cmds, objs


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


def build(arch: str | None = None, verbose: bool | None = None, out: Path | str | None = None) -> Path:
    """Compile and link the library to ``out`` (default: the in-tree ``_lib`` path).  The
    result is written under a temporary name and renamed into place, so a concurrent
    loader never maps a half-written file."""
    archs = target_archs(arch)
    verbose = verbose_from_env() if verbose is None else verbose
    out = Path(out) if out is not None else OUT
    out.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="pi05w4a4_build_") as work:
        cmds, objs = compile_commands(archs, Path(work))
        workers = max(1, min(len(cmds), os.cpu_count() or 1))
        with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
            for fut in [pool.submit(_run, c, verbose) for c in cmds]:
                fut.result()
        fd, tmp = tempfile.mkstemp(prefix=out.name + ".", suffix=".tmp", dir=out.parent)
        os.close(fd)
        try:
            _run([hipcc()] + [f"--offload-arch={a}" for a in archs] + ["-shared", "-fPIC", "-o", tmp] + objs,
                 verbose)
            os.chmod(tmp, 0o755)
            os.replace(tmp, out)
        finally:
            if os.path.exists(tmp):
                os.unlink(tmp)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--arch", default=None, help="offload target(s); default PYTORCH_ROCM_ARCH, GPU_ARCHS, gfx950")
    ap.add_argument("--verbose", action="store_true", default=None)
    ap.add_argument("--out", default=None)
    args = ap.parse_args()
    out = build(args.arch, args.verbose, args.out)
    print(f"built {out}")


if __name__ == "__main__":
    sys.exit(main())
