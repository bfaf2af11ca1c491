"""Markdown summaries of rocprofv3 output for the W4A4 kernels.

    python -m pi05_fast.w4a4.profiling trace <kernel_trace.csv> [--match REGEX] [--top N]
    python -m pi05_fast.w4a4.profiling counters <counter_collection.csv> ... [--match REGEX]
    python -m pi05_fast.w4a4.profiling forward <kernel_trace.csv> [--steps N]
    python -m pi05_fast.w4a4.profiling traffic <FETCH_SIZE counters.csv> <WRITE_SIZE counters.csv>

``trace`` reads a ``rocprofv3 --kernel-trace --output-format csv`` file and lists, per
kernel and grid, the launch count and the mean / median / min duration.  ``forward``
takes the trace of a run that ends with N replays of one captured forward (``bench.py
--forward-only``), finds the replay period (the shortest dispatch sequence that repeats at
the end of the trace) and breaks the last N replays down per kernel.  ``counters``
reads the ``--pmc`` files of one or more runs (rocprofv3 writes one row per dispatch and
counter, summed over the XCDs and shader engines) and prints, per kernel and grid, the
median of each counter over the dispatches and the figures derived from them on MI355X
(8 XCDs x 4 shader engines, 256 CUs, 1024 SIMDs):

    clock_ghz   = SQ_BUSY_CYCLES / 32 / duration           (cycles with a wave present,
                                                             per shader engine)
    busy_cycles = SQ_BUSY_CYCLES / 32                       (the dispatch's cycles)
    mfma_busy   = SQ_VALU_MFMA_BUSY_CYCLES / (1024 * busy_cycles)
    int8_tops   = SQ_INSTS_VALU_MFMA_MOPS_I8 * 512 / duration
    clock_peak  = 5.0 POPS * clock_ghz / 2.4                (dense int8 at that clock)
    waves_cu    = 4 * SQ_WAVE_CYCLES / (256 * busy_cycles)  (mean resident waves per CU)
    valu_per_wave = SQ_INSTS_VALU / SQ_WAVES
    valu_active = 4 * SQ_ACTIVE_INST_VALU / (4 * 256 * busy_cycles)  (per-SIMD VALU issue share)
    fetch_kib / write_kib = FETCH_SIZE / WRITE_SIZE per dispatch

The duration of a counter dispatch is its End - Start timestamp in that (serialised)
run, so it can exceed the kernel's time in a plain trace.  ``traffic`` takes the
FETCH_SIZE run and the WRITE_SIZE run of ``bench.py --only-kernel ...,copy`` and prints
each 776-token kernel class's HBM-side bytes per launch, scaled by what the same counter
reads for the 64 MiB device copy, against its algorithmic bytes.
"""

from __future__ import annotations

import argparse
import csv
import functools
import re
import shutil
import statistics
import subprocess
import sys
from collections import defaultdict

N_SE = 32          # 8 XCDs x 4 shader engines
N_CU = 256
N_SIMD = 1024
INT8_PEAK_POPS = 5.0
PEAK_CLOCK_GHZ = 2.4

csv.field_size_limit(1 << 24)


_MANGLED = re.compile(r"_ZN4w4a4(?:12_GLOBAL__N_1)?(\d+)")
_TEMPLATE_ARG = re.compile(r"L([ib])(\d+)E")


@functools.lru_cache(maxsize=None)
def _demangle(name: str) -> str:
    """c++filt, else (it does not know _Float16 parameters) the w4a4 kernel name and its
    integer / bool template arguments read from the mangled name."""
    if not name.startswith("_Z"):
        return name
    tool = shutil.which("c++filt")
    if tool is not None:
        out = subprocess.run([tool, name], capture_output=True, text=True).stdout.strip()
        if out and not out.startswith("_Z"):
            return out
    m = _MANGLED.match(name)
    if m is None:
        return name
    n = int(m.group(1))
    ident = name[m.end():m.end() + n]
    rest = name[m.end() + n:]
    args = []
    if rest.startswith("I"):
        rest = rest[1:]
        while True:
            t = _TEMPLATE_ARG.match(rest)
            if t is None:
                break
            args.append(t.group(2) if t.group(1) == "i" else ("true" if t.group(2) == "1" else "false"))
            rest = rest[t.end():]
    return f"w4a4::{ident}<{', '.join(args)}>" if args else f"w4a4::{ident}"


def short_name(name: str) -> str:
    """Kernel name without the argument list and the namespace noise."""
    base = re.sub(r"^void\s+", "", _demangle(name))
    base = base.replace("(anonymous namespace)::", "").replace("_GLOBAL__N_1::", "")
    depth = 0
    for i, ch in enumerate(base):
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            base = base[:i]
            break
    return base[:110]


def read_trace(path: str, match: str | None = None) -> dict:
    rows = defaultdict(list)
    pat = re.compile(match) if match else None
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if pat and not pat.search(name):
                continue
            grid = (int(r["Grid_Size_X"]) // max(int(r["Workgroup_Size_X"]), 1), int(r["Workgroup_Size_X"]))
            dur_us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            rows[(short_name(name), grid)].append(dur_us)
    return rows


def trace_table(path: str, match: str | None = None, top: int = 30) -> str:
    rows = read_trace(path, match)
    items = sorted(rows.items(), key=lambda kv: -sum(kv[1]))[:top]
    out = [f"| kernel | workgroups x size | calls | mean us | median us | min us | total us |",
           "|---|---|---:|---:|---:|---:|---:|"]
    for (name, (wgs, wg)), d in items:
        out.append(f"| `{name}` | {wgs} x {wg} | {len(d)} | {statistics.fmean(d):.3f} | "
                   f"{statistics.median(d):.3f} | {min(d):.3f} | {sum(d):.1f} |")
    return "\n".join(out)


def _trace_rows(path: str) -> list[tuple[str, tuple, int, int]]:
    out = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            grid = (int(r["Grid_Size_X"]) // max(int(r["Workgroup_Size_X"]), 1), int(r["Workgroup_Size_X"]))
            out.append((short_name(r["Kernel_Name"]), grid, int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    out.sort(key=lambda t: t[2])
    return out


def forward_table(path: str, steps: int) -> str:
    rows = _trace_rows(path)
    keys = [(n, g) for n, g, _, _ in rows]
    period = next((p for p in range(10, len(keys) // 2 + 1) if keys[-p:] == keys[-2 * p:-p]), None)
    if period is None:
        raise SystemExit("no repeating forward found at the end of the trace")
    last = rows[-steps * period:]
    busy = sum(e - s for _, _, s, e in last) / 1e6 / steps
    span = (max(e for *_, e in last) - min(s for _, _, s, _ in last)) / 1e6 / steps
    per = defaultdict(list)
    for n, g, s, e in last:
        per[(n, g)].append((e - s) / 1e3)
    out = [f"Last {steps} replays: {period} dispatches per forward; kernel time {busy:.3f} ms per forward, "
           f"first start to last end {span:.3f} ms per forward, idle gaps {span - busy:.3f} ms per forward.",
           "",
           "| kernel | workgroups x size | per forward | avg us | min us | max us | ms per forward | % |",
           "|---|---|---:|---:|---:|---:|---:|---:|"]
    for (n, (wgs, wg)), d in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        tot = sum(d) / 1e3 / steps
        out.append(f"| `{n}` | {wgs} x {wg} | {len(d) // steps} | {statistics.fmean(d):.3f} | {min(d):.3f} | "
                   f"{max(d):.3f} | {tot:.4f} | {100 * tot / busy:.1f} |")
    return "\n".join(out)


def read_counters(paths: list[str], match: str | None = None) -> dict:
    """{(kernel, workgroups, wg size): {counter: [values], "_dur_ns": [..]}}"""
    res = defaultdict(lambda: defaultdict(list))
    pat = re.compile(match) if match else None
    for path in paths:
        seen = set()
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"]
                if pat and not pat.search(name):
                    continue
                wg = int(r["Workgroup_Size"])
                key = (short_name(name), int(r["Grid_Size"]) // max(wg, 1), wg)
                res[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
                did = (r["Dispatch_Id"], key)
                if did not in seen:
                    seen.add(did)
                    res[key]["_dur_ns"].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
                    res[key]["_vgpr"].append(int(r["VGPR_Count"]))
                    res[key]["_agpr"].append(int(r["Accum_VGPR_Count"]))
                    res[key]["_lds"].append(int(r["LDS_Block_Size"]))
    return res


def derived(med: dict) -> dict:
    d = {}
    dur = med.get("_dur_ns")
    busy = med.get("SQ_BUSY_CYCLES")
    if dur and busy:
        cyc = busy / N_SE
        d["clock_ghz"] = cyc / dur
        if "SQ_VALU_MFMA_BUSY_CYCLES" in med:
            d["mfma_busy"] = med["SQ_VALU_MFMA_BUSY_CYCLES"] / (N_SIMD * cyc)
        if "SQ_WAVE_CYCLES" in med:
            d["waves_cu"] = 4 * med["SQ_WAVE_CYCLES"] / (N_CU * cyc)
        if "SQ_ACTIVE_INST_VALU" in med:
            d["valu_active"] = 4 * med["SQ_ACTIVE_INST_VALU"] / (N_SIMD * cyc)
        d["clock_peak_tops"] = INT8_PEAK_POPS * 1e3 * d["clock_ghz"] / PEAK_CLOCK_GHZ
    if dur and med.get("SQ_INSTS_VALU_MFMA_MOPS_I8"):
        d["int8_tops"] = med["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512 / dur / 1e3
    if med.get("SQ_WAVES") and "SQ_INSTS_VALU" in med:
        d["valu_per_wave"] = med["SQ_INSTS_VALU"] / med["SQ_WAVES"]
    return d


def counter_table(paths: list[str], match: str | None = None) -> str:
    res = read_counters(paths, match)
    out = []
    for key, cs in res.items():
        name, wgs, wg = key
        med = {c: statistics.median(v) for c, v in cs.items()}
        n = len(cs["_dur_ns"])
        # rocprofv3's VGPR_Count / Accum_VGPR_Count fields as recorded (its own granularity,
        # not the kernel descriptor's register count)
        out.append(f"### `{name}`  ({wgs} workgroups x {wg}; {n} dispatches; rocprofv3 VGPR_Count "
                   f"{med['_vgpr']:.0f}, Accum_VGPR_Count {med['_agpr']:.0f}, LDS {med['_lds']:.0f} B)")
        out.append("")
        out.append("| counter | median per dispatch |")
        out.append("|---|---:|")
        out.append(f"| duration (ns) | {med['_dur_ns']:.0f} |")
        for c in sorted(k for k in med if not k.startswith("_")):
            out.append(f"| {c} | {med[c]:.1f} |")
        for c, v in derived(med).items():
            out.append(f"| *{c}* | {v:.4g} |")
        out.append("")
    return "\n".join(out)


def _gemm_alg_bytes(m: int, k: int, n: int, out_bytes: float) -> float:
    """Codes + scales/corrections of A and B, plus the output (as bench.py counts them)."""
    return m * k / 2 + 4 * m + n * k / 2 + 4 * n + out_bytes


def _gemm_e3m2_bytes(m: int, k: int, n: int, out_bytes: float) -> float:
    """The same for E3M2 operands (6 bits per code), the form the FP6-MFMA GEMM reads."""
    return m * k * 0.75 + 4 * m + n * k * 0.75 + 4 * n + out_bytes


# The kernel classes of the 776-token prefix-LM forward (one decoder layer's launches), as
# bench.py --only-kernel names them: class -> (kernel name, workgroups, algorithmic bytes,
# what they are).  gemm_w4a4_kernel<MI, NI, NWAVES, KW, GELU, RING, WPE, QKV_PREP, QFUSE,
# E3M2, QPRO, NKB>, fwht_quant_kernel<LOGK, LOGT, ROWS, NORM, E3M2>.
_M = 776
TRAFFIC_CLASSES = {
    "gate_up_gelu": ("gemm_w4a4_kernel<7, 4, 4, 1, true, 2, 2, false, false, true, false, 0>", 896,
                     _gemm_e3m2_bytes(_M, 2048, 32768, 2.0 * _M * 16384),
                     "E3M2 codes A 1.19 MB + gate and up weights 50.33 MB + scales; fp16 h 25.43 MB"),
    "gate_up": ("gemm_w4a4_kernel<7, 4, 4, 1, false, 2, 2, false, false, true, false, 0>", 896,
                _gemm_e3m2_bytes(_M, 2048, 32768, 2.0 * _M * 32768),
                "E3M2 codes A 1.19 MB + weights 50.33 MB + scales; fp16 gate and up 50.86 MB"),
    "gate_up_gelu_int4": ("gemm_w4a4_kernel<7, 4, 4, 1, true, 2, 2, false, false, false, false, 0>", 896,
                          _gemm_alg_bytes(_M, 2048, 32768, 2.0 * _M * 16384),
                          "codes A 0.79 MB + gate and up weights 33.55 MB + scales/corrections; fp16 h 25.43 MB"),
    "gate_up_int4": ("gemm_w4a4_kernel<7, 4, 4, 1, false, 2, 2, false, false, false, false, 0>", 896,
                     _gemm_alg_bytes(_M, 2048, 32768, 2.0 * _M * 32768),
                     "codes A 0.79 MB + weights 33.55 MB + scales/corrections; fp16 gate and up 50.86 MB"),
    "down_residual": ("gemm_w4a4_kernel<7, 4, 8, 8, false, 2, 2, false, false, false, false, 16>", 224,
                      _gemm_alg_bytes(_M, 16384, 2048, 2.0 * 2.0 * _M * 2048),
                      "codes A 6.36 MB + down weights 16.78 MB + scales/corrections + fp16 residual 3.18 MB; "
                      "fp16 out 3.18 MB"),
    "qkv": ("gemm_w4a4_kernel<2, 2, 4, 1, false, 3, 2, false, false, false, false, 0>", 500,
            _gemm_alg_bytes(_M, 2048, 2560, 2.0 * _M * 2560), "codes A 0.79 MB + weights 2.62 MB; fp16 q/k/v 3.97 MB"),
    "qkv_rope": ("gemm_w4a4_kernel<4, 4, 4, 4, false, 2, 2, true, false, false, false, 4>", 520,
                 _gemm_alg_bytes(_M, 2048, 2560, 2.0 * _M * 2560) + 2 * _M * 256 * 2 * 2 + 2 * 832 * 256 * 2,
                 "as qkv + rotary tables 0.79 MB read + key states 0.40 MB and K/V^T 0.85 MB written"),
    "o_residual": ("gemm_w4a4_kernel<4, 4, 4, 4, false, 2, 2, false, false, false, false, 4>", 416,
                   _gemm_alg_bytes(_M, 2048, 2048, 2.0 * 2.0 * _M * 2048),
                   "codes A 0.79 MB + weights 2.10 MB + residual 3.18 MB; out 3.18 MB"),
    "quant_k16384": ("fwht_quant_kernel<14, 8, 1, false, false>", 776, 2.0 * _M * 16384 + _M * 16384 / 2 + 4 * _M,
                     "fp16 x 25.43 MB; codes 6.36 MB + scales"),
    "rmsnorm_quant_k2048": ("fwht_quant_kernel<11, 6, 4, true, false>", 194,
                            2.0 * _M * 2048 + 2 * 2048 + _M * 2048 / 2 + 4 * _M,
                            "fp16 x 3.18 MB + norm weight; codes 0.79 MB + scales"),
    "rmsnorm_quant_e3m2": ("fwht_quant_kernel<11, 6, 4, true, true>", 194,
                           2.0 * _M * 2048 + 2 * 2048 + _M * 2048 * 0.75 + 4 * _M,
                           "fp16 x 3.18 MB + norm weight; E3M2 codes 1.19 MB + scales"),
}
COPY_KIB = 65536.0  # the calibration copy (bench.py --only-kernel copy): 64 MiB read and written


def _mean_counter(res: dict, counter: str, name: str, grid: int) -> tuple[float, int]:
    for (kn, wgs, _), cs in res.items():
        if name in kn and wgs == grid and counter in cs:
            return statistics.fmean(cs[counter]), len(cs[counter])
    raise KeyError(f"{counter} of {name} with {grid} workgroups not in the counter file")


def traffic_table(fetch_csv: str, write_csv: str) -> str:
    """FETCH_SIZE / WRITE_SIZE per launch of each class, scaled by what the same counters
    read for the 64 MiB device copy of the same runs (``__amd_rocclr_copyBuffer`` with 256
    workgroups), against the algorithmic bytes; ends with the ``traffic_bytes_per_launch``
    lines that bench.py reads."""
    rf, rw = read_counters([fetch_csv]), read_counters([write_csv])
    cf, ncf = _mean_counter(rf, "FETCH_SIZE", "copyBuffer", 256)
    cw, ncw = _mean_counter(rw, "WRITE_SIZE", "copyBuffer", 256)
    sf, sw = COPY_KIB / cf, COPY_KIB / cw
    out = [f"Calibration: the 64 MiB copy reads FETCH_SIZE {cf:.1f} KiB (n={ncf}) and WRITE_SIZE {cw:.1f} KiB "
           f"(n={ncw}) per dispatch, so FETCH_SIZE is scaled by {sf:.4f} and WRITE_SIZE by {sw:.4f}.", "",
           "| class | kernel | FETCH_SIZE KiB (mean) | WRITE_SIZE KiB (mean) | read MB (scaled) | write MB (scaled) "
           "| total MB | algorithmic MB | ratio | algorithmic bytes |",
           "|---|---|---:|---:|---:|---:|---:|---:|---:|---|"]
    tb = {}
    for cls, (kn, grid, alg, what) in TRAFFIC_CLASSES.items():
        f, nf = _mean_counter(rf, "FETCH_SIZE", kn, grid)
        w, nw = _mean_counter(rw, "WRITE_SIZE", kn, grid)
        rb, wb = f * 1024 * sf, w * 1024 * sw
        tb[cls] = rb + wb
        out.append(f"| {cls} | `{kn}` {grid} WGs | {f:.1f} (n={nf}) | {w:.1f} (n={nw}) | {rb / 1e6:.2f} | "
                   f"{wb / 1e6:.2f} | {(rb + wb) / 1e6:.2f} | {alg / 1e6:.2f} | {(rb + wb) / alg:.2f} | {what} |")
    out.append("")
    out.extend(f"traffic_bytes_per_launch[{k}]: {v:.0f}" for k, v in tb.items())
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="rocprofv3 summaries for the W4A4 kernels")
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    t.add_argument("--match", default=None)
    t.add_argument("--top", type=int, default=30)
    fw = sub.add_parser("forward")
    fw.add_argument("csv")
    fw.add_argument("--steps", type=int, default=20)
    c = sub.add_parser("counters")
    c.add_argument("csv", nargs="+")
    c.add_argument("--match", default=None)
    tr = sub.add_parser("traffic")
    tr.add_argument("fetch_csv")
    tr.add_argument("write_csv")
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        print(trace_table(a.csv, a.match, a.top))
    elif a.cmd == "forward":
        print(forward_table(a.csv, a.steps))
    elif a.cmd == "traffic":
        print(traffic_table(a.fetch_csv, a.write_csv))
    else:
        print(counter_table(a.csv, a.match))
    return 0


if __name__ == "__main__":
    sys.exit(main())
