"""The rocprofv3 summary helpers (pi05_fast.w4a4.profiling) on small synthetic CSV files
written in rocprofv3's column layout: kernel-name shortening, the per-kernel trace and
counter tables, and the traffic table's copy calibration and algorithmic ratios."""

from __future__ import annotations

import csv

import pytest

from pi05_fast.w4a4 import profiling as prof

GEMM = "_ZN4w4a412_GLOBAL__N_116gemm_w4a4_kernelILi7ELi4ELi4ELi1ELb1ELi2ELi2ELb0ELb0EEEvNS_10GemmParamsE"
COPY = "__amd_rocclr_copyBuffer"

COUNTER_FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
                  "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
                  "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp",
                  "End_Timestamp"]


def _write_counters(path, rows):
    """rows: (dispatch, kernel, workgroups, wg size, counter, value, duration ns)"""
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COUNTER_FIELDS)
        w.writeheader()
        for d, name, wgs, wg, c, v, dur in rows:
            w.writerow({"Correlation_Id": d, "Dispatch_Id": d, "Agent_Id": "Agent 1", "Queue_Id": 1,
                        "Process_Id": 1, "Thread_Id": 1, "Grid_Size": wgs * wg, "Kernel_Id": 1,
                        "Kernel_Name": name, "Workgroup_Size": wg, "LDS_Block_Size": 0, "Scratch_Size": 0,
                        "VGPR_Count": 128, "Accum_VGPR_Count": 0, "SGPR_Count": 32, "Counter_Name": c,
                        "Counter_Value": v, "Start_Timestamp": 1000 * d, "End_Timestamp": 1000 * d + dur})


def test_short_name_demangles_template_arguments():
    assert prof.short_name(GEMM) == "w4a4::gemm_w4a4_kernel<7, 4, 4, 1, true, 2, 2, false, false>"


def test_counter_table_derives_clock_and_mfma_busy(tmp_path):
    p = tmp_path / "c.csv"
    dur = 40000  # ns
    busy = 2.0 * dur * prof.N_SE  # SQ_BUSY_CYCLES summed over 32 SEs at 2.0 GHz
    mfma = 0.5 * prof.N_SIMD * 2.0 * dur
    _write_counters(p, [(1, GEMM, 896, 256, "SQ_BUSY_CYCLES", busy, dur),
                        (1, GEMM, 896, 256, "SQ_VALU_MFMA_BUSY_CYCLES", mfma, dur),
                        (1, GEMM, 896, 256, "SQ_INSTS_VALU", 3584 * 3000, dur),
                        (1, GEMM, 896, 256, "SQ_WAVES", 3584, dur)])
    res = prof.read_counters([str(p)])
    (key, cs), = res.items()
    assert key == ("w4a4::gemm_w4a4_kernel<7, 4, 4, 1, true, 2, 2, false, false>", 896, 256)
    d = prof.derived({c: v[0] for c, v in cs.items()})
    assert d["clock_ghz"] == pytest.approx(2.0)
    assert d["mfma_busy"] == pytest.approx(0.5)
    assert d["valu_per_wave"] == pytest.approx(3000)
    assert d["clock_peak_tops"] == pytest.approx(5000 * 2.0 / 2.4)
    table = prof.counter_table([str(p)])
    assert "| *mfma_busy* | 0.5 |" in table and "| duration (ns) | 40000 |" in table


def test_traffic_table_calibrates_with_the_copy(tmp_path):
    """FETCH_SIZE reading half of the copy's bytes is scaled by 2; the ratio is taken
    against the class's algorithmic bytes."""
    fetch, write = tmp_path / "f.csv", tmp_path / "w.csv"
    frows, wrows = [], []
    d = 1
    for cls, (name, wgs, nbytes, _) in prof.TRAFFIC_CLASSES.items():
        # plain (unmangled) names are kept as they are by read_counters
        frows.append((d, name, wgs, 256, "FETCH_SIZE", nbytes / 2048 / 2, 1000))  # half, in KiB
        wrows.append((d, name, wgs, 256, "WRITE_SIZE", nbytes / 2048, 1000))
        d += 1
    frows.append((d, COPY, 256, 512, "FETCH_SIZE", prof.COPY_KIB / 2, 1000))
    wrows.append((d, COPY, 256, 512, "WRITE_SIZE", prof.COPY_KIB, 1000))
    _write_counters(fetch, frows)
    _write_counters(write, wrows)
    out = prof.traffic_table(str(fetch), str(write))
    assert "FETCH_SIZE is scaled by 2.0000 and WRITE_SIZE by 1.0000" in out
    got = {ln.split("[")[1].split("]")[0]: float(ln.split(":")[1])
           for ln in out.splitlines() if ln.startswith("traffic_bytes_per_launch[")}
    assert set(got) == set(prof.TRAFFIC_CLASSES)
    for cls, (_, _, nbytes, _) in prof.TRAFFIC_CLASSES.items():
        assert got[cls] == pytest.approx(nbytes, rel=1e-9), cls  # half read + half written
    assert "| 1.00 |" in out


def test_traffic_classes_algorithmic_bytes():
    """The 776-token byte counts stated in the table's descriptions."""
    c = prof.TRAFFIC_CLASSES
    assert c["gate_up_gelu_int4"][2] / 1e6 == pytest.approx(59.91, abs=0.01)
    assert c["gate_up_int4"][2] / 1e6 == pytest.approx(85.34, abs=0.01)
    assert c["gate_up_gelu"][2] / 1e6 == pytest.approx(77.09, abs=0.01)  # E3M2 operands: 6 bits per code
    assert c["gate_up"][2] / 1e6 == pytest.approx(102.51, abs=0.01)
    assert c["rmsnorm_quant_e3m2"][2] / 1e6 == pytest.approx(4.38, abs=0.01)
    assert c["down_residual"][2] / 1e6 == pytest.approx(29.50, abs=0.01)
    assert c["o_residual"][2] / 1e6 == pytest.approx(9.26, abs=0.01)
    assert c["quant_k16384"][2] / 1e6 == pytest.approx(31.79, abs=0.01)
    assert c["rmsnorm_quant_k2048"][2] / 1e6 == pytest.approx(3.98, abs=0.01)


# The forward's GEMM instances as the launchers name them (mangled, twelve template
# arguments: <MI, NI, NWAVES, KW, GELU, RING, WPE, QKV_PREP, QFUSE, E3M2, QPRO, NKB>).
def _mangled(args):
    enc = "".join(f"Lb{int(a)}E" if isinstance(a, bool) else f"Li{a}E" for a in args)
    return f"_ZN4w4a412_GLOBAL__N_116gemm_w4a4_kernelI{enc}EEvNS_10GemmParamsE"


FORWARD_GEMMS = {
    "gate_up_gelu": (7, 4, 4, 1, True, 2, 2, False, False, True, False, 0),
    "down_residual": (7, 4, 8, 8, False, 2, 2, False, False, False, False, 16),
    "qkv_rope": (4, 4, 4, 4, False, 2, 2, True, False, False, False, 4),
    "o_residual": (4, 4, 4, 4, False, 2, 2, False, False, False, False, 4),
}


@pytest.mark.parametrize("cls", sorted(FORWARD_GEMMS))
def test_forward_gemm_names_match_their_classes(cls):
    """The profiling tables and bench.py's in-forward breakdown find each forward GEMM by
    its name: the demangled name is the traffic class's, and bench.kernel_class maps both
    the mangled and the demangled name to the class."""
    import importlib.util
    import pathlib

    spec = importlib.util.spec_from_file_location("_bench", pathlib.Path(__file__).resolve().parents[1] / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    name = _mangled(FORWARD_GEMMS[cls])
    short = prof.short_name(name)
    assert short == "w4a4::" + prof.TRAFFIC_CLASSES[cls][0]
    assert bench.kernel_class(name) == cls
    assert bench.kernel_class(short) == cls
