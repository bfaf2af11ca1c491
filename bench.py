#!/usr/bin/env python3
"""Benchmark: W4A4 PaliGemma-2B-shaped prefix LM on one MI355X.

    python bench.py [--steps K] [--warmup W] [--tokens 776] [--batch 1] [--layers 18]

Workload: the 18-layer Gemma-2B-shaped prefix LM (hidden 2048, 8x256 heads, 1 KV head,
intermediate 16384) over a 776-token prefix, batch 1, with all q/k/v/o/gate/up/down
projections running the W4A4 path (quantize + int8-MFMA GEMM) and attention fp16 eager.
Weights are synthetic packed INT4 (random codes with the statistics of a packed
N(0, 0.02) weight), inputs synthetic N(0, 1/sqrt(2048)) prefix embeddings.

Timed region: K replays of the whole forward captured in one HIP graph (inputs resident
in HBM), bracketed by device synchronisation.  `value` = ms per prefix forward.
Per-GEMM timings come from a second, eager timed region in which HIP events (recorded on
the stream the kernels run on) bracket every GEMM launch; they give int8 TOPS and the
fraction of the MI355X dense int8 MFMA peak per GEMM class and the `roofline` object of
the dominant kernel.  `cpu_baseline` times the CPU oracle (numpy) on one decoder layer's
W4A4 work at the same M and scales it to the full depth.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "pi05-pytorch-fast_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "W4A4 prefix-LM ms @776 tok; int8 TOPS & % MFMA peak per GEMM (1 MI355X)"
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, published
HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, published


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=776)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--layers", type=int, default=18)
    ap.add_argument("--kernel-steps", type=int, default=10, help="eager forwards for per-GEMM events")
    ap.add_argument("--no-graph", action="store_true", help="time eager forwards instead of graph replays")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline")
    ap.add_argument("--fuse-gelu", action="store_true", help="gate/up with the fused GELU*up epilogue")
    return ap.parse_args()


def gemm_class(kind: str, k: int, ns: list[int]) -> str:
    if kind == "quant":
        return f"quant_k{k}"
    if kind == "gemm3":
        return "qkv"
    if kind in ("gemm2", "gemm2_gelu"):
        return "gate_up"
    return "down" if k > 2048 else "o"


def gemm_ops(kind: str, m: int, k: int, ns: list[int]) -> float:
    return 2.0 * m * k * sum(ns)


class EventRecorder:
    """HIP events around each GEMM / quant launch on the launching (current) stream."""

    def __init__(self, torch):
        self.torch = torch
        self.open: dict[str, tuple] = {}
        self.done: list[tuple] = []

    def __call__(self, kind, phase, m, k, ns):
        key = (kind, k, tuple(ns))
        if phase == "begin":
            ev = self.torch.cuda.Event(enable_timing=True)
            ev.record()
            self.open[key] = (ev, m)
        else:
            ev0, m0 = self.open.pop(key)
            ev1 = self.torch.cuda.Event(enable_timing=True)
            ev1.record()
            self.done.append((kind, m0, k, list(ns), ev0, ev1))

    def summary(self, steps: int) -> dict:
        self.torch.cuda.synchronize()
        acc: dict[str, dict] = {}
        for kind, m, k, ns, e0, e1 in self.done:
            cls = gemm_class(kind, k, ns)
            d = acc.setdefault(cls, {"times_us": [], "m": m, "k": k, "n": sum(ns), "kind": kind})
            d["times_us"].append(e0.elapsed_time(e1) * 1e3)
        out = {}
        for cls, d in acc.items():
            avg = sum(d["times_us"]) / len(d["times_us"])
            calls_per_step = len(d["times_us"]) / steps
            m, k, n = d["m"], d["k"], d["n"]
            entry = {"m": m, "k": k, "n": n, "calls_per_forward": calls_per_step, "avg_us": round(avg, 3)}
            if cls.startswith("quant"):
                nbytes = 2.0 * m * k + m * k / 2 + 4 * m
                gbs = nbytes / (avg * 1e-6) / 1e9
                entry.update(bytes=nbytes, gbs=round(gbs, 1), frac_hbm=round(gbs / HBM_PEAK_GBS, 4))
            else:
                ops = 2.0 * m * n * k
                tops = ops / (avg * 1e-6) / 1e12
                entry.update(ops=ops, tops=round(tops, 1), frac_int8_peak=round(tops / INT8_PEAK_TOPS, 4))
            out[cls] = entry
        return out


def cpu_baseline(tokens: int, batch: int, layers: int, budget_s: float) -> dict:
    """CPU oracle (numpy) on one decoder layer's W4A4 work at M = tokens*batch, scaled to
    `layers`.  Per GEMM: quantize the activation (fp32 FWHT + INT4), exact integer matmul
    (fp32 BLAS), dequant to fp16."""
    import numpy as np

    from oracle import w4a4_oracle as orc

    try:
        from threadpoolctl import threadpool_info

        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    m = tokens * batch
    rng = np.random.default_rng(20260923)

    def act(k):
        x = rng.standard_normal((m, k), dtype=np.float32)
        x[:, rng.permutation(k)[: max(1, k // 100)]] *= 20.0
        return x.astype(np.float16)

    def wcodes(n, k):
        return np.clip(np.rint(rng.standard_normal((n, k), dtype=np.float32) * 2), -7, 7).astype(np.int8)

    shapes = [("qkv", 2048, 2560), ("o", 2048, 2048), ("gate_up", 2048, 32768), ("down", 16384, 2048)]
    data = [(name, act(k), wcodes(n, k), np.full(n, 0.01, np.float32)) for name, k, n in shapes]

    def one_layer():
        for _, x, wc, sw in data:
            q, sa = orc.quant_activation(x)
            orc.dequant_fp16(orc.gemm_acc_int32(q, wc), sa, sw)

    times = []
    t_start = time.perf_counter()
    one_layer()  # warm-up
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        one_layer()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 4 * budget_s:
            break
    per_layer = statistics.median(times)
    return {
        "value": round(per_layer * layers * 1e3, 1),
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"one decoder layer of W4A4 work at M={m} (4 activation quants + QKV/o/gate-up/down "
            f"integer GEMMs + fp16 dequant), median of {len(times)} runs x {layers} layers; "
            f"numpy oracle, fp32-BLAS exact integer matmul, {threads} threads, "
            f"os.cpu_count()={os.cpu_count()}; attention/norms not included"
        ),
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the W4A4 path is "
            "measured at one GPU's share, multi-GPU sharding is design-only.",
            file=sys.stderr,
        )
        return 2

    import torch

    from pi05_fast.w4a4 import extension as ext
    from pi05_fast.w4a4.prefix_lm import build_prefix_lm, prefix_inputs, prefix_ops

    if args.fuse_gelu:
        os.environ["PI05_W4A4_FUSE_GELU"] = "1"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ext.preload()
    model, _ = build_prefix_lm(dev, num_layers=args.layers)
    x = prefix_inputs(args.batch, args.tokens, dev)
    s = args.tokens
    # Prefix-LM mask over the prefix: every prefix token sees every other one (additive 4D).
    mask = torch.zeros(args.batch, 1, s, s, dtype=torch.float16, device=dev)

    with torch.no_grad():
        y_eager = model(x, mask)
        torch.cuda.synchronize()
        graph = None
        if not args.no_graph:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):
                    model(x, mask)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            try:
                with torch.cuda.graph(graph):
                    y_graph = model(x, mask)
            except Exception as exc:  # capture unsupported: time eager forwards instead
                print(f"bench: graph capture failed ({exc!r}); timing eager forwards", file=sys.stderr)
                graph = None
                torch.cuda.synchronize()
        graph_exact = None
        if graph is not None:
            # Replays interleaved with eager work must all give the same output, and that
            # output must match the eager forward.
            first = None
            for i in range(3):
                graph.replay()
                torch.cuda.synchronize()
                if first is None:
                    first = y_graph.clone()
                    graph_exact = bool(torch.equal(first, y_eager))
                    err = ((first.float() - y_eager.float()).norm() / y_eager.float().norm()).item()
                    if not err <= 1e-3:
                        raise RuntimeError(f"graph replay differs from the eager forward (rel_l2={err:.3e})")
                elif not torch.equal(y_graph, first):
                    raise RuntimeError(f"graph replay {i} differs from replay 0")
                model(x, mask)
                torch.cuda.synchronize()

        # Eager forwards, for reference (host-dispatch bound).
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(max(3, args.steps // 4)):
            model(x, mask)
        torch.cuda.synchronize()
        eager_ms = (time.perf_counter() - t0) * 1e3 / max(3, args.steps // 4)

        def step():
            if graph is not None:
                graph.replay()
            else:
                model(x, mask)

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / args.steps

        # Per-GEMM kernel times: eager forwards with HIP events around every launch.
        rec = EventRecorder(torch)
        ext._launch_hook = rec
        try:
            torch.cuda.synchronize()
            for _ in range(args.kernel_steps):
                model(x, mask)
            kernels = rec.summary(args.kernel_steps)
        finally:
            ext._launch_hook = None

    ops = prefix_ops(args.tokens, args.batch, args.layers)
    total_ops = sum(ops.values())
    gemm_classes = [c for c in kernels if not c.startswith("quant")]
    dominant = max(gemm_classes, key=lambda c: kernels[c]["avg_us"] * kernels[c]["calls_per_forward"])
    dk = kernels[dominant]
    roofline = {
        "bound": "mfma",
        "kernel": dominant,
        "achieved": dk["tops"],
        "peak": INT8_PEAK_TOPS,
        "unit": "TFLOP/s",
        "frac": round(dk["tops"] / INT8_PEAK_TOPS, 4),
        "traffic": None,
        "per_launch_ops": dk["ops"],
        "avg_launch_us": dk["avg_us"],
    }
    out = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic: random packed INT4 weights (codes ~ round(N(0,2)) in [-7,7], scales ~0.01), "
                "N(0,1/sqrt(2048)) fp16 prefix embeddings",
        "config": {
            "workload": f"PaliGemma-2B-shaped W4A4 prefix LM forward, {args.layers} layers, "
                        f"{args.tokens} tokens x batch {args.batch}",
            "tokens": args.tokens,
            "batch": args.batch,
            "layers": args.layers,
            "timed": "hip-graph replay" if graph is not None else "eager",
            "fused_gelu_up": bool(args.fuse_gelu),
            "graph_replay_bit_exact_vs_eager": graph_exact,
        },
        "eager_ms_per_forward": round(eager_ms, 3),
        "w4a4_gop_per_forward": round(total_ops / 1e9, 1),
        "effective_tops_whole_forward": round(total_ops / (ms * 1e-3) / 1e12, 1),
        "gemms": kernels,
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.tokens, args.batch, args.layers, args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
