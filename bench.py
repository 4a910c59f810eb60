#!/usr/bin/env python3
"""Benchmark of the three-layer multi-head GAT forward on one MI355X.

A step is one full forward D_in -> 8x32 -> 8x32 -> 1xC over the whole graph,
inputs resident in HBM.  Default workload: the 64.3M-edge power-law graph
(2,449,029 nodes, 100 -> 8x32 -> 8x32 -> 1x47, bf16 storage with FP32
softmax/accumulation).  Prints ONE JSON line (rank 0).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload large|skew|arxiv|smoke]
                  [--precision bf16|fp32] [--dataflow auto|transform_first|aggregate_first]
                  [--no-cpu-baseline] [--cpu-threads T] [--cpu-warmups 2] [--cpu-repeats 7]

Besides the contract fields the line carries, per layer, the aggregation's
and the projection's time and fraction of the HBM (and MFMA) peaks
("layers"), the dominant projection against both peaks ("roofline_gemm"),
the cold-start times ("cold_start_ms") and the host CPU baseline with its
protocol and host description ("cpu_baseline").
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "gat-tfs_amd"))

METRIC = "3-layer GAT fwd latency (ms), GEdge/s & % HBM roofline, 2.5M/64M-edge graphs"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_FP32_PEAK_TFLOPS = 157.3


def agg_bytes(n, e, heads, dim, s_z, s_out, r_gather=True):
    """Algorithmic bytes of one transform-first aggregation launch: rowptr,
    col, R gathers (K floats per edge), L/M/den per node, the gathered Z rows
    and the output rows.  bf16 layers of 8 heads x 32 features form R from the
    gathered bf16 Z row itself, so their launches have no R gathers."""
    r = 4 * heads * e if r_gather else 0
    return 8 * (n + 1) + 4 * e + r + 4 * heads * n + e * heads * dim * s_z + n * heads * dim * s_out


def pmc_traffic(workload, precision):
    """HBM bytes per launch of the layer-2 aggregation, measured with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE and calibrated against a device
    copy of known size; read from the committed summary (None if absent)."""
    for f in sorted((ROOT / "profiles").glob("*pmc*.md")):
        for line in f.read_text().splitlines():
            if line.startswith("bench-traffic: "):
                rec = json.loads(line[len("bench-traffic: "):])
                if rec.get("workload") == workload and rec.get("precision") == precision:
                    return rec
    return None


def cpu_baseline(workload, precision, threads, warmups, repeats):
    """The oracle's B0 forward timed on the host cores (oracle/cpu_baseline.py),
    in a child process started before this one touches the GPU, so that its
    OpenMP threads are placed one per physical core of the first socket."""
    cmd = [sys.executable, str(ROOT / "oracle" / "cpu_baseline.py"), "--workload", workload, "--precision", precision,
           "--threads", str(threads), "--warmups", str(warmups), "--repeats", str(repeats)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError(f"CPU baseline failed ({r.returncode}): {r.stderr[-2000:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="large")
    ap.add_argument("--precision", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--dataflow", default="auto", choices=["auto", "transform_first", "aggregate_first"],
                    help="per-layer dataflow; aggregate_first applies where the layer supports it")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="CPU baseline threads (default: the first socket's physical cores, at most OMP_NUM_THREADS)")
    ap.add_argument("--cpu-warmups", type=int, default=2)
    ap.add_argument("--cpu-repeats", type=int, default=7)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run one 1 GiB device-to-device copy first (counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1).", file=sys.stderr)
        sys.exit(2)

    cpu = None
    if not args.no_cpu_baseline:
        print("# CPU baseline (child process) ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.workload, args.precision, args.cpu_threads, args.cpu_warmups, args.cpu_repeats)

    import torch
    import gatgpu
    from gatgpu import inputs

    w = inputs.WORKLOADS[args.workload]
    t0 = time.perf_counter()
    row, col = w.graph()
    x = w.features()
    model = w.model()
    gen_s = time.perf_counter() - t0
    n, e = w.n, int(row[-1])
    prec = gatgpu.BF16 if args.precision == "bf16" else gatgpu.FP32
    flow = {"auto": gatgpu.AUTO, "transform_first": gatgpu.TRANSFORM_FIRST,
            "aggregate_first": gatgpu.AGGREGATE_FIRST}[args.dataflow]

    ctx = gatgpu.Context(0)
    ctx.set_graph(row, col)
    ctx.set_model(model)
    ctx.set_input(x)
    static = ctx.static_times()
    print(f"# workload {w.name}: N={n} E={e} gen {gen_s:.1f}s", file=sys.stderr, flush=True)

    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    # The first forward allocates the per-layer device buffers: the cold forward.
    _, _, cold_ms = ctx.model_forward(prec, flow, want_logits=False, timed=True)
    for _ in range(max(args.warmup - 1, 0)):
        ctx.model_forward(prec, flow, want_logits=False, timed=False)
    torch.cuda.synchronize()
    ctx.synchronize()
    step_ms, layer_times = [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        _, times, total = ctx.model_forward(prec, flow, want_logits=False, timed=True)
        step_ms.append(total)
        layer_times.append(times)
    ctx.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = float(np.mean(step_ms))  # HIP-event model time (first kernel of layer 1 to last of layer 3)
    value = 3 * e / (ms * 1e-3) / 1e9
    # Cold-start: the static steps (graph checks, uploads, degree schedule,
    # weight preparation, feature permutation), the first forward, and the
    # logits copied back to the host after a forward.
    ctx.model_forward(prec, flow, want_logits=True, timed=False)
    cold = {k: round(v, 3) for k, v in ctx.static_times().items()}
    cold.update({k: round(static[k], 3) for k in static if k != "logits_d2h_ms"})
    cold["first_forward_ms"] = round(cold_ms, 3)

    bf16 = prec == gatgpu.BF16
    s_z = 2 if bf16 else 4
    # The output layer's projection ran inside layer 2's aggregation (its
    # output rows never stored): layer 2's kernel writes layer 3's Z rows and
    # L/R instead of its own output rows.
    fused23 = not ctx.has_stage(1, "out")
    layers = []
    for l, p in enumerate(model):
        K, d, D = p["heads"], p["dim"], p["in"]
        W = K * d
        t = {k: float(np.mean([lt[l][k] for lt in layer_times])) for k in layer_times[0][l]}
        af = t["lr_ms"] > 0  # aggregate-first layers report the L/R front end as lr_ms
        hidden = l < 2
        s_out = 2 if (bf16 and hidden) else 4
        s_x = 4 if (l == 0 or not bf16) else 2  # layer 1 reads the FP32 features; later layers the bf16 output
        if af:
            agg_b = 8 * (n + 1) + 4 * e + 4 * K * e + 4 * K * n + e * D * 2 + n * W * s_out
        else:
            no_r = bf16 and ((K, d) == (8, 32) or (K, d) == (1, 64))  # R formed from the gathered Z row
            agg_b = agg_bytes(n, e, K, d, s_z, s_out, r_gather=not no_r)
            if fused23 and l == 1:
                nxt = model[2]
                agg_b += n * (nxt["heads"] * nxt["dim"] * 2 + 8 * nxt["heads"]) - n * W * s_out
        rec = {"layer": l + 1, "dataflow": "aggregate_first" if af else "transform_first",
               "aggregate_ms": round(t["aggregate_ms"], 4), "aggregate_bytes": int(agg_b),
               "aggregate_gbs": round(agg_b / (t["aggregate_ms"] * 1e-3) / 1e9, 1),
               "aggregate_frac": round(agg_b / (t["aggregate_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "total_ms": round(t["total_ms"], 4)}
        if fused23 and l == 1:
            rec["fused"] = "layer-3 projection in the epilogue (32-row tiles on MFMA); layer-2 output rows not stored"
        if af:
            rec["lr_front_end_ms"] = round(t["lr_ms"], 4)
        elif fused23 and l == 2:
            rec["projection"] = "fused into the layer-2 aggregation"
        else:
            flop = 2 * n * D * W
            gb = n * D * s_x + D * W * s_x + n * W * s_z + 8 * K * n
            pm = t["projection_ms"]
            rec.update({"projection_ms": round(pm, 4), "projection_tflops": round(flop / (pm * 1e-3) / 1e12, 1),
                        "projection_mfma_frac": round(flop / (pm * 1e-3) / 1e12 / (MFMA_BF16_PEAK_TFLOPS if bf16 else
                                                                                   MFMA_FP32_PEAK_TFLOPS), 4),
                        "projection_bytes": int(gb),
                        "projection_hbm_frac": round(gb / (pm * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        layers.append(rec)
    # Dominant kernel: the layer-2 aggregation (fused prescan/softmax/SpMM/ELU).
    dom = layers[1]
    pmc = pmc_traffic(w.name, args.precision)
    gemm = max((r for r in layers if "projection_ms" in r), key=lambda r: r["projection_ms"])
    out = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "GEdge/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if bf16 else "f32",
        "data": "synthetic",
        "config": {"workload": f"{w.name}: 3-layer GAT {w.din}->{w.heads}x{w.dim}->{w.heads}x{w.dim}->1x{w.classes}, "
                               f"N={n}, E={e} (incl. self-loops), max in-degree {int(np.diff(row).max())}",
                   "precision": args.precision, "wall_ms_per_step": round(wall / args.steps * 1e3, 4)},
        "roofline": {"bound": "hbm", "achieved": dom["aggregate_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["aggregate_frac"],
                     "traffic": int(pmc["bytes_per_launch"]) if pmc else None,
                     "kernel": "layer-2 aggregation", "algorithmic_bytes": dom["aggregate_bytes"],
                     "avg_ms": dom["aggregate_ms"]},
        "roofline_gemm": {"kernel": f"layer-{gemm['layer']} projection", "bound": "hbm",
                          "flop": int(2 * n * model[gemm["layer"] - 1]["in"] * model[gemm["layer"] - 1]["heads"]
                                      * model[gemm["layer"] - 1]["dim"]),
                          "avg_ms": gemm["projection_ms"], "achieved_tflops": gemm["projection_tflops"],
                          "peak_tflops": MFMA_BF16_PEAK_TFLOPS if bf16 else MFMA_FP32_PEAK_TFLOPS,
                          "mfma_frac": gemm["projection_mfma_frac"], "hbm_bytes": gemm["projection_bytes"],
                          "hbm_frac": gemm["projection_hbm_frac"]},
        "layers": layers,
        "cold_start_ms": cold,
    }
    ctx.close()
    if cpu is not None:
        out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
