#!/usr/bin/env python3
"""Benchmark of the three-layer multi-head GAT forward on one MI355X.

A step is one full forward D_in -> 8x32 -> 8x32 -> 1xC over the whole graph,
inputs resident in HBM.  Default workload: the 64.3M-edge power-law graph
(2,449,029 nodes, 100 -> 8x32 -> 8x32 -> 1x47, bf16 storage with FP32
softmax/accumulation).  Prints ONE JSON line (rank 0).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload large|skew|arxiv|smoke]
                  [--precision bf16|fp32] [--dataflow auto|transform_first|aggregate_first]
                  [--no-cpu-baseline] [--cpu-threads T] [--cpu-warmups 2] [--cpu-repeats 7]
                  [--no-arxiv] [--arxiv-steps 50]

Besides the contract fields the line carries, per layer, the aggregation's
and the projection's time and fraction of the HBM (and MFMA) peaks
("layers"), the dominant projection against both peaks ("roofline_gemm"),
the cold-start times ("cold_start_ms") and the host CPU baseline with its
protocol and host description ("cpu_baseline").  With the default workload
it also times the 2.5M-edge graph of the metric (169,343 nodes, 2,484,941
edges, 128 -> 8x32 -> 8x32 -> 1x40) in bf16 and FP32, beside its own host
CPU baseline ("arxiv"; --no-arxiv skips it).
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


def source_digest(paths):
    """SHA-256 over the given source files (repository-relative), in order."""
    import hashlib

    h = hashlib.sha256()
    for rel in paths:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()


def pmc_traffic(workload, precision):
    """HBM bytes per launch of the layer-2 aggregation, measured with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE and calibrated against a device
    copy of known size; read from the committed summary.  The summary names
    the kernel sources it was measured on and their digest: if those sources
    have changed since, the figure is stale and is not reported (None, with
    the reason)."""
    for f in sorted((ROOT / "profiles").glob("*pmc*.md")):
        for line in f.read_text().splitlines():
            if line.startswith("bench-traffic: "):
                rec = json.loads(line[len("bench-traffic: "):])
                if rec.get("workload") == workload and rec.get("precision") == precision:
                    srcs = rec.get("sources")
                    if not srcs or source_digest(srcs) != rec.get("sources_sha256"):
                        return None, f"{f.name}: measured on other kernel sources than this tree's"
                    return rec, f.name
    return None, "no counter summary for this workload"


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


def run_forwards(gatgpu, torch, w, precision, flow, steps, warmup, calibrate_copy=False):
    """Uploads workload w, runs `warmup` untimed forwards (the first one, which
    allocates the per-layer buffers, timed as the cold forward) and `steps`
    timed forwards (the model time only: an event before the first kernel and
    after the last), then `steps` more with an event at every stage boundary
    for the per-layer times.  Returns the HIP-event times and the cold-start
    record."""
    t0 = time.perf_counter()
    row, col = w.graph()
    x = w.features()
    model = w.model()
    gen_s = time.perf_counter() - t0
    prec = gatgpu.BF16 if precision == "bf16" else gatgpu.FP32
    ctx = gatgpu.Context(0)
    ctx.set_graph(row, col)
    ctx.set_model(model)
    ctx.set_input(x)
    static = ctx.static_times()
    print(f"# workload {w.name} {precision}: N={w.n} E={int(row[-1])} gen {gen_s:.1f}s", file=sys.stderr, flush=True)
    if calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    _, _, cold_ms = ctx.model_forward(prec, flow, want_logits=False, timed=True)
    for _ in range(max(warmup - 1, 0)):
        ctx.model_forward(prec, flow, want_logits=False, timed=False)
    torch.cuda.synchronize()
    ctx.synchronize()
    step_ms, layer_times = [], []
    t0 = time.perf_counter()
    for _ in range(steps):
        # The model time alone: two HIP events, the forward's first and last.
        _, _, total = ctx.model_forward(prec, flow, want_logits=False, timed=True, stages=False)
        step_ms.append(total)
    ctx.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # The per-layer breakdown from as many forwards again, after the timed
    # region: their events at every stage boundary add 0.02-0.03 ms to a
    # forward of the 2.5M-edge graph.
    staged_ms = []
    for _ in range(steps):
        _, times, total = ctx.model_forward(prec, flow, want_logits=False, timed=True)
        layer_times.append(times)
        staged_ms.append(total)
    ctx.synchronize()
    # Cold-start: the static steps (graph checks, uploads, degree schedule,
    # weight preparation, feature permutation), the first forward, and the
    # logits copied back to the host after a forward.
    ctx.model_forward(prec, flow, want_logits=True, timed=False)
    cold = {k: round(v, 3) for k, v in ctx.static_times().items()}
    cold.update({k: round(static[k], 3) for k in static if k != "logits_d2h_ms"})
    cold["first_forward_ms"] = round(cold_ms, 3)
    # The output layer's projection ran inside layer 2's aggregation (its
    # output rows never stored): layer 2's kernel writes layer 3's Z rows and
    # L/R instead of its own output rows.
    fused23 = not ctx.has_stage(1, "out")
    ctx.close()
    ms = float(np.mean(step_ms))  # HIP-event model time (first kernel of layer 1 to last of layer 3)
    return {"row": row, "model": model, "n": w.n, "e": int(row[-1]), "ms": ms, "wall_s": wall,
            "staged_ms": float(np.mean(staged_ms)),
            "layer_times": layer_times, "cold": cold, "fused23": fused23, "bf16": prec == gatgpu.BF16}


def device_copy_gbs(torch, nbytes, reps=5):
    """Rate of a device-to-device copy of nbytes (the runtime's blit kernel,
    as torch's copy_ issues it): 2 nbytes moved per copy, median of reps,
    timed with events on torch's stream.  The streaming reference for the
    projections, which read one table and write another."""
    n = nbytes // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        dst.copy_(src)
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    del src, dst
    torch.cuda.empty_cache()
    ms = float(np.median(ts))
    return {"bytes_per_copy": 2 * 4 * n, "ms": round(ms, 4), "gbs": round(2 * 4 * n / (ms * 1e-3) / 1e9, 1)}


def layer_records(r):
    """Per-layer aggregation and projection times with their bytes, FLOP and
    fractions of the HBM and MFMA peaks."""
    n, e, model, bf16, fused23 = r["n"], r["e"], r["model"], r["bf16"], r["fused23"]
    s_z = 2 if bf16 else 4
    layers = []
    for l, p in enumerate(model):
        K, d, D = p["heads"], p["dim"], p["in"]
        W = K * d
        t = {k: float(np.mean([lt[l][k] for lt in r["layer_times"]])) for k in r["layer_times"][0][l]}
        af = t["lr_ms"] > 0  # aggregate-first layers report the L/R front end as lr_ms
        hidden = l < 2
        s_out = 2 if (bf16 and hidden) else 4
        s_x = 4 if (l == 0 or not bf16) else 2  # layer 1 reads the FP32 features; later layers the bf16 output
        gather_b = None
        if af:
            # Algorithmic (B_AF): the bf16 input rows of D features per edge.
            agg_b = 8 * (n + 1) + 4 * e + 4 * K * e + 4 * K * n + e * D * 2 + n * W * s_out
            # As read: the sum form gathers 256-byte table rows (128 bf16
            # slots; R in the row tail up to 112 inputs, else from its own
            # array: 4K bytes more per edge) and keeps L, max and den per node.
            r_arr = 4 * K * e if D > 112 else 0
            gather_b = 8 * (n + 1) + 4 * e + 256 * e + r_arr + 12 * K * n + n * W * s_out
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
        if gather_b is not None:
            rec.update({"aggregate_bytes_basis": "algorithmic: D bf16 input features per edge",
                        "gather_table_bytes": int(gather_b),
                        "gather_table_frac": round(gather_b / (t["aggregate_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
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
    return layers


# The reference's published B0 forwards on this graph size (ogbn-arxiv,
# 16 Sapphire Rapids cores; baseline/docs/FOUR_PATHS_GITHUB_INDEX.md:7-8).
REFERENCE_ARXIV_B0_MS = {"bf16": 68.437, "fp32": 73.996}


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
    ap.add_argument("--no-arxiv", action="store_true",
                    help="skip the 2.5M-edge graph's bf16 and FP32 forwards (run only with the default workload)")
    ap.add_argument("--arxiv-steps", type=int, default=50)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run one 1 GiB device-to-device copy first (counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1).", file=sys.stderr)
        sys.exit(2)
    with_arxiv = args.workload == "large" and not args.no_arxiv

    # CPU baselines first, each in a child process, before the GPU is touched.
    cpu, cpu_arxiv = None, {}
    if not args.no_cpu_baseline:
        print("# CPU baseline (child process) ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.workload, args.precision, args.cpu_threads, args.cpu_warmups, args.cpu_repeats)
        if with_arxiv:
            for prec in ("bf16", "fp32"):
                cpu_arxiv[prec] = cpu_baseline("arxiv", prec, args.cpu_threads, args.cpu_warmups, args.cpu_repeats)

    import torch
    import gatgpu
    from gatgpu import inputs

    flow = {"auto": gatgpu.AUTO, "transform_first": gatgpu.TRANSFORM_FIRST,
            "aggregate_first": gatgpu.AGGREGATE_FIRST}[args.dataflow]
    w = inputs.WORKLOADS[args.workload]
    r = run_forwards(gatgpu, torch, w, args.precision, flow, args.steps, args.warmup, args.calibrate_copy)
    n, e, model, bf16 = r["n"], r["e"], r["model"], r["bf16"]
    ms = r["ms"]
    value = 3 * e / (ms * 1e-3) / 1e9
    layers = layer_records(r)
    # Dominant kernel: the layer-2 aggregation (fused prescan/softmax/SpMM/ELU).
    dom = layers[1]
    pmc, pmc_src = pmc_traffic(w.name, args.precision)
    gemm = max((x for x in layers if "projection_ms" in x), key=lambda x: x["projection_ms"])
    # A device copy of the projection's input table size: the rate a stream of
    # reads and writes of that size reaches on this part.
    copy = device_copy_gbs(torch, int(n * model[gemm["layer"] - 1]["in"] * (2 if bf16 else 4)))
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
                               f"N={n}, E={e} (incl. self-loops), max in-degree {int(np.diff(r['row']).max())}",
                   "precision": args.precision, "wall_ms_per_step": round(r["wall_s"] / args.steps * 1e3, 4),
                   "ms_per_step_with_stage_events": round(r["staged_ms"], 4)},
        "roofline": {"bound": "hbm", "achieved": dom["aggregate_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["aggregate_frac"],
                     "traffic": int(pmc["bytes_per_launch"]) if pmc else None,
                     "traffic_source": pmc_src,
                     "kernel": "layer-2 aggregation", "algorithmic_bytes": dom["aggregate_bytes"],
                     "avg_ms": dom["aggregate_ms"]},
        "roofline_gemm": {"kernel": f"layer-{gemm['layer']} projection", "bound": "hbm",
                          "flop": int(2 * n * model[gemm["layer"] - 1]["in"] * model[gemm["layer"] - 1]["heads"]
                                      * model[gemm["layer"] - 1]["dim"]),
                          "avg_ms": gemm["projection_ms"], "achieved_tflops": gemm["projection_tflops"],
                          "peak_tflops": MFMA_BF16_PEAK_TFLOPS if bf16 else MFMA_FP32_PEAK_TFLOPS,
                          "mfma_frac": gemm["projection_mfma_frac"], "hbm_bytes": gemm["projection_bytes"],
                          "hbm_frac": gemm["projection_hbm_frac"], "device_copy": copy,
                          "copy_frac": round(gemm["projection_bytes"] / (gemm["projection_ms"] * 1e-3) / 1e9 / copy["gbs"], 4)},
        "layers": layers,
        "cold_start_ms": r["cold"],
    }
    if cpu is not None:
        out["cpu_baseline"] = cpu
    if with_arxiv:
        wa = inputs.WORKLOADS["arxiv"]
        rec = {"workload": f"arxiv: 3-layer GAT {wa.din}->{wa.heads}x{wa.dim}->{wa.heads}x{wa.dim}->1x{wa.classes}, "
                           f"N={wa.n}, E={wa.edges} (incl. self-loops), max in-degree {wa.max_degree}",
               "note": "Z (87-173 MB) fits the 256 MB Infinity Cache at this size: the fractions are of the HBM "
                       "peak but the gathers are served from that cache"}
        for prec in ("bf16", "fp32"):
            ra = run_forwards(gatgpu, torch, wa, prec, gatgpu.AUTO, args.arxiv_steps, 5)
            ea = ra["e"]
            entry = {"ms_per_forward": round(ra["ms"], 4), "gedge_s": round(3 * ea / (ra["ms"] * 1e-3) / 1e9, 4),
                     "ms_per_forward_with_stage_events": round(ra["staged_ms"], 4),
                     "steps": args.arxiv_steps, "warmup": 5,
                     "layers": [{k: x[k] for k in ("layer", "dataflow", "aggregate_ms", "aggregate_bytes",
                                                   "aggregate_frac", "projection_ms", "total_ms") if k in x}
                                for x in layer_records(ra)],
                     "reference_published_b0_ms": REFERENCE_ARXIV_B0_MS[prec]}
            if prec in cpu_arxiv:
                c = cpu_arxiv[prec]
                entry["cpu_b0"] = {k: c[k] for k in ("ms_per_forward", "p95_ms", "cores", "kind", "sample")}
                entry["speedup_vs_cpu_b0"] = round(c["ms_per_forward"] / ra["ms"], 1)
            rec[prec] = entry
        out["arxiv"] = rec
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
