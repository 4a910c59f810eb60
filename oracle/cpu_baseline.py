#!/usr/bin/env python3
"""Host CPU baseline of bench.py: the oracle's B0 three-layer forward, timed.

TEST INFRASTRUCTURE.  bench.py's cpu_baseline leg starts this script as a
child process, before it touches the GPU, so that the OpenMP runtime of the
oracle library starts in a process of its own with the reference's thread
placement: one thread per physical core of the first socket, packed on
consecutive cores (OMP_PROC_BIND=close, OMP_PLACES=cores), at most
OMP_NUM_THREADS threads; 2 warm-ups and 7 timed repeats, median and p95
(baseline/scripts/arxiv_payload.sh:5-38, baseline/bench/main.cpp:46,171-182).
The forward is the oracle's restatement of standard_bf16 / standard_fp32
(baseline/src/baseline_standard.cpp:3-108) on the same synthetic workload as
the GPU run.  Prints one JSON line.
"""
import os

# Read by libgomp when the oracle library loads it, below.
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")

import argparse  # noqa: E402
import json  # noqa: E402
import math  # noqa: E402
import sys  # noqa: E402
import time  # noqa: E402
from pathlib import Path  # noqa: E402

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "gat-tfs_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def host_info():
    """CPU model, sockets, physical cores of the CPUs this process may run on
    (its affinity mask), NUMA nodes and whether AMX tiles exist."""
    model, flags = "unknown", set()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    cpus = sorted(os.sched_getaffinity(0))
    cores = {}  # socket -> core ids
    first = None
    for c in cpus:
        topo = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
        try:
            pkg = int((topo / "physical_package_id").read_text())
            core = int((topo / "core_id").read_text())
        except (OSError, ValueError):
            pkg, core = 0, c
        if first is None:
            first = pkg
        cores.setdefault(pkg, set()).add(core)
    node_dir = Path("/sys/devices/system/node")
    nodes = len(list(node_dir.glob("node[0-9]*"))) if node_dir.exists() else 0
    return {"cpu_model": model, "amx_tile": "amx_tile" in flags, "cpus_allowed": len(cpus), "sockets": len(cores),
            "physical_cores_per_socket": {str(k): len(v) for k, v in sorted(cores.items())},
            "first_socket_physical_cores": len(cores.get(first, ())), "numa_nodes": nodes}


def pct(samples, q):
    """Percentile as the reference computes it (baseline/bench/main.cpp:26)."""
    x = sorted(samples)
    return x[min(len(x) - 1, max(0, math.ceil(q * len(x)) - 1))]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="large")
    ap.add_argument("--precision", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--threads", type=int, default=0, help="0: first socket's physical cores, at most OMP_NUM_THREADS")
    ap.add_argument("--warmups", type=int, default=2)
    ap.add_argument("--repeats", type=int, default=7)
    args = ap.parse_args()

    host = host_info()
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    phys = host["first_socket_physical_cores"] or os.cpu_count() or 1
    threads = args.threads or (min(phys, cap) if cap > 0 else phys)

    import numpy as np

    import oracle
    from gatgpu import inputs

    w = inputs.WORKLOADS[args.workload]
    row, col = w.graph()
    x = w.features()
    model = w.model()
    bf16 = args.precision == "bf16"
    n, e = int(row.size - 1), int(row[-1])
    # Prepared outside the timer like prepare() (common.cpp:97-119) and the
    # workspaces like Workspace::allocate (common.cpp:126-134).
    wq = [oracle.quantize_bf16(p["w"]) if bf16 else p["w"] for p in model]
    ws = [oracle.standard_workspace(n, p) for p in model]

    def forward():
        h = x
        for l, p in enumerate(model):
            st, _ = oracle.standard_layer(row, col, h, p, l < 2, bf16, threads, wq[l], ws[l])
            h = st["out"]
        return h

    for _ in range(args.warmups):
        forward()
    times = []
    for _ in range(args.repeats):
        t0 = time.perf_counter()
        out = forward()
        times.append(time.perf_counter() - t0)
    if not np.isfinite(out).all():
        raise SystemExit("CPU baseline produced non-finite logits")
    med, p95 = pct(times, 0.5), pct(times, 0.95)
    rec = {"value": round(3 * e / med / 1e9, 6), "unit": "GEdge/s", "cores": threads, "kind": "port",
           "sample": f"full {w.name} graph, three-layer B0 forward ({'standard_bf16' if bf16 else 'standard_fp32'}), "
                     f"{args.warmups} warm-ups + {args.repeats} timed repeats, median",
           "ms_per_forward": round(med * 1e3, 3), "p95_ms": round(p95 * 1e3, 3),
           "samples_ms": [round(t * 1e3, 3) for t in times],
           "host": {k: host[k] for k in ("cpu_model", "sockets", "physical_cores_per_socket", "cpus_allowed",
                                         "numa_nodes")},
           "tfs": ("not runnable: host lacks amx_tile (the reference's tfs_bf16 path is AMX-only)"
                   if not host["amx_tile"] else
                   "not run: the reference's tfs_bf16 path needs oneMKL and icpx, absent from this image")}
    rec["host"].update({"threads": threads, "binding": f"OMP_PROC_BIND={os.environ['OMP_PROC_BIND']} "
                                                       f"OMP_PLACES={os.environ['OMP_PLACES']}",
                        "numa_policy": "first touch (no interleave)"})
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
