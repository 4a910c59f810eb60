"""bench.py's bookkeeping without a GPU: the per-layer byte counts and the
check that ties the committed HBM-traffic figure to the kernel sources it
was measured on."""
import json

import bench


def fake_run(bf16=True, fused23=True):
    """A run record of the 100 -> 8x32 -> 8x32 -> 1x47 model with layer 1
    aggregate-first, as run_forwards returns it (times in ms)."""
    n, e = 1000, 20000
    model = [{"in": 100, "heads": 8, "dim": 32}, {"in": 256, "heads": 8, "dim": 32}, {"in": 256, "heads": 1, "dim": 47}]
    lt = [{"lr_ms": 0.1, "aggregate_ms": 1.0, "total_ms": 1.1, "projection_ms": 0.0},
          {"lr_ms": 0.0, "aggregate_ms": 2.0, "total_ms": 2.5, "projection_ms": 0.5},
          {"lr_ms": 0.0, "aggregate_ms": 0.5, "total_ms": 0.5, "projection_ms": 0.0}]
    return {"n": n, "e": e, "model": model, "bf16": bf16, "fused23": fused23, "layer_times": [lt, lt]}


def test_layer_records_bytes():
    r = fake_run()
    n, e = r["n"], r["e"]
    rec = bench.layer_records(r)
    # aggregate-first layer 1: B_AF with D = 100 bf16 features per edge and
    # bf16 hidden output rows; the table rows as read are 256 bytes per edge
    # (R in their tail, D <= 112) plus L, max and den per node.
    assert rec[0]["dataflow"] == "aggregate_first"
    assert rec[0]["aggregate_bytes"] == 8 * (n + 1) + 4 * e + 32 * e + 32 * n + 200 * e + 512 * n
    assert rec[0]["gather_table_bytes"] == 8 * (n + 1) + 4 * e + 256 * e + 96 * n + 512 * n
    assert rec[0]["lr_front_end_ms"] == 0.1
    # layer 2, transform-first with R from the gathered bf16 Z rows and the
    # output layer's projection in its epilogue: Z rows of 512 bytes per edge,
    # L/max/den per node, layer 3's 94-byte Z row and its L/R instead of the
    # layer-2 output row.
    want2 = 8 * (n + 1) + 4 * e + 32 * n + 512 * e + 512 * n + n * (94 + 8) - 512 * n
    assert rec[1]["aggregate_bytes"] == want2
    assert abs(rec[1]["aggregate_frac"] - want2 / 2e-3 / 8e12) < 1e-4
    assert rec[1]["projection_ms"] == 0.5
    assert rec[2]["projection"] == "fused into the layer-2 aggregation"
    # one-head output layer: R gathered (47 classes are not a 1 x 64 row), FP32 logits
    assert rec[2]["aggregate_bytes"] == 8 * (n + 1) + 4 * e + 4 * e + 4 * n + 94 * e + 188 * n


def test_traffic_record_tied_to_kernel_sources(tmp_path, monkeypatch):
    src = tmp_path / "k.hip"
    src.write_text("kernel v1\n")
    (tmp_path / "profiles").mkdir()
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    rec = {"workload": "large", "precision": "bf16", "bytes_per_launch": 123, "sources": ["k.hip"],
           "sources_sha256": bench.source_digest(["k.hip"])}
    (tmp_path / "profiles" / "x_pmc.md").write_text("text\nbench-traffic: " + json.dumps(rec) + "\n")
    got, where = bench.pmc_traffic("large", "bf16")
    assert got["bytes_per_launch"] == 123 and where == "x_pmc.md"
    assert bench.pmc_traffic("large", "fp32")[0] is None
    src.write_text("kernel v2\n")  # the kernel changed after the counters were taken
    got, where = bench.pmc_traffic("large", "bf16")
    assert got is None and "other kernel sources" in where


def test_committed_traffic_record_names_its_sources():
    """The committed summary carries the digest of the sources it was
    measured on (whether they still match is the bench's concern)."""
    rec = None
    for f in (bench.ROOT / "profiles").glob("*pmc*.md"):
        for line in f.read_text().splitlines():
            if line.startswith("bench-traffic: "):
                rec = json.loads(line[len("bench-traffic: "):])
    assert rec is not None and rec["sources"] and len(rec["sources_sha256"]) == 64
    for s in rec["sources"]:
        assert (bench.ROOT / s).exists()
