"""OGB node-property raw CSVs -> GATBIN1 (offline; no download).

Same inputs, graph construction and outputs as the reference converter
(implementation/tools/prepare_arxiv.py:18-50):

    python -m gatgpu.ogb --source <dataset dir holding raw/> --output g.gatbin [--dataset ogbn-arxiv]

reads raw/node-feat.csv.gz (float32 features), raw/edge.csv.gz (src,dst pairs)
and raw/node-label.csv.gz (one label per node, for the class count), and
writes a destination-row CSR that is undirected (every edge in both
directions), deduplicated, with exactly one self-loop per node and sorted
column indices, plus `<output>.json` with the dataset summary.  The labels
file can be passed to `python -m gatgpu.evaluate --labels` as it is.
"""
from __future__ import annotations

import argparse
import gzip
import json
from pathlib import Path

import numpy as np

from . import formats


def _csv(path, dtype):
    with gzip.open(path, "rt") as f:
        a = np.loadtxt(f, delimiter=",", dtype=dtype, ndmin=2)
    return a


def undirected_csr(n, src, dst):
    """(row u64[n+1], col u32[e]) of the symmetrised, deduplicated graph with
    one self-loop per node, rows = destinations, columns sorted."""
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    loops = np.arange(n, dtype=np.int64)
    rows = np.concatenate((dst, src, loops))
    cols = np.concatenate((src, dst, loops))
    keys = np.unique(rows * n + cols)  # sorted by (row, col), duplicates gone
    r, c = keys // n, keys % n
    row = np.zeros(n + 1, np.uint64)
    np.cumsum(np.bincount(r, minlength=n), out=row[1:])
    return row, c.astype(np.uint32)


def convert(source, output, dataset="ogbn-arxiv"):
    raw = Path(source) / "raw"
    x = np.ascontiguousarray(_csv(raw / "node-feat.csv.gz", np.float32), "<f4")
    edges = _csv(raw / "edge.csv.gz", np.int64)
    labels = _csv(raw / "node-label.csv.gz", np.int64).reshape(-1)
    n, d = x.shape
    if edges.shape[1] != 2 or labels.shape[0] != n:
        raise ValueError("edge list must be pairs and labels one per node")
    if edges.size and (edges.min() < 0 or edges.max() >= n):
        raise ValueError("edge endpoint out of range")
    row, col = undirected_csr(n, edges[:, 0], edges[:, 1])
    classes = int(labels.max() + 1)
    output = Path(output)
    output.parent.mkdir(parents=True, exist_ok=True)
    formats.save_graph(output, row, col, x, classes)
    meta = dict(dataset=dataset, source=str(source), nodes=int(n), edges=int(col.size), in_features=int(d),
                classes=classes, graph="undirected, deduplicated, one self-loop per node", dtype="float32",
                format="GATBIN1")
    output.with_suffix(".json").write_text(json.dumps(meta, indent=2) + "\n")
    return meta


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--source", type=Path, required=True)
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--dataset", default="ogbn-arxiv")
    a = ap.parse_args(argv)
    print(json.dumps(convert(a.source, a.output, a.dataset)))


if __name__ == "__main__":
    main()
