"""Node-classification evaluation of model logits, outside any timing.

Same command line, checks and JSON report as the reference's evaluator
(baseline/scripts/evaluate_task.py:6-50):

    python -m gatgpu.evaluate --output logits.f32 --nodes N --classes C \\
        --labels labels.npy|.csv[.gz] --split ids.npy|.csv[.gz] \\
        [--reference r0_logits.f32 [--max-accuracy-drop 0.01]]

logits are FP32 little-endian [N][C] (gat_bench --output, or
gatgpu.Context.model_forward).  The split holds development/test node ids,
not a mask.  Prints one JSON line; with --max-accuracy-drop the exit status is
0 on PASS and 1 on FAIL.
"""
from __future__ import annotations

import argparse
import json
import sys

import numpy as np


def _array(path):
    if path.endswith(".npy"):
        return np.load(path, allow_pickle=False)
    return np.loadtxt(path, delimiter=",")


def _logits(path, nodes, classes):
    data = np.fromfile(path, dtype="<f4")
    if data.size != nodes * classes or not np.isfinite(data).all():
        raise ValueError("invalid/nonfinite logits")
    return data.reshape(nodes, classes)


def _integers(a):
    if not np.isfinite(a).all():
        raise ValueError("invalid label/split sizes or finite values")
    as_int = a.astype(np.int64)
    if np.any(a != as_int):
        raise ValueError("labels/split must be integers")
    return as_int


def evaluate(output, nodes, classes, labels, split, reference=None, max_accuracy_drop=None):
    """Returns (report dict, passed or None).  labels/split: arrays or paths."""
    labels = np.asarray(_array(labels) if isinstance(labels, str) else labels).reshape(-1)
    split = np.asarray(_array(split) if isinstance(split, str) else split).reshape(-1)
    if labels.size != nodes:
        raise ValueError("invalid label/split sizes or finite values")
    labels = _integers(labels)
    split = _integers(split)
    if split.size == 0 or split.min() < 0 or split.max() >= nodes or np.unique(split).size != split.size:
        raise ValueError("invalid or duplicate split IDs")
    truth = labels[split]
    if truth.min() < 0 or truth.max() >= classes:
        raise ValueError("split labels out of bounds")
    pred = _logits(output, nodes, classes)[split].argmax(axis=1)
    report = {"accuracy": float(np.mean(pred == truth)), "split_nodes": int(split.size), "gate": "UNCONFIGURED"}
    if reference:
        ref_pred = _logits(reference, nodes, classes)[split].argmax(axis=1)
        ref_acc = float(np.mean(ref_pred == truth))
        report.update(reference_accuracy=ref_acc, accuracy_drop=ref_acc - report["accuracy"],
                      prediction_agreement=float(np.mean(pred == ref_pred)))
    if max_accuracy_drop is None:
        return report, None
    if not reference or not np.isfinite(max_accuracy_drop) or max_accuracy_drop < 0:
        raise ValueError("accuracy drop gate needs reference and a finite nonnegative threshold")
    passed = report["accuracy_drop"] <= max_accuracy_drop
    report["gate"] = "PASS" if passed else "FAIL"
    return report, passed


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--output", required=True, help="FP32 row-major model logits")
    ap.add_argument("--nodes", type=int, required=True)
    ap.add_argument("--classes", type=int, required=True)
    ap.add_argument("--labels", required=True)
    ap.add_argument("--split", required=True, help="development/test node IDs, not a boolean mask")
    ap.add_argument("--reference", help="FP32 R0 logits for the accuracy-drop gate")
    ap.add_argument("--max-accuracy-drop", type=float)
    a = ap.parse_args(argv)
    report, passed = evaluate(a.output, a.nodes, a.classes, a.labels, a.split, a.reference, a.max_accuracy_drop)
    print(json.dumps(report))
    return 0 if passed is None or passed else 1


if __name__ == "__main__":
    sys.exit(main())
