"""Binary formats of the reference harness, read and written from Python.

GATBIN1  graph      magic[8], u64 n, u64 e, u32 din, u32 classes,
                    u64 row[n+1], u32 col[e], f32 x[n*din]
                    (baseline/src/common.cpp:31-44)
GATWGT1  weights    magic[8], u32 count, then per layer u32 {in, heads, dim},
                    f32 W[in*heads*dim], f32 aL[heads*dim], f32 aR[heads*dim]
                    (common.cpp:63-79)
GATFIX1  fixture    magic[8], u64 {n, e, in, heads, dim}, u64 row[n+1],
                    u32 col[e], f32 W, aL, aR, f32 input[n*in], f32 p[e*heads],
                    f32 den[n*heads]  (common.cpp:171-194)

All little-endian.  Readers apply the reference's checks (Graph::validate,
Param::validate, load_model's three-layer shape, load_fixture's CSR,
checkpoint, range and denominator checks) and raise ValueError with the
reference's message.  Large arrays are read with numpy.fromfile, without a
Python-level copy.
"""
from __future__ import annotations

import struct

import numpy as np

INT32_MAX = 2**31 - 1


def _magic(f, want: bytes, what: str):
    got = f.read(8)
    if len(got) != 8 or got[:7] != want:
        raise ValueError(f"bad {what} magic")


def _read(f, dtype, count):
    a = np.fromfile(f, dtype=dtype, count=count)
    if a.size != count:
        raise ValueError("truncated file")
    return a


def _require_finite(a, name):
    if not np.isfinite(a).all():
        raise ValueError(f"nonfinite {name} index={int(np.flatnonzero(~np.isfinite(a.reshape(-1)))[0])}")


# ---------------------------------------------------------------- graph
def validate_graph(g):
    """Graph::validate (baseline/src/common.cpp:23-30)."""
    n, e, din, classes = g["n"], g["e"], g["din"], g["classes"]
    row, col, x = g["row"], g["col"], g["x"]
    if not n or n > INT32_MAX or din <= 0 or classes <= 0 or row.size != n + 1 or col.size != e or x.size != n * din:
        raise ValueError("invalid graph sizes")
    if row[0] != 0 or row[-1] != e:
        raise ValueError("bad CSR bounds")
    if np.any(row[1:] < row[:-1]):
        raise ValueError("nonmonotone CSR")
    if e and int(col.max()) >= n:
        raise ValueError("source index out of bounds")
    _require_finite(x, "graph input")


def load_graph(path):
    with open(path, "rb") as f:
        _magic(f, b"GATBIN1", "graph")
        n, e, din, classes = struct.unpack("<QQII", f.read(24))
        if not n or n > INT32_MAX or not din or not classes or din > INT32_MAX or classes > INT32_MAX:
            raise ValueError("bad graph dimensions")
        row = _read(f, "<u8", n + 1)
        col = _read(f, "<u4", e)
        x = _read(f, "<f4", n * din).reshape(n, din)
    g = dict(n=int(n), e=int(e), din=int(din), classes=int(classes), row=row, col=col, x=x)
    validate_graph(g)
    return g


def save_graph(path, row, col, x, classes):
    row = np.ascontiguousarray(row, "<u8")
    col = np.ascontiguousarray(col, "<u4")
    x = np.ascontiguousarray(x, "<f4")
    g = dict(n=x.shape[0], e=col.size, din=x.shape[1], classes=int(classes), row=row, col=col, x=x)
    validate_graph(g)
    with open(path, "wb") as f:
        f.write(b"GATBIN1\0")
        f.write(struct.pack("<QQII", g["n"], g["e"], g["din"], g["classes"]))
        for a in (row, col, x):
            a.tofile(f)


# ---------------------------------------------------------------- weights
def validate_param(p):
    """Param::validate (baseline/src/common.cpp:45-49)."""
    din, K, d = p["in"], p["heads"], p["dim"]
    W = K * d
    if din <= 0 or K <= 0 or K > 8 or d <= 0 or d > 64 or np.size(p["w"]) != din * W or np.size(p["al"]) != W \
            or np.size(p["ar"]) != W:
        raise ValueError("invalid parameter shape (heads <=8, head_dim <=64)")
    for k, name in (("w", "W"), ("al", "aL"), ("ar", "aR")):
        _require_finite(np.asarray(p[k]), name)


def model_shapes(din, classes):
    """(in, heads, dim) of the three layers (common.cpp:54, :74)."""
    return [(din, 8, 32), (256, 8, 32), (256, 1, classes)]


def load_model(path, din=None, classes=None):
    """GATWGT1; with din/classes, load_model's three-layer shape check."""
    model = []
    with open(path, "rb") as f:
        _magic(f, b"GATWGT1", "weights")
        (count,) = struct.unpack("<I", f.read(4))
        if din is not None and count != 3:
            raise ValueError("model must have 3 layers")
        for l in range(count):
            s = struct.unpack("<III", f.read(12))
            if din is not None and s != model_shapes(din, classes)[l]:
                raise ValueError("checkpoint model shape mismatch")
            W = s[1] * s[2]
            p = {"in": s[0], "heads": s[1], "dim": s[2], "w": _read(f, "<f4", s[0] * W).reshape(s[0], W),
                 "al": _read(f, "<f4", W), "ar": _read(f, "<f4", W)}
            validate_param(p)
            model.append(p)
    return model


def save_model(path, model):
    with open(path, "wb") as f:
        f.write(b"GATWGT1\0")
        f.write(struct.pack("<I", len(model)))
        for p in model:
            validate_param(p)
            f.write(struct.pack("<III", p["in"], p["heads"], p["dim"]))
            for k in ("w", "al", "ar"):
                np.ascontiguousarray(p[k], "<f4").tofile(f)


# ---------------------------------------------------------------- fixture
def save_fixture(path, row, col, p, inp, P, den):
    n, e = row.size - 1, col.size
    K = p["heads"]
    if np.size(inp) != n * p["in"] or np.size(P) != e * K or np.size(den) != n * K:
        raise ValueError("bad fixture sizes")
    with open(path, "wb") as f:
        f.write(b"GATFIX1\0")
        f.write(struct.pack("<5Q", n, e, p["in"], K, p["dim"]))
        for a, t in ((row, "<u8"), (col, "<u4"), (p["w"], "<f4"), (p["al"], "<f4"), (p["ar"], "<f4"), (inp, "<f4"),
                     (P, "<f4"), (den, "<f4")):
            np.ascontiguousarray(a, t).tofile(f)


def load_fixture(path, row, col, p):
    """load_fixture (baseline/src/common.cpp:184-194) -> dict(input, p, den)."""
    n, e, K = row.size - 1, col.size, p["heads"]
    with open(path, "rb") as f:
        _magic(f, b"GATFIX1", "fixture")
        s = struct.unpack("<5Q", f.read(40))
        if s != (n, e, p["in"], K, p["dim"]):
            raise ValueError("fixture shape mismatch")
        if not np.array_equal(_read(f, "<u8", n + 1), row) or not np.array_equal(_read(f, "<u4", e), col):
            raise ValueError("fixture CSR mismatch")
        for k in ("w", "al", "ar"):
            if not np.array_equal(_read(f, "<f4", np.size(p[k])), np.asarray(p[k], np.float32).reshape(-1)):
                raise ValueError("fixture checkpoint mismatch")
        inp = _read(f, "<f4", n * p["in"]).reshape(n, p["in"])
        P = _read(f, "<f4", e * K).reshape(e, K)
        den = _read(f, "<f4", n * K).reshape(n, K)
    _require_finite(inp, "fixture input")
    _require_finite(P, "fixture p")
    _require_finite(den, "fixture denominator")
    if np.any(P < 0) or np.any(P > 1):
        raise ValueError("fixture p outside [0,1]")
    # The reference sums each row in edge order in FP32; a pairwise FP32 sum
    # differs from it by far less than the 1e-5 relative tolerance.
    starts = row[:-1].astype(np.int64)
    nonempty = row[1:] > row[:-1]
    sums = np.zeros((n, K), np.float32)
    if e:
        sums[nonempty] = np.add.reduceat(P, starts[nonempty], axis=0)
    bad = np.abs(sums - den) > np.float32(1e-5) * np.maximum(np.float32(1), sums)
    bad |= nonempty[:, None] & (den <= 0)
    if bad.any():
        raise ValueError("fixture denominator mismatch")
    return dict(input=inp, p=P, den=den)
