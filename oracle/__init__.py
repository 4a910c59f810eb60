"""CPU oracle for the three-layer GAT forward -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package, and only as the checker or the timed CPU baseline.
The product (``gat-tfs_amd/``) never imports it.

The numerical work lives in ``gat_oracle.cpp`` (built by ``oracle/Makefile``
into ``liboracle_v3.so`` / ``liboracle_v4.so``); this module loads it with
ctypes and adds the file formats and an FP64 NumPy restatement of the
reference's independent oracle (baseline/tests/oracle.py).
"""
from __future__ import annotations

import ctypes
import struct
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB = None


def _cpu_has_avx512() -> bool:
    try:
        flags = Path("/proc/cpuinfo").read_text().split("flags")[1].split("\n")[0].split()
    except (OSError, IndexError):
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512cd"))


def build() -> None:
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    """Load the oracle library (v4 = AVX-512 build when the host supports it)."""
    global _LIB
    if _LIB is None:
        name = "liboracle_v4.so" if _cpu_has_avx512() else "liboracle_v3.so"
        path = HERE / name
        if not path.exists():
            build()
        L = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        u64, i32 = ctypes.c_uint64, ctypes.c_int
        L.or_rne.argtypes = [P, P, u64]
        L.or_exp_cw.argtypes = [ctypes.c_float]
        L.or_exp_cw.restype = ctypes.c_float
        L.or_expm1_neg.argtypes = [ctypes.c_float]
        L.or_expm1_neg.restype = ctypes.c_float
        L.or_random_param.argtypes = [i32, i32, i32, i32, P, P, P]
        L.or_boundary_param.argtypes = [i32, i32, i32, P, P, P]
        L.or_boundary_features.argtypes = [u64, P]
        L.or_ref_layer.argtypes = [u64, P, P, P, i32, i32, i32, P, P, P, i32] + [P] * 9
        L.or_fp64_layer.argtypes = [u64, P, P, P, i32, i32, i32, P, P, P, i32] + [P] * 6
        L.or_standard_layer.argtypes = [u64, P, P, P, i32, i32, i32, P, P, P, i32, i32, i32] + [P] * 8
        L.or_fixed_p_layer.argtypes = [u64, P, P, P, i32, i32, i32, P, P, P, i32, P, P]
        L.or_b1_layer.argtypes = [u64, P, P, P, i32, i32, i32, P, P, P, i32, P]
        L.or_degree_schedule.argtypes = [u64, P, P, P]
        L.or_permute_csr.argtypes = [u64, P, P, P, P, P]
        L.or_choose_R.argtypes = [u64, u64, P]
        L.or_choose_R.restype = i32
        L.or_errors.argtypes = [P, P, u64, P]
        L.or_errors.restype = i32
        L.or_max_threads.restype = i32
        _LIB = L
    return _LIB


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ----------------------------------------------------------------- formats
def save_graph(path, row, col, x, classes):
    """GATBIN1 writer: baseline/src/common.cpp:40-44."""
    row = np.ascontiguousarray(row, dtype="<u8")
    col = np.ascontiguousarray(col, dtype="<u4")
    x = np.ascontiguousarray(x, dtype="<f4")
    n, din = x.shape
    with open(path, "wb") as f:
        f.write(b"GATBIN1\0")
        f.write(struct.pack("<QQII", n, col.size, din, classes))
        f.write(row.tobytes())
        f.write(col.tobytes())
        f.write(x.tobytes())


def load_graph(path):
    """GATBIN1 reader: baseline/src/common.cpp:31-39, baseline/tests/oracle.py:12-17."""
    with open(path, "rb") as f:
        magic = f.read(8)
        if not magic.startswith(b"GATBIN1"):
            raise ValueError("bad graph magic")
        n, e, din, classes = struct.unpack("<QQII", f.read(24))
        row = np.fromfile(f, dtype="<u8", count=n + 1)
        col = np.fromfile(f, dtype="<u4", count=e)
        x = np.fromfile(f, dtype="<f4", count=n * din).reshape(n, din)
    if row.size != n + 1 or col.size != e or x.size != n * din:
        raise ValueError("truncated file")
    return dict(n=n, e=e, din=din, classes=classes, row=row, col=col, x=x)


def save_model(path, model):
    """GATWGT1 writer: baseline/src/common.cpp:63-68."""
    with open(path, "wb") as f:
        f.write(b"GATWGT1\0")
        f.write(struct.pack("<I", len(model)))
        for p in model:
            f.write(struct.pack("<III", p["in"], p["heads"], p["dim"]))
            for k in ("w", "al", "ar"):
                f.write(np.ascontiguousarray(p[k], dtype="<f4").tobytes())


def load_model(path):
    """GATWGT1 reader: baseline/src/common.cpp:69-79, baseline/tests/oracle.py:18-27."""
    with open(path, "rb") as f:
        if not f.read(8).startswith(b"GATWGT1"):
            raise ValueError("bad weights magic")
        (count,) = struct.unpack("<I", f.read(4))
        model = []
        for _ in range(count):
            din, heads, dim = struct.unpack("<III", f.read(12))
            w = np.fromfile(f, dtype="<f4", count=din * heads * dim).reshape(din, heads * dim)
            al = np.fromfile(f, dtype="<f4", count=heads * dim)
            ar = np.fromfile(f, dtype="<f4", count=heads * dim)
            model.append({"in": din, "heads": heads, "dim": dim, "w": w, "al": al, "ar": ar})
    return model


# ----------------------------------------------------------------- weights and test graphs
def random_param(din, heads, dim, rng_seed):
    w = np.empty((din, heads * dim), np.float32)
    al = np.empty(heads * dim, np.float32)
    ar = np.empty(heads * dim, np.float32)
    lib().or_random_param(din, heads, dim, rng_seed, _p(w), _p(al), _p(ar))
    return {"in": din, "heads": heads, "dim": dim, "w": w, "al": al, "ar": ar}


def random_model(din, classes, seed):
    """random_model: baseline/src/common.cpp:50-62 (layer seeds seed+11*layer)."""
    return [random_param(din if l == 0 else 256, 8 if l < 2 else 1, 32 if l < 2 else classes, seed + 11 * l)
            for l in range(3)]


def boundary_param(D, K, d):
    w = np.empty((D, K * d), np.float32)
    al = np.empty(K * d, np.float32)
    ar = np.empty(K * d, np.float32)
    lib().or_boundary_param(D, K, d, _p(w), _p(al), _p(ar))
    return {"in": D, "heads": K, "dim": d, "w": w, "al": al, "ar": ar}


def boundary_graph(D):
    """The 35-node degree-edge-case graph of baseline/tests/boundaries.cpp:10-14."""
    degs = [0, 1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 129]
    n = 35
    row = [0]
    col = []
    for i in range(n):
        c = degs[i % 13]
        col.extend((i * 3 + e * 7) % n for e in range(c))
        row.append(len(col))
    x = np.empty((n, D), np.float32)
    lib().or_boundary_features(n * D, _p(x))
    return dict(n=n, e=len(col), din=D, classes=40, row=np.array(row, np.uint64),
                col=np.array(col, np.uint32), x=x)


# ----------------------------------------------------------------- layer oracles
def _graph_args(row, col):
    row = np.ascontiguousarray(row, np.uint64)
    col = np.ascontiguousarray(col, np.uint32)
    return row, col


def ref_layer(row, col, x, p, hidden, edge_stages=False):
    """R0 FP32 layer (baseline/src/ref_fp32.cpp:3-26) -> dict of stage arrays."""
    row, col = _graph_args(row, col)
    x = np.ascontiguousarray(x, np.float32)
    n = row.size - 1
    K, W = p["heads"], p["heads"] * p["dim"]
    out = {k: np.empty((n, W), np.float32) for k in ("z", "out")}
    for k in ("left", "right", "max", "den"):
        out[k] = np.empty((n, K), np.float32)
    for k in ("score", "p", "alpha"):
        out[k] = np.empty((col.size, K), np.float32) if edge_stages else None
    lib().or_ref_layer(n, _p(row), _p(col), _p(x), p["in"], K, p["dim"], _p(p["w"]), _p(p["al"]), _p(p["ar"]),
                       int(hidden), _p(out["z"]), _p(out["left"]), _p(out["right"]), _p(out["max"]),
                       _p(out["den"]), _p(out["score"]), _p(out["p"]), _p(out["alpha"]), _p(out["out"]))
    return out


def fp64_layer(row, col, x, p, hidden):
    """Independent FP64 layer (baseline/tests/boundaries.cpp:15-21)."""
    row, col = _graph_args(row, col)
    x = np.ascontiguousarray(x, np.float32)
    n = row.size - 1
    K, W = p["heads"], p["heads"] * p["dim"]
    o = {k: np.empty((n, W), np.float64) for k in ("z", "out")}
    for k in ("left", "right", "max", "den"):
        o[k] = np.empty((n, K), np.float64)
    lib().or_fp64_layer(n, _p(row), _p(col), _p(x), p["in"], K, p["dim"], _p(p["w"]), _p(p["al"]), _p(p["ar"]),
                        int(hidden), _p(o["z"]), _p(o["left"]), _p(o["right"]), _p(o["max"]), _p(o["den"]),
                        _p(o["out"]))
    return o


def quantize_bf16(a):
    """FP32 values rounded to bf16 (RNE) and widened back (common.cpp:80-93, quantized())."""
    a = np.ascontiguousarray(a, np.float32)
    bits = np.empty(a.shape, np.uint16)
    lib().or_rne(_p(a), _p(bits), a.size)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def rne_bits(a):
    a = np.ascontiguousarray(a, np.float32)
    bits = np.empty(a.shape, np.uint16)
    lib().or_rne(_p(a), _p(bits), a.size)
    return bits


def standard_workspace(n, p):
    """Stage buffers of one B0 layer, allocated and touched once (the
    Workspace::allocate of baseline/src/common.cpp:126-134, outside timing)."""
    K, W = p["heads"], p["heads"] * p["dim"]
    ws = {"z": np.zeros((n, W), np.float32), "out": np.zeros((n, W), np.float32),
          "xq": np.zeros((n, p["in"]), np.float32)}
    for k in ("left", "right", "max", "den"):
        ws[k] = np.zeros((n, K), np.float32)
    return ws


def standard_layer(row, col, x, p, hidden, bf16, threads=0, wq=None, ws=None):
    """B0 strong standard layer (baseline/src/baseline_standard.cpp:98-108).

    Returns (stages, times_ms) with times = convert, projection, lr,
    max_prescan, aggregate, finish, total.  ``wq`` is the bf16-rounded W
    (prepared outside the timer, like prepare() in common.cpp:97-119); ``ws``
    a standard_workspace() reused across calls.
    """
    row, col = _graph_args(row, col)
    x = np.ascontiguousarray(x, np.float32)
    n = row.size - 1
    w = p["w"]
    if bf16:
        w = quantize_bf16(w) if wq is None else wq
    st = ws if ws is not None else standard_workspace(n, p)
    t = np.zeros(7, np.float64)
    lib().or_standard_layer(n, _p(row), _p(col), _p(x), p["in"], p["heads"], p["dim"],
                            _p(np.ascontiguousarray(w, np.float32)), _p(p["al"]), _p(p["ar"]), int(hidden),
                            int(bf16), int(threads), _p(st["xq"]), _p(st["z"]), _p(st["left"]), _p(st["right"]),
                            _p(st["max"]), _p(st["den"]), _p(st["out"]), _p(t))
    return st, t


def fixed_p_layer(row, col, x, p, P, den, bf16):
    """Fixed-p operator (baseline/bench/main.cpp:103-150): Z = XW (bf16-rounded
    X and W with FP32 Z when bf16, else FP32), out = sum_e P[e] Z[col[e]] / den.
    P [e][heads] in CSR edge order, den [n][heads] -> dict(z, out)."""
    row, col = _graph_args(row, col)
    x = np.ascontiguousarray(x, np.float32)
    P = np.ascontiguousarray(P, np.float32)
    den = np.ascontiguousarray(den, np.float32)
    n = row.size - 1
    W = p["heads"] * p["dim"]
    o = {k: np.empty((n, W), np.float32) for k in ("z", "out")}
    lib().or_fixed_p_layer(n, _p(row), _p(col), _p(x), p["in"], p["heads"], p["dim"], _p(p["w"]), _p(P), _p(den),
                           int(bool(bf16)), _p(o["z"]), _p(o["out"]))
    return o


def b1_layer(row, col, xq, p, wq, P, den, hidden):
    """Neighbour-step TFS with bf16-rounded p x (baseline/src/baseline_tfs.cpp:16-110;
    emulation of baseline/bench/main.cpp:139-143).  xq, wq: bf16-rounded FP32;
    P [e][heads], den [n][heads] -> out [n][heads*dim]."""
    row, col = _graph_args(row, col)
    xq = np.ascontiguousarray(xq, np.float32)
    wq = np.ascontiguousarray(wq, np.float32)
    P = np.ascontiguousarray(P, np.float32)
    den = np.ascontiguousarray(den, np.float32)
    n = row.size - 1
    out = np.empty((n, p["heads"] * p["dim"]), np.float32)
    lib().or_b1_layer(n, _p(row), _p(col), _p(xq), p["in"], p["heads"], p["dim"], _p(wq), _p(P), _p(den),
                      int(bool(hidden)), _p(out))
    return out


def ref_model(row, col, x, model):
    """Three R0 layers chained on their own outputs (bench/main.cpp:87-88)."""
    stages = []
    h = x
    for l, p in enumerate(model):
        s = ref_layer(row, col, h, p, hidden=l < 2)
        stages.append(s)
        h = s["out"]
    return stages


# ----------------------------------------------------------------- schedule and metrics
def degree_schedule(row):
    row = np.ascontiguousarray(row, np.uint64)
    n = row.size - 1
    perm = np.empty(n, np.uint32)
    steps = np.zeros(1, np.uint64)
    lib().or_degree_schedule(n, _p(row), _p(perm), _p(steps))
    return perm, int(steps[0])


def permute_csr(row, col, perm):
    row, col = _graph_args(row, col)
    n = row.size - 1
    prow = np.empty(n + 1, np.uint64)
    pcol = np.empty(col.size, np.uint32)
    lib().or_permute_csr(n, _p(row), _p(col), _p(np.ascontiguousarray(perm, np.uint32)), _p(prow), _p(pcol))
    return prow, pcol


def choose_R(row):
    row = np.ascontiguousarray(row, np.uint64)
    return int(lib().or_choose_R(row.size - 1, int(row[-1]), _p(row)))


ERROR_KEYS = ("max_abs", "mean_abs", "relative_l2", "rmse", "p50", "p90", "p99")


def errors(ref, got):
    """errors(): baseline/src/common.cpp:141-150 -> dict (+ 'finite')."""
    ref = np.ascontiguousarray(ref, np.float32).ravel()
    got = np.ascontiguousarray(got, np.float32).ravel()
    if ref.size == 0 or ref.size != got.size:
        raise ValueError("comparison size mismatch")
    o = np.zeros(7, np.float64)
    fin = lib().or_errors(_p(ref), _p(got), ref.size, _p(o))
    d = dict(zip(ERROR_KEYS, o.tolist()))
    d["finite"] = bool(fin)
    return d


# ----------------------------------------------------------------- NumPy FP64 three-layer oracle
def numpy_fp64_layer(row, col, x, p, hidden):
    """FP64 NumPy layer restating baseline/tests/oracle.py:28-54 (vectorised
    per head over all edges instead of a Python row loop)."""
    row = np.asarray(row, np.int64)
    col = np.asarray(col, np.int64)
    n = row.size - 1
    K, d = p["heads"], p["dim"]
    w = np.asarray(p["w"], np.float64)
    al = np.asarray(p["al"], np.float64).reshape(K, d)
    ar = np.asarray(p["ar"], np.float64).reshape(K, d)
    z = (np.asarray(x, np.float64) @ w).reshape(n, K, d)
    left = np.einsum("nhd,hd->nh", z, al)
    right = np.einsum("nhd,hd->nh", z, ar)
    dst = np.repeat(np.arange(n), np.diff(row))
    score = left[dst] + right[col]
    score = np.where(score >= 0, score, 0.2 * score)
    mx = np.full((n, K), -np.inf)
    np.maximum.at(mx, dst, score)
    deg = np.diff(row)
    mx[deg == 0] = 0.0
    pe = np.exp(score - mx[dst])
    den = np.zeros((n, K))
    np.add.at(den, dst, pe)
    alpha = pe / den[dst]
    out = np.zeros((n, K, d))
    np.add.at(out, dst, alpha[:, :, None] * z[col])
    if hidden:
        out = np.where(out >= 0, out, np.expm1(np.minimum(out, 0)))
    return dict(z=z.reshape(n, K * d), left=left, right=right, max=mx, den=den, score=score, p=pe,
                alpha=alpha, out=out.reshape(n, K * d))
