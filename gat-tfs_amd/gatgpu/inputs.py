"""Seeded synthetic graphs, features and weights (ctypes over libgathost.so).

The named workloads are the benchmark and parity configurations of this
project: the 1024-node smoke graph, the arxiv-sized power-law graph (169,343
nodes / 2,484,941 CSR entries, max in-degree 13,162 as the reference's arxiv
logs report), the 64M-edge power-law graph and the R-MAT skew graph.  Every
graph is a destination-row CSR with one self-loop per node.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import PKG_ROOT

HOSTLIB_PATH = PKG_ROOT / "lib" / "libgathost.so"
_H = None


def hostlib():
    global _H
    if _H is None:
        if not HOSTLIB_PATH.exists():
            raise FileNotFoundError(f"{HOSTLIB_PATH} is not built; run `make -C {PKG_ROOT}`")
        H = ctypes.CDLL(str(HOSTLIB_PATH))
        P, u64, u32, i32, f64 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_double
        H.gathost_uniform_rows.argtypes = [u64, u32, u64, P]
        H.gathost_uniform_rows.restype = u64
        H.gathost_powerlaw_rows.argtypes = [u64, u64, u32, u64, P]
        H.gathost_powerlaw_rows.restype = u64
        H.gathost_fill_sources.argtypes = [u64, P, u64, P]
        H.gathost_rmat.argtypes = [i32, u64, f64, f64, f64, u64, P, P]
        H.gathost_rmat.restype = u64
        H.gathost_normal.argtypes = [u64, u64, P]
        H.gathost_glorot_param.argtypes = [i32, i32, i32, u64, P, P, P]
        H.gathost_random_param.argtypes = [i32, i32, i32, i32, P, P, P]
        _H = H
    return _H


def uniform_graph(n, mean_degree, seed):
    row = np.empty(n + 1, np.uint64)
    e = hostlib().gathost_uniform_rows(n, mean_degree, seed, row.ctypes.data)
    col = np.empty(e, np.uint32)
    hostlib().gathost_fill_sources(n, row.ctypes.data, seed, col.ctypes.data)
    return row, col


def powerlaw_graph(n, edges, max_degree, seed):
    row = np.empty(n + 1, np.uint64)
    e = hostlib().gathost_powerlaw_rows(n, edges, max_degree, seed, row.ctypes.data)
    if e != edges:
        raise ValueError("infeasible power-law request")
    col = np.empty(e, np.uint32)
    hostlib().gathost_fill_sources(n, row.ctypes.data, seed, col.ctypes.data)
    return row, col


def rmat_graph(scale, edges, a, b, c, seed):
    n = 1 << scale
    row = np.empty(n + 1, np.uint64)
    e = hostlib().gathost_rmat(scale, edges, a, b, c, seed, row.ctypes.data, None)
    col = np.empty(e, np.uint32)
    hostlib().gathost_rmat(scale, edges, a, b, c, seed, row.ctypes.data, col.ctypes.data)
    return row, col


def normal(shape, seed):
    out = np.empty(shape, np.float32)
    hostlib().gathost_normal(out.size, seed, out.ctypes.data)
    return out


def glorot_param(din, heads, dim, seed):
    w = np.empty((din, heads * dim), np.float32)
    al = np.empty(heads * dim, np.float32)
    ar = np.empty(heads * dim, np.float32)
    hostlib().gathost_glorot_param(din, heads, dim, seed, w.ctypes.data, al.ctypes.data, ar.ctypes.data)
    return {"in": din, "heads": heads, "dim": dim, "w": w, "al": al, "ar": ar}


def random_param(din, heads, dim, rng_seed):
    w = np.empty((din, heads * dim), np.float32)
    al = np.empty(heads * dim, np.float32)
    ar = np.empty(heads * dim, np.float32)
    hostlib().gathost_random_param(din, heads, dim, rng_seed, w.ctypes.data, al.ctypes.data, ar.ctypes.data)
    return {"in": din, "heads": heads, "dim": dim, "w": w, "al": al, "ar": ar}


def model_dims(din, hidden_heads, hidden_dim, classes):
    """Layer shapes D_in -> K x d -> K x d -> 1 x C."""
    w = hidden_heads * hidden_dim
    return [(din, hidden_heads, hidden_dim), (w, hidden_heads, hidden_dim), (w, 1, classes)]


def glorot_model(din, hidden_heads, hidden_dim, classes, seed):
    return [glorot_param(i, k, d, seed + 11 * l)
            for l, (i, k, d) in enumerate(model_dims(din, hidden_heads, hidden_dim, classes))]


def random_model(din, classes, seed):
    """random_model (baseline/src/common.cpp:50-62): seeds seed+11*layer."""
    return [random_param(din if l == 0 else 256, 8 if l < 2 else 1, 32 if l < 2 else classes, seed + 11 * l)
            for l in range(3)]


@dataclass(frozen=True)
class Workload:
    name: str
    kind: str            # "uniform" | "powerlaw" | "rmat"
    n: int
    edges: int           # CSR entries incl. self-loops (powerlaw), drawn edges (rmat), mean degree (uniform)
    max_degree: int
    din: int
    heads: int
    dim: int
    classes: int
    seed: int = 11

    def graph(self):
        if self.kind == "uniform":
            return uniform_graph(self.n, self.edges, self.seed)
        if self.kind == "powerlaw":
            return powerlaw_graph(self.n, self.edges, self.max_degree, self.seed)
        scale = self.n.bit_length() - 1
        return rmat_graph(scale, self.edges, 0.57, 0.19, 0.19, self.seed)

    def features(self):
        return normal((self.n, self.din), self.seed + 1)

    def model(self):
        return glorot_model(self.din, self.heads, self.dim, self.classes, self.seed + 2)


WORKLOADS = {
    # 3-layer 128 -> 8x32 -> 8x32 -> 1x40 on a 1024-node uniform graph, mean in-degree 16.
    "smoke": Workload("smoke", "uniform", 1024, 16, 0, 128, 8, 32, 40),
    # 169,343 nodes / 2,484,941 CSR entries, Zipf-like in-degree, max 13,162.
    "arxiv": Workload("arxiv", "powerlaw", 169_343, 2_484_941, 13_162, 128, 8, 32, 40),
    # 2,449,029 nodes / 64.3M CSR entries (mean ~26), max in-degree 17,000.
    "large": Workload("large", "powerlaw", 2_449_029, 64_300_000, 17_000, 100, 8, 32, 47),
    # R-MAT (0.57, 0.19, 0.19, 0.05), 2^22 nodes, 100M drawn edges + self-loops, deduplicated.
    "skew": Workload("skew", "rmat", 1 << 22, 100_000_000, 0, 128, 8, 64, 64),
}
