"""Python binding of libgatgpu (the gfx950 GAT forward) over its C ABI.

The binding is a thin ctypes layer over ``include/gatgpu.h``: host arrays are
NumPy, every device buffer is owned by the library context.  There is no
fallback: if ``lib/libgatgpu.so`` is missing or no gfx950 device is present,
the calls raise.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG_ROOT = Path(__file__).resolve().parent.parent  # gat-tfs_amd/
LIB_PATH = PKG_ROOT / "lib" / "libgatgpu.so"

OK, EINVAL, ESTATE, ENODEV, ENOMEM, EDEVICE, ENONFINITE, EOVERFLOW = 0, -1, -2, -3, -4, -5, -6, -7
FP32, BF16 = 0, 1
AUTO, TRANSFORM_FIRST, AGGREGATE_FIRST, TFS_B1 = 0, 1, 2, 3
STAGE_Z, STAGE_LEFT, STAGE_RIGHT, STAGE_MAX, STAGE_DEN, STAGE_OUT, STAGE_XBF = range(7)
OPT_BLOCK_ROW_MIN_DEGREE, OPT_SPLIT_ROW_MIN_DEGREE, OPT_SPLIT_CHUNK_EDGES, OPT_KEEP_INPUT_BF16 = 1, 2, 3, 5
OPT_FUSE_NEXT_PROJECTION = 6

STATIC_SCRATCH_BYTES = 64 << 20  # GATGPU_STATIC_SCRATCH_BYTES

STAGE_NAMES = {"z": STAGE_Z, "left": STAGE_LEFT, "right": STAGE_RIGHT, "max": STAGE_MAX,
               "den": STAGE_DEN, "out": STAGE_OUT, "xbf": STAGE_XBF}

# Every symbol include/gatgpu.h declares.
EXPORTS = (
    "gatgpu_create", "gatgpu_destroy", "gatgpu_last_error", "gatgpu_set_graph", "gatgpu_set_layer",
    "gatgpu_set_input", "gatgpu_degree_schedule", "gatgpu_permuted_csr", "gatgpu_choose_R",
    "gatgpu_layer_forward", "gatgpu_model_forward", "gatgpu_get_stage", "gatgpu_stage_size",
    "gatgpu_set_option", "gatgpu_synchronize", "gatgpu_stream", "gatgpu_set_fixed_p", "gatgpu_fixed_p_forward",
    "gatgpu_get_static_times", "gatgpu_validate_graph", "gatgpu_layer_forward_static",
    "gatgpu_static_scratch_need",
)


class Times(ctypes.Structure):
    """gatgpu_times (field names of gat::Times, baseline/include/gat.hpp:68-76)."""
    _fields_ = [(name, ctypes.c_double) for name in (
        "convert_ms", "projection_ms", "lr_ms", "max_prescan_ms", "aggregate_ms", "normalize_ms",
        "activation_ms", "total_ms")]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


class StaticTimes(ctypes.Structure):
    """gatgpu_static_times: wall times (ms) of the static, untimed steps."""
    _fields_ = [(name, ctypes.c_double) for name in (
        "graph_check_ms", "graph_h2d_ms", "degree_sort_ms", "model_prepare_ms", "input_h2d_ms",
        "input_permute_ms", "logits_d2h_ms")]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


class GatGpuError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"gatgpu error {code}: {msg}")
        self.code = code


_LIB = None


def load_library(path: os.PathLike | None = None):
    """Loads libgatgpu.so (raises if it has not been built)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built; run `make -C {PKG_ROOT}` (or __graft_entry__.build())")
    L = ctypes.CDLL(str(p))
    P, u64, i32, i64 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int64
    L.gatgpu_create.argtypes = [i32, ctypes.POINTER(P)]
    L.gatgpu_destroy.argtypes = [P]
    L.gatgpu_last_error.argtypes = [P]
    L.gatgpu_last_error.restype = ctypes.c_char_p
    L.gatgpu_set_graph.argtypes = [P, u64, u64, P, P]
    L.gatgpu_set_layer.argtypes = [P, i32, i32, i32, i32, P, P, P]
    L.gatgpu_set_input.argtypes = [P, u64, i32, P]
    L.gatgpu_degree_schedule.argtypes = [P, P, P]
    L.gatgpu_permuted_csr.argtypes = [P, P, P]
    L.gatgpu_choose_R.argtypes = [P, ctypes.POINTER(i32)]
    L.gatgpu_layer_forward.argtypes = [P, i32, i32, i32, i32, P, P]
    L.gatgpu_model_forward.argtypes = [P, i32, i32, P, P, ctypes.POINTER(ctypes.c_double)]
    L.gatgpu_get_stage.argtypes = [P, i32, i32, P]
    L.gatgpu_stage_size.argtypes = [P, i32, i32, ctypes.POINTER(u64)]
    L.gatgpu_set_option.argtypes = [P, i32, i64]
    L.gatgpu_synchronize.argtypes = [P]
    L.gatgpu_stream.argtypes = [P]
    L.gatgpu_set_fixed_p.argtypes = [P, i32, P, P]
    L.gatgpu_fixed_p_forward.argtypes = [P, i32, i32, i32, P, P]
    L.gatgpu_stream.restype = P
    L.gatgpu_get_static_times.argtypes = [P, ctypes.POINTER(StaticTimes)]
    L.gatgpu_validate_graph.argtypes = [u64, u64, P, P]
    L.gatgpu_layer_forward_static.argtypes = [P, i32, i32, i32, P, P]
    L.gatgpu_static_scratch_need.argtypes = [P, i32, i32, i32, ctypes.POINTER(u64)]
    for name in EXPORTS:
        if name not in ("gatgpu_last_error", "gatgpu_stream"):
            getattr(L, name).restype = i32
    if path is None:
        _LIB = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data


def validate_graph(row, col, n=None, e=None):
    """gatgpu_validate_graph: raises GatGpuError for a CSR set_graph would
    reject (no device needed).  n and e default to the arrays' sizes."""
    L = load_library()
    row = np.ascontiguousarray(row, np.uint64)
    col = np.ascontiguousarray(col, np.uint32)
    n = row.size - 1 if n is None else n
    e = col.size if e is None else e
    rc = L.gatgpu_validate_graph(n, e, _ptr(row), _ptr(col))
    if rc != OK:
        raise GatGpuError(rc, L.gatgpu_last_error(None).decode())


class Context:
    """One device context (gatgpu_ctx)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = ctypes.c_void_p()
        rc = self.lib.gatgpu_create(device, ctypes.byref(h))
        if rc != OK:
            raise GatGpuError(rc, self.lib.gatgpu_last_error(None).decode())
        self.h = h
        self.n = 0
        self.e = 0
        self.layers = [None, None, None]

    def _check(self, rc):
        if rc != OK:
            raise GatGpuError(rc, self.lib.gatgpu_last_error(self.h).decode())

    def close(self):
        if self.h:
            self.lib.gatgpu_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- static inputs
    def set_graph(self, row, col):
        row = np.ascontiguousarray(row, np.uint64)
        col = np.ascontiguousarray(col, np.uint32)
        n = row.size - 1
        self._check(self.lib.gatgpu_set_graph(self.h, n, col.size, _ptr(row), _ptr(col)))
        self.n, self.e = n, col.size

    def set_layer(self, layer, p):
        w = np.ascontiguousarray(p["w"], np.float32)
        al = np.ascontiguousarray(p["al"], np.float32)
        ar = np.ascontiguousarray(p["ar"], np.float32)
        self._check(self.lib.gatgpu_set_layer(self.h, layer, p["in"], p["heads"], p["dim"], _ptr(w), _ptr(al),
                                              _ptr(ar)))
        self.layers[layer] = (p["in"], p["heads"], p["dim"])

    def set_model(self, model):
        for l, p in enumerate(model):
            self.set_layer(l, p)

    def set_input(self, x):
        x = np.ascontiguousarray(x, np.float32)
        self._check(self.lib.gatgpu_set_input(self.h, x.shape[0], x.shape[1], _ptr(x)))

    def set_option(self, key, value):
        self._check(self.lib.gatgpu_set_option(self.h, key, int(value)))

    # -- schedule
    def degree_schedule(self):
        perm = np.empty(self.n, np.uint32)
        steps = np.zeros(1, np.uint64)
        self._check(self.lib.gatgpu_degree_schedule(self.h, _ptr(perm), _ptr(steps)))
        return perm, int(steps[0])

    def permuted_csr(self):
        prow = np.empty(self.n + 1, np.uint64)
        pcol = np.empty(self.e, np.uint32)
        self._check(self.lib.gatgpu_permuted_csr(self.h, _ptr(prow), _ptr(pcol)))
        return prow, pcol

    def choose_R(self):
        r = ctypes.c_int()
        self._check(self.lib.gatgpu_choose_R(self.h, ctypes.byref(r)))
        return r.value

    # -- forward
    def layer_forward(self, layer, precision=FP32, dataflow=AUTO, hidden=True, input=None):
        t = Times()
        inp = None if input is None else np.ascontiguousarray(input, np.float32)
        self._check(self.lib.gatgpu_layer_forward(self.h, layer, precision, dataflow, int(hidden), _ptr(inp),
                                                  ctypes.byref(t)))
        return t.as_dict()

    def set_fixed_p(self, layer, p, den):
        """Fixture weights for the fixed-p operator: p [e][heads] in CSR edge
        order, den [n][heads] (GATFIX1 fields, baseline/src/common.cpp:171-194)."""
        p = np.ascontiguousarray(p, np.float32)
        den = np.ascontiguousarray(den, np.float32)
        self._check(self.lib.gatgpu_set_fixed_p(self.h, layer, _ptr(p), _ptr(den)))

    def fixed_p_forward(self, layer, precision=BF16, dataflow=TRANSFORM_FIRST, input=None):
        t = Times()
        inp = None if input is None else np.ascontiguousarray(input, np.float32)
        self._check(self.lib.gatgpu_fixed_p_forward(self.h, layer, precision, dataflow, _ptr(inp), ctypes.byref(t)))
        return t.as_dict()

    def model_forward(self, precision=FP32, dataflow=AUTO, want_logits=True, timed=True, stages=True):
        """timed: the model time (HIP events, first kernel to last); stages:
        also the per-layer times, which add an event at every stage boundary."""
        logits = None
        if want_logits:
            logits = np.empty((self.n, self.layers[2][1] * self.layers[2][2]), np.float32)
        per_layer = timed and stages
        times = (Times * 3)() if per_layer else None
        total = ctypes.c_double(0.0)
        self._check(self.lib.gatgpu_model_forward(self.h, precision, dataflow, _ptr(logits),
                                                  times if per_layer else None,
                                                  ctypes.byref(total) if timed else None))
        return logits, ([t.as_dict() for t in times] if per_layer else None), total.value

    def has_stage(self, layer, which):
        """True when the last forward left this stage (gatgpu_stage_size > 0)."""
        code = STAGE_NAMES[which] if isinstance(which, str) else which
        cnt = ctypes.c_uint64()
        self._check(self.lib.gatgpu_stage_size(self.h, layer, code, ctypes.byref(cnt)))
        return cnt.value > 0

    def stage(self, layer, which):
        code = STAGE_NAMES[which] if isinstance(which, str) else which
        cnt = ctypes.c_uint64()
        self._check(self.lib.gatgpu_stage_size(self.h, layer, code, ctypes.byref(cnt)))
        if cnt.value == 0:
            return None
        out = np.empty(cnt.value, np.float32)
        self._check(self.lib.gatgpu_get_stage(self.h, layer, code, _ptr(out)))
        return out.reshape(self.n, -1)

    def layer_forward_static(self, layer, precision, hidden, x_dev, out_dev):
        """gatgpu_layer_forward_static on device pointers (ints): x [n][in],
        out [n][heads*dim], FP32, original node order.  Enqueued on the
        context's stream; call synchronize() before reading out."""
        self._check(self.lib.gatgpu_layer_forward_static(self.h, layer, precision, int(hidden), x_dev, out_dev))

    def static_scratch_need(self, layer, precision, hidden):
        b = ctypes.c_uint64()
        self._check(self.lib.gatgpu_static_scratch_need(self.h, layer, precision, int(hidden), ctypes.byref(b)))
        return b.value

    def static_times(self):
        t = StaticTimes()
        self._check(self.lib.gatgpu_get_static_times(self.h, ctypes.byref(t)))
        return t.as_dict()

    def synchronize(self):
        self._check(self.lib.gatgpu_synchronize(self.h))
