"""Full-size parity of the three-layer forward with the R0 oracle.

The 64.3M-edge power-law graph (2,449,029 nodes, max in-degree 17,000,
100 -> 8x32 -> 8x32 -> 1x47) is the benchmark workload.  Its logits are
compared with the oracle's R0 chain (baseline/src/ref_fp32.cpp:3-26, three
layers each consuming its own previous output as baseline/bench/main.cpp:87-98
chains them): bf16 path within relative L2 1e-2, FP32 path within max-abs
1e-4.  Each layer's output is compared too, and layers 2 and 3 are checked
row by row against a float64 evaluation of the exact-max softmax over the
GPU's own stages on sampled rows (the heaviest included).

The R-MAT graph (2^22 nodes, 100.6M edges, 128 -> 8x64 -> 8x64 -> 1x64) gets
the same R0 check of every layer for its bf16 and FP32 forwards.
"""
import numpy as np
import pytest

import gatgpu
import oracle
from gatgpu import inputs

pytestmark = pytest.mark.gpu

FP32_MAX_ABS = 1e-4
BF16_REL_L2 = 1e-2


def r0_chain(row, col, x, model):
    """Outputs of the three R0 layers, each fed the previous R0 output."""
    outs = []
    h = x
    for l, p in enumerate(model):
        h = oracle.ref_layer(row, col, h, p, hidden=l < 2)["out"]
        outs.append(h)
    return outs


def b0_chain(row, col, x, model):
    """Outputs of the oracle's B0 standard_bf16 chain (baseline_standard.cpp:98-108)."""
    outs = []
    h = x
    for l, p in enumerate(model):
        st, _ = oracle.standard_layer(row, col, h, p, l < 2, True)
        h = st["out"].copy()
        outs.append(h)
    return outs


@pytest.fixture(scope="module")
def large():
    w = inputs.WORKLOADS["large"]
    row, col = w.graph()
    x = w.features()
    m = w.model()
    return dict(w=w, row=row, col=col, x=x, m=m, r0=r0_chain(row, col, x, m))


def forward(ctx, g, precision, dataflow=gatgpu.AUTO):
    ctx.set_graph(g["row"], g["col"])
    ctx.set_model(g["m"])
    ctx.set_input(g["x"])
    logits, _, _ = ctx.model_forward(precision, dataflow)
    return logits


def report(tag, layer, e):
    print(f"{tag} layer={layer} rel_l2={e['relative_l2']:.6g} max_abs={e['max_abs']:.6g} "
          f"mean_abs={e['mean_abs']:.6g} p99={e['p99']:.6g}", flush=True)


def test_large_bf16_logits_vs_r0(gpu_ctx, large):
    """The benchmark forward (AUTO: layer 1 aggregate-first, layers 2-3
    transform-first) within relative L2 1e-2 of R0, end to end and per layer
    (each layer chained on its own path's previous output; layer 2's output
    is stored when the output projection is not fused into its aggregation).
    The benchmark's fused forward gives the same logits bit for bit.  The
    oracle's B0 standard_bf16 chain is printed beside it for scale."""
    gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 0)
    try:
        logits = forward(gpu_ctx, large, gatgpu.BF16)
    finally:
        gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 1)
    assert gpu_ctx.stage(0, "z") is None  # layer 1 ran aggregate-first
    b0 = b0_chain(large["row"], large["col"], large["x"], large["m"])
    for l in range(3):
        got = logits if l == 2 else gpu_ctx.stage(l, "out")
        e = oracle.errors(large["r0"][l], got)
        report("large_bf16_gpu_vs_r0", l + 1, e)
        report("large_bf16_b0_vs_r0", l + 1, oracle.errors(large["r0"][l], b0[l]))
        assert e["finite"] and e["relative_l2"] < BF16_REL_L2, (l, e)
    assert np.array_equal(logits, gpu_ctx.stage(2, "out"))
    fused, _, _ = gpu_ctx.model_forward(gatgpu.BF16, gatgpu.AUTO)
    assert gpu_ctx.stage(1, "out") is None  # the output projection ran in layer 2's aggregation
    assert np.array_equal(fused, logits)


def test_large_fp32_logits_vs_r0(gpu_ctx, large):
    """FP32 path (FP32 MFMA projections, FP32 Z and softmax state) within
    max-abs 1e-4 of R0 for every layer and the logits."""
    logits = forward(gpu_ctx, large, gatgpu.FP32)
    for l in range(3):
        got = logits if l == 2 else gpu_ctx.stage(l, "out")
        e = oracle.errors(large["r0"][l], got)
        report("large_fp32_gpu_vs_r0", l + 1, e)
        assert e["finite"] and e["max_abs"] < FP32_MAX_ABS, (l, e)


def check_tf_layer_rows(ctx, layer, hidden, p, row, col, rows):
    """Transform-first bf16 layer on sampled rows: the row max equals the
    scalar max of LeakyReLU(L + R) over the GPU's own L/R bit for bit, the
    denominator a float64 sum of p, and the output the float64
    sum_j p Z_j / den over the GPU's own bf16 Z rows (FP32 summation error,
    plus one bf16 rounding of hidden outputs)."""
    K, d = p["heads"], p["dim"]
    Z = ctx.stage(layer, "z").astype(np.float64)
    L, R = ctx.stage(layer, "left"), ctx.stage(layer, "right")
    M, den, out = ctx.stage(layer, "max"), ctx.stage(layer, "den"), ctx.stage(layer, "out")
    for i in rows:
        js = col[int(row[i]):int(row[i + 1])].astype(np.int64)
        s = L[i][None, :] + R[js]
        s = np.where(s >= 0, s, np.float32(0.2) * s).astype(np.float32)
        assert np.array_equal(M[i], s.max(axis=0)), (layer, i)
        pe = np.exp(s.astype(np.float64) - M[i].astype(np.float64))
        dsum = pe.sum(axis=0)
        assert np.all(np.abs(den[i] - dsum) <= 1e-5 * dsum), (layer, i)
        zj = Z[js][:, :K * d].reshape(len(js), K, d)
        y = (np.einsum("jh,jhc->hc", pe, zj) / dsum[:, None]).reshape(-1)
        mag = (np.einsum("jh,jhc->hc", pe, np.abs(zj)) / dsum[:, None]).reshape(-1)
        if hidden:
            y = np.where(y >= 0, y, np.expm1(y))
        tol = (np.abs(y) * 2.0 ** -8 if hidden else 0.0) + 1e-4 * mag + 1e-6
        assert np.all(np.abs(out[i] - y) <= tol), (layer, i, np.max(np.abs(out[i] - y) - tol))


def test_large_layers_2_3_sampled_rows(gpu_ctx, large):
    """Layers 2 (8 x 32, R formed from the bf16 Z row) and 3 (one head of 47,
    R carried in the Z row, logits written to original rows) of the benchmark
    forward, on 2000 sampled rows plus the 64 heaviest (split into chunks)."""
    gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 0)  # layer 2 stores its output rows
    try:
        forward(gpu_ctx, large, gatgpu.BF16)
    finally:
        gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 1)
    row, col = large["row"], large["col"]
    deg = np.diff(row.astype(np.int64))
    rng = np.random.default_rng(11)
    rows = np.concatenate((rng.choice(large["w"].n, 2000, replace=False), np.argsort(deg)[-64:]))
    for layer, hidden in ((1, True), (2, False)):
        check_tf_layer_rows(gpu_ctx, layer, hidden, large["m"][layer], row, col, rows)


@pytest.fixture(scope="module")
def skew():
    w = inputs.WORKLOADS["skew"]
    row, col = w.graph()
    x = w.features()
    m = w.model()
    return dict(w=w, row=row, col=col, x=x, m=m, r0=r0_chain(row, col, x, m))


def test_skew_bf16_logits_vs_r0(gpu_ctx, skew):
    """R-MAT forward (layer 1 aggregate-first with heads of 64, layers 2-3
    transform-first, 9 109 split rows, 3.0M rows of at most 4 edges) within
    relative L2 1e-2 of R0."""
    logits = forward(gpu_ctx, skew, gatgpu.BF16)
    for l, h in enumerate(skew["r0"]):
        got = logits if l == 2 else gpu_ctx.stage(l, "out")
        e = oracle.errors(h, got)
        report("skew_bf16_gpu_vs_r0", l + 1, e)
        assert e["finite"] and e["relative_l2"] < BF16_REL_L2, (l, e)


def test_skew_fp32_logits_vs_r0(gpu_ctx, skew):
    """R-MAT FP32 forward (FP32 MFMA projections, 8 x 64 FP32 rows, the
    one-head output layer; every layer transform-first) within max-abs 1e-4 of
    R0 on every layer, as the 64.3M-edge graph's."""
    logits = forward(gpu_ctx, skew, gatgpu.FP32)
    for l, h in enumerate(skew["r0"]):
        got = logits if l == 2 else gpu_ctx.stage(l, "out")
        e = oracle.errors(h, got)
        report("skew_fp32_gpu_vs_r0", l + 1, e)
        assert e["finite"] and e["max_abs"] < FP32_MAX_ABS, (l, e)
