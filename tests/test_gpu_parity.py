"""Parity of the gfx950 path (through the C ABI) with the CPU oracle.

Gates: FP32 path max-abs <= 1e-4 (and rel-L2 <= 1e-4 where the reference's
boundary test uses it) against R0; bf16 path rel-L2 <= 1e-2 against R0 FP32;
the degree permutation, neighbor_steps and the permuted CSR bit-exact.
"""
import numpy as np
import pytest

import gatgpu
import oracle
from gatgpu import inputs
from make_smoke1024 import smoke1024

pytestmark = pytest.mark.gpu

FP32_MAX_ABS = 1e-4
BF16_REL_L2 = 1e-2


# 0 for the split options restores the per-kernel split plans.
DEFAULT_OPTIONS = {gatgpu.OPT_BLOCK_ROW_MIN_DEGREE: 512, gatgpu.OPT_SPLIT_ROW_MIN_DEGREE: 0,
                   gatgpu.OPT_SPLIT_CHUNK_EDGES: 0}
# Schedules that route the small graphs' rows through every kernel variant:
# default, every row a block (generic path), rows >= 16 split into 64-edge chunks.
SCHEDULES = [{}, {gatgpu.OPT_BLOCK_ROW_MIN_DEGREE: 1},
             {gatgpu.OPT_SPLIT_ROW_MIN_DEGREE: 16, gatgpu.OPT_SPLIT_CHUNK_EDGES: 64}]


def run_layer(ctx, row, col, x, p, hidden, precision, options=None, dataflow=gatgpu.TRANSFORM_FIRST):
    ctx.set_graph(row, col)
    for k, v in (options or {}).items():
        ctx.set_option(k, v)
    ctx.set_layer(0, p)
    ctx.set_input(x)
    ctx.layer_forward(0, precision, dataflow, hidden)
    out = {k: ctx.stage(0, k) for k in ("left", "right", "max", "den", "out")}
    for k in options or {}:
        ctx.set_option(k, DEFAULT_OPTIONS[k])
    return out


# ---------------------------------------------------------------- schedule
def four_digit_graph():
    """4 096 rows whose degrees need all four 8-bit digits of the radix sort:
    two rows of more than 2^24 edges that differ only in their low digit, a
    row of 2^17 + 3 and rows of 65 535, 65 536, 65 792 (0x10100) and twice
    70 000 (equal degrees: ascending ids), among rows of 0..23 edges.  About
    34M edges, sources uniform."""
    rng = np.random.default_rng(5)
    n = 4096
    deg = rng.integers(0, 24, n).astype(np.uint64)
    for i, d in {17: (1 << 24) + 5, 3000: (1 << 24) + 1, 5: (1 << 17) + 3, 900: 70000, 901: 70000,
                 77: 65536, 4095: 65535, 1000: 0x10100}.items():
        deg[i] = d
    row = np.zeros(n + 1, np.uint64)
    np.cumsum(deg, out=row[1:])
    col = rng.integers(0, n, int(row[-1]), dtype=np.uint32)
    return row, col


def schedule_graph(case):
    if case == "boundary35":
        g = oracle.boundary_graph(17)
        return g["row"], g["col"]
    if case == "smoke1024":
        g = smoke1024()
        return g["row"], g["col"]
    if case == "four_digits":
        return four_digit_graph()
    return inputs.WORKLOADS[case].graph()


# Radix passes the sort needs (one per 8-bit digit of the maximum degree):
# boundary35..large 1-2, skew (max in-degree 132 270) 3, four_digits 4.
@pytest.mark.parametrize("case", ["boundary35", "smoke1024", "smoke", "arxiv", "large", "skew", "four_digits"])
def test_degree_schedule_bit_exact(gpu_ctx, case):
    row, col = schedule_graph(case)
    maxdeg = int(np.diff(row).max())
    if case == "skew":
        assert (1 << 16) <= maxdeg < (1 << 24)
    if case == "four_digits":
        assert maxdeg >= (1 << 24)
    gpu_ctx.set_graph(row, col)
    perm, steps = gpu_ctx.degree_schedule()
    operm, osteps = oracle.degree_schedule(row)
    assert np.array_equal(perm, operm)
    assert steps == osteps
    prow, pcol = gpu_ctx.permuted_csr()
    oprow, opcol = oracle.permute_csr(row, col, operm)
    assert np.array_equal(prow, oprow)
    assert np.array_equal(pcol, opcol)
    assert gpu_ctx.choose_R() == oracle.choose_R(row)


# ---------------------------------------------------------------- boundary shapes
SHAPES = [(D, K, d) for D in (17, 33, 128, 256) for K in (1, 2, 4, 8) for d in (7, 32, 40, 47)]
# The other input widths of the FP32 MFMA projection (D = 2 KH, KH = 16, 32, 48, 96), up to 8 x 64.
SHAPES += [(32, 8, 32), (64, 4, 40), (96, 8, 64), (192, 2, 47), (192, 1, 64), (256, 8, 64)]


@pytest.mark.parametrize("D,K,d", SHAPES)
def test_boundary_shapes_fp32(gpu_ctx, D, K, d):
    """baseline/tests/boundaries.cpp:27-35 on the GPU path: FP32 within 1e-4 of
    R0 (max-abs and rel-L2), exact zeros for the empty row, and the row max
    equal bit for bit to the scalar max of LeakyReLU(L+R) over the GPU's own L/R."""
    g = oracle.boundary_graph(D)
    p = oracle.boundary_param(D, K, d)
    r = oracle.ref_layer(g["row"], g["col"], g["x"], p, False)
    for opts in SCHEDULES:
        got = run_layer(gpu_ctx, g["row"], g["col"], g["x"], p, False, gatgpu.FP32, opts)
        e = oracle.errors(r["out"], got["out"])
        assert e["finite"] and e["max_abs"] < FP32_MAX_ABS and e["relative_l2"] < FP32_MAX_ABS, (opts, e)
        for k in ("left", "right", "max"):
            assert oracle.errors(r[k], got[k])["max_abs"] < FP32_MAX_ABS, k
        assert oracle.errors(r["den"], got["den"])["relative_l2"] < 1e-5
        assert np.all(got["out"][0] == 0) and np.all(got["den"][0] == 0)
        row, col = g["row"], g["col"]
        L, R = got["left"], got["right"]
        for i in range(g["n"]):
            b, e_ = int(row[i]), int(row[i + 1])
            sc = L[i][None, :] + R[col[b:e_]]
            sc = np.where(sc >= 0, sc, np.float32(0.2) * sc).astype(np.float32)
            m = np.zeros(K, np.float32) if b == e_ else sc.max(axis=0)
            assert np.array_equal(m, got["max"][i])


@pytest.mark.parametrize("D,K,d", [(17, 8, 7), (128, 8, 32), (256, 1, 47), (33, 4, 40), (128, 8, 64),
                                   (256, 8, 64), (128, 1, 64), (512, 1, 64), (512, 8, 64)])
def test_boundary_shapes_bf16_and_hidden(gpu_ctx, D, K, d):
    g = oracle.boundary_graph(D)
    p = oracle.boundary_param(D, K, d)
    for hidden in (False, True):
        r = oracle.ref_layer(g["row"], g["col"], g["x"], p, hidden)
        for opts in SCHEDULES:
            got = run_layer(gpu_ctx, g["row"], g["col"], g["x"], p, hidden, gatgpu.FP32, opts)
            assert oracle.errors(r["out"], got["out"])["max_abs"] < FP32_MAX_ABS, opts
            got = run_layer(gpu_ctx, g["row"], g["col"], g["x"], p, hidden, gatgpu.BF16, opts)
            e = oracle.errors(r["out"], got["out"])
            assert e["finite"] and e["relative_l2"] < BF16_REL_L2, (opts, e)
            assert np.all(got["out"][0] == 0)


def test_adversarial_scores(gpu_ctx):
    """boundaries.cpp:44-52 through inputs (see test_oracle.adversarial_layer)."""
    from test_oracle import adversarial_layer

    g = oracle.boundary_graph(2)
    deg = np.diff(g["row"])
    for scenario in range(5):
        x, p = adversarial_layer(g["n"], scenario)
        got = run_layer(gpu_ctx, g["row"], g["col"], x, p, False, gatgpu.FP32)
        assert np.isfinite(got["out"]).all(), scenario
        assert np.all(got["den"][deg == 0] == 0)
        assert np.all(got["den"][deg > 0] >= 1), scenario
        r = oracle.ref_layer(g["row"], g["col"], x, p, False)
        scale = max(1.0, float(np.abs(r["out"]).max()))
        assert oracle.errors(r["out"], got["out"])["max_abs"] < FP32_MAX_ABS * scale, scenario


def peak_graph():
    """250 nodes; node 249 is the score peak of the late-peak scenario.  Row
    degrees cycle through 0..249 edges (one to four 64-edge chunks); rows
    i % 3 == 0 list the peak as their last source (in their last chunk),
    rows i % 3 == 1 as their first, rows i % 3 == 2 not at all."""
    n = 250
    degs = [0, 1, 2, 15, 16, 17, 63, 64, 65, 127, 128, 129, 130, 191, 192, 193, 200, 249]
    row, col = [0], []
    for i in range(n):
        c = degs[i % len(degs)]
        if c:
            base = [(i * 3 + k * 7) % (n - 1) for k in range(c - 1)]
            col.extend({0: base + [n - 1], 1: [n - 1] + base}.get(i % 3, base + [(i * 3 + 5) % (n - 1)]))
        row.append(len(col))
    return np.array(row, np.uint64), np.array(col, np.uint32)


def adversarial_layer_bf16_exact(n, scenario, K, d):
    """The score scenarios of baseline/tests/boundaries.cpp:46-48 with every
    input, weight and projected value exact in bf16, so the bf16 paths see
    the same scores as the FP32 oracle: x = [1, t], W = 1, Z[i,:] = 1 + t_i,
    L[i,h] = (1 + t_i) aL[h,0], R[j,h] = (1 + t_j) aR[h,1].
    0: equal scores (aR = 0); 1: late peak (t = -255 except the last node,
    +255: non-peak weights underflow to 0); 2: ramp t = i - 17; 3/4: L offset
    +-8192 (t = 0 / t = round(8 sin i))."""
    t = np.zeros(n, np.float32)
    if scenario == 1:
        t[:] = -255.0
        t[-1] = 255.0
    elif scenario == 2:
        t = np.arange(n, dtype=np.float32) - 17
    elif scenario == 4:
        t = np.round(np.sin(np.arange(n)) * 8).astype(np.float32)
    x = np.stack([np.ones(n, np.float32), t], axis=1)
    w = np.ones((2, K * d), np.float32)
    al = np.zeros(K * d, np.float32)
    ar = np.zeros(K * d, np.float32)
    for h in range(K):
        al[h * d] = {3: 8192.0, 4: -8192.0}.get(scenario, float(h) - 4)
        ar[h * d + 1] = 0.0 if scenario == 0 else 1.0
    assert np.array_equal(oracle.quantize_bf16(x), x) and np.array_equal(oracle.quantize_bf16(x @ w), x @ w)
    return x, {"in": 2, "heads": K, "dim": d, "w": w, "al": al, "ar": ar}


ADVERSARIAL_PATHS = [("fp32_tf", gatgpu.FP32, gatgpu.TRANSFORM_FIRST), ("bf16_tf", gatgpu.BF16, gatgpu.TRANSFORM_FIRST),
                     ("bf16_af", gatgpu.BF16, gatgpu.AGGREGATE_FIRST)]


# (K, d, D_in, path): D_in 256 takes the 8 x 64 bf16 layer onto the
# W-stationary projection, whose aggregation recomputes R from gathered Z rows.
SPLIT_ADVERSARIAL_CASES = ([(K, d, 2, p[0]) for K, d in ((8, 32), (8, 64)) for p in ADVERSARIAL_PATHS] +
                           [(8, 64, 256, "bf16_tf")])


@pytest.mark.parametrize("K,d,din,path", SPLIT_ADVERSARIAL_CASES)
def test_adversarial_scores_split_rows(gpu_ctx, K, d, din, path):
    """boundaries.cpp:44-52 on the 8-head kernels: the transform-first 8 x 32 /
    8 x 64 aggregation (FP32 and bf16; 8 x 64 bf16 also with 256 inputs, R
    recomputed from each gathered Z row) and the aggregate-first sum form,
    under every schedule; with rows >= 16 split into 64-edge chunks, the
    multi-chunk rows take each chunk's own maximum and the last chunk to
    arrive rescales the partials, and the peak sits in a row's last chunk,
    its first, or nowhere.  Every non-empty row has den >= 1, empty rows have
    den 0 and output 0, outputs are finite, the row max equals the scalar max
    of LeakyReLU(L + R) over the GPU's own L/R bit for bit, and the output
    agrees with R0 (inputs exact in bf16, so bf16 and FP32 see one set of
    scores)."""
    _, precision, flow = next(p for p in ADVERSARIAL_PATHS if p[0] == path)
    row, col = peak_graph()
    n = row.size - 1
    deg = np.diff(row).astype(np.int64)
    dst = np.repeat(np.arange(n), deg)
    for scenario in range(5):
        x, p = adversarial_layer_bf16_exact(n, scenario, K, d)
        if din > x.shape[1]:
            # Zero inputs and weight rows: the same exact Z.
            x = np.concatenate((x, np.zeros((n, din - x.shape[1]), np.float32)), axis=1)
            w = np.zeros((din, K * d), np.float32)
            w[:p["in"]] = p["w"]
            p = dict(p, **{"in": din, "w": w})
        r = oracle.ref_layer(row, col, x, p, False)
        scale = max(1.0, float(np.abs(r["out"]).max()))
        for opts in SCHEDULES:
            got = run_layer(gpu_ctx, row, col, x, p, False, precision, opts, flow)
            tag = (scenario, opts)
            assert np.isfinite(got["out"]).all(), tag
            assert np.all(got["den"][deg == 0] == 0) and np.all(got["out"][deg == 0] == 0), tag
            assert np.all(got["den"][deg > 0] >= 1), tag
            s = got["left"][dst] + got["right"][col]
            s = np.where(s >= 0, s, np.float32(0.2) * s).astype(np.float32)
            m = np.full((n, K), -np.inf, np.float32)
            np.maximum.at(m, dst, s)
            assert np.array_equal(got["max"], np.where(deg[:, None] > 0, m, 0).astype(np.float32)), tag
            e = oracle.errors(r["out"], got["out"])
            assert e["max_abs"] < 1e-3 * scale and e["relative_l2"] < 1e-4, (tag, e)


# ---------------------------------------------------------------- repeated runs on one graph
SPLIT_16_64 = {gatgpu.OPT_SPLIT_ROW_MIN_DEGREE: 16, gatgpu.OPT_SPLIT_CHUNK_EDGES: 64}


@pytest.mark.parametrize("flow", [gatgpu.AGGREGATE_FIRST, gatgpu.TRANSFORM_FIRST])
@pytest.mark.parametrize("split", [False, True])
def test_rerun_without_set_graph(gpu_ctx, flow, split):
    """The sum form takes its tiles from counters (169 343 rows: 5 292 tiles,
    beyond the statically assigned ones) and split rows are merged by the
    last chunk to arrive; each launch must leave those counters at zero for
    the next one.  On the arxiv-sized graph a bf16 128 -> 8 x 32 layer runs on
    inputs x1, x2, x1 with no set_graph in between: the second run equals a
    run of x2 right after set_graph bit for bit, the third equals the first,
    and the second is within tolerance of R0 on bf16-rounded x2 and W."""
    w = inputs.WORKLOADS["arxiv"]
    row, col = w.graph()
    p = inputs.glorot_param(128, 8, 32, 41)
    xs = [inputs.normal((w.n, 128), 42), inputs.normal((w.n, 128), 43)]
    opts = SPLIT_16_64 if split else {}

    def fresh():
        gpu_ctx.set_graph(row, col)
        for k, v in opts.items():
            gpu_ctx.set_option(k, v)
        gpu_ctx.set_layer(0, p)

    def run(x):
        gpu_ctx.layer_forward(0, gatgpu.BF16, flow, False, input=x)
        return gpu_ctx.stage(0, "out"), gpu_ctx.stage(0, "den")

    try:
        fresh()
        runs = [run(xs[0]), run(xs[1]), run(xs[0])]
        fresh()
        ref2 = run(xs[1])
    finally:
        for k in opts:
            gpu_ctx.set_option(k, DEFAULT_OPTIONS[k])
    assert not np.array_equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[1], ref2):
        assert np.array_equal(a, b)
    for a, b in zip(runs[2], runs[0]):
        assert np.array_equal(a, b)
    qp = dict(p, w=oracle.quantize_bf16(p["w"]))
    r = oracle.ref_layer(row, col, oracle.quantize_bf16(xs[1]), qp, False)
    e = oracle.errors(r["out"], runs[1][0])
    assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e


@pytest.mark.parametrize("flow", [gatgpu.AGGREGATE_FIRST, gatgpu.TRANSFORM_FIRST])
def test_short_rows_rerun_without_set_graph(gpu_ctx, flow):
    """The rows of at most 4 edges run in a launch of their own after the
    others; the sum form's two launches take tiles from the same counters, each
    leaving them at zero.  On 140 000 rows, half of them with 1..4 edges and
    half with 5..40 (about 2 200 tiles each, beyond the statically assigned
    ones), a bf16 100 -> 8 x 64 layer runs on x1, x2, x1 with no set_graph in
    between: the second run equals x2 on a fresh graph bit for bit, the third
    equals the first, and the second is within tolerance of R0."""
    n = 140_000
    rng = np.random.default_rng(61)
    deg = np.where(rng.random(n) < 0.5, rng.integers(1, 5, n), rng.integers(5, 41, n))
    row = np.zeros(n + 1, np.uint64)
    row[1:] = np.cumsum(deg)
    col = rng.integers(0, n, int(row[-1])).astype(np.uint32)
    p = inputs.glorot_param(100, 8, 64, 62)
    xs = [inputs.normal((n, 100), 63), inputs.normal((n, 100), 64)]

    def fresh():
        gpu_ctx.set_graph(row, col)
        gpu_ctx.set_layer(0, p)

    def run(x):
        gpu_ctx.layer_forward(0, gatgpu.BF16, flow, True, input=x)
        return gpu_ctx.stage(0, "out"), gpu_ctx.stage(0, "den"), gpu_ctx.stage(0, "max")

    fresh()
    runs = [run(xs[0]), run(xs[1]), run(xs[0])]
    fresh()
    ref2 = run(xs[1])
    assert not np.array_equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[1], ref2):
        assert np.array_equal(a, b)
    for a, b in zip(runs[2], runs[0]):
        assert np.array_equal(a, b)
    if flow == gatgpu.AGGREGATE_FIRST:
        qp = dict(p, w=oracle.quantize_bf16(p["w"]))
        r = oracle.ref_layer(row, col, oracle.quantize_bf16(xs[1]), qp, True)
        ref, tol = oracle.quantize_bf16(r["out"]), 4e-3
    else:
        r = oracle.ref_layer(row, col, xs[1], p, True)
        ref, tol = r["out"], BF16_REL_L2
    e = oracle.errors(ref, runs[1][0])
    assert e["finite"] and e["relative_l2"] < tol, e


def test_model_rerun_without_set_graph(gpu_ctx):
    """Chained bf16 forwards on the arxiv-sized graph (layer 1 aggregate-first,
    layer 2 transform-first with the output layer's projection in its
    epilogue, split rows on every layer) with set_input between them and no
    set_graph: the logits of x2 after x1 equal those of x2 on a fresh graph
    bit for bit, and x1 again gives x1's logits."""
    w = inputs.WORKLOADS["arxiv"]
    row, col = w.graph()
    m = w.model()
    xs = [w.features(), inputs.normal((w.n, w.din), 44)]

    def fresh():
        gpu_ctx.set_graph(row, col)
        gpu_ctx.set_model(m)

    def run(x):
        gpu_ctx.set_input(x)
        return gpu_ctx.model_forward(gatgpu.BF16, gatgpu.AGGREGATE_FIRST)[0]

    gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 2)  # fused on this graph size too
    try:
        fresh()
        l1, l2, l3 = run(xs[0]), run(xs[1]), run(xs[0])
        assert not gpu_ctx.has_stage(1, "out")
        fresh()
        ref2 = run(xs[1])
    finally:
        gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 1)
    assert not np.array_equal(l1, l2)
    assert np.array_equal(l2, ref2) and np.array_equal(l3, l1)
    ref = oracle.ref_model(row, col, xs[1], m)[2]["out"]
    e = oracle.errors(ref, l2)
    assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e


# ---------------------------------------------------------------- full models
def model_parity(ctx, row, col, x, model, precision):
    ctx.set_graph(row, col)
    ctx.set_model(model)
    ctx.set_input(x)
    logits, times, total = ctx.model_forward(precision, gatgpu.AUTO)
    ref = oracle.ref_model(row, col, x, model)
    return logits, ref, times, total


def test_smoke1024_model_fp32_and_checksum(gpu_ctx):
    g = smoke1024()
    m = oracle.random_model(128, 40, 11)
    logits, ref, times, total = model_parity(gpu_ctx, g["row"], g["col"], g["x"], m, gatgpu.FP32)
    e = oracle.errors(ref[2]["out"], logits)
    assert e["finite"] and e["max_abs"] < FP32_MAX_ABS, e
    assert abs(float(logits.astype(np.float64).sum()) - 221.971286) < 1e-3
    assert total > 0 and all(t["aggregate_ms"] > 0 for t in times)
    for l in range(3):
        for k in ("left", "right", "max", "den"):
            s = gpu_ctx.stage(l, k)
            assert oracle.errors(ref[l][k], s)["relative_l2"] < 1e-5, (l, k)


def test_smoke1024_model_bf16(gpu_ctx):
    g = smoke1024()
    m = oracle.random_model(128, 40, 11)
    logits, ref, _, _ = model_parity(gpu_ctx, g["row"], g["col"], g["x"], m, gatgpu.BF16)
    e = oracle.errors(ref[2]["out"], logits)
    assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e


@pytest.mark.parametrize("precision", [gatgpu.FP32, gatgpu.BF16])
def test_model_time_without_stage_events(gpu_ctx, precision):
    """total_ms alone (no per-layer records): the forward records only its
    first and last events and still returns the model time; the logits and
    stages equal those of a forward with every stage timed."""
    g = smoke1024()
    gpu_ctx.set_graph(g["row"], g["col"])
    gpu_ctx.set_model(oracle.random_model(128, 40, 11))
    gpu_ctx.set_input(g["x"])
    staged, times, t_staged = gpu_ctx.model_forward(precision, gatgpu.AUTO)
    den_staged = gpu_ctx.stage(1, "den").copy()
    bare, none, t_bare = gpu_ctx.model_forward(precision, gatgpu.AUTO, stages=False)
    assert none is None and len(times) == 3
    assert 0 < t_bare < 1e3 and 0 < t_staged < 1e3
    assert np.array_equal(bare, staged)
    assert np.array_equal(gpu_ctx.stage(1, "den"), den_staged)
    # untimed forwards still return no time
    assert gpu_ctx.model_forward(precision, gatgpu.AUTO, want_logits=False, timed=False)[2] == 0.0


@pytest.mark.parametrize("name", ["smoke", "arxiv"])
@pytest.mark.parametrize("precision", [gatgpu.FP32, gatgpu.BF16])
def test_workload_model_parity(gpu_ctx, name, precision):
    w = inputs.WORKLOADS[name]
    row, col = w.graph()
    x = w.features()
    m = w.model()
    logits, ref, _, _ = model_parity(gpu_ctx, row, col, x, m, precision)
    e = oracle.errors(ref[2]["out"], logits)
    if precision == gatgpu.FP32:
        assert e["finite"] and e["max_abs"] < FP32_MAX_ABS, e
    else:
        assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e


@pytest.mark.parametrize("classes", [20, 32, 47, 64])
@pytest.mark.parametrize("precision", [gatgpu.FP32, gatgpu.BF16])
def test_model_logits_rows_in_original_order(gpu_ctx, classes, precision):
    """The last layer writes its FP32 rows straight to original node order
    with the one-head kernel's padded stride (32 or 64 floats, zeros past the
    classes); the logits copied back, the OUT stage of layer 3 and a per-layer
    forward chained on the model's own layer-2 output agree bit for bit, and
    the logits match R0 (FP32 max-abs 1e-4, bf16 rel-L2 1e-2).  A ragged
    graph (empty rows, split rows), 128 -> 8 x 32 -> 8 x 32 -> 1 x classes."""
    row, col = ragged_graph(3001, 40 + classes)
    x = inputs.normal((3001, 128), 7)
    model = inputs.random_model(128, classes, 13)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_model(model)
    gpu_ctx.set_input(x)
    gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 0)  # keep layer 2's output for the chained check
    try:
        logits, _, _ = gpu_ctx.model_forward(precision, gatgpu.TRANSFORM_FIRST)
        out = gpu_ctx.stage(2, "out")
        assert logits.shape == (3001, classes) and np.array_equal(logits, out)
        gpu_ctx.layer_forward(2, precision, gatgpu.TRANSFORM_FIRST, False)
        assert np.array_equal(gpu_ctx.stage(2, "out"), logits)
    finally:
        gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 1)
    ref = oracle.ref_model(row, col, x, model)[2]["out"]
    e = oracle.errors(ref, logits)
    if precision == gatgpu.FP32:
        assert e["finite"] and e["max_abs"] < FP32_MAX_ABS, e
    else:
        assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e


# ---------------------------------------------------------------- output projection fused into layer 2
def ragged_graph(n, seed):
    """CSR with empty rows, rows of one to a few hundred edges and two rows
    of about 1 500 and 3 000 edges; n is not a multiple of the 32-row tile."""
    rng = np.random.default_rng(seed)
    deg = rng.integers(0, 40, n)
    deg[rng.choice(n, n // 10, replace=False)] = 0
    deg[rng.choice(n, 20, replace=False)] = rng.integers(100, 400, 20)
    deg[3], deg[n - 2] = 1500, 3000
    row = np.zeros(n + 1, np.uint64)
    row[1:] = np.cumsum(deg)
    col = rng.integers(0, n, int(row[-1])).astype(np.uint32)
    return row, col


def fused_and_unfused(ctx, row, col, x, model, options=None):
    """bf16 model forward (layers 2-3 transform-first) with the output layer's
    projection fused into layer 2's aggregation (option 2: on any graph) and
    without (0): logits and the stages of layers 2 and 3 of each run."""
    ctx.set_graph(row, col)
    for k, v in (options or {}).items():
        ctx.set_option(k, v)
    ctx.set_model(model)
    ctx.set_input(x)
    runs = {}
    for fuse in (0, 2):
        ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, fuse)
        logits, _, _ = ctx.model_forward(gatgpu.BF16, gatgpu.TRANSFORM_FIRST)
        runs[fuse] = (logits, {(l, k): ctx.stage(l, k) for l in (1, 2)
                               for k in ("z", "left", "right", "max", "den", "out")})
    ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 1)
    for k in options or {}:
        ctx.set_option(k, DEFAULT_OPTIONS[k])
    return runs


@pytest.mark.parametrize("classes", [40, 20, 60])
@pytest.mark.parametrize("sched", range(len(SCHEDULES)))
def test_fused_output_projection_bit_exact(gpu_ctx, classes, sched):
    """Layer 3's projection inside layer 2's aggregation (32-row tiles staged
    in LDS, the same MFMA sequence as the projection kernel; split rows
    projected after the launch): logits and layer 3's Z (up to its width), L,
    R, max and den equal the unfused run bit for bit, as do layer 2's max and
    den; layer 2's output stage is absent when fused.  Classes 20 use one
    32-column block, 40 and 60 two; a ragged graph (empty rows, heavy rows,
    n % 32 != 0) under the three schedules (default, block rows, rows >= 16
    split into 64-edge chunks)."""
    row, col = ragged_graph(3001, 5 + classes)
    x = inputs.normal((3001, 128), 3)
    model = inputs.random_model(128, classes, 11)
    runs = fused_and_unfused(gpu_ctx, row, col, x, model, SCHEDULES[sched])
    (l0, s0), (l1, s1) = runs[0], runs[2]
    assert np.isfinite(l0).all() and np.array_equal(l0, l1)
    for (l, k), v in s0.items():
        if (l, k) == (1, "out"):
            assert v is not None and s1[(l, k)] is None
            continue
        assert np.array_equal(v, s1[(l, k)]), (l, k)
    ref = oracle.ref_model(row, col, x, model)[2]["out"]
    e = oracle.errors(ref, l1)
    assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e


def test_fused_output_projection_arxiv(gpu_ctx):
    """The 169K-node power-law model (128 -> 8x32 -> 8x32 -> 1x40, split rows
    of up to 13K edges): fused and unfused logits bit-equal."""
    w = inputs.WORKLOADS["arxiv"]
    row, col = w.graph()
    runs = fused_and_unfused(gpu_ctx, row, col, w.features(), w.model())
    assert np.array_equal(runs[0][0], runs[2][0])
    assert np.array_equal(runs[0][1][(2, "z")], runs[2][1][(2, "z")])
    assert runs[2][1][(1, "out")] is None


def test_fusion_default_by_graph_size(gpu_ctx):
    """The default fuses the output projection into layer 2 only on graphs of
    at least 16M edges: the 2.5M-edge graph keeps layer 2's output rows."""
    w = inputs.WORKLOADS["arxiv"]
    row, col = w.graph()
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_model(w.model())
    gpu_ctx.set_input(w.features())
    gpu_ctx.model_forward(gatgpu.BF16, gatgpu.AUTO, want_logits=False)
    assert gpu_ctx.has_stage(1, "out")
    with pytest.raises(gatgpu.GatGpuError):
        gpu_ctx.set_option(gatgpu.OPT_FUSE_NEXT_PROJECTION, 3)


def test_layer2_micro_fp32(gpu_ctx):
    """Single layer 256 -> 8x32 on the arxiv-sized graph, N(0,1) input."""
    w = inputs.WORKLOADS["arxiv"]
    row, col = w.graph()
    x = inputs.normal((w.n, 256), 5)
    p = inputs.glorot_param(256, 8, 32, 6)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(1, p)
    gpu_ctx.layer_forward(1, gatgpu.FP32, gatgpu.TRANSFORM_FIRST, True, input=x)
    got = gpu_ctx.stage(1, "out")
    r = oracle.ref_layer(row, col, x, p, True)
    e = oracle.errors(r["out"], got)
    assert e["finite"] and e["max_abs"] < FP32_MAX_ABS, e


# ---------------------------------------------------------------- single-head one-pass layer
def exact_max_aggregate(row, col, z, L, R, hidden):
    """FP64 restatement of max_prescan + standard_aggregate + finish
    (baseline/src/baseline_standard.cpp:44-97) over given Z, L, R (one head)."""
    n = row.size - 1
    out = np.zeros(z.shape, np.float64)
    mx = np.zeros(n, np.float32)
    den = np.zeros(n, np.float64)
    for i in range(n):
        b, e = int(row[i]), int(row[i + 1])
        if b == e:
            continue
        s = L[i, 0] + R[col[b:e], 0]
        s = np.where(s >= 0, s, np.float32(0.2) * s).astype(np.float32)
        mx[i] = s.max()
        p = np.exp(s.astype(np.float64) - np.float64(mx[i]))
        den[i] = p.sum()
        out[i] = (p[:, None] * z[col[b:e]].astype(np.float64)).sum(0) / den[i]
    if hidden:
        out = np.where(out >= 0, out, np.expm1(out))
    return mx, den, out


@pytest.mark.parametrize("ramp", [False, True])
def test_single_head_bf16_one_pass(gpu_ctx, ramp):
    """bf16 single-head layers (C <= 60) read each source's Z line once, with R
    in the line, and keep the softmax online.  The row max must still equal
    leaky(L + max R) bit for bit, and den/out must match the exact-max formula
    evaluated over the GPU's own Z, L, R.  With `ramp`, R rises with the source
    id, so every batch of a row raises the running maximum (a rescale per
    batch).  Rows up to 3000 edges run whole (split threshold lifted) and split
    into chunks (default schedule)."""
    n, d = 20000, 47
    row, col = inputs.powerlaw_graph(n, 400000, 3000, 5)
    if ramp:
        rng = np.random.default_rng(3)
        x = np.stack([np.arange(n, dtype=np.float32) * np.float32(6.0 / n), np.ones(n, np.float32)], 1)
        p = {"in": 2, "heads": 1, "dim": d, "w": rng.standard_normal((2, d)).astype(np.float32),
             "al": rng.standard_normal(d).astype(np.float32), "ar": rng.standard_normal(d).astype(np.float32)}
        if float(p["w"][0] @ p["ar"]) < 0:
            p["ar"] = -p["ar"]
    else:
        x = inputs.normal((n, 64), 8)
        p = inputs.glorot_param(64, 1, d, 9)
    for opts in ({}, {gatgpu.OPT_SPLIT_ROW_MIN_DEGREE: 1 << 30}):
        for hidden in (False, True):
            got = run_layer(gpu_ctx, row, col, x, p, hidden, gatgpu.BF16, opts)
            z = gpu_ctx.stage(0, "z")
            L, R = got["left"].reshape(n, 1), got["right"].reshape(n, 1)
            if ramp:
                assert np.mean(np.diff(R[:, 0]) >= 0) > 0.99
            mx, den, out = exact_max_aggregate(row, col, z, L, R, hidden)
            assert np.array_equal(got["max"].reshape(n), mx), opts
            assert oracle.errors(den, got["den"].reshape(n))["relative_l2"] < 1e-5, opts
            g_out = got["out"].reshape(n, d)
            if hidden:
                # hidden bf16 layers store their output in bf16: one rounding
                assert np.all(np.abs(g_out - out) <= np.abs(out) * (2.0 ** -8 * 1.001) + 1e-6), opts
            else:
                e = oracle.errors(out, g_out)
                assert e["finite"] and e["relative_l2"] < 1e-5, (opts, e)
            r = oracle.ref_layer(row, col, x, p, hidden)
            assert oracle.errors(r["out"], got["out"])["relative_l2"] < BF16_REL_L2


# ---------------------------------------------------------------- fixed-p operator
FIXED_SHAPES = [(128, 8, 32), (256, 8, 64), (256, 1, 47), (33, 4, 40), (17, 8, 7), (64, 2, 32)]


@pytest.mark.parametrize("graph", ["boundary", "powerlaw"])
@pytest.mark.parametrize("D,K,d", FIXED_SHAPES)
def test_fixed_p_operator(gpu_ctx, graph, D, K, d):
    """The fixed-p operator (baseline/bench/main.cpp:103-150) with R0's p/den
    as the fixture: FP32 within 1e-4 of the oracle's FP32 master, bf16 within
    rel-L2 1e-2 of the oracle's bf16-input operator, DEN equal to the fixture
    bit for bit, on every schedule (whole rows, split chunks)."""
    if graph == "boundary":
        g = oracle.boundary_graph(D)
        row, col, x = g["row"], g["col"], g["x"]
        p = oracle.boundary_param(D, K, d)
    else:
        row, col = inputs.powerlaw_graph(4000, 90000, 1500, 3)
        x = inputs.normal((row.size - 1, D), 4)
        p = inputs.glorot_param(D, K, d, 5)
    r = oracle.ref_layer(row, col, x, p, False, edge_stages=True)
    m32 = oracle.fixed_p_layer(row, col, x, p, r["p"], r["den"], False)["out"]
    m16 = oracle.fixed_p_layer(row, col, x, p, r["p"], r["den"], True)["out"]
    b1 = oracle.b1_layer(row, col, oracle.quantize_bf16(x), p, oracle.quantize_bf16(p["w"]), r["p"], r["den"], False)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_fixed_p(0, r["p"], r["den"])
    for opts in SCHEDULES:
        for k, v in opts.items():
            gpu_ctx.set_option(k, v)
        gpu_ctx.fixed_p_forward(0, gatgpu.FP32, input=x)
        e = oracle.errors(m32, gpu_ctx.stage(0, "out"))
        assert e["finite"] and e["max_abs"] < FP32_MAX_ABS, (opts, e)
        assert np.array_equal(gpu_ctx.stage(0, "den"), r["den"])
        gpu_ctx.fixed_p_forward(0, gatgpu.BF16, input=x)
        e = oracle.errors(m16, gpu_ctx.stage(0, "out"))
        assert e["finite"] and e["relative_l2"] < BF16_REL_L2, (opts, e)
        if d == 32 and D <= 128 and K in (1, 2, 4, 8):
            # The reference's tfs_op of the same mode (baseline_tfs.cpp with fixed_p):
            # bf16(p x) W summed in FP32, against the oracle's emulation; and the
            # FP32-product aggregate-first form against the bf16-input master.
            gpu_ctx.fixed_p_forward(0, gatgpu.BF16, gatgpu.TFS_B1, input=x)
            e = oracle.errors(b1, gpu_ctx.stage(0, "out"))
            assert e["finite"] and e["relative_l2"] < 1e-5, (opts, e)
            assert np.array_equal(gpu_ctx.stage(0, "den"), r["den"])
            gpu_ctx.fixed_p_forward(0, gatgpu.BF16, gatgpu.AGGREGATE_FIRST, input=x)
            e = oracle.errors(m16, gpu_ctx.stage(0, "out"))
            assert e["finite"] and e["relative_l2"] < 1e-5, (opts, e)
        for k in opts:
            gpu_ctx.set_option(k, DEFAULT_OPTIONS[k])


def test_fixed_p_rejects_bad_fixtures(gpu_ctx):
    """load_fixture's checks (baseline/src/common.cpp:189-192) and call order."""
    g = oracle.boundary_graph(33)
    p = oracle.boundary_param(33, 4, 8)
    r = oracle.ref_layer(g["row"], g["col"], g["x"], p, False, edge_stages=True)
    gpu_ctx.set_graph(g["row"], g["col"])
    gpu_ctx.set_layer(0, p)
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.fixed_p_forward(0, gatgpu.FP32, input=g["x"])
    assert err.value.code == gatgpu.ESTATE
    bad = r["p"].copy()
    bad[3, 1] = 1.5
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.set_fixed_p(0, bad, r["den"])
    assert err.value.code == gatgpu.EINVAL and "outside [0,1]" in str(err.value)
    bad_den = r["den"].copy()
    bad_den[np.diff(g["row"]).argmax(), 0] *= 1.01
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.set_fixed_p(0, r["p"], bad_den)
    assert err.value.code == gatgpu.EINVAL and "denominator" in str(err.value)
    gpu_ctx.set_fixed_p(0, r["p"], r["den"])
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.fixed_p_forward(0, gatgpu.BF16, gatgpu.AGGREGATE_FIRST, input=g["x"])
    assert err.value.code == gatgpu.EINVAL
    gpu_ctx.set_layer(0, p)  # drops the fixture
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.fixed_p_forward(0, gatgpu.FP32, input=g["x"])
    assert err.value.code == gatgpu.ESTATE


# ---------------------------------------------------------------- error codes
def test_error_codes(gpu_ctx):
    g = oracle.boundary_graph(17)
    row, col = g["row"].copy(), g["col"].copy()
    bad = row.copy()
    bad[3] = bad[-1] + 1
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.set_graph(bad, col)
    assert err.value.code == gatgpu.EINVAL
    badc = col.copy()
    badc[0] = g["n"]
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.set_graph(row, badc)
    assert err.value.code == gatgpu.EINVAL
    gpu_ctx.set_graph(row, col)
    x = g["x"].copy()
    x[0, 0] = np.nan
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.set_input(x)
    assert err.value.code == gatgpu.ENONFINITE
    p = oracle.boundary_param(17, 8, 7)
    for heads, dim in ((9, 7), (8, 65)):
        q = dict(p, heads=heads, dim=dim, w=np.zeros((17, heads * dim), np.float32),
                 al=np.zeros(heads * dim, np.float32), ar=np.zeros(heads * dim, np.float32))
        with pytest.raises(gatgpu.GatGpuError) as err:
            gpu_ctx.set_layer(0, q)
        assert err.value.code == gatgpu.EINVAL
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.set_layer(3, p)
    assert err.value.code == gatgpu.EINVAL
    with pytest.raises(gatgpu.GatGpuError) as err:  # split chunks of at least 64 edges (0: per-kernel plans)
        gpu_ctx.set_option(gatgpu.OPT_SPLIT_CHUNK_EDGES, 32)
    assert err.value.code == gatgpu.EINVAL
    ctx2 = gatgpu.Context(0)
    with pytest.raises(gatgpu.GatGpuError) as err:
        ctx2.layer_forward(0)
    assert err.value.code == gatgpu.ESTATE
    ctx2.close()


@pytest.mark.parametrize("D,K,d", [(128, 8, 32), (100, 8, 32), (256, 8, 32), (256, 1, 47), (128, 8, 64), (33, 4, 40),
                                   (256, 8, 64), (384, 8, 64), (512, 8, 64), (512, 1, 64)])
def test_bf16_projection_stages(gpu_ctx, D, K, d):
    """bf16 MFMA projection against R0 run on bf16-rounded X and W: Z within one
    bf16 ulp of RNE(FP32 Z) (accumulation order may flip a rounding), L from
    the hi/lo B_LR block within 1e-5 relative L2 of the FP32 dots of Z.  R the
    same, except for 8 heads x 32 features and one head x 64, where R is the
    dot of the stored bf16 Z row with a_r (the aggregation then needs no R
    gathers): that R is
    checked against the float64 dot of the GPU's own Z stage to FP32
    summation accuracy, and against R0 to the bf16 rounding of Z."""
    check_bf16_projection(gpu_ctx, inputs.WORKLOADS["smoke"], D, K, d)


# 1021 rows: the last 32-row tile holds 29 rows and its last lane quad one, so
# the stores that leave whole lines after an in-quad transpose (rows 4a + j
# written by lane quad a, rows past n repeating row n - 1) meet partial tiles.
ODD_ROWS = inputs.Workload("odd1021", "uniform", 1021, 16, 0, 128, 8, 32, 40)


@pytest.mark.parametrize("D", [100, 256])
def test_projection_partial_tiles(gpu_ctx, D):
    """The 8 x 32 projection (whole-line Z stores, R from the stored Z) on a
    graph whose row count is not a multiple of 32 or 4: the same bounds as on
    whole tiles."""
    check_bf16_projection(gpu_ctx, ODD_ROWS, D, 8, 32)


# Row counts for the W-stationary 8 x 64 projection: its blocks come in pairs
# (half the CUs, 128 on MI355X) and each pair takes every pairs-th 32-row
# tile, so 32 t - 7 rows give the pairs t // 128 or t // 128 + 1 tiles each:
# 1 to 9 tiles per pair across these graphs, every tail of its 4-tile loop,
# and a partial last tile.
WS_TILES = [192, 320, 448, 576, 832, 1088]


@pytest.mark.parametrize("tiles", WS_TILES)
def test_ws_projection_tile_counts(gpu_ctx, tiles):
    """The 512 -> 8 x 64 projection (W held in registers, the tiles' input in an
    LDS ring) on graphs that give its block pairs 1 to 9 tiles: Z within one
    bf16 ulp plus the FP32 accumulation-order bound of the float64 product of
    the bf16-rounded operands, L (the dot of the FP32 Z row with a_L,
    lr_from_z, baseline_standard.cpp:7-20) within the FP32 bounds of that
    product's dots, and R (from the stored bf16 Z, as the aggregation
    recomputes it) within FP32 summation accuracy of the Z stage's dots."""
    n, D, K, d = 32 * tiles - 7, 512, 8, 64
    row, col = inputs.uniform_graph(n, 2, 5)
    x = inputs.normal((n, D), 17)
    p = inputs.glorot_param(D, K, d, 18)
    xq = oracle.quantize_bf16(x).astype(np.float64)
    wq = oracle.quantize_bf16(p["w"]).astype(np.float64)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_input(x)
    gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, False)
    z64 = xq @ wq
    absdot = np.abs(xq) @ np.abs(wq)
    zref = oracle.quantize_bf16(z64.astype(np.float32)).astype(np.float64)
    z = gpu_ctx.stage(0, "z").astype(np.float64)
    ulp = np.ldexp(1.0, np.frexp(np.abs(zref))[1] - 8)
    assert np.all(np.abs(z - zref) <= ulp + 4 * D * 2.0 ** -24 * absdot)
    a64 = p["al"].astype(np.float64).reshape(K, d)
    want = (z64.reshape(n, K, d) * a64).sum(axis=2)
    # FP32 Z (the Z check's accumulation-order bound) times a, then 64-term
    # FP32 sums; a factor 2 of margin.
    bound = ((4 * D + 2 * d) * 2.0 ** -24 * (absdot.reshape(n, K, d) * np.abs(a64)).sum(axis=2)) * 2 + 1e-30
    got = gpu_ctx.stage(0, "left").astype(np.float64).reshape(n, K)
    bad = np.abs(got - want) > bound
    assert not bad.any(), ("left", int(bad.sum()), np.argwhere(bad)[0])
    # R from the stored bf16 Z (what the aggregation recomputes from a
    # gathered row): the float64 dot of the Z stage with a_R, to FP32
    # summation accuracy.
    terms = z.reshape(n, K, d) * p["ar"].astype(np.float64).reshape(K, d)
    want = terms.sum(axis=2)
    bound = 4 * d * 2.0 ** -24 * np.abs(terms).sum(axis=2) + 1e-30
    got = gpu_ctx.stage(0, "right").astype(np.float64).reshape(n, K)
    bad = np.abs(got - want) > bound
    assert not bad.any(), ("right", int(bad.sum()), np.argwhere(bad)[0])


@pytest.mark.parametrize("D", [100, 64])
def test_aggregate_first_partial_tiles(gpu_ctx, D):
    """The aggregate-first front end writes the gather-table rows (rounded X and
    R) as whole lines; on 1021 rows every row, including the last partial
    tile's, feeds the sum form as on whole tiles: outputs and L equal R0 on
    bf16-rounded X and W."""
    w = ODD_ROWS
    row, col = w.graph()
    x = inputs.normal((w.n, D), 23)
    p = inputs.glorot_param(D, 8, 32, 24)
    qp = dict(p, w=oracle.quantize_bf16(p["w"]))
    xq = oracle.quantize_bf16(x)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_input(x)
    for hidden in (False, True):
        r = oracle.ref_layer(row, col, xq, qp, hidden)
        gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.AGGREGATE_FIRST, hidden)
        out = gpu_ctx.stage(0, "out")
        e = oracle.errors(oracle.quantize_bf16(r["out"]) if hidden else r["out"], out)
        assert e["finite"] and e["relative_l2"] < (4e-3 if hidden else 1e-4), (hidden, e)
        assert oracle.errors(r["left"], gpu_ctx.stage(0, "left"))["relative_l2"] < 1e-5
        assert oracle.errors(r["right"], gpu_ctx.stage(0, "right"))["relative_l2"] < 1e-5
        for k_ in ("max", "den"):
            assert oracle.errors(r[k_], gpu_ctx.stage(0, k_))["relative_l2"] < 1e-4, (hidden, k_)


def short_row_graph(n, seed, heavy):
    """Rows of 0..4 edges (a third of them one edge), and with `heavy` a tenth
    of the rows with 5..40; distinct random sources."""
    rng = np.random.default_rng(seed)
    deg = rng.choice(np.array([0, 1, 1, 2, 3, 4]), size=n)
    if heavy:
        pick = rng.choice(n, n // 10, replace=False)
        deg[pick] = rng.integers(5, 41, pick.size)
    row = np.zeros(n + 1, np.uint64)
    row[1:] = np.cumsum(deg)
    col = np.concatenate([rng.choice(n, int(k), replace=False) for k in deg]).astype(np.uint32)
    return row, col


@pytest.mark.parametrize("D,d,heavy", [(100, 32, True), (128, 64, True), (100, 32, False)])
def test_sum_form_short_rows(gpu_ctx, D, d, heavy):
    """Rows of at most 4 edges share one 16-edge batch four at a time, in a
    launch of their own (without heavier rows, the only one).  On a graph of
    mostly such rows, empty rows included: the row max equals max_j
    LeakyReLU(L_i + R_j) over the GPU's own L and R bit for bit, an empty row
    gives max, den and output 0, and den and the bf16 outputs equal R0 on
    bf16-rounded X and W, over all rows and over the short rows alone."""
    n = 2011
    row, col = short_row_graph(n, 5, heavy)
    deg = np.diff(row.astype(np.int64))
    assert np.mean(deg <= 4) > 0.85 and np.any(deg == 0)
    x = inputs.normal((n, D), 41)
    p = inputs.glorot_param(D, 8, d, 42)
    qp = dict(p, w=oracle.quantize_bf16(p["w"]))
    r = oracle.ref_layer(row, col, oracle.quantize_bf16(x), qp, True)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_input(x)
    gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.AGGREGATE_FIRST, True)
    out, den, M = (gpu_ctx.stage(0, k) for k in ("out", "den", "max"))
    L, R = gpu_ctx.stage(0, "left"), gpu_ctx.stage(0, "right")
    want = np.zeros_like(M)
    for i in np.nonzero(deg)[0]:  # FP32 as the kernel forms it: L + R, then max(s, 0.2 s)
        s = L[i] + R[col[int(row[i]):int(row[i + 1])]]
        want[i] = np.max(np.maximum(s, np.float32(0.2) * s), axis=0)
    assert np.array_equal(M.view(np.uint32), want.view(np.uint32))
    empty = deg == 0
    assert np.all(M[empty] == 0) and np.all(den[empty] == 0) and np.all(out[empty] == 0)
    ref_out = oracle.quantize_bf16(r["out"])
    short = deg <= 4
    for sel in (slice(None), short):
        e = oracle.errors(ref_out[sel], out[sel])
        assert e["finite"] and e["relative_l2"] < 4e-3, e
        assert oracle.errors(r["den"][sel], den[sel])["relative_l2"] < 1e-5


TINY_GRAPHS = {
    "one_node": ([0, 1], [0]),
    "one_empty_node": ([0, 0], []),
    "three_nodes_one_empty": ([0, 2, 2, 5], [0, 2, 1, 2, 0]),
    "seven_nodes": ([0, 1, 3, 3, 7, 8, 12, 17], [0, 0, 1, 0, 1, 2, 3, 4, 0, 2, 4, 5, 6, 5, 4, 3, 2]),
}


@pytest.mark.parametrize("name", sorted(TINY_GRAPHS))
def test_short_rows_tiny_graphs(gpu_ctx, name):
    """Fewer rows than one tile or one four-row group, empty rows among them
    (a graph with no edges at all included): the sum form (100 -> 8 x 32,
    hidden) and the 8 x 64 bf16 transform-first layer equal R0 (on bf16-rounded
    X and W for the sum form), the row max equals max_j LeakyReLU(L_i + R_j)
    over the GPU's own L and R bit for bit and den a float64 softmax over them,
    and an empty row gives max, den and output 0."""
    row = np.array(TINY_GRAPHS[name][0], np.uint64)
    col = np.array(TINY_GRAPHS[name][1], np.uint32)
    n = row.size - 1
    empty = np.diff(row.astype(np.int64)) == 0
    for D, d, flow, hidden in ((100, 32, gatgpu.AGGREGATE_FIRST, True), (100, 64, gatgpu.TRANSFORM_FIRST, False)):
        x = inputs.normal((n, D), 51)
        p = inputs.glorot_param(D, 8, d, 52)
        qp = dict(p, w=oracle.quantize_bf16(p["w"]))
        got = run_layer(gpu_ctx, row, col, x, p, hidden, gatgpu.BF16, dataflow=flow)
        if flow == gatgpu.AGGREGATE_FIRST:
            r = oracle.ref_layer(row, col, oracle.quantize_bf16(x), qp, hidden)
            ref, tol = oracle.quantize_bf16(r["out"]), 4e-3
        else:
            r = oracle.ref_layer(row, col, x, p, hidden)
            ref, tol = r["out"], BF16_REL_L2
        assert np.all(got["max"][empty] == 0) and np.all(got["den"][empty] == 0) and np.all(got["out"][empty] == 0)
        if (~empty).any():
            e = oracle.errors(ref[~empty], got["out"][~empty])
            assert e["finite"] and e["relative_l2"] < tol, (name, flow, e)
        L, R = got["left"], got["right"]
        for i in np.nonzero(~empty)[0]:
            s = L[i][None, :] + R[col[int(row[i]):int(row[i + 1])]]
            s = np.maximum(s, np.float32(0.2) * s)
            assert np.array_equal(s.max(axis=0), got["max"][i]), (flow, i)
            d64 = np.exp(s.astype(np.float64) - got["max"][i].astype(np.float64)).sum(axis=0)
            assert np.all(np.abs(got["den"][i] - d64) <= 1e-5 * d64), (flow, i)


@pytest.mark.parametrize("heavy", [True, False])
def test_transform_first_short_rows(gpu_ctx, heavy):
    """8 x 64 bf16 rows (R in its own array): rows of at most 4 edges go four
    to a wave in a launch of their own (without heavier rows, the only one).
    Over the GPU's own Z, L and R: the row max bit for bit, den and the FP32
    output rows against a float64 softmax within FP32 summation error, empty
    rows 0; and the outputs against R0."""
    n = 2011
    row, col = short_row_graph(n, 7, heavy)
    deg = np.diff(row.astype(np.int64))
    x = inputs.normal((n, 100), 43)
    p = inputs.glorot_param(100, 8, 64, 44)
    got = run_layer(gpu_ctx, row, col, x, p, False, gatgpu.BF16)
    Z = gpu_ctx.stage(0, "z").astype(np.float64).reshape(n, 8, 64)
    L, R, M, den, out = (got[k] for k in ("left", "right", "max", "den", "out"))
    out = out.reshape(n, 8, 64)
    for i in range(n):
        b, e_ = int(row[i]), int(row[i + 1])
        if b == e_:
            assert np.all(M[i] == 0) and np.all(den[i] == 0) and np.all(out[i] == 0), i
            continue
        src = col[b:e_]
        s = L[i][None, :] + R[src]
        s = np.maximum(s, np.float32(0.2) * s)
        assert np.array_equal(s.max(axis=0), M[i]), i
        w = np.exp(s.astype(np.float64) - M[i].astype(np.float64))  # [edges][heads]
        d64 = w.sum(axis=0)
        assert np.all(np.abs(den[i] - d64) <= 1e-5 * d64), i
        acc = np.einsum("eh,ehf->hf", w, Z[src])
        mag = np.einsum("eh,ehf->hf", w, np.abs(Z[src])) / d64[:, None]
        assert np.all(np.abs(out[i] - acc / d64[:, None]) <= 1e-5 * mag + 1e-30), i
    r = oracle.ref_layer(row, col, x, p, False)
    e = oracle.errors(r["out"], got["out"])
    assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e


def check_bf16_projection(gpu_ctx, w, D, K, d):
    row, col = w.graph()
    x = inputs.normal((w.n, D), 3)
    p = inputs.glorot_param(D, K, d, 4)
    qp = dict(p, w=oracle.quantize_bf16(p["w"]))
    r = oracle.ref_layer(row, col, oracle.quantize_bf16(x), qp, False)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_input(x)
    gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, False)
    z = gpu_ctx.stage(0, "z").astype(np.float64)
    zref = oracle.quantize_bf16(r["z"]).astype(np.float64)
    # One bf16 ulp of the result plus the FP32 accumulation-order bound
    # (D * 2^-24 * sum |x w|, with margin) for results that cancel.
    expo = np.frexp(np.abs(zref))[1]
    ulp = np.ldexp(1.0, expo - 8)
    absdot = np.abs(oracle.quantize_bf16(x)).astype(np.float64) @ np.abs(qp["w"]).astype(np.float64)
    tol = ulp + 4 * D * 2.0 ** -24 * absdot
    bad = np.abs(z - zref) > tol
    if bad.any():
        i, f = np.argwhere(bad)[0]
        pytest.fail(f"{int(bad.sum())} Z entries off, first [{i},{f}] gpu={z[i, f]!r} ref={zref[i, f]!r} "
                    f"fp32={r['z'][i, f]!r} tol={tol[i, f]!r}")
    assert np.mean(z != zref) < 0.01
    e = oracle.errors(r["left"], gpu_ctx.stage(0, "left"))
    assert e["relative_l2"] < 1e-5, ("left", e)
    right = gpu_ctx.stage(0, "right").astype(np.float64)
    # R from the stored Z: 8 x 32, one head x 64, and 8 x 64 on the
    # W-stationary path (16 to 32 k steps).
    if (K, d) in ((8, 32), (1, 64)) or ((K, d) == (8, 64) and D in (256, 384, 512)):
        terms = z.reshape(w.n, K, d) * p["ar"].astype(np.float64).reshape(K, d)
        want = terms.sum(axis=2)
        bound = 4 * d * 2.0 ** -24 * np.abs(terms).sum(axis=2) + 1e-30
        assert np.all(np.abs(right.reshape(w.n, K) - want) <= bound)
        # bf16 rounding of Z: relative error <= 2^-9 per term.
        e = oracle.errors(r["right"], gpu_ctx.stage(0, "right"))
        assert e["relative_l2"] < 4e-3, ("right", e)
    else:
        e = oracle.errors(r["right"], gpu_ctx.stage(0, "right"))
        assert e["relative_l2"] < 1e-5, ("right", e)


AF_SHAPES = [(100, 8, 32), (128, 8, 32), (33, 4, 32), (17, 1, 32), (128, 2, 32), (64, 8, 32)]
# The sum form beyond 112 inputs (R from its own array) and with heads of 64.
SUM_FORM_SHAPES = [(116, 8, 32), (120, 8, 64), (128, 8, 64), (100, 8, 64)]


@pytest.mark.parametrize("D,K,d", AF_SHAPES + SUM_FORM_SHAPES)
def test_aggregate_first_layer(gpu_ctx, D, K, d):
    """Aggregate-first (tfs_online_fused semantics, exact max): equals R0 run on
    bf16-rounded X and W (the AF path projects FP32 sums of bf16 inputs with
    hi/lo bf16 MFMA operands), for every schedule incl. split-row chunks."""
    w = inputs.WORKLOADS["smoke"]
    row, col = w.graph()
    x = inputs.normal((w.n, D), 13)
    p = inputs.glorot_param(D, K, d, 14)
    qp = dict(p, w=oracle.quantize_bf16(p["w"]))
    xq = oracle.quantize_bf16(x)
    for hidden in (False, True):
        r = oracle.ref_layer(row, col, xq, qp, hidden)
        r32 = oracle.ref_layer(row, col, x, p, hidden)
        for opts in SCHEDULES:
            gpu_ctx.set_graph(row, col)
            for k_, v_ in opts.items():
                gpu_ctx.set_option(k_, v_)
            gpu_ctx.set_layer(0, p)
            gpu_ctx.set_input(x)
            gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.AGGREGATE_FIRST, hidden)
            out = gpu_ctx.stage(0, "out")
            assert gpu_ctx.stage(0, "z") is None  # no Z in the aggregate-first dataflow
            for k_ in opts:
                gpu_ctx.set_option(k_, DEFAULT_OPTIONS[k_])
            # hidden outputs are stored bf16 (the next layer's input): allow its rounding
            e = oracle.errors(oracle.quantize_bf16(r["out"]) if hidden else r["out"], out)
            assert e["finite"] and e["relative_l2"] < (4e-3 if hidden else 1e-4), (hidden, opts, e)
            assert oracle.errors(r32["out"], out)["relative_l2"] < BF16_REL_L2
            for k_ in ("max", "den"):
                assert oracle.errors(r[k_], gpu_ctx.stage(0, k_))["relative_l2"] < 1e-4, (k_, opts)


def test_sum_form_chained_bf16_input(gpu_ctx):
    """A hidden 4 x 32 layer's bf16 output (128 features) feeding a 128 -> 8 x 64
    aggregate-first layer: the chained rows are the gather table as they are.
    Equals R0 on the GPU's own layer-1 output and the bf16-rounded W."""
    w = inputs.WORKLOADS["smoke"]
    row, col = w.graph()
    x = inputs.normal((w.n, 64), 31)
    p0 = inputs.glorot_param(64, 4, 32, 32)
    p1 = inputs.glorot_param(128, 8, 64, 33)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p0)
    gpu_ctx.set_layer(1, p1)
    gpu_ctx.set_input(x)
    gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, True)
    h0 = gpu_ctx.stage(0, "out")
    assert np.array_equal(h0, oracle.quantize_bf16(h0))  # stored bf16
    qp = dict(p1, w=oracle.quantize_bf16(p1["w"]))
    for hidden in (True, False):
        gpu_ctx.layer_forward(1, gatgpu.BF16, gatgpu.AGGREGATE_FIRST, hidden)
        assert gpu_ctx.stage(1, "z") is None
        r = oracle.ref_layer(row, col, h0, qp, hidden)
        out = gpu_ctx.stage(1, "out")
        e = oracle.errors(oracle.quantize_bf16(r["out"]) if hidden else r["out"], out)
        assert e["finite"] and e["relative_l2"] < (4e-3 if hidden else 1e-4), (hidden, e)


@pytest.mark.parametrize("D,K,d", AF_SHAPES)
def test_tfs_b1_layer(gpu_ctx, D, K, d):
    """Faithful neighbour-step TFS (baseline/src/baseline_tfs.cpp:16-110): the
    row max is exact (equal bit for bit to the scalar max of LeakyReLU(L + R)
    over the GPU's own L/R), and the output equals the oracle's emulation
    sum_e sum_k bf16(p x) W / den with p from the same L/R and max."""
    w = inputs.WORKLOADS["smoke"]
    row, col = w.graph()
    x = inputs.normal((w.n, D), 23)
    p = inputs.glorot_param(D, K, d, 24)
    xq, wq = oracle.quantize_bf16(x), oracle.quantize_bf16(p["w"])
    deg = np.diff(row).astype(np.int64)
    dst = np.repeat(np.arange(w.n), deg)
    for hidden in (False, True):
        r32 = oracle.ref_layer(row, col, x, p, hidden)
        for opts in SCHEDULES:
            gpu_ctx.set_graph(row, col)
            for k_, v_ in opts.items():
                gpu_ctx.set_option(k_, v_)
            gpu_ctx.set_layer(0, p)
            gpu_ctx.set_input(x)
            gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.TFS_B1, hidden)
            for k_ in opts:
                gpu_ctx.set_option(k_, DEFAULT_OPTIONS[k_])
            L, R, M = gpu_ctx.stage(0, "left"), gpu_ctx.stage(0, "right"), gpu_ctx.stage(0, "max")
            s = L[dst] + R[col]
            s = np.where(s >= 0, s, np.float32(0.2) * s).astype(np.float32)
            mfull = np.full((w.n, K), -np.inf, np.float32)
            np.maximum.at(mfull, dst, s)
            mref = np.where(deg[:, None] > 0, mfull, 0).astype(np.float32)
            assert np.array_equal(M, mref), opts
            P = np.exp(s - M[dst]).astype(np.float32)
            den = np.zeros((w.n, K), np.float32)
            np.add.at(den, dst, P)
            want = oracle.b1_layer(row, col, xq, p, wq, P, den, hidden)
            got = gpu_ctx.stage(0, "out")
            e = oracle.errors(oracle.quantize_bf16(want) if hidden else want, got)
            assert e["finite"] and e["relative_l2"] < (4e-3 if hidden else 1e-4), (hidden, opts, e)
            assert oracle.errors(r32["out"], got)["relative_l2"] < BF16_REL_L2


def test_aggregate_first_matches_transform_first_on_arxiv(gpu_ctx):
    w = inputs.WORKLOADS["arxiv"]
    row, col = w.graph()
    x = w.features()
    m = w.model()
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_model(m)
    gpu_ctx.set_input(x)
    tf, _, _ = gpu_ctx.model_forward(gatgpu.BF16, gatgpu.TRANSFORM_FIRST)
    # layer 1 aggregate-first, layers 2-3 cannot (in = 256 > 128) and take transform-first
    gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.AGGREGATE_FIRST, True)
    gpu_ctx.layer_forward(1, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, True)
    gpu_ctx.layer_forward(2, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, False)
    auto = gpu_ctx.stage(2, "out")
    ref = oracle.ref_model(row, col, x, m)[2]["out"]
    for got in (tf, auto):
        e = oracle.errors(ref, got)
        assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e
    assert oracle.errors(tf, auto)["relative_l2"] < BF16_REL_L2
    # The chained model runs aggregate-first where a layer supports it (layer 1
    # here) and transform-first elsewhere: the same bits as the chain above.
    af, _, _ = gpu_ctx.model_forward(gatgpu.BF16, gatgpu.AGGREGATE_FIRST)
    assert np.array_equal(af, auto)
    with pytest.raises(gatgpu.GatGpuError) as err:
        gpu_ctx.layer_forward(1, gatgpu.BF16, gatgpu.AGGREGATE_FIRST, True)  # in = 256
    assert err.value.code == gatgpu.EINVAL


def test_large_model_auto_sum_form(gpu_ctx):
    """Full-size check of the 100 -> 8x32 layer on the 64.3M-edge graph, where
    AUTO takes the aggregate-first sum form (U_h = sum p X_j, then U_h W_h):
    on 2000 sampled rows plus the 64 heaviest (split into chunks), the row max
    equals the scalar max of LeakyReLU(L + R) over the GPU's own L/R bit for
    bit, the denominator and the bf16 output equal a float64 recomputation from
    the bf16-rounded X and W (to one bf16 rounding of the staged sums and of
    the output),
    and the logits stay within the bf16 tolerance of the transform-first model."""
    w = inputs.WORKLOADS["large"]
    row, col = w.graph()
    x = w.features()
    m = w.model()
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_model(m)
    gpu_ctx.set_input(x)
    auto, _, _ = gpu_ctx.model_forward(gatgpu.BF16, gatgpu.AUTO)
    assert gpu_ctx.stage(0, "z") is None  # layer 1 ran aggregate-first
    L, R = gpu_ctx.stage(0, "left"), gpu_ctx.stage(0, "right")
    M, den, out = gpu_ctx.stage(0, "max"), gpu_ctx.stage(0, "den"), gpu_ctx.stage(0, "out")
    p0 = m[0]
    K, d = p0["heads"], p0["dim"]
    wq = oracle.quantize_bf16(p0["w"]).astype(np.float64)
    deg = np.diff(row.astype(np.int64))
    rng = np.random.default_rng(5)
    rows = np.concatenate((rng.choice(w.n, 2000, replace=False), np.argsort(deg)[-64:]))
    for i in rows:
        b, e = int(row[i]), int(row[i + 1])
        js = col[b:e].astype(np.int64)
        s = L[i][None, :] + R[js]
        s = np.where(s >= 0, s, np.float32(0.2) * s).astype(np.float32)
        assert np.array_equal(M[i], s.max(axis=0)), i
        p = np.exp(s.astype(np.float64) - M[i].astype(np.float64))
        dsum = p.sum(axis=0)
        assert np.all(np.abs(den[i] - dsum) <= 1e-5 * dsum), i
        xq = oracle.quantize_bf16(x[js]).astype(np.float64)
        u = p.T @ xq / dsum[:, None]  # [K][D]
        y = np.concatenate([u[h] @ wq[:, h * d:(h + 1) * d] for h in range(K)])
        mag = np.concatenate([np.abs(u[h]) @ np.abs(wq[:, h * d:(h + 1) * d]) for h in range(K)])
        y = np.where(y >= 0, y, np.expm1(y))
        # one bf16 rounding of the output and of the staged sums U / den
        tol = np.abs(y) * 2.0 ** -8 + mag * 2.0 ** -8 + 1e-6
        assert np.all(np.abs(out[i] - y) <= tol), (i, np.max(np.abs(out[i] - y) - tol))
    tf, _, _ = gpu_ctx.model_forward(gatgpu.BF16, gatgpu.TRANSFORM_FIRST)
    e = oracle.errors(tf, auto)
    assert e["finite"] and e["relative_l2"] < BF16_REL_L2, e


def test_skew_model_properties(gpu_ctx):
    """Full-size check on the R-MAT graph (2^22 nodes, 100.6M edges, max
    in-degree 132 270, 9 109 split rows; 128 -> 8x64 -> 8x64 -> 1x64, bf16):
    on 1000 sampled rows plus the 32 heaviest, for layer 1 (aggregate-first sum
    form, R from its own array) the row max equals the scalar max of
    LeakyReLU(L + R) bit for bit and the denominator and the bf16 output equal
    a float64 recomputation from the bf16-rounded X and W (to one bf16
    rounding of the staged sums and of the output); for layer 2 (8 x 64) and layer 3
    (one head of 64), the row max equals the scalar max of LeakyReLU(L + R)
    over the GPU's own L/R bit for bit, the denominator equals a float64 sum of
    p, and the output equals the float64 sum_j p Z_j / den over the GPU's own
    bf16 Z rows (to FP32 summation error and one bf16 rounding of hidden
    outputs)."""
    w = inputs.WORKLOADS["skew"]
    row, col = w.graph()
    x = w.features()
    m = w.model()
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_model(m)
    gpu_ctx.set_input(x)
    logits, _, _ = gpu_ctx.model_forward(gatgpu.BF16, gatgpu.AUTO)
    assert np.isfinite(logits).all()
    deg = np.diff(row.astype(np.int64))
    rng = np.random.default_rng(7)
    rows = np.concatenate((rng.choice(w.n, 1000, replace=False), np.argsort(deg)[-32:]))
    assert gpu_ctx.stage(0, "z") is None  # layer 1 ran aggregate-first
    L, R = gpu_ctx.stage(0, "left"), gpu_ctx.stage(0, "right")
    M, den, out = gpu_ctx.stage(0, "max"), gpu_ctx.stage(0, "den"), gpu_ctx.stage(0, "out")
    K, d = m[0]["heads"], m[0]["dim"]
    wq = oracle.quantize_bf16(m[0]["w"]).astype(np.float64)
    for i in rows:
        js = col[int(row[i]):int(row[i + 1])].astype(np.int64)
        s = L[i][None, :] + R[js]
        s = np.where(s >= 0, s, np.float32(0.2) * s).astype(np.float32)
        assert np.array_equal(M[i], s.max(axis=0)), (0, i)
        p = np.exp(s.astype(np.float64) - M[i].astype(np.float64))
        dsum = p.sum(axis=0)
        assert np.all(np.abs(den[i] - dsum) <= 1e-5 * dsum), (0, i)
        xq = oracle.quantize_bf16(x[js]).astype(np.float64)
        u = p.T @ xq / dsum[:, None]  # [K][D]
        y = np.concatenate([u[h] @ wq[:, h * d:(h + 1) * d] for h in range(K)])
        mag = np.concatenate([np.abs(u[h]) @ np.abs(wq[:, h * d:(h + 1) * d]) for h in range(K)])
        y = np.where(y >= 0, y, np.expm1(y))
        tol = np.abs(y) * 2.0 ** -8 + mag * 2.0 ** -8 + 1e-6
        assert np.all(np.abs(out[i] - y) <= tol), (0, i, np.max(np.abs(out[i] - y) - tol))
    for layer, hidden in ((1, True), (2, False)):
        K, d = m[layer]["heads"], m[layer]["dim"]
        Z = gpu_ctx.stage(layer, "z").astype(np.float64)
        L, R = gpu_ctx.stage(layer, "left"), gpu_ctx.stage(layer, "right")
        M, den, out = gpu_ctx.stage(layer, "max"), gpu_ctx.stage(layer, "den"), gpu_ctx.stage(layer, "out")
        for i in rows:
            js = col[int(row[i]):int(row[i + 1])].astype(np.int64)
            s = L[i][None, :] + R[js]
            s = np.where(s >= 0, s, np.float32(0.2) * s).astype(np.float32)
            assert np.array_equal(M[i], s.max(axis=0)), (layer, i)
            p = np.exp(s.astype(np.float64) - M[i].astype(np.float64))
            dsum = p.sum(axis=0)
            assert np.all(np.abs(den[i] - dsum) <= 1e-5 * dsum), (layer, i)
            zj = Z[js][:, :K * d].reshape(len(js), K, d)
            y = (np.einsum("jh,jhc->hc", p, zj) / dsum[:, None]).reshape(-1)
            mag = (np.einsum("jh,jhc->hc", p, np.abs(zj)) / dsum[:, None]).reshape(-1)
            if hidden:
                y = np.where(y >= 0, y, np.expm1(y))
            # FP32 sums over up to 132K edges (256-edge chunks added in order)
            tol = (np.abs(y) * 2.0 ** -8 if hidden else 0.0) + 1e-4 * mag + 1e-6
            assert np.all(np.abs(out[i] - y) <= tol), (layer, i, np.max(np.abs(out[i] - y) - tol))
