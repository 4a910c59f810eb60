"""Bit-exact bf16 rounding at every site of the gfx950 path.

The reference rounds FP32 to bf16 with convert() = rne() (round to nearest
even, baseline/src/common.cpp:80-93) and gates the vector conversion bit for
bit against rne() on the mantissa-midpoint ties of
baseline/tests/boundaries.cpp:25-26.  Here every place the path rounds is
compared bit for bit with the oracle's rne_bits:

* the input conversion (stage XBF): the convert kernels (k_to_bf16,
  k_to_bf16_pad), the fused conversion inside the fast and the wide bf16
  projections, and the aggregate-first gather table, on 2^20 random finite
  bit patterns plus the boundary ties, their tails and the extremes;
* the Z store of the bf16 projections: rows with one nonzero input, so that
  every Z entry is one exact FP32 product x * w whose rounding is known;
* the hidden-layer output stores of each aggregation kernel: scores all zero
  (aL = aR = 0, so p = 1) and power-of-two degrees, so that the value before
  rounding, sum_j Z_j / deg, is exact and positive (ELU is the identity).
"""
import numpy as np
import pytest

import gatgpu
import oracle
from gatgpu import inputs

pytestmark = pytest.mark.gpu

# baseline/tests/boundaries.cpp:25: u = 0x3f808000 + i * 0x10000, i = 0..36
TIES = (0x3F808000 + np.arange(37, dtype=np.uint64) * 0x10000).astype(np.uint32)


def special_patterns():
    """Ties (both signs), the values either side of each tie, and extremes
    (zeros, the smallest subnormal, FLT_MAX, ties that round to infinity)."""
    t = np.concatenate([TIES, TIES | 0x80000000])
    extra = np.array([0, 0x80000000, 1, 0x80000001, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F7E8000,
                      0x00008000, 0x00018000, 0x007FFFFF, 0x00800000, 0x3F800000, 0xBF808000], np.uint32)
    return np.concatenate([t, t - 1, t + 1, extra]).astype(np.uint32)


def finite_patterns(count, seed):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 1 << 32, size=count, dtype=np.uint64).astype(np.uint32)
    exp = (u >> 23) & 0xFF
    u = np.where(exp == 0xFF, u & ~np.uint32(0x40000000), u)  # Inf/NaN exponent -> finite
    s = special_patterns()
    u[:s.size] = s
    return u.view(np.float32)


def bits(a):
    """bf16 bits of FP32 values that are bf16 (the stages widen bf16 exactly)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    assert np.all(u & 0xFFFF == 0), "stage value is not a widened bf16"
    return (u >> 16).astype(np.uint16)


def rne(a):
    return oracle.rne_bits(np.ascontiguousarray(a, np.float32))


def assert_bits_equal(got_bits, want_bits, what):
    bad = got_bits != want_bits
    if bad.any():
        i = np.argwhere(bad)[0]
        pytest.fail(f"{what}: {int(bad.sum())} of {bad.size} differ, first at {tuple(i)}: "
                    f"got 0x{int(got_bits[tuple(i)]):04x} want 0x{int(want_bits[tuple(i)]):04x}")


# (D, K, d, dataflow, keep) -> the rounding site the layer's FP32 input goes through
CONVERT_SITES = [
    (33, 8, 32, gatgpu.TRANSFORM_FIRST, False),   # k_to_bf16_pad (rows not 16-byte multiples)
    (256, 8, 32, gatgpu.TRANSFORM_FIRST, False),  # k_to_bf16 (16 k steps x 8 head blocks: not fused)
    (128, 8, 32, gatgpu.TRANSFORM_FIRST, True),   # fused in k_proj_fast (8 x 32, R from Z)
    (100, 8, 32, gatgpu.TRANSFORM_FIRST, True),   # fused in k_proj_fast, 7 k steps, tail zeroed
    (128, 1, 47, gatgpu.TRANSFORM_FIRST, True),   # fused in k_proj_fast, 2 head blocks
    (128, 8, 64, gatgpu.TRANSFORM_FIRST, True),   # fused in k_proj_wide (two output groups)
    (100, 8, 32, gatgpu.AGGREGATE_FIRST, False),  # L/R front end writing the gather table (R tail)
    (128, 8, 64, gatgpu.AGGREGATE_FIRST, False),  # gather table without R tail
    (64, 4, 32, gatgpu.AGGREGATE_FIRST, False),   # neighbour-step form: k_to_bf16_pad into its rows
]


@pytest.mark.parametrize("D,K,d,flow,keep", CONVERT_SITES)
def test_input_conversion_bit_exact(gpu_ctx, D, K, d, flow, keep):
    n = (1 << 20) // D + 1
    x = finite_patterns(n * D, 1000 + D).reshape(n, D)
    row, col = inputs.uniform_graph(n, 4, 7)
    p = inputs.glorot_param(D, K, d, 3)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_option(gatgpu.OPT_KEEP_INPUT_BF16, int(keep))
    try:
        gpu_ctx.set_layer(0, p)
        gpu_ctx.set_input(x)
        gpu_ctx.layer_forward(0, gatgpu.BF16, flow, False)
        xbf = gpu_ctx.stage(0, "xbf")
    finally:
        gpu_ctx.set_option(gatgpu.OPT_KEEP_INPUT_BF16, 0)
    assert xbf is not None and xbf.shape == (n, D)
    assert_bits_equal(bits(xbf), rne(x), f"convert D={D} {K}x{d} flow={flow}")


def test_fused_convert_not_kept_by_default(gpu_ctx):
    """Without the option the fused projection keeps the rounded rows in
    registers only: no XBF stage, and the same Z bits as with it."""
    n, D = 4096, 128
    row, col = inputs.uniform_graph(n, 8, 2)
    x = inputs.normal((n, D), 4)
    p = inputs.glorot_param(D, 8, 32, 5)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_input(x)
    gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, True)
    assert gpu_ctx.stage(0, "xbf") is None
    z0, o0 = gpu_ctx.stage(0, "z"), gpu_ctx.stage(0, "out")
    gpu_ctx.set_option(gatgpu.OPT_KEEP_INPUT_BF16, 1)
    try:
        gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, True)
        assert np.array_equal(gpu_ctx.stage(0, "z"), z0) and np.array_equal(gpu_ctx.stage(0, "out"), o0)
        assert_bits_equal(bits(gpu_ctx.stage(0, "xbf")), rne(x), "kept rows")
    finally:
        gpu_ctx.set_option(gatgpu.OPT_KEEP_INPUT_BF16, 0)


def bf16_values(rng, shape, lo_exp, hi_exp, signed):
    """Random bf16-representable FP32 values: 8-bit significands, exponents in [lo_exp, hi_exp)."""
    m = 1.0 + rng.integers(0, 128, size=shape) / 128.0
    e = rng.integers(lo_exp, hi_exp, size=shape)
    v = np.ldexp(m, e)
    if signed:
        v = np.where(rng.random(shape) < 0.5, -v, v)
    return v.astype(np.float32)


def one_hot_rows(rng, n, D, lo_exp, hi_exp, signed, k0=None):
    """Rows with a single nonzero bf16 value, at feature k0 (or i mod D)."""
    x = np.zeros((n, D), np.float32)
    k = np.full(n, k0) if k0 is not None else np.arange(n) % D
    x[np.arange(n), k] = bf16_values(rng, n, lo_exp, hi_exp, signed)
    return x, k


# Shapes by projection kernel: fast (8 x 32 with R from Z; one head with R in
# the row), wide (8 x 64: two groups; 512 inputs), and the general MFMA kernel.
Z_SHAPES = [(128, 8, 32), (256, 1, 40), (64, 1, 64), (128, 8, 64), (512, 8, 64), (48, 4, 40), (100, 2, 32)]


@pytest.mark.parametrize("D,K,d", Z_SHAPES)
def test_projection_z_store_bit_exact(gpu_ctx, D, K, d):
    """Z of a bf16 projection is the RNE of its FP32 accumulator.  With one
    nonzero input per row the accumulator is the exact product x * w
    (8-bit significands, exponents within +-20: no overflow or underflow)."""
    rng = np.random.default_rng(D * 100 + K * 10 + d)
    n = max(2048, (1 << 19) // (K * d))
    x, k = one_hot_rows(rng, n, D, -20, 20, True)
    p = inputs.glorot_param(D, K, d, 9)
    p["w"] = bf16_values(rng, (D, K * d), -20, 20, True)
    row, col = inputs.uniform_graph(n, 4, 3)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_input(x)
    gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, False)
    exact = x[np.arange(n), k][:, None] * p["w"][k]  # float32 products of 8-bit significands: exact
    assert np.array_equal(exact.astype(np.float64), x[np.arange(n), k][:, None].astype(np.float64) * p["w"][k])
    assert_bits_equal(bits(gpu_ctx.stage(0, "z")), rne(exact), f"Z store {D}->{K}x{d}")


def pow2_graph(n, max_log2, seed):
    """Rows of degree 2^(i mod (max_log2 + 1)), uniform random sources."""
    rng = np.random.default_rng(seed)
    deg = (1 << (np.arange(n) % (max_log2 + 1))).astype(np.uint64)
    row = np.zeros(n + 1, np.uint64)
    row[1:] = np.cumsum(deg)
    col = rng.integers(0, n, size=int(row[-1])).astype(np.uint32)
    return row, col, deg


def zero_attention(p):
    return dict(p, al=np.zeros_like(p["al"]), ar=np.zeros_like(p["ar"]))


SCHEDULES = [{}, {gatgpu.OPT_BLOCK_ROW_MIN_DEGREE: 1},
             {gatgpu.OPT_SPLIT_ROW_MIN_DEGREE: 16, gatgpu.OPT_SPLIT_CHUNK_EDGES: 64}]
DEFAULTS = {gatgpu.OPT_BLOCK_ROW_MIN_DEGREE: 512, gatgpu.OPT_SPLIT_ROW_MIN_DEGREE: 0,
            gatgpu.OPT_SPLIT_CHUNK_EDGES: 0}


def run_with(ctx, opts, fn):
    for k, v in opts.items():
        ctx.set_option(k, v)
    try:
        return fn()
    finally:
        for k in opts:
            ctx.set_option(k, DEFAULTS[k])


# Transform-first hidden bf16 layers by aggregation kernel: k_agg_vec (8 x 32
# with R from Z, 8 x 64), k_agg_k1 (one head, R in the row), the generic
# wave/block kernels (4 x 40).
TF_OUT_SHAPES = [(128, 8, 32), (128, 8, 64), (128, 1, 47), (64, 4, 40)]


@pytest.mark.parametrize("D,K,d", TF_OUT_SHAPES)
def test_aggregation_output_store_bit_exact(gpu_ctx, D, K, d):
    """Hidden bf16 outputs are the RNE of the normalised sum: with p = 1 and
    power-of-two degrees (up to 2048, split and block rows included), the
    value before rounding is sum_j Z_j / deg exactly (Z_j in [1, 4] with
    8-bit significands), whatever the summation order."""
    rng = np.random.default_rng(D + K + d)
    n = 6144
    row, col, deg = pow2_graph(n, 11, 5)
    x, _ = one_hot_rows(rng, n, D, 0, 1, False)
    p = zero_attention(inputs.glorot_param(D, K, d, 2))
    p["w"] = bf16_values(rng, (D, K * d), 0, 1, False)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_input(x)
    for opts in SCHEDULES:
        def run():
            gpu_ctx.layer_forward(0, gatgpu.BF16, gatgpu.TRANSFORM_FIRST, True)
            return gpu_ctx.stage(0, "z").astype(np.float64), gpu_ctx.stage(0, "out"), gpu_ctx.stage(0, "den")
        z, out, den = run_with(gpu_ctx, opts, run)
        assert np.all(den == deg[:, None].astype(np.float32)), opts
        s = np.zeros((n, K * d))
        np.add.at(s, np.repeat(np.arange(n), deg.astype(np.int64)), z[col.astype(np.int64)])
        pre = s / deg[:, None].astype(np.float64)
        assert np.array_equal(pre.astype(np.float32).astype(np.float64), pre)  # exact in FP32
        assert_bits_equal(bits(out), rne(pre.astype(np.float32)), f"output store {D}->{K}x{d} {opts}")


# Aggregate-first hidden layers: the sum form (8 x 32, 8 x 64: U rounded to
# bf16, then (U W_h) / den, rounded again; with a power-of-two den the first
# rounding is that of U / den) and the neighbour-step form
# (4 x 32: sum_j p (X_j W_h) / den; TFS_B1: bf16(p X_j) W_h), all inputs at
# one feature k0 so that each output is one exact product.
AF_OUT = [(100, 8, 32, gatgpu.AGGREGATE_FIRST), (128, 8, 64, gatgpu.AGGREGATE_FIRST),
          (64, 4, 32, gatgpu.AGGREGATE_FIRST), (64, 4, 32, gatgpu.TFS_B1), (100, 8, 32, gatgpu.TFS_B1)]


@pytest.mark.parametrize("D,K,d,flow", AF_OUT)
def test_aggregate_first_output_store_bit_exact(gpu_ctx, D, K, d, flow):
    rng = np.random.default_rng(D * K + d + flow)
    n, k0 = 4096, 3
    row, col, deg = pow2_graph(n, 6, 8)  # degrees up to 64: the neighbour-step sums stay exact
    x, _ = one_hot_rows(rng, n, D, 0, 1, False, k0=k0)
    p = zero_attention(inputs.glorot_param(D, K, d, 4))
    p["w"] = bf16_values(rng, (D, K * d), 0, 1, False)
    gpu_ctx.set_graph(row, col)
    gpu_ctx.set_layer(0, p)
    gpu_ctx.set_input(x)
    for opts in SCHEDULES:
        def run():
            gpu_ctx.layer_forward(0, gatgpu.BF16, flow, True)
            return gpu_ctx.stage(0, "out"), gpu_ctx.stage(0, "den")
        out, den = run_with(gpu_ctx, opts, run)
        assert np.all(den == deg[:, None].astype(np.float32)), opts
        u = np.zeros(n)
        np.add.at(u, np.repeat(np.arange(n), deg.astype(np.int64)), x[col.astype(np.int64), k0].astype(np.float64))
        mean = (u / deg).astype(np.float32)  # exact: 8-bit values in [1, 2), power-of-two degrees
        w0 = p["w"][k0].astype(np.float64)
        if flow == gatgpu.AGGREGATE_FIRST and K == 8:
            # sum form: U enters the MFMA as one bf16 (hidden output), and U / den
            # has the same significand (den a power of two)
            s = (oracle.rne_bits(mean).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        else:
            s = mean.astype(np.float64)  # sum_j x_j w / den: each term and the sum exact
        pre = s[:, None] * w0[None, :]
        assert np.array_equal(pre.astype(np.float32).astype(np.float64), pre)
        assert_bits_equal(bits(out), rne(pre.astype(np.float32)), f"AF output store {D}->{K}x{d} flow={flow} {opts}")
