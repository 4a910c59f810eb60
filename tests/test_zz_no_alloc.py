"""gatgpu_layer_forward_static: the allocation-free transform-first layer.

It runs the kernels of gatgpu_layer_forward with every intermediate in the
library's static scratch array, on device-resident rows in original node
order.  Its output must equal the OUT stage of gatgpu_layer_forward on the
same input bit for bit (same kernels, same per-row summation order), on two
calls in a row, the second on a smaller graph, so that what the first call
left in the array (counters, partial sums) cannot leak into the second.
Layers whose intermediates exceed the array are rejected before any launch.
"""
import numpy as np
import pytest
import torch

import gatgpu
import oracle
from gatgpu import inputs

pytestmark = pytest.mark.gpu

# (D, K, d, precision, hidden): the 8-head vector kernel (R from Z; R gathered),
# the one-head kernel (R in the row), the generic kernels, the FP32 MFMA and
# tiled projections.
CASES = [(128, 8, 32, gatgpu.BF16, True), (256, 8, 64, gatgpu.BF16, False), (256, 1, 47, gatgpu.BF16, False),
         (64, 4, 40, gatgpu.BF16, True), (128, 8, 32, gatgpu.FP32, True), (33, 2, 7, gatgpu.FP32, False),
         (256, 1, 47, gatgpu.BF16, True)]
# Split rows from 16 edges in chunks of 64: the scratch partial sums and counters are used.
SPLIT = {gatgpu.OPT_SPLIT_ROW_MIN_DEGREE: 16, gatgpu.OPT_SPLIT_CHUNK_EDGES: 64}


def graphs():
    big = inputs.powerlaw_graph(6000, 120000, 1500, 3)
    small = inputs.powerlaw_graph(1500, 20000, 400, 4)
    return [big, small]


@pytest.fixture(scope="module")
def ctx():
    c = gatgpu.Context(0)
    yield c
    c.close()


def static_out(ctx, x, width, precision, hidden):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda")
    od = torch.full((x.shape[0], width), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.layer_forward_static(0, precision, hidden, xd.data_ptr(), od.data_ptr())
    ctx.synchronize()
    return od.cpu().numpy()


@pytest.mark.parametrize("D,K,d,precision,hidden", CASES)
@pytest.mark.parametrize("split", [False, True])
def test_static_layer_equals_layer_forward(ctx, D, K, d, precision, hidden, split):
    p = inputs.glorot_param(D, K, d, 7)
    for call, (row, col) in enumerate(graphs()):  # two calls, the second smaller
        n = row.size - 1
        x = inputs.normal((n, D), 11 + call)
        ctx.set_graph(row, col)
        if split:
            for k, v in SPLIT.items():
                ctx.set_option(k, v)
        try:
            ctx.set_layer(0, p)
            need = ctx.static_scratch_need(0, precision, hidden)
            assert 0 < need <= gatgpu.STATIC_SCRATCH_BYTES
            ctx.layer_forward(0, precision, gatgpu.TRANSFORM_FIRST, hidden, input=x)
            want = ctx.stage(0, "out")
            got = static_out(ctx, x, K * d, precision, hidden)
        finally:
            for k in SPLIT:
                ctx.set_option(k, 0)
        assert np.array_equal(got, want), (call, oracle.errors(want, got))
        r = oracle.ref_layer(row, col, x, p, hidden)["out"]
        e = oracle.errors(r, got)
        assert e["finite"] and (e["max_abs"] < 1e-4 if precision == gatgpu.FP32 else e["relative_l2"] < 1e-2), e


def test_static_layer_rejects_oversized_layer(ctx):
    """A 169,343-node graph with 8 x 32 bf16 (Z alone is 87 MB) exceeds the
    64 MiB array: EOVERFLOW, and the output buffer is left untouched."""
    row, col = inputs.WORKLOADS["arxiv"].graph()
    n = row.size - 1
    ctx.set_graph(row, col)
    ctx.set_layer(0, inputs.glorot_param(128, 8, 32, 1))
    assert ctx.static_scratch_need(0, gatgpu.BF16, True) > gatgpu.STATIC_SCRATCH_BYTES
    xd = torch.zeros((n, 128), dtype=torch.float32, device="cuda")
    od = torch.full((n, 256), 7.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    with pytest.raises(gatgpu.GatGpuError) as err:
        ctx.layer_forward_static(0, gatgpu.BF16, True, xd.data_ptr(), od.data_ptr())
    assert err.value.code == gatgpu.EOVERFLOW and "static scratch" in str(err.value)
    ctx.synchronize()
    assert bool(torch.all(od == 7.0))


def test_static_scratch_need_before_setup():
    """Without a graph, or without the layer's weights, the size query
    returns GATGPU_ESTATE."""
    with gatgpu.Context(0) as fresh:
        with pytest.raises(gatgpu.GatGpuError) as err:
            fresh.static_scratch_need(0, gatgpu.BF16, True)
        assert err.value.code == gatgpu.ESTATE
        row, col = inputs.WORKLOADS["smoke"].graph()
        fresh.set_graph(row, col)
        with pytest.raises(gatgpu.GatGpuError) as err:
            fresh.static_scratch_need(1, gatgpu.BF16, True)
        assert err.value.code == gatgpu.ESTATE
