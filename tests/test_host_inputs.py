"""Synthetic inputs: exact sizes, self-loops, distinct sorted sources, determinism."""
import numpy as np
import pytest

import oracle
from gatgpu import inputs


def check_csr(row, col, n):
    assert row[0] == 0 and row[-1] == col.size and np.all(np.diff(row.astype(np.int64)) >= 1)
    assert col.max() < n
    for i in np.linspace(0, n - 1, 50).astype(np.int64):
        c = col[row[i]:row[i + 1]].astype(np.int64)
        assert i in c
        assert np.all(np.diff(c) > 0)


def test_uniform_graph():
    row, col = inputs.uniform_graph(1024, 16, 11)
    check_csr(row, col, 1024)
    deg = np.diff(row)
    assert 14.5 < deg.mean() < 17.5 and deg.max() <= 31
    row2, col2 = inputs.uniform_graph(1024, 16, 11)
    assert np.array_equal(row, row2) and np.array_equal(col, col2)


def test_powerlaw_exact_edges_and_max_degree():
    row, col = inputs.powerlaw_graph(20_000, 300_000, 3_000, 5)
    check_csr(row, col, 20_000)
    deg = np.diff(row)
    assert row[-1] == 300_000 and deg.max() == 3_000


def test_rmat_dedup_selfloops():
    row, col = inputs.rmat_graph(12, 40_000, 0.57, 0.19, 0.19, 3)
    n = 1 << 12
    check_csr(row, col, n)
    assert row[-1] <= 40_000 + n
    # skewed: the heaviest row is far above the mean
    deg = np.diff(row)
    assert deg.max() > 10 * deg.mean()


def test_normal_and_glorot_ranges():
    z = inputs.normal((1000, 100), 7)
    assert abs(float(z.mean())) < 0.02 and abs(float(z.std()) - 1) < 0.02
    p = inputs.glorot_param(128, 8, 32, 9)
    assert np.abs(p["w"]).max() <= np.sqrt(6 / (128 + 256))
    assert np.abs(p["al"]).max() <= np.sqrt(6 / (8 + 32))


def test_host_random_model_equals_oracle_random_model():
    """Two restatements of random_model (common.cpp:50-62) agree bit for bit."""
    a = inputs.random_model(128, 40, 11)
    b = oracle.random_model(128, 40, 11)
    for pa, pb in zip(a, b):
        for k in ("w", "al", "ar"):
            assert np.array_equal(pa[k], pb[k])
