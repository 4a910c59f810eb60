"""The C-ABI libraries load and export every declared symbol (no GPU needed)."""
import re
from pathlib import Path

import numpy as np
import pytest

import gatgpu
from gatgpu import inputs

ROOT = Path(__file__).resolve().parent.parent


def declared(header):
    text = (ROOT / "include" / header).read_text()
    return sorted(set(re.findall(r"\b(gat(?:gpu|host)_[a-z_A-Z0-9]+)\s*\(", text)))


def test_gatgpu_exports_every_declared_symbol():
    lib = gatgpu.load_library()
    names = declared("gatgpu.h")
    assert set(names) == set(gatgpu.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name


def test_gathost_exports_every_declared_symbol():
    lib = inputs.hostlib()
    for name in declared("gathost.h"):
        assert hasattr(lib, name), name


def test_create_without_gpu_reports_no_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; covered by the GPU tests")
    with pytest.raises(gatgpu.GatGpuError) as err:
        gatgpu.Context(0)
    assert err.value.code == gatgpu.ENODEV


def test_destroy_accepts_null_and_last_error_without_context():
    lib = gatgpu.load_library()
    assert lib.gatgpu_destroy(None) == gatgpu.OK
    assert isinstance(lib.gatgpu_last_error(None), bytes)


def test_validate_graph_without_device():
    """gatgpu_validate_graph: Graph::validate's checks (baseline/src/common.cpp:
    23-30, the negative cases of baseline/tests/boundaries.cpp:54-56) and the
    32-bit in-degree limit of the degree schedule, with no GPU."""
    import oracle

    g = oracle.boundary_graph(17)
    row, col = g["row"], g["col"]
    gatgpu.validate_graph(row, col)
    bad = row.copy()
    bad[3] = bad[-1] + 1
    with pytest.raises(gatgpu.GatGpuError) as err:
        gatgpu.validate_graph(bad, col)
    assert err.value.code == gatgpu.EINVAL and "nonmonotone" in str(err.value)
    badc = col.copy()
    badc[0] = g["n"]
    with pytest.raises(gatgpu.GatGpuError) as err:
        gatgpu.validate_graph(row, badc)
    assert err.value.code == gatgpu.EINVAL and "out of bounds" in str(err.value)
    with pytest.raises(gatgpu.GatGpuError) as err:  # row[n] != e
        gatgpu.validate_graph(row, col[:-1])
    assert err.value.code == gatgpu.EINVAL
    # A row of 2^32 in-edges: rejected from the row array alone (rows are
    # checked before sources, so the one-entry source array is never read).
    e = (1 << 32) + 1
    big = np.array([0, 1 << 32, e], np.uint64)
    with pytest.raises(gatgpu.GatGpuError) as err:
        gatgpu.validate_graph(big, np.zeros(1, np.uint32), n=2, e=e)
    assert err.value.code == gatgpu.EOVERFLOW and "row 0" in str(err.value)
    ok = np.array([0, (1 << 32) - 1], np.uint64)  # 2^32 - 1 passes the row checks ...
    with pytest.raises(gatgpu.GatGpuError) as err:  # ... so a source beyond n is then found
        gatgpu.validate_graph(ok, np.full(2, 5, np.uint32), n=1, e=(1 << 32) - 1)
    assert err.value.code == gatgpu.EINVAL and "out of bounds" in str(err.value)
