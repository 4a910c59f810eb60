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
