"""Shared fixtures.  GPU tests are marked ``gpu`` and call the library
through its C-ABI (ctypes); CPU tests cover the oracle, the golden vectors
and the library's exports."""
from __future__ import annotations

import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "gnc-x_amd"))

import pyoracle  # noqa: E402
import synth  # noqa: E402

_spec_root = ROOT / "gnc-x_amd"
import importlib.util  # noqa: E402

if "gncx_amd" not in sys.modules:
    _spec = importlib.util.spec_from_file_location("gncx_amd", _spec_root / "__init__.py",
                                                   submodule_search_locations=[str(_spec_root)])
    _mod = importlib.util.module_from_spec(_spec)
    sys.modules["gncx_amd"] = _mod
    _spec.loader.exec_module(_mod)
gncx = sys.modules["gncx_amd"]

GOLDEN = ROOT / "tests" / "golden" / "ref_vectors.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); calls the C-ABI library")


@pytest.fixture(scope="session")
def oracle():
    return pyoracle.Oracle()


@pytest.fixture(scope="session")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.fixture(scope="session")
def ref():
    if not pyoracle.REF_SO.exists():
        pytest.skip("reference library not built (reference sources absent)")
    return pyoracle.Reference()


@pytest.fixture(scope="session")
def lib():
    """The product library; GPU tests only.  Fails (not skips) when the
    library is missing or no device is visible."""
    lib = gncx.load()
    rc = lib.gncx_hip_init(0)
    assert rc == 0, f"gncx_hip_init failed: {rc} {lib.gncx_hip_last_error().decode()}"
    return lib


@pytest.fixture(scope="session")
def torch_mod():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch


def ptr(a) -> int:
    return 0 if a is None else a.ctypes.data


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
