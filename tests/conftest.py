"""Shared pytest setup: markers, import paths and the golden-vector loader."""

from __future__ import annotations

import json
import os
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "tensor.cx_amd" / "python"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_present() -> bool:
    """True when a HIP device is usable (checked through the built C ABI)."""
    try:
        import tensorcx_hip_capi as capi
        return capi.available()
    except Exception:  # noqa: BLE001 - any load failure means no usable device
        return False


@pytest.fixture(scope="session")
def golden():
    manifest = json.loads((GOLDEN / "golden.json").read_text())
    arrays = np.load(GOLDEN / "golden.npz", allow_pickle=False)
    return manifest, arrays


def bits(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x)
    return x.view(np.uint32) if x.dtype == np.float32 else x


def assert_bits_equal(actual, expected, context=""):
    actual, expected = np.asarray(actual), np.asarray(expected)
    assert actual.shape == expected.shape, f"{context}: shape {actual.shape} != {expected.shape}"
    assert actual.dtype == expected.dtype, f"{context}: dtype {actual.dtype} != {expected.dtype}"
    if not np.array_equal(bits(actual), bits(expected)):
        diff = np.flatnonzero(bits(actual).reshape(-1) != bits(expected).reshape(-1))
        raise AssertionError(
            f"{context}: {diff.size} of {actual.size} elements differ; first at {diff[0]}: "
            f"{actual.reshape(-1)[diff[0]]!r} != {expected.reshape(-1)[diff[0]]!r}")


def require_gpu():
    import tensorcx_hip_capi as capi
    if not capi.LIB_PATH.exists():
        pytest.fail(f"{capi.LIB_PATH} is not built: run `python tensor.cx_amd/build.py`")
    if not gpu_present():
        if os.environ.get("TENSORCX_REQUIRE_HIP") == "1":
            pytest.fail("TENSORCX_REQUIRE_HIP=1 but no usable HIP device")
        pytest.skip("no HIP device")
