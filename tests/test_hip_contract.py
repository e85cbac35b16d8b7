"""The HipBackend::execute ABI contract on the device (tests/cpp/hip_backend_contract.cpp).

Malformed BackendExecution requests (wrong op class, launch metadata on a
primitive, wrong arity, tensors that are not contiguous device-0 hip tensors,
axes, shapes, dtypes and parameters the plans reject) must return
kInvalidArgument before any allocation, with output slots untouched; then
every hot-path family runs outside and twice inside a bounded pool with
bit-identical results and known answers, the mirror of the reference's
tests/cpp/test_cuda_backend_contract.cpp:416-443, 568-599, 604-625.
"""

from __future__ import annotations

import os
import pathlib
import subprocess

import pytest

from conftest import require_gpu

pytestmark = pytest.mark.gpu

CONTRACT = pathlib.Path(__file__).resolve().parent / "cpp" / "_bin" / "hip_backend_contract"


def test_backend_contract_on_device():
    require_gpu()
    if not CONTRACT.exists():
        pytest.fail(f"{CONTRACT} is not built: run `python tensor.cx_amd/build.py`")
    env = dict(os.environ, TENSORCX_REQUIRE_HIP="1")
    print("running", CONTRACT, flush=True)
    result = subprocess.run([str(CONTRACT)], capture_output=True, text=True, timeout=110, env=env)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "malformed requests rejected before allocation" in result.stdout
    assert "matched inside a bounded pool" in result.stdout
    assert "HIP backend contract passed" in result.stdout
