"""tcx_hip_reduce_noalloc against tcx_hip_reduce, through the C ABI.

The no-allocation entry point runs the kernels of tcx_hip_reduce with the
segment partials in the library's static per-device scratch instead of a
workspace. Two calls in a row (the second on a smaller input), and more
after them, must each match the workspace entry point bit for bit: the
partials and their combine order are the same.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import require_gpu
from hip_cases import SUM_BAR, assert_bits, sum_error

pytestmark = pytest.mark.gpu

# Segmented plans (rows too few to fill the GPU): the full-tensor sum of the
# C3 config, then smaller inputs, one with rows not a multiple of 4 floats
# (the scalar-load path).
SHAPES = [(1, 8192 * 8192), (3, 2_000_000), (1, 300_001), (5, 70_000)]


@pytest.fixture(scope="module")
def capi():
    require_gpu()
    import tensorcx_hip_capi
    return tensorcx_hip_capi


def run_pair(capi, op, x):
    rows, cols = x.shape
    dtype = capi.TCX_INT32 if x.dtype == np.int32 else capi.TCX_FLOAT32
    out_dtype = np.int32 if (op == "argmax" or x.dtype == np.int32) else np.float32
    dx = capi.DeviceArray.from_numpy(x)
    ws = capi.reduce_workspace(op, dtype, rows, cols, 1)
    assert ws is not None and ws.nbytes <= capi.REDUCE_NOALLOC_MAX_WORKSPACE
    with_ws, without = capi.DeviceArray((rows,), out_dtype), capi.DeviceArray((rows,), out_dtype)
    capi.reduce(op, dtype, dx.ptr, with_ws.ptr, rows, cols, 1, workspace=ws)
    capi.reduce_noalloc(op, dtype, dx.ptr, without.ptr, rows, cols, 1)
    capi.synchronize()
    return with_ws.numpy(), without.numpy()


@pytest.mark.parametrize("op", ["sum", "mean", "max", "min", "argmax"])
def test_noalloc_matches_workspace_entry_f32(capi, op):
    rng = np.random.default_rng(31)
    for shape in SHAPES:  # consecutive calls share the scratch
        x = rng.standard_normal(shape).astype(np.float32)
        reference, actual = run_pair(capi, op, x)
        assert_bits(actual, reference, f"{op} {shape}")
        if op == "sum":  # and both sit within the sum bar of the oracle's sequential sum
            err = sum_error(actual, oracle.sum(x, -1), x, shape[0], shape[1], 1)
            assert err <= SUM_BAR, f"{op} {shape}: {err:.3e}"


@pytest.mark.parametrize("op", ["sum", "max", "argmax"])
def test_noalloc_matches_workspace_entry_i32(capi, op):
    rng = np.random.default_rng(32)
    for shape in SHAPES[1:]:
        x = rng.integers(-2**31, 2**31 - 1, shape, dtype=np.int64).astype(np.int32)
        reference, actual = run_pair(capi, op, x)
        assert_bits(actual, reference, f"i32 {op} {shape}")


def test_noalloc_special_values_and_ties(capi):
    # NaN-first, first-index ties and signed zeros across segment and block
    # boundaries, where the last block's combine decides.
    x = np.zeros((2, 1_000_000), np.float32)
    x[0, 999_999] = -0.0
    x[0, 4096 * 7 + 3] = 5.0
    x[0, 4096 * 300 % 1_000_000] = 5.0
    x[1, 700_000] = np.nan
    x[1, 900_000] = np.nan
    for op in ("max", "min", "argmax"):
        reference, actual = run_pair(capi, op, x)
        assert_bits(actual, reference, op)
    reference, actual = run_pair(capi, "sum", x)
    assert actual[0] == 10.0 and np.isnan(actual[1]) and np.isnan(reference[1])


def test_noalloc_column_plans_match(capi):
    # Strided reductions whose rows are split over blocks keep their split
    # partials in the scratch; consecutive calls shrink.
    rng = np.random.default_rng(34)
    for outer, rows, inner in [(1, 4096, 4096), (1, 100_000, 3), (2, 1000, 1030), (1, 8192, 64)]:
        x = rng.standard_normal(outer * rows * inner).astype(np.float32)
        x[::977] = 2.0
        dx = capi.DeviceArray.from_numpy(x)
        for op in ("sum", "mean", "max", "argmax"):
            ws = capi.reduce_workspace(op, capi.TCX_FLOAT32, outer, rows, inner)
            assert ws is not None and ws.nbytes <= capi.REDUCE_NOALLOC_MAX_WORKSPACE
            out_dtype = np.int32 if op == "argmax" else np.float32
            a = capi.DeviceArray((outer * inner,), out_dtype)
            b = capi.DeviceArray((outer * inner,), out_dtype)
            capi.reduce(op, capi.TCX_FLOAT32, dx.ptr, a.ptr, outer, rows, inner, workspace=ws)
            capi.reduce_noalloc(op, capi.TCX_FLOAT32, dx.ptr, b.ptr, outer, rows, inner)
            capi.synchronize()
            assert_bits(b.numpy(), a.numpy(), f"column {op} {(outer, rows, inner)}")
            if op == "max":
                assert_bits(b.numpy(), oracle.max(x.reshape(outer, rows, inner), 1).reshape(-1), "column max")


def test_noalloc_unsegmented_plans_match(capi):
    # Plans without segments need no scratch and run the same kernels.
    rng = np.random.default_rng(33)
    x = rng.standard_normal((9000, 700)).astype(np.float32)
    dx = capi.DeviceArray.from_numpy(x)
    assert capi.reduce_workspace("sum", capi.TCX_FLOAT32, 9000, 700, 1) is None
    a, b = capi.DeviceArray((9000,)), capi.DeviceArray((9000,))
    capi.reduce("sum", capi.TCX_FLOAT32, dx.ptr, a.ptr, 9000, 700, 1)
    capi.reduce_noalloc("sum", capi.TCX_FLOAT32, dx.ptr, b.ptr, 9000, 700, 1)
    capi.synchronize()
    assert_bits(b.numpy(), a.numpy(), "unsegmented")
