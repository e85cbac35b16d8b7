"""Strided reductions (a middle axis, inner > 1) on the hip device.

A reduction over an axis with elements after it reads x as [outer, R, inner]
(the reference's reduce_axis_impl, cpu_backend.cpp:1099-1249, walks the same
three extents). More than 64 rows run col_kernel: column tiles of 64 or 256
columns, waves folding contiguous runs of rows, and rows split over blocks
(partials folded in split order) when tiles are few. max/min/argmax and
int32 sums must match the oracle bit for bit, with ties, NaNs and signed
zeros placed across wave-run and split boundaries; float32 sums and means
are held to the sum bar (max|d| / sum|x| <= 1e-5 per output, a mean's error
taken times its count). Up to 64 rows keep the reference's order exactly.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import require_gpu
from hip_cases import SUM_BAR, assert_bits, sum_error

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cx():
    require_gpu()
    import tensorcx
    return tensorcx


@pytest.fixture(scope="module")
def capi():
    require_gpu()
    import tensorcx_hip_capi
    return tensorcx_hip_capi


def check_f32(cx, x, axis, context):
    _, outer, red, inner = oracle.reduction_dims(x.shape, axis)
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, axis).numpy(), getattr(oracle, op)(x, axis), f"{op} {context}")
    for op in ("sum", "mean"):
        actual = getattr(cx, op)(h, axis).numpy()
        expected = getattr(oracle, op)(x, axis)
        if red <= 64:
            assert_bits(actual, expected, f"{op} {context}")
        else:
            scale = np.float64(red if op == "mean" else 1)
            err = sum_error(actual * scale, expected * scale, x, outer, red, inner)
            assert err <= SUM_BAR, f"{op} {context}: {err:.3e}"


def plant_specials(x, rng):
    """Ties, NaNs of both signs, signed zeros and infinities in columns of
    x viewed as [R, C], at rows near wave-run and split boundaries."""
    rows, cols = x.shape
    marks = sorted({1, 63, 64, 127, 128, 129, rows // 8, rows // 3, rows // 2, rows - 2, rows - 1})
    marks = [r for r in marks if 0 <= r < rows]
    for c in range(0, cols, 7):
        kind = (c // 7) % 6
        if kind == 0:      # tie of the column's extreme at two boundary rows
            x[marks[1], c] = x[marks[-2], c] = 50.0
            x[marks[2], c] = x[marks[-1], c] = -50.0
        elif kind == 1:    # two NaNs, the first one negative
            x[marks[len(marks) // 2], c] = np.float32(np.nan) * -1
            x[marks[-1], c] = np.nan
        elif kind == 2:    # zeros of both signs only: the first one kept
            x[:, c] = -0.0
            x[marks[-2], c] = 0.0
        elif kind == 3:    # every value -inf
            x[:, c] = -np.inf
        elif kind == 4:    # +inf late, -inf early
            x[marks[-1], c] = np.inf
            x[0, c] = -np.inf
        else:              # many ties
            x[:, c] = rng.integers(-1, 2, rows)


# (shape, axis): tiles of 256 columns (inner a multiple of 4) and of 64, the
# last tile partly past the end, one tile split many ways, many tiles with no
# split, outer > 1, 65 rows (the smallest strided plan) and 64 (exact order).
SHAPES = [
    ((8192, 64), 0),          # 64 columns, waves stepping 4 rows: 32 splits
    ((300, 2052), 0),         # 9 tiles of 256, 4 columns in the last
    ((2, 1000, 1030), 1),     # tiles of 64 (1030 is not a multiple of 4)
    ((5, 3001, 7), 1),        # 7 columns of an 8-wide tile, stepping 8 rows
    ((4096, 4096), 0),        # 16 tiles x 32 splits
    ((65, 600), 0),           # 65 rows
    ((64, 600), 0),           # exact order
    ((3, 777, 2, 2), 1),      # inner 4 from two axes
    ((100_000, 3), 0),        # 3 columns of a 4-wide tile, stepping 16 rows
    ((70, 2, 2), 0),          # inner 4 stepping 64 rows, 70 rows: one split
    ((1000, 12), 0),          # 12 columns of a 16-wide tile (16-byte loads)
]


@pytest.mark.parametrize("shape,axis", SHAPES)
def test_column_reductions_random(cx, shape, axis):
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    check_f32(cx, x, axis, f"{shape} axis {axis}")


@pytest.mark.parametrize("shape,axis", SHAPES)
def test_column_reductions_special_values(cx, shape, axis):
    rng = np.random.default_rng(7 + sum(shape))
    x = rng.integers(-3, 4, shape).astype(np.float32)
    # View the reduced axis as rows and everything after it as columns.
    moved = np.moveaxis(x, axis, -1)
    flat = moved.reshape(-1, shape[axis]).T.copy()          # [R, outer * inner]
    plant_specials(flat, rng)
    x = np.moveaxis(flat.T.reshape(moved.shape), -1, axis).copy()
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, axis).numpy(), getattr(oracle, op)(x, axis), f"{op} {shape}")
    # NaN columns stay NaN, infinities stay infinite, integer sums are exact.
    s = cx.sum(h, axis).numpy()
    expected = oracle.sum(x, axis)
    assert np.array_equal(np.isnan(s), np.isnan(expected)), f"sum NaN positions {shape}"
    finite = np.isfinite(expected)
    assert_bits(s[finite], expected[finite], f"integer sum {shape}")


@pytest.mark.parametrize("shape,axis", [((8192, 64), 0), ((300, 2052), 0), ((2, 1000, 1030), 1),
                                        ((100_000, 3), 0), ((70, 9, 33), 0)])
def test_column_reductions_int32(cx, shape, axis):
    rng = np.random.default_rng(40 + sum(shape))
    x = rng.integers(-2**31, 2**31 - 1, shape, dtype=np.int64).astype(np.int32)
    x.reshape(-1)[:: 11] = np.iinfo(np.int32).max
    x.reshape(-1)[5:: 13] = np.iinfo(np.int32).min
    h = cx.tensor(x, device="hip")
    for op in ("sum", "max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, axis).numpy(), getattr(oracle, op)(x, axis), f"i32 {op} {shape}")


def test_column_unaligned_base_takes_the_scalar_tiles(capi):
    # A base 4 bytes past a 16-byte boundary with inner a multiple of 4: the
    # 64-column kernel runs with the 256-column plan's splits.
    rng = np.random.default_rng(44)
    R, C = 3000, 132
    x = rng.standard_normal(R * C + 1).astype(np.float32)
    x[1 + 5 * C + 17] = np.nan
    x[1 + 2999 * C + 40] = 99.0
    x[1 + 100 * C + 40] = 99.0
    dx = capi.DeviceArray.from_numpy(x)
    view = x[1:].reshape(R, C)
    for op in ("sum", "max", "min", "argmax"):
        out_dtype = np.int32 if op == "argmax" else np.float32
        out = capi.DeviceArray((C,), out_dtype)
        ws = capi.reduce_workspace(op, capi.TCX_FLOAT32, 1, R, C)
        capi.reduce(op, capi.TCX_FLOAT32, dx.ptr + 4, out.ptr, 1, R, C, workspace=ws)
        capi.synchronize()
        actual = out.numpy()
        expected = getattr(oracle, op)(view, 0)
        if op == "sum":
            assert sum_error(actual, expected, view, 1, R, C) <= SUM_BAR
        else:
            assert_bits(actual, expected, f"unaligned {op}")


# Selections of several reduced runs (after folding): more than 64 elements
# per output fold one run at a time, innermost first, through the row and
# column kernels (argmax gathers the selected axes innermost and takes a row
# argmax); at most 64 run the exact-order metadata kernel.
SELECTIONS = [
    ((16, 64, 300), (0, 2)),           # R K R: 4800 per output
    ((32, 8, 16, 16), (0, 2, 3)),      # the per-channel statistics shape
    ((4, 100, 3, 50), (1, 3)),         # K R K R
    ((3, 40, 5, 70, 2), (0, 2, 4)),    # R K R K R
    ((6, 5, 7, 9), (0, 2)),            # 42 per output: metadata kernel
    ((2, 1, 500, 1, 3, 130), (0, 2, 5)),
]


@pytest.mark.parametrize("shape,axes", SELECTIONS)
def test_multi_run_selections(cx, shape, axes):
    from hip_cases import check_case
    rng = np.random.default_rng(sum(shape))
    x = rng.integers(-3, 4, shape).astype(np.float32)   # ties across runs
    flat = x.reshape(-1)
    flat[rng.integers(0, flat.size, 3)] = 9.0
    flat[rng.integers(0, flat.size, 2)] = np.nan
    h = cx.tensor(x, device="hip")
    for op in ("max", "min"):
        assert_bits(getattr(cx, op)(h, axes).numpy(), getattr(oracle, op)(x, axes), f"{op} {shape} {axes}")
    assert_bits(cx.Tensor(cx._core._argmax_axes(h._impl, list(axes))).numpy(), oracle.argmax(x, axes),
                f"argmax {shape} {axes}")
    y = rng.standard_normal(shape).astype(np.float32)
    hy = cx.tensor(y, device="hip")
    for op in ("sum", "mean", "max", "min"):
        check_case(f"{op} {shape} {axes}", op, [y], {"axes": list(axes)}, getattr(cx, op)(hy, axes).numpy(),
                   getattr(oracle, op)(y, axes))
    assert_bits(cx.Tensor(cx._core._argmax_axes(hy._impl, list(axes))).numpy(), oracle.argmax(y, axes),
                f"argmax random {shape} {axes}")
    yi = rng.integers(-2**31, 2**31 - 1, shape, dtype=np.int64).astype(np.int32)
    hi = cx.tensor(yi, device="hip")
    for op in ("sum", "max", "min"):
        assert_bits(getattr(cx, op)(hi, axes).numpy(), getattr(oracle, op)(yi, axes), f"i32 {op} {shape} {axes}")
    assert_bits(cx.Tensor(cx._core._argmax_axes(hi._impl, list(axes))).numpy(), oracle.argmax(yi, axes),
                f"i32 argmax {shape} {axes}")


@pytest.mark.parametrize("width", [2, 3, 4, 7, 8, 16, 31, 32, 33, 48, 63, 64])
def test_short_rows_exact_order(cx, width):
    # Contiguous rows of at most 64 elements: 64 rows per wave staged in LDS,
    # each folded in the reference's order, so float32 sums are bit-exact
    # too. 1000 rows leave a partial last tile; ties, NaNs and signed zeros
    # sit in the rows.
    rng = np.random.default_rng(width)
    rows = 1000
    x = rng.standard_normal((rows, width)).astype(np.float32) * np.float32(1e3)
    x[1, :] = 0.0
    x[1, width - 1] = -0.0
    x[2, width // 2] = np.nan
    x[3, :] = 7.0
    x[4, :] = -np.inf
    x[rows - 1, 0] = np.inf
    h = cx.tensor(x, device="hip")
    for op in ("sum", "mean", "max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1), f"{op} width {width}")
    xi = rng.integers(-2**31, 2**31 - 1, (rows, width), dtype=np.int64).astype(np.int32)
    hi = cx.tensor(xi, device="hip")
    for op in ("sum", "max", "min", "argmax"):
        assert_bits(getattr(cx, op)(hi, 1).numpy(), getattr(oracle, op)(xi, 1), f"i32 {op} width {width}")


@pytest.mark.parametrize("width", [65, 66, 67, 128, 130, 255, 257, 511, 512, 513, 700, 1021, 1024, 1027, 1500, 2047, 2048, 2049, 4099, 8191, 40001])
def test_unaligned_rows_head_body_tail(cx, width):
    # Rows whose length is not a multiple of 4 start at every 4-byte offset:
    # each wave segment splits into a head (to the next 16-byte boundary), a
    # float4 body and a tail. Ties, NaNs and signed zeros sit in the heads
    # and tails, where the fold must keep the lowest index. Rows of up to 512
    # elements are packed 16, 32 or 64 lanes per row, 9 rows leaving a wave
    # partly filled.
    rows = 9
    rng = np.random.default_rng(width)
    x = rng.integers(-3, 4, (rows, width)).astype(np.float32)
    flat = x.reshape(-1)
    for r in range(rows):
        x[r, 0] = 9.0                        # head ties the body's later 9
        x[r, width // 2] = 9.0
        x[r, width - 1] = -9.0               # tail ties an earlier -9
        x[r, 1] = -9.0
    x[3, width - 2] = np.nan                 # NaN in a tail
    x[4, 0] = np.nan                         # NaN in a head
    x[4, width - 1] = np.nan
    x[5, :] = -0.0
    x[5, width - 1] = 0.0
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1), f"{op} width {width}")
    y = rng.standard_normal((rows, width)).astype(np.float32)
    hy = cx.tensor(y, device="hip")
    for op in ("sum", "mean"):
        actual, expected = getattr(cx, op)(hy, 1).numpy(), getattr(oracle, op)(y, 1)
        scale = np.float64(width if op == "mean" else 1)
        assert sum_error(actual * scale, expected * scale, y, rows, width, 1) <= SUM_BAR, f"{op} {width}"
    yi = rng.integers(-2**31, 2**31 - 1, (rows, width), dtype=np.int64).astype(np.int32)
    hi = cx.tensor(yi, device="hip")
    for op in ("sum", "max", "min", "argmax"):
        assert_bits(getattr(cx, op)(hi, 1).numpy(), getattr(oracle, op)(yi, 1), f"i32 {op} width {width}")
    assert_bits(cx.sum(hi).numpy(), oracle.sum(yi, None), f"i32 full sum {width}")
