"""Softmax / RMSNorm / LayerNorm over a middle axis (inner > 1) on the hip device.

The row of (outer o, column j) is R elements, inner apart (the reference's
softmax_impl / rmsnorm_impl / layernorm_impl walk the same [outer, R, inner]
extents, cpu_backend.cpp:125-240). col_norm_kernel folds per-column
statistics over runs of rows (softmax: a running maximum and rescaled sum;
LayerNorm: count, mean and squared deviations, combined pairwise), then
writes every element from them; with few column tiles the rows are split
over blocks (statistics in a workspace, a fold launch, a write launch).
Every result is held to the row ops' bar, allclose(rtol=1e-5, atol=1e-5),
against the oracle's sequential restatement, with and without the affine
weight and bias, and with NaN, infinities, overflowing squares and constant
columns placed at wave-run and split boundaries.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import require_gpu
from hip_cases import SUM_BAR, assert_bits, assert_close, sum_error

pytestmark = pytest.mark.gpu

BAR = dict(rtol=1e-5, atol=1e-5)


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


def check_all(cx, x, axis, context, rng, eps=1e-5):
    h = cx.tensor(x, device="hip")
    n = x.shape[axis]
    g = rng.uniform(0.5, 1.5, size=n).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, size=n).astype(np.float32)
    gh, bh = cx.tensor(g, device="hip"), cx.tensor(b, device="hip")
    with np.errstate(all="ignore"):
        assert_close(cx.softmax(h, axis).numpy(), oracle.softmax(x, axis), context=f"softmax {context}", **BAR)
        assert_close(cx.rmsnorm(h, axis, eps).numpy(), oracle.rmsnorm(x, axis, eps), context=f"rmsnorm {context}",
                     **BAR)
        assert_close(cx.layernorm(h, axis, eps).numpy(), oracle.layernorm(x, axis, eps),
                     context=f"layernorm {context}", **BAR)
        assert_close(cx.layernorm(h, axis, eps, weight=gh, bias=bh).numpy(),
                     oracle.affine_norm(x, axis, eps, g, b), context=f"affine layernorm {context}", **BAR)
        assert_close(cx.rmsnorm(h, axis, eps, weight=gh).numpy(),
                     oracle.affine_norm(x, axis, eps, g, None, rms=True), context=f"affine rmsnorm {context}",
                     **BAR)


# (shape, axis): split plans (few column tiles: the backend passes a
# workspace) and unsplit ones; 256-column tiles (16-byte loads), 64-column
# tiles, and narrow columns whose waves step several rows at a time.
SHAPES = [
    ((8192, 64), 0),          # 64 columns, waves stepping 4 rows: 32 splits
    ((300, 2052), 0),         # 9 tiles of 256 (4 columns in the last): 4 splits
    ((2, 1000, 1030), 1),     # tiles of 64 (inner not a multiple of 4): 8 splits
    ((5, 3001, 7), 1),        # 7 columns of an 8-wide tile, stepping 8 rows: 4 splits
    ((64, 4096), 0),          # 64 rows: unsplit
    ((3, 777, 2, 2), 1),      # inner 4, stepping 64 rows: unsplit
    ((20_000, 3), 0),         # 3 columns of a 4-wide tile: 8 splits
    ((16, 512, 256), 1),      # 16 tiles: 8 splits
    ((7, 70, 9), 1),          # small
    ((2, 1, 5), 1),           # one row
]


@pytest.mark.parametrize("shape,axis", SHAPES)
def test_column_row_ops_random(cx, shape, axis):
    rng = np.random.default_rng(sum(shape) + axis)
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    check_all(cx, x, axis, f"{shape} axis {axis}", rng)


def plant_specials(x):
    """Non-finite and constant columns of x viewed as [R, C]."""
    rows, cols = x.shape
    marks = sorted({0, 1, 63, 64, 127, 128, rows // 3, rows // 2, rows - 2, rows - 1})
    marks = [r for r in marks if 0 <= r < rows]
    second, next_to_last = marks[min(1, len(marks) - 1)], marks[max(len(marks) - 2, 0)]
    for c in range(cols):
        kind = c % 9
        if kind == 0:
            x[marks[len(marks) // 2], c] = np.nan
        elif kind == 1:
            x[marks[-1], c] = np.inf                 # +inf last
        elif kind == 2:
            x[0, c] = -np.inf                        # -inf first
        elif kind == 3:
            x[:, c] = -np.inf                        # every value -inf
        elif kind == 4:
            x[second, c], x[next_to_last, c] = np.inf, -np.inf
        elif kind == 5:
            x[:, c] *= np.float32(1e20)              # squares overflow
        elif kind == 6:
            x[:, c] = 2.5                            # constant column
        elif kind == 7:
            x[:, c] = 2.5
            x[marks[-1], c] = 2.5000002              # equal but the last


@pytest.mark.parametrize("shape,axis", SHAPES)
def test_column_row_ops_special_values(cx, shape, axis):
    rng = np.random.default_rng(100 + sum(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    moved = np.moveaxis(x, axis, -1)
    flat = moved.reshape(-1, shape[axis]).T.copy()     # [R, outer * inner]
    plant_specials(flat)
    x = np.moveaxis(flat.T.reshape(moved.shape), -1, axis).copy()
    check_all(cx, x, axis, f"special {shape}", rng)


def test_column_softmax_long_rows_against_float64(cx):
    # 100000 rows in 64 splits. The reference's sequential float32 sum of
    # 100000 exponentials drifts: the oracle is 3.3e-5 (1.1e-4 relative)
    # from the float64 softmax at the column's largest output, past the bar.
    # The split fold stays within the bar of float64.
    rng = np.random.default_rng(100_003)
    x = (rng.standard_normal((100_000, 3)) * 3).astype(np.float32)
    x64 = x.astype(np.float64)
    truth = np.exp(x64 - x64.max(0))
    truth /= truth.sum(0)
    got = cx.softmax(cx.tensor(x, device="hip"), 0).numpy()
    assert_close(got, truth, context="softmax 100000 rows against float64", **BAR)
    assert_close(cx.rmsnorm(cx.tensor(x, device="hip"), 0).numpy(),
                 x64 / np.sqrt((x64 * x64).mean(0) + 1e-5), context="rmsnorm 100000 rows", **BAR)
    mean = x64.mean(0)
    assert_close(cx.layernorm(cx.tensor(x, device="hip"), 0).numpy(),
                 (x64 - mean) / np.sqrt(((x64 - mean) ** 2).mean(0) + 1e-5), context="layernorm 100000 rows", **BAR)


@pytest.mark.parametrize("eps", [0.0, 1e-5])
def test_column_constant_rows(cx, eps):
    # Constant columns with eps 0 (NaN for LayerNorm, as the reference) and
    # eps > 0 (zeros), split and unsplit.
    for shape, axis in (((4000, 12), 0), ((50, 300), 0)):
        x = np.full(shape, 2.5, np.float32)
        x[:, 3] = -7.0
        x[-1, 5] = 2.5000002
        x[:, 7] = 0.0
        check_all(cx, x, axis, f"constant {shape} eps {eps}", np.random.default_rng(3), eps)


def run_capi(capi, op, ptr, out, outer, rows, inner, gamma=None, beta=None, ws=False):
    workspace = capi.rownorm_workspace(outer, rows, inner) if ws else None
    if op == "softmax":
        (capi.softmax_ws(ptr, out, outer, rows, inner, workspace) if ws
         else capi.softmax(ptr, out, outer, rows, inner))
    elif op == "rmsnorm":
        (capi.rmsnorm_ws(ptr, gamma, out, outer, rows, inner, 1e-5, workspace) if ws
         else capi.rmsnorm(ptr, gamma, out, outer, rows, inner, 1e-5))
    else:
        (capi.layernorm_ws(ptr, gamma, beta, out, outer, rows, inner, 1e-5, workspace) if ws
         else capi.layernorm(ptr, gamma, beta, out, outer, rows, inner, 1e-5))
    capi.synchronize()
    return workspace


def test_column_row_ops_unaligned_and_unsplit(capi):
    # Through the C ABI: a base 4 bytes past a 16-byte boundary (4-byte
    # kernel with the splits planned for 16-byte loads), and the entry
    # points without a workspace (one unsplit launch), against the oracle.
    rng = np.random.default_rng(9)
    outer, rows, inner = 2, 3000, 132
    x = rng.standard_normal(outer * rows * inner + 1).astype(np.float32)
    x[1 + 17] = np.nan
    g = rng.uniform(0.5, 1.5, rows).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, rows).astype(np.float32)
    dx, dg, db = capi.DeviceArray.from_numpy(x), capi.DeviceArray.from_numpy(g), capi.DeviceArray.from_numpy(b)
    view = x[1:].reshape(outer, rows, inner)
    assert capi.lib().tcx_hip_rownorm_workspace_bytes(outer, rows, inner) > 0
    expected = {"softmax": oracle.softmax(view, 1),
                "rmsnorm": oracle.affine_norm(view, 1, 1e-5, g, None, rms=True),
                "layernorm": oracle.affine_norm(view, 1, 1e-5, g, b)}
    for op in ("softmax", "rmsnorm", "layernorm"):
        for ws in (False, True):
            out = capi.DeviceArray((outer * rows * inner + 1,))
            run_capi(capi, op, dx.ptr + 4, out.ptr + 4, outer, rows, inner, dg.ptr, db.ptr, ws)
            got = out.numpy()[1:].reshape(outer, rows, inner)
            assert_close(got, expected[op], context=f"unaligned {op} ws={ws}", **BAR)
    # A workspace smaller than the query is refused before any launch.
    small = capi.DeviceBuffer(64)
    out = capi.DeviceArray((outer * rows * inner,))
    with pytest.raises(capi.HipError):
        capi.softmax_ws(dx.ptr, out.ptr, outer, rows, inner, small)



def test_strided_random_shapes_and_bases(capi):
    # Seeded random [outer, R, inner] inputs reduced and normalised over the
    # middle axis through the C ABI: R and inner log-uniform (1-20000 rows,
    # 2-9000 columns, so column tiles narrower than a wave, partial tiles,
    # unsplit and split rows all occur), bases 0-3 floats past a 16-byte
    # boundary, the row ops with and without a workspace. Softmax, RMSNorm +
    # weight and LayerNorm + weight/bias meet the row-op bar, widened by the
    # oracle's own distance from float64 truth, against both truth and the
    # oracle: the reference's float32 steps drift from float64 where a few
    # terms dominate a sum or where x - mean cancels (two nearly equal
    # elements), and the kernel may drift as far. Max and argmax are
    # bit-exact, sums within the sum bar.
    rng = np.random.default_rng(37)
    failures = []
    for case in range(40):
        R = int(np.exp(rng.uniform(0.0, np.log(20000.0))))
        inner = int(np.exp(rng.uniform(np.log(2.0), np.log(9000.0))))
        outer = int(max(1, min(int(rng.integers(1, 9)), 2_000_000 // (R * inner))))
        if R * inner > 2_000_000:
            R = max(1, 2_000_000 // inner)
        off, ws = int(rng.integers(0, 4)), case % 2 == 1
        n = outer * R * inner
        flat = (rng.standard_normal(n + off) * 3).astype(np.float32)
        x = flat[off:].reshape(outer, R, inner)
        g = rng.uniform(0.5, 1.5, R).astype(np.float32)
        b = rng.uniform(-0.1, 0.1, R).astype(np.float32)
        dx, dg, db = (capi.DeviceArray.from_numpy(t) for t in (flat, g, b))
        out = capi.DeviceArray((n + off,))
        xp, op_ = dx.ptr + 4 * off, out.ptr + 4 * off
        context = f"case {case}: [{outer}, {R}, {inner}] base +{off} floats workspace={ws}"
        x64 = x.astype(np.float64)
        g64, b64 = g.astype(np.float64)[None, :, None], b.astype(np.float64)[None, :, None]
        e = np.exp(x64 - x64.max(axis=1, keepdims=True))
        mean = x64.mean(axis=1, keepdims=True)
        ln = (x64 - mean) / np.sqrt(((x64 - mean) ** 2).mean(axis=1, keepdims=True) + 1e-5)
        rms = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5)
        cases = {"softmax": (None, None, oracle.softmax(x, 1), e / e.sum(axis=1, keepdims=True)),
                 "rmsnorm": (dg.ptr, None, oracle.affine_norm(x, 1, 1e-5, g, None, rms=True), rms * g64),
                 "layernorm": (dg.ptr, db.ptr, oracle.affine_norm(x, 1, 1e-5, g, b), ln * g64 + b64)}
        try:
            for op, (gp, bp, expected, truth) in cases.items():
                run_capi(capi, op, xp, op_, outer, R, inner, gp, bp, ws)
                got = out.numpy()[off:].reshape(outer, R, inner)
                drift = float(np.max(np.abs(expected - truth) / np.maximum(np.abs(truth), 1e-30)))
                assert_close(got, truth, 1e-5 + drift, 1e-5, f"{op} vs float64 {context} (oracle drift {drift:.1e})")
                assert_close(got, expected, 1e-5 + drift, 1e-5, f"{op} {context} (oracle drift {drift:.1e})")
            res = capi.DeviceArray((outer * inner,))
            for op in ("max", "argmax", "sum"):
                workspace = capi.reduce_workspace(op, capi.TCX_FLOAT32, outer, R, inner)
                capi.reduce(op, capi.TCX_FLOAT32, xp, res.ptr, outer, R, inner, workspace)
                capi.synchronize()
                got = res.numpy().reshape(outer, inner)
                if op == "max":
                    assert_bits(got, oracle.max(x, 1), f"max {context}")
                elif op == "argmax":
                    assert_bits(got.view(np.int32), oracle.argmax(x, 1), f"argmax {context}")
                else:
                    err = sum_error(got, oracle.sum(x, 1), x, outer, R, inner)
                    assert err <= SUM_BAR, f"sum {context}: {err:.3e}"
        except AssertionError as error:
            failures.append(str(error))
    assert not failures, "\n".join(failures[:10])


@pytest.mark.parametrize("width", [1, 2, 3, 4, 5, 7, 8, 16, 31, 32, 33, 64, 100, 127, 128])
def test_packed_short_rows(cx, width):
    # Contiguous rows of at most 128 elements pack 64 / L rows per wave (L
    # lanes per row); 1001 rows leave a partly filled last wave. Special
    # rows: a NaN, infinities, a constant row (LayerNorm's fill), overflowing
    # squares.
    rng = np.random.default_rng(width)
    x = (rng.standard_normal((1001, width)) * 3).astype(np.float32)
    x[0, width // 2] = np.nan
    x[1, width - 1] = np.inf
    x[2, 0] = -np.inf
    x[3] = -np.inf
    x[4] = 2.5
    x[5] *= np.float32(1e20)
    check_all(cx, x, 1, f"packed width {width}", rng)
    for eps in (0.0, 1e-5):
        check_all(cx, np.full((70, width), 2.5, np.float32), 1, f"constant width {width} eps {eps}", rng, eps)
