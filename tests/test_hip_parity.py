"""GPU parity of the hip device against the CPU oracle and reference golden
vectors, through tensorcx -> HipBackend::execute -> C ABI -> gfx950 kernels.

Bars are those of tests/hip_cases.py. Sizes: golden vectors (small, from the
reference CPU backend), random edge shapes (oracle), and the BASELINE.json
configs at full size (oracle, multithreaded but bit-identical).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import require_gpu
from hip_cases import (assert_bits, assert_close, assert_matmul, check_case, host, run_hip,
                       sum_error)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cx():
    require_gpu()
    import tensorcx
    return tensorcx


# ------------------------------------------------------------- golden vectors
def test_golden_vectors(cx, golden):
    manifest, arrays = golden
    failures = []
    for entry in manifest:
        inputs = [arrays[k] for k in entry["inputs"]]
        name, op, kw = entry["name"], entry["op"], entry["kwargs"]
        if "error" in entry:
            with pytest.raises(ValueError):
                host(run_hip(cx, op, inputs, kw))
            continue
        try:
            actual = host(run_hip(cx, op, inputs, kw))
            expected = (tuple(arrays[k] for k in entry["outputs"]) if "outputs" in entry
                        else arrays[entry["output"]])
            check_case(name, op, inputs, kw, actual, expected)
        except AssertionError as error:
            failures.append(str(error))
    assert not failures, f"{len(failures)} golden cases failed:\n" + "\n".join(failures[:20])


# ------------------------------------------------------------- matmul
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (2, 3, 4), (15, 17, 31), (17, 16, 15), (32, 33, 16),
                                   (0, 3, 4), (3, 0, 4), (3, 4, 0), (65, 129, 67), (128, 128, 128),
                                   (129, 255, 257), (300, 64, 200), (700, 300, 500), (512, 512, 512),
                                   (768, 768, 768), (1000, 1000, 1000), (1000, 1004, 996)])
def test_matmul_shapes(cx, m, k, n):
    rng = np.random.default_rng(7)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    expected = oracle.matmul(a, b)
    if k == 0:
        assert_bits(actual, expected, "k=0")
    else:
        assert_matmul(actual, expected, a, b, f"{m}x{k}x{n}")


@pytest.mark.parametrize("size", [1000, 1100])
def test_matmul_direct64_k_tail_isolation(cx, size):
    # Direct-to-LDS tiles with a K tail: 1000 = 15 x 64 + 40 (256 tiles of
    # 64x64) and 1100 = 17 x 64 + 12 (324 tiles of 64x64, whose last round of
    # 68 runs the 32x64 tiles). An infinity at the start of the next row,
    # which the tail of a row's last k-tile would read, must not reach that
    # row (it is zeroed, not 0 * inf).
    rng = np.random.default_rng(14)
    a = rng.standard_normal((size, size)).astype(np.float32)
    b = rng.standard_normal((size, size)).astype(np.float32)
    a[5, 0] = np.inf           # row 4's tail reads a[5, 0..] past its K
    a[9, size - 1] = -np.inf   # row 9 itself: -inf times its B row
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    with np.errstate(invalid="ignore"):
        truth = a.astype(np.float64) @ b.astype(np.float64)
    assert np.all(np.isfinite(actual[4])) and np.all(np.isfinite(actual[10]))
    bad = [5, 9]
    assert np.array_equal(np.isinf(actual[bad]), np.isinf(truth[bad]))
    assert np.array_equal(np.isnan(actual[bad]), np.isnan(truth[bad]))
    keep = np.setdiff1d(np.arange(size), bad)
    assert_matmul(actual[keep], truth[keep], a[keep], b, "direct64 finite rows")
    # Transposed B (a linear's weight): the weight row after a column's row.
    w = rng.standard_normal((size, size)).astype(np.float32)
    w[7, 0] = np.inf
    lin = cx.linear(cx.tensor(a[keep], device="hip"), cx.tensor(w, device="hip")).numpy()
    with np.errstate(invalid="ignore"):
        lt = a[keep].astype(np.float64) @ w.astype(np.float64).T
    assert np.all(np.isfinite(lin[:, 6])) and np.array_equal(np.isinf(lin[:, 7]), np.isinf(lt[:, 7]))
    others = np.setdiff1d(np.arange(size), [7])
    assert_matmul(lin[:, others], lt[:, others], a[keep], w[others].T, "direct64 linear finite columns")


@pytest.mark.parametrize("batches", [2, 4])
def test_matmul_direct64_kn_b_k_tail_isolation(cx, batches):
    # A [k, n] B with K = 700 = 10 x 64 + 60: batch 0's last k-tile spans
    # k rows 640..703, and rows 700..703 of that span are batch 1's B rows
    # 0..3. Infinities there must read as zero for batch 0 (not 0 * inf), and
    # still reach batch 1's outputs as the reference's sums give them. Two
    # batches make 160 tiles of 64x64; four make 320, whose last round of 64
    # runs the 32x64 tiles.
    rng = np.random.default_rng(16)
    a = rng.standard_normal((batches, 500, 700)).astype(np.float32)
    b = rng.standard_normal((batches, 700, 600)).astype(np.float32)
    b[1, 0:4, :] = np.inf
    b[1, 2, 5] = -np.inf
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    for i in [0] + list(range(2, batches)):
        assert np.all(np.isfinite(actual[i]))
        assert_matmul(actual[i], a[i].astype(np.float64) @ b[i].astype(np.float64), a[i], b[i], f"batch {i}")
    with np.errstate(invalid="ignore"):
        truth = a[1].astype(np.float64) @ b[1].astype(np.float64)
    assert np.array_equal(np.isnan(actual[1]), np.isnan(truth))
    assert np.array_equal(np.isinf(actual[1]), np.isinf(truth))


@pytest.mark.parametrize("sa,sb", [((4, 500, 700), (4, 700, 600)), ((3, 1000, 1000), (1000, 1000)),
                                   ((8192, 1000), (1000, 4)), ((4, 1000), (1000, 8192)),
                                   ((999, 1001), (1001, 1003)), ((1200, 1204), (1204, 1196)),
                                   ((1599, 1600), (1600, 1596)), ((2, 700, 1100), (2, 1100, 1012))])
def test_matmul_direct64_batched(cx, sa, sb):
    # Batched 64x64-tile shapes, skinny shapes (a 4-wide n runs the
    # streaming kernel, a 4-wide m with a [k, n] B the small kernel's 32x32
    # tiles, all but 4 rows of each tile past the edge), an unaligned k
    # (1001) that takes the register-staged 64x64 tile instead, and shapes
    # whose last round of 64x64 tiles holds at most 128 (4 x 500x600: 320
    # tiles; 1200 x 1196: 361; 1599 x 1596: 625, three rounds; 2 x 700 x
    # 1012: 352), which run 32x64 tiles with edges in m, n and k.
    rng = np.random.default_rng(15)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(actual, a.astype(np.float64) @ b.astype(np.float64), a, b, f"direct64 {sa}x{sb}")


# Shapes of fewer than 128 output tiles of 64x64 with 16-byte rows run the
# register-direct small kernel: 32x32 tiles, the K split over 1 to 16 waves
# (one 16-k chunk per wave at least), edges through buffer range checks
# ((16384, 512) x (512, 4), 4 columns against 16384 rows, runs the streaming
# kernel).
@pytest.mark.parametrize("sa,sb", [((1, 4), (4, 4)), ((31, 4), (4, 36)), ((33, 20), (20, 36)),
                                   ((100, 300), (300, 200)), ((64, 4096), (4096, 64)), ((2, 3, 60), (60, 40)),
                                   ((7, 33, 68), (68, 12)), ((500, 600), (600, 400)), ((512, 512), (512, 512)),
                                   ((3, 1, 40, 36), (1, 5, 36, 44)), ((256, 2048), (2048, 512)),
                                   ((16384, 512), (512, 4)), ((4, 1000), (1000, 16384))])
def test_matmul_small_kernel(cx, sa, sb):
    rng = np.random.default_rng(21)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(actual, np.matmul(a.astype(np.float64), b.astype(np.float64)), a, b, f"small {sa}x{sb}")


def test_matmul_small_kernel_skinny_batched(cx):
    # 64 batches of 200 x 4 outputs: 256 tiles of 64x64, mostly padding, so
    # the small kernel's 32x32 tiles (eight waves each) take them; 200 rows
    # per batch are too few for the streaming kernel.
    rng = np.random.default_rng(24)
    a = rng.standard_normal((64, 200, 512)).astype(np.float32)
    b = rng.standard_normal((64, 512, 4)).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(actual, np.matmul(a.astype(np.float64), b.astype(np.float64)), a, b, "small skinny batched")


def test_matmul_random_shapes_every_route(cx):
    # Seeded random shapes across every GEMM route (small 32x32 tiles, the
    # skinny route, 64x64 direct and register-staged tiles, aligned and
    # unaligned rows, transposed B, batches with broadcast), each against
    # float64 truth at the matmul bar.
    rng = np.random.default_rng(25)
    failures = []
    for case in range(96):
        m, n, k = (int(v) for v in rng.integers(1, 700, 3))
        if case % 3 == 0:  # 16-byte rows
            n, k = 4 * ((n + 3) // 4), 4 * ((k + 3) // 4)
        batch = int(rng.integers(1, 4)) if case % 4 == 1 else 0
        linear = case % 5 == 2
        a = rng.standard_normal(((batch,) if batch else ()) + (m, k)).astype(np.float32)
        if linear:
            w = rng.standard_normal((n, k)).astype(np.float32)
            got = cx.linear(cx.tensor(a, device="hip"), cx.tensor(w, device="hip")).numpy()
            b = w.T
        else:
            b = rng.standard_normal(((batch,) if batch and case % 8 == 1 else ()) + (k, n)).astype(np.float32)
            got = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
        truth = np.matmul(a.astype(np.float64), b.astype(np.float64))
        try:
            assert_matmul(got, truth, a, b, f"case {case}: a {a.shape} b {b.shape} linear={linear}")
        except AssertionError as error:
            failures.append(str(error))
    assert not failures, "\n".join(failures[:10])


def test_matmul_random_streaming_and_split_routes(cx):
    # Seeded random shapes aimed at the streaming kernel (one side of at most
    # 32 against 256+ rows, both B layouts, batches) and at the K splits
    # (multiples of 128 with few tiles or a badly filled last round), each
    # against float64 truth at the matmul bar.
    rng = np.random.default_rng(26)
    failures = []
    for case in range(40):
        kind = case % 4
        k = 4 * int(rng.integers(1, 600))
        if kind == 0:    # linear with at most 32 rows of x
            m, n = int(rng.integers(1, 33)), int(rng.integers(256, 3000))
        elif kind == 1:  # at most 32 columns of B
            m, n = int(rng.integers(256, 3000)), int(rng.integers(1, 33))
        elif kind == 2:  # few 128x128 tiles, long K: split K
            m, n, k = 128 * int(rng.integers(1, 9)), 128 * int(rng.integers(1, 9)), 128 * int(rng.integers(8, 33))
        else:            # 256+ tiles with a partial last round
            m, n, k = 128 * int(rng.integers(16, 24)), 128 * int(rng.integers(16, 24)), 128 * int(rng.integers(3, 7))
        batch = int(rng.integers(2, 4)) if case % 5 == 3 and kind != 3 else 0
        lead = (batch,) if batch else ()
        a = rng.standard_normal(lead + (m, k)).astype(np.float32)
        if kind == 0:
            w = rng.standard_normal((n, k)).astype(np.float32)
            got = cx.linear(cx.tensor(a, device="hip"), cx.tensor(w, device="hip")).numpy()
            b = w.T
        else:
            b = rng.standard_normal(lead + (k, n)).astype(np.float32)
            got = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
        truth = np.matmul(a.astype(np.float64), b.astype(np.float64))
        try:
            assert_matmul(got, truth, a, b, f"case {case}: a {a.shape} b {b.shape} kind {kind}")
        except AssertionError as error:
            failures.append(str(error))
    assert not failures, "\n".join(failures[:10])


def test_matmul_small_kernel_k_tail_isolation(cx):
    # K = 60: each row's last 16-k chunk spans k 48..63, and k 60..63 of a
    # [k, n] B are the next batch's rows 0..3, of an A row the next row's
    # first four values. Infinities there must read as zero (not 0 * inf) and
    # still reach their own outputs as the float64 sums give them.
    rng = np.random.default_rng(22)
    a = rng.standard_normal((2, 40, 60)).astype(np.float32)
    b = rng.standard_normal((2, 60, 36)).astype(np.float32)
    b[1, 0:4, :] = np.inf
    b[1, 2, 5] = -np.inf
    a[0, 7, 0:4] = np.inf  # row 6's tail would read these
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    with np.errstate(invalid="ignore"):
        truth = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert np.all(np.isfinite(np.delete(actual[0], 7, axis=0)))
    assert np.array_equal(np.isnan(actual), np.isnan(truth))
    assert np.array_equal(np.isinf(actual), np.isinf(truth))
    keep = np.setdiff1d(np.arange(40), [7])
    assert_matmul(actual[0][keep], truth[0][keep], a[0][keep], b[0], "small batch 0")
    # Transposed B (a linear's weight [n, k]): the next weight row's start.
    w = rng.standard_normal((36, 60)).astype(np.float32)
    w[5, 0:4] = np.inf
    x = a[1]
    lin = cx.linear(cx.tensor(x, device="hip"), cx.tensor(w, device="hip")).numpy()
    with np.errstate(invalid="ignore"):
        lt = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.all(np.isfinite(lin[:, 4])) and np.array_equal(np.isinf(lin[:, 5]), np.isinf(lt[:, 5]))
    assert_matmul(lin[:, :5], lt[:, :5], x, w[:5].T, "small linear finite columns")


@pytest.mark.parametrize("k", [4, 16, 28, 64, 132, 1024, 4100])
def test_linear_small_kernel_bias_activation(cx, k):
    # Every K split width (1 to 16 waves), a transposed B, and the fused bias
    # and SiLU / GELU epilogue split over the block's waves.
    rng = np.random.default_rng(23 + k)
    x = rng.standard_normal((70, k)).astype(np.float32)
    w = rng.standard_normal((52, k)).astype(np.float32)
    bias = rng.standard_normal(52).astype(np.float32)
    xh, wh, bh = (cx.tensor(v, device="hip") for v in (x, w, bias))
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert_matmul(cx.linear(xh, wh, bh).numpy(), exact + bias, x, w.T, f"small linear k={k}")
    z = exact + bias
    bound = 1.1e-4 * np.sqrt(k) * np.sqrt(np.mean(x * x)) * np.sqrt(np.mean(w * w)) + 1e-6
    silu = cx.hip.linear_act(xh, wh, bh, "silu").numpy()
    assert np.max(np.abs(silu - z / (1.0 + np.exp(-z)))) <= bound
    gelu = cx.hip.linear_act(xh, wh, bh, "gelu").numpy()
    expected = 0.5 * z * (1.0 + np.tanh(0.7978845608028654 * (z + 0.044715 * z ** 3)))
    assert np.max(np.abs(gelu - expected)) <= bound


# One skinny operand against a long one (at least 256 rows) runs the
# streaming kernel: at most 32 rows of A against a transposed B (a linear), or
# at most 32 columns of B in either layout. The long operand's rows are read
# once, 16 per block, K split over 1 to 16 waves; rows past the edge and k
# past K read zero. A linear whose blocks all stay resident stages both
# operands in LDS (5, 16, 17, 32 and 2 rows here, the last over 11008 W rows
# at two waves per block); 4 rows over 14336 (one wave per block) and 20 over
# 20000 (too many blocks to stay resident) keep the register kernel. 33 rows
# (and columns) are the first past it.
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (5, 1000, 300), (16, 256, 4), (17, 4100, 1028),
                                   (32, 2048, 64), (32, 300, 8), (33, 3000, 516), (2, 11008, 512),
                                   (4, 14336, 64), (20, 20000, 68)])
def test_linear_streaming_skinny_rows(cx, m, n, k):
    rng = np.random.default_rng(40 + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    xh, wh, bh = (cx.tensor(v, device="hip") for v in (x, w, bias))
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert_matmul(cx.linear(xh, wh).numpy(), exact, x, w.T, f"streaming linear {m}x{n}x{k}")
    z = exact + bias
    bound = 1.1e-4 * np.sqrt(k) * np.sqrt(np.mean(x * x)) * np.sqrt(np.mean(w * w)) + 1e-6
    silu = cx.hip.linear_act(xh, wh, bh, "silu").numpy()
    assert np.max(np.abs(silu - z / (1.0 + np.exp(-z)))) <= bound


@pytest.mark.parametrize("batch,m,n,k", [(3, 12, 700, 520), (2, 24, 300, 1000), (1, 20, 300, 1000),
                                         (4, 3, 1000, 256), (1, 16, 4096, 4096), (1, 32, 2048, 2048)])
def test_linear_streaming_batched_transposed(cx, batch, m, n, k):
    # x W^T through the C ABI with a batch axis on both operands, and again
    # with the weight broadcast (batch stride 0): the LDS-staged streaming
    # kernel at one and two row groups of x, one to four waves per block, a
    # K tail (520, 1000) and rows of W past the last 16-row block (700, 300),
    # with a bias and SiLU in the second pass; 3 rows of x over 1000 W rows
    # keep two waves per block.
    import tensorcx_hip_capi as capi
    rng = np.random.default_rng(90 + m)
    x = rng.standard_normal((batch, m, k)).astype(np.float32)
    w = rng.standard_normal((batch, n, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    dx, db = capi.DeviceArray.from_numpy(x), capi.DeviceArray.from_numpy(bias)
    for shared in (False, True):
        wb = w[:1] if shared else w
        dw = capi.DeviceArray.from_numpy(wb)
        out = capi.DeviceArray((batch, m, n))
        act = "silu" if shared else "none"
        d = capi.gemm_desc(m, n, k, batch_shape=(batch,), lhs_batch_strides=(m * k,),
                           rhs_batch_strides=(0 if shared else n * k,), rhs_transposed=True,
                           bias=db.ptr if shared else None, activation=act)
        capi.gemm(dx.ptr, dw.ptr, out.ptr, d)
        capi.synchronize()
        got = out.numpy()
        wf = np.broadcast_to(wb, w.shape).astype(np.float64)
        exact = np.matmul(x.astype(np.float64), np.swapaxes(wf, 1, 2))
        if not shared:
            for i in range(batch):
                assert_matmul(got[i], exact[i], x[i], wf[i].T, f"streaming batch {i} {m}x{n}x{k}")
        else:
            z = exact + bias
            bound = 1.1e-4 * np.sqrt(k) * np.sqrt(np.mean(x * x)) * np.sqrt(np.mean(w[0] * w[0])) + 1e-6
            assert np.max(np.abs(got - z / (1.0 + np.exp(-z)))) <= bound


@pytest.mark.parametrize("sa,sb", [((4096, 4096), (4096, 1)), ((1000, 300), (300, 7)), ((300, 16), (16, 32)),
                                   ((3, 500, 68), (3, 68, 20)), ((2, 1, 400, 132), (3, 132, 28)),
                                   ((8192, 1000), (1000, 4)), ((257, 4100), (4100, 17)), ((600, 200), (200, 33))])
def test_matmul_streaming_skinny_columns(cx, sa, sb):
    # [k, n] B of at most 64 columns (its rows read as columns of the skinny
    # operand), batches with broadcast, and the same shapes as a linear with
    # the weight [n, k].
    rng = np.random.default_rng(50 + sb[-1])
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(actual, np.matmul(a.astype(np.float64), b.astype(np.float64)), a, b, f"streaming {sa}x{sb}")
    if b.ndim == 2:
        w = np.ascontiguousarray(b.T)
        lin = cx.linear(cx.tensor(a, device="hip"), cx.tensor(w, device="hip")).numpy()
        assert_matmul(lin, np.matmul(a.astype(np.float64), b.astype(np.float64)), a, b, f"streaming linear {sa}")


@pytest.mark.parametrize("n,k", [(4096, 4096), (1, 4), (7, 4100), (300, 8), (2000, 1028), (11008, 512),
                                 (5000, 64)])
def test_gemv_one_row_and_one_column(cx, n, k):
    # One row of x against a weight [n, k] (the decode-time linear), and one
    # column of B in both layouts: rows streamed in whole cache lines, K
    # split over 1, 2 or 4 waves by the row count.
    rng = np.random.default_rng(70 + n)
    x = rng.standard_normal((1, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    xh, wh, bh = (cx.tensor(v, device="hip") for v in (x, w, bias))
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert_matmul(cx.linear(xh, wh).numpy(), exact, x, w.T, f"gemv linear {n}x{k}")
    z = exact + bias
    bound = 1.1e-4 * np.sqrt(k) * np.sqrt(np.mean(x * x)) * np.sqrt(np.mean(w * w)) + 1e-6
    gelu = cx.hip.linear_act(xh, wh, bh, "gelu").numpy()
    expected = 0.5 * z * (1.0 + np.tanh(0.7978845608028654 * (z + 0.044715 * z ** 3)))
    assert np.max(np.abs(gelu - expected)) <= bound
    col = np.ascontiguousarray(x.T)
    got = cx.matmul(wh, cx.tensor(col, device="hip")).numpy()
    assert_matmul(got, w.astype(np.float64) @ col.astype(np.float64), w, col, f"gemv column {n}x{k}")
    got_t = cx.linear(wh, xh).numpy()
    assert_matmul(got_t, w.astype(np.float64) @ col.astype(np.float64), w, col, f"gemv column linear {n}x{k}")


def test_gemv_batched_and_special_values(cx):
    # A batch axis on both operands and broadcast on one; a NaN and an inf in
    # one row each, and a dyadic case that must be exact in any order.
    rng = np.random.default_rng(77)
    a = rng.standard_normal((3, 500, 260)).astype(np.float32)
    b = rng.standard_normal((3, 260, 1)).astype(np.float32)
    a[1, 7, 100] = np.nan
    a[2, 9, 3] = np.inf
    got = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    with np.errstate(invalid="ignore"):
        truth = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert np.array_equal(np.isnan(got), np.isnan(truth)) and np.array_equal(np.isinf(got), np.isinf(truth))
    finite = np.isfinite(truth)
    assert np.max(np.abs(got[finite] - truth[finite])) <= 1e-4 * np.sqrt(260) * 1.1
    shared = rng.standard_normal((260, 1)).astype(np.float32)
    got2 = cx.matmul(cx.tensor(a[0:1], device="hip"), cx.tensor(shared, device="hip")).numpy()
    assert_matmul(got2[0], a[0].astype(np.float64) @ shared.astype(np.float64), a[0], shared, "gemv broadcast")
    i = np.arange(3000 * 1000)
    w = ((i % 11 - 5) / 8).astype(np.float32).reshape(3000, 1000)
    x = ((np.arange(1000) % 7 - 3) / 16).astype(np.float32).reshape(1, 1000)
    lin = cx.linear(cx.tensor(x, device="hip"), cx.tensor(w, device="hip")).numpy()
    assert_bits(lin, (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32), "gemv dyadic")


def test_streaming_k_tail_and_row_isolation(cx):
    # K = 60: the last 16-k chunk spans k 48..63; k 60..63 of a row are the
    # next row's first values (and past the last row, memory past the
    # operand). Infinities there must read as zero, not 0 * inf, and still
    # reach their own outputs as the float64 sums give them.
    rng = np.random.default_rng(60)
    x = rng.standard_normal((9, 60)).astype(np.float32)
    w = rng.standard_normal((300, 60)).astype(np.float32)
    w[5, 0:4] = np.inf       # row 4's tail would read these
    x[3, 0:4] = -np.inf      # x row 2's tail would read these
    with np.errstate(invalid="ignore"):
        truth = x.astype(np.float64) @ w.astype(np.float64).T
    lin = cx.linear(cx.tensor(x, device="hip"), cx.tensor(w, device="hip")).numpy()
    assert np.array_equal(np.isnan(lin), np.isnan(truth))
    assert np.array_equal(np.isinf(lin), np.isinf(truth))
    assert np.all(np.isfinite(lin[2, :5])) and np.all(np.isfinite(lin[:3, 4]))
    rows = [0, 1, 2, 4, 5, 6, 7, 8]
    cols = np.setdiff1d(np.arange(300), [5])
    assert_matmul(lin[np.ix_(rows, cols)], truth[np.ix_(rows, cols)], x[rows], w[cols].T, "streaming finite part")
    # Skinny columns of a [k, n] B: A rows stream, B's columns are gathered.
    a = rng.standard_normal((400, 60)).astype(np.float32)
    a[11, 0:4] = np.inf      # row 10's tail would read these
    b = rng.standard_normal((60, 12)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        t2 = a.astype(np.float64) @ b.astype(np.float64)
    got = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert np.array_equal(np.isnan(got), np.isnan(t2)) and np.all(np.isfinite(got[10]))
    keep = np.setdiff1d(np.arange(400), [11])
    assert_matmul(got[keep], t2[keep], a[keep], b, "streaming columns finite part")


def test_streaming_dyadic_exact(cx):
    # Exact in any summation order: pins the streaming kernel's k mapping,
    # row placement and wave-ordered combine bit for bit, in all three roles.
    i = np.arange(40 * 1000)
    x = ((i % 11 - 5) / 8).astype(np.float32).reshape(40, 1000)
    j = np.arange(1000 * 600)
    w = ((j % 7 - 3) / 16).astype(np.float32).reshape(600, 1000)
    truth = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    lin = cx.linear(cx.tensor(x, device="hip"), cx.tensor(w, device="hip")).numpy()
    assert_bits(lin, truth, "streaming dyadic linear")
    got = cx.matmul(cx.tensor(w, device="hip"), cx.tensor(np.ascontiguousarray(x.T), device="hip")).numpy()
    assert_bits(got, np.ascontiguousarray(truth.T), "streaming dyadic columns")
    lin2 = cx.linear(cx.tensor(w, device="hip"), cx.tensor(x, device="hip")).numpy()
    assert_bits(lin2, np.ascontiguousarray(truth.T), "streaming dyadic linear columns")


def test_matmul_small_kernel_dyadic_exact(cx):
    # Exact in any summation order: pins the small kernel's k mapping, tile
    # placement and the wave-ordered combine bit for bit.
    i = np.arange(96 * 200)
    a = ((i % 11 - 5) / 8).astype(np.float32).reshape(96, 200)
    j = np.arange(200 * 68)
    b = ((j % 7 - 3) / 16).astype(np.float32).reshape(200, 68)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_bits(actual, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32), "small dyadic")
    lin = cx.linear(cx.tensor(a, device="hip"), cx.tensor(np.ascontiguousarray(b.T), device="hip")).numpy()
    assert_bits(lin, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32), "small dyadic linear")


@pytest.mark.parametrize("sa,sb", [((1024, 8192), (8192, 1024)), ((2048, 4096), (4096, 2048)),
                                   ((4, 512, 8192), (4, 8192, 512)), ((3072, 2048), (2048, 2048)),
                                   ((1536, 1536), (1536, 1536))])
def test_matmul_split_k(cx, sa, sb):
    # Few output tiles and a long K, or a last round of tiles that would leave
    # most CUs idle (3072 x 2048: 384 tiles, two splits; 1536^3: 144 tiles,
    # four splits): K split over blocks through the pool workspace, checked
    # against float64 truth at the matmul bar.
    rng = np.random.default_rng(11)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(actual, a.astype(np.float64) @ b.astype(np.float64), a, b, f"split {sa}x{sb}")


def test_matmul_split_k_special_values(cx):
    # Non-finite values in different K splits: +inf alone, +inf and -inf in two
    # splits of one row, NaN. The partials add as the unsplit sum would:
    # NaN / inf positions and signs as float64 truth, the rest at the bar.
    rng = np.random.default_rng(13)
    a = rng.standard_normal((1024, 8192)).astype(np.float32)
    b = rng.standard_normal((8192, 1024)).astype(np.float32)
    a[0, 10] = np.inf
    a[1, 100], a[1, 5000] = np.inf, -np.inf
    a[2, 7000] = np.nan
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    with np.errstate(invalid="ignore"):
        truth = a.astype(np.float64) @ b.astype(np.float64)
    head = slice(0, 3)
    assert np.array_equal(np.isnan(actual[head]), np.isnan(truth[head]))
    assert np.array_equal(np.isinf(actual[head]), np.isinf(truth[head]))
    inf = np.isinf(truth[head])
    assert np.array_equal(np.sign(actual[head][inf]), np.sign(truth[head][inf]))
    assert_matmul(actual[3:], truth[3:], a[3:], b, "split special values, finite rows")


def test_gemm_split_k_matches_unsplit(cx):
    # The C ABI with and without the workspace, linear form with bias + SiLU:
    # both within the bar of float64 truth, and of each other.
    import tensorcx_hip_capi as capi
    rng = np.random.default_rng(12)
    x = rng.standard_normal((2048, 4096)).astype(np.float32)
    w = rng.standard_normal((1024, 4096)).astype(np.float32)
    bias = rng.standard_normal(1024).astype(np.float32)
    dx, dw, db = (capi.DeviceArray.from_numpy(t) for t in (x, w, bias))
    d = capi.gemm_desc(2048, 1024, 4096, rhs_transposed=True, bias=db.ptr, activation="silu")
    ws = capi.gemm_workspace(d)
    assert ws is not None and ws.nbytes == 4 * 2048 * 1024 * 4
    outs = []
    for workspace in (None, ws):
        out = capi.DeviceArray((2048, 1024))
        capi.gemm(dx.ptr, dw.ptr, out.ptr, d, None, workspace)
        capi.synchronize()
        outs.append(out.numpy())
    pre = x.astype(np.float64) @ w.astype(np.float64).T + bias
    truth = pre / (1 + np.exp(-pre))
    scale = 1e-4 * np.sqrt(4096) * np.sqrt(np.mean(x.astype(np.float64) ** 2) * np.mean(w.astype(np.float64) ** 2))
    for out in outs:
        assert np.max(np.abs(out - truth)) <= scale
    assert np.max(np.abs(outs[0] - outs[1])) <= scale


def test_matmul_dyadic_is_exact(cx):
    # Dyadic inputs make every partial sum exact, so any order matches bitwise.
    i = np.arange(6 * 130 * 70)
    a = ((i % 11 - 5) / 8).astype(np.float32).reshape(6, 130, 70)
    j = np.arange(6 * 70 * 90)
    b = ((j % 7 - 3) / 8).astype(np.float32).reshape(6, 70, 90)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_bits(actual, oracle.matmul(a, b), "dyadic batched")


@pytest.mark.parametrize("sa,sb", [((4096, 32), (32, 4096)), ((4096, 96), (96, 4096)),
                                   ((8, 1024, 512), (512, 2048)), ((2, 1, 2048, 256), (1, 4, 256, 2048))])
def test_matmul_full_tiles(cx, sa, sb):
    """Shapes of >= 256 full 128x128 tiles take the direct-to-LDS kernel: one
    k-tile, an odd k-tile count, a broadcast batch on either side. Checked
    against float64 products under the matmul bar."""
    rng = np.random.default_rng(17)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(actual, np.matmul(a.astype(np.float64), b.astype(np.float64)), a, b, f"{sa}@{sb}")


@pytest.mark.parametrize("sa,sb", [((32, 1024, 1024), (32, 1024, 1024)), ((65, 384, 96), (65, 96, 384)),
                                   ((72, 512, 96), (96, 512)), ((600, 256, 128), (600, 128, 256)),
                                   ((34, 256, 4096), (34, 4096, 256))])
def test_matmul_persistent_tiles(cx, sa, sb):
    """More full items than blocks that fit at once: the direct kernel runs a
    persistent grid, each block taking several items and issuing the next
    item's loads before its stores. On 128x128 tiles (512 blocks): the
    bench's batched config (2048 items, four per block), an item count that is
    not a multiple of 8 (585, plain order) with an odd k-tile count, the XCD
    order with an odd k-tile count and a broadcast B (1152 items), up to five
    items per block (2400), and K split over 4 items per tile (136 tiles, 544
    items). Checked against float64 products."""
    rng = np.random.default_rng(19)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(actual, np.matmul(a.astype(np.float64), b.astype(np.float64)), a, b, f"{sa}@{sb}")


@pytest.mark.parametrize("n,linear", [(1024, False), (4096, False), (2048, True)])
def test_matmul_full_tiles_special_values(cx, n, linear):
    # Non-finite values through the direct 128x128 kernel: one item per block
    # (1024 columns, 512 items), the persistent grid (4096 columns, four items
    # per block) and the transposed-B linear. A +inf, a -inf and a NaN in rows of A and a
    # +inf in a column of B: NaN / inf positions and signs as float64 truth,
    # the finite rest at the matmul bar.
    rng = np.random.default_rng(31)
    a = rng.standard_normal((8192, 64)).astype(np.float32)
    b = rng.standard_normal((64, n)).astype(np.float32)
    a[5, 3], a[300, 10], a[4000, 63] = np.inf, -np.inf, np.nan
    b[7, n - 1] = np.inf
    ah = cx.tensor(a, device="hip")
    if linear:
        actual = cx.linear(ah, cx.tensor(np.ascontiguousarray(b.T), device="hip")).numpy()
    else:
        actual = cx.matmul(ah, cx.tensor(b, device="hip")).numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        truth = a.astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(np.isnan(actual), np.isnan(truth))
    assert np.array_equal(np.isinf(actual), np.isinf(truth))
    inf = np.isinf(truth)
    assert np.array_equal(np.sign(actual[inf]), np.sign(truth[inf]))
    rows = np.setdiff1d(np.arange(8192), [5, 300, 4000])
    assert_matmul(actual[rows][:, :n - 1], truth[rows][:, :n - 1], a[rows], b[:, :n - 1], "special full tiles")


def test_matmul_persistent_tiles_dyadic_exact(cx):
    # Exact in any order: pins the item -> tile map of the persistent grid bit
    # for bit (585 items of 128x128, plain order, three k-tiles).
    i = np.arange(65 * 384 * 96)
    a = ((i % 13 - 6) / 8).astype(np.float32).reshape(65, 384, 96)
    j = np.arange(65 * 96 * 384)
    b = ((j % 9 - 4) / 16).astype(np.float32).reshape(65, 96, 384)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_bits(actual, np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32),
                "dyadic persistent")


def test_gemm_persistent_bias_activation(cx):
    # The C ABI with a [k, n] B, bias and SiLU over 2048 full tiles: the
    # persistent kernel's bias path (bias loads before the next item's tile
    # loads), against float64 truth at the matmul bar.
    import tensorcx_hip_capi as capi
    rng = np.random.default_rng(20)
    x = rng.standard_normal((8192, 64)).astype(np.float32)
    w = rng.standard_normal((64, 4096)).astype(np.float32)
    bias = rng.standard_normal(4096).astype(np.float32)
    dx, dw, db = (capi.DeviceArray.from_numpy(t) for t in (x, w, bias))
    out = capi.DeviceArray((8192, 4096))
    capi.gemm(dx.ptr, dw.ptr, out.ptr, capi.gemm_desc(8192, 4096, 64, bias=db.ptr, activation="silu"))
    capi.synchronize()
    pre = x.astype(np.float64) @ w.astype(np.float64) + bias
    truth = pre / (1 + np.exp(-pre))
    scale = 1e-4 * np.sqrt(64) * np.sqrt(np.mean(x.astype(np.float64) ** 2) * np.mean(w.astype(np.float64) ** 2))
    assert np.max(np.abs(out.numpy() - truth)) <= scale


def test_matmul_dyadic_full_tiles_exact(cx):
    # Exact in any order: pins the k permutation, swizzles and tile placement
    # of the direct-to-LDS kernel bit for bit.
    i = np.arange(4096 * 160)
    a = ((i % 13 - 6) / 8).astype(np.float32).reshape(4096, 160)
    j = np.arange(160 * 4096)
    b = ((j % 9 - 4) / 16).astype(np.float32).reshape(160, 4096)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_bits(actual, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32), "dyadic full tiles")


@pytest.mark.parametrize("sa,sb", [((2, 1, 5, 7), (3, 7, 4)), ((4, 33, 65), (65, 17)),
                                   ((65,), (65, 9)), ((9, 65), (65,)), ((3, 1, 40, 36), (1, 5, 36, 44))])
def test_matmul_broadcast(cx, sa, sb):
    rng = np.random.default_rng(3)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(actual, oracle.matmul(a, b), a, b, f"{sa}@{sb}")


def test_matmul_errors(cx):
    a = cx.tensor(np.ones((2, 3), np.float32), device="hip")
    with pytest.raises(ValueError):
        cx.matmul(a, a)
    with pytest.raises(ValueError):
        cx.matmul(cx.tensor(np.ones((2, 2), np.int32), device="hip"),
                  cx.tensor(np.ones((2, 2), np.int32), device="hip"))


# ------------------------------------------------------------- reductions
@pytest.mark.parametrize("shape", [(3, 65), (7, 300), (5, 1000), (2, 4097), (64, 8192), (1, 100003),
                                   (3, 5, 70), (11, 40)])
def test_reductions_random(cx, shape):
    rng = np.random.default_rng(11)
    x = rng.standard_normal(shape).astype(np.float32)
    h = cx.tensor(x, device="hip")
    for axis in range(-len(shape), len(shape)):
        _, outer, red, inner = oracle.reduction_dims(shape, axis)
        for op in ("max", "min", "argmax"):
            actual = getattr(cx, op)(h, axis).numpy()
            assert_bits(actual, getattr(oracle, op)(x, axis), f"{op} {shape} axis {axis}")
        for op in ("sum", "mean"):
            actual = getattr(cx, op)(h, axis).numpy()
            expected = getattr(oracle, op)(x, axis)
            if red <= 64:
                assert_bits(actual, expected, f"{op} {shape} axis {axis}")
            else:
                scale = red if op == "mean" else 1
                assert sum_error(actual * scale, expected * scale, x, outer, red, inner) <= 1e-5
    full = cx.sum(h).numpy()
    assert sum_error(full.reshape(1), oracle.sum(x, None).reshape(1), x, 1, x.size, 1) <= 1e-5


def test_extrema_ties_nan_and_signed_zero(cx):
    x = np.zeros((6, 777), np.float32)
    x[0, 100] = x[0, 500] = 3.0                   # tie -> lowest index
    x[1, :] = -np.inf                             # all -inf
    x[2, 300], x[2, 10] = np.nan, -1.0
    x[2, 600] = np.float32(np.nan) * -1           # a second NaN later
    x[3, :] = -0.0
    x[3, 400] = 0.0                               # +0/-0 equal, first kept
    x[4, 5:] = 7.0
    x[5, 776] = 9.0
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1), op)
        assert_bits(getattr(cx, op)(h, None).numpy(), getattr(oracle, op)(x, None), f"{op} all")


@pytest.mark.parametrize("width", [1024, 1028, 4096, 32768])
def test_extrema_special_values_vector_rows(cx, width):
    """16-byte rows: ties across float4 components, lanes and loop steps, signed
    zeros, infinities and NaNs (which send the wave to the exact re-scan)."""
    rows = 12
    x = np.zeros((rows, width), np.float32)
    x[0, 5] = x[0, 6] = 3.0                       # tie inside one lane's float4
    x[1, 7] = x[1, 3] = 3.0                       # tie across lanes
    x[2, 8 + 256] = x[2, 8] = 3.0                 # tie across loop steps
    x[3, :] = -0.0
    x[3, width // 2] = 0.0                        # +0/-0 equal: first (-0) kept
    x[4, :] = -np.inf
    x[5, :] = np.inf
    x[6, 300], x[6, 10] = np.nan, -1.0
    x[6, width - 1] = np.float32(np.nan) * -1     # a second NaN later
    x[7, width - 1] = 9.0                         # extreme at the last element
    x[7, width - 4] = -9.0
    x[8, width - 2] = np.nan                      # NaN in the tail group only
    x[9] = np.random.default_rng(12).integers(-3, 4, width)  # many ties
    x[10, ::97] = 5.0
    x[10, ::89] = -5.0
    x[11] = np.random.default_rng(13).standard_normal(width)
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1), f"{op} width {width}")
    # One long row split into segments, with a NaN in a late segment.
    y = np.random.default_rng(14).integers(-2, 3, 1 << 20).astype(np.float32)
    hy = cx.tensor(y, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(hy, None).numpy(), getattr(oracle, op)(y, None), f"{op} long row")
    y[777777] = np.nan
    hy = cx.tensor(y, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(hy, None).numpy(), getattr(oracle, op)(y, None), f"{op} long row NaN")


@pytest.mark.parametrize("width", [1 << 20, (1 << 20) + 3])
def test_extrema_segment_combine_special_values(cx, width):
    """Rows split into segments: the finish step's (rank key, index) fold must
    keep the first of equal keys across segments (ties, -0 against +0, every
    value -inf, two NaNs of different sign) and let a real int32 extreme,
    whose key is 0, beat an empty candidate."""
    x = np.zeros((6, width), np.float32)
    x[0, :] = -0.0
    x[0, 900000] = 0.0                            # +0 in a late segment: first -0 kept
    x[1, :] = -np.inf
    x[2, 700000] = x[2, 900000] = 5.0             # tie across segments
    x[2, 300000] = x[2, 800000] = -7.0
    x[3, 800000] = np.float32(np.nan) * -1
    x[3, 300000] = np.nan                         # the first NaN is the positive one
    x[4, :] = np.inf
    x[4, 1000] = -0.0
    x[5] = np.random.default_rng(15).integers(-2, 3, width)
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1), f"{op} f32 width {width}")
        assert_bits(getattr(cx, op)(h, None).numpy(), getattr(oracle, op)(x, None), f"{op} f32 all")
    imin, imax = np.iinfo(np.int32).min, np.iinfo(np.int32).max
    y = np.zeros((4, width), np.int32)
    y[0, :] = imin                                # max: key 0 everywhere, index 0
    y[1, :] = imax                                # min: key 0 everywhere, index 0
    y[2, 600000] = y[2, 950000] = imax            # tie across segments
    y[2, 100000] = y[2, 400000] = imin
    y[3] = np.random.default_rng(16).integers(imin, imax, width, dtype=np.int64).astype(np.int32)
    hy = cx.tensor(y, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(hy, 1).numpy(), getattr(oracle, op)(y, 1), f"{op} i32 width {width}")
        assert_bits(getattr(cx, op)(hy, None).numpy(), getattr(oracle, op)(y, None), f"{op} i32 all")


@pytest.mark.parametrize("shape", [(5, 9000), (1, 8193), (700, 16384), (3, 40004), (2, 65548), (448, 32768),
                                   (447, 32768), (2000, 4100)])
def test_row_reduction_block_items(cx, shape):
    """Rows cut into 4-wave block items: empty and short trailing wave
    segments (9000 = 3 x 3072 - 216, 8193 unaligned), one item per row with
    and without a full grid, items split into partials (fewer than 448 rows),
    and extrema whose ties and NaNs straddle wave-segment boundaries."""
    rows, cols = shape
    rng = np.random.default_rng(cols)
    x = rng.integers(-3, 4, shape).astype(np.float32)   # many ties
    for r in range(min(rows, 4)):
        for edge in (3072, 4096, 8192, cols - 1):
            if edge < cols:
                x[r, edge] = 9.0 if r % 2 == 0 else -9.0
    if rows > 1:
        x[1, cols // 2] = np.nan
        x[1, cols - 1] = np.float32(np.nan) * -1
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, -1).numpy(), getattr(oracle, op)(x, -1), f"{op} {shape}")
    y = rng.standard_normal(shape).astype(np.float32)
    hy = cx.tensor(y, device="hip")
    for op in ("sum", "mean"):
        actual = getattr(cx, op)(hy, -1).numpy()
        expected = getattr(oracle, op)(y, -1)
        scale = cols if op == "mean" else 1
        assert sum_error(actual * scale, expected * scale, y, rows, cols, 1) <= 1e-5, f"{op} {shape}"
    yi = rng.integers(-2**31, 2**31 - 1, shape, dtype=np.int64).astype(np.int32)
    hi = cx.tensor(yi, device="hip")
    for op in ("sum", "max", "argmax"):
        assert_bits(getattr(cx, op)(hi, -1).numpy(), getattr(oracle, op)(yi, -1), f"i32 {op} {shape}")


@pytest.mark.parametrize("width", [65, 100, 128, 129, 193, 256, 257, 385, 512, 513, 769, 1023, 1025, 1537,
                                   2047, 2048])
def test_packed_row_reductions_special_values(cx, width):
    """Rows of 65-2048 elements: 8 to 64 lanes per row with 16-byte loads at
    any alignment, 1 to 8 loads per lane (each width is the first or last of
    one shape). A float4 that runs past a row reads the next row's first
    elements and must mask them: those are NaN, +inf or -inf here. Ties inside
    a float4, across lanes and across loop steps, signed zeros, the extreme at
    the last element, a partial last wave (11 rows), and int32 rows whose sums
    wrap."""
    rows = 11
    rng = np.random.default_rng(width)
    x = rng.integers(-3, 4, (rows, width)).astype(np.float32)   # many ties
    x[1, 0] = np.nan                       # row 0's last float4 may read it
    x[2, 0:3] = np.inf                     # row 1's
    x[3, 0] = -np.inf                      # row 2's
    x[4, 1] = x[4, 2] = 9.0                # tie inside a float4
    x[5, 4] = x[5, 0] = 9.0                # tie across lanes
    x[6, width - 1] = 9.0                  # extreme at the last element
    x[7, :] = -0.0
    x[7, width // 2] = 0.0                 # +0/-0 equal: first (-0) kept
    x[8, width - 2] = np.nan               # NaN late in the row
    x[9, 4 * 8 * (width // 64)] = 9.0      # a later loop step
    x[9, 0] = 9.0
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1), f"{op} width {width}")
    with np.errstate(invalid="ignore"):
        for op in ("sum", "mean"):
            actual, expected = getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1)
            assert np.array_equal(np.isnan(actual), np.isnan(expected)), op
            assert np.array_equal(np.isinf(actual), np.isinf(expected)), op
            fin = np.isfinite(expected)
            scale = width if op == "mean" else 1
            assert sum_error(actual[fin] * scale, expected[fin] * scale, x[fin], int(fin.sum()), width, 1) <= 1e-5
    y = rng.standard_normal((rows, width)).astype(np.float32)
    hy = cx.tensor(y, device="hip")
    assert sum_error(cx.sum(hy, 1).numpy(), oracle.sum(y, 1), y, rows, width, 1) <= 1e-5
    yi = rng.integers(-2**31, 2**31 - 1, (rows, width), dtype=np.int64).astype(np.int32)
    hi = cx.tensor(yi, device="hip")
    for op in ("sum", "max", "min", "argmax"):
        assert_bits(getattr(cx, op)(hi, 1).numpy(), getattr(oracle, op)(yi, 1), f"i32 {op} width {width}")


def test_int32_reductions_wrap(cx):
    rng = np.random.default_rng(3)
    x = rng.integers(-2**31, 2**31 - 1, size=(300, 1031), dtype=np.int64).astype(np.int32)
    h = cx.tensor(x, device="hip")
    for axis in (0, 1):
        for op in ("sum", "max", "min", "argmax"):
            assert_bits(getattr(cx, op)(h, axis).numpy(), getattr(oracle, op)(x, axis), f"{op} {axis}")
    assert_bits(cx.sum(h).numpy(), oracle.sum(x, None), "i32 full sum")
    with pytest.raises(ValueError):
        cx.mean(h, 1)


def test_multi_axis_and_canonical_order(cx):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 6, 9)).astype(np.float32)
    h = cx.tensor(x, device="hip")
    for axes in ((0, 2), (2, 0), (0, 1), (1, 2), (0, 1, 2)):
        for op in ("sum", "max", "mean", "min"):
            # Exact order except adjacent runs longer than 64 (tree order, sum bar).
            check_case(f"{op} {axes}", op, [x], {"axes": list(axes)},
                       getattr(cx, op)(h, axes).numpy(), getattr(oracle, op)(x, axes))
    pins = np.array([[1e20, 1], [-1e20, 3]], np.float32)
    assert cx.sum(cx.tensor(pins, device="hip")).numpy() == 3.0
    big = np.array([[3e38, 3e38], [-3e38, -3e38]], np.float32)
    assert np.isposinf(cx.mean(cx.tensor(big, device="hip")).numpy())


@pytest.mark.parametrize("name", ["sum", "max", "mean"])
def test_high_rank_and_empty_metadata(cx, name):
    # tests/python/test_multi_axis_reductions.py:143-163 of the reference on
    # hip: a rank-300 selection folds to one 6-element row; a zero-size
    # tensor whose reduced iteration space would overflow int64 has no outputs
    # to compute; a selection whose output shape overflows is rejected.
    x = cx.tensor(np.arange(6, dtype=np.float32), device="hip").reshape((2,) + (1,) * 298 + (3,))
    y = getattr(x, name)((299, 0), keepdims=True)
    assert y.shape == (1,) * 300 and y.device == "hip"
    assert y.reshape(()).numpy() == {"sum": 15.0, "max": 5.0, "mean": 2.5}[name]
    assert getattr(x, name)((299, 0)).shape == (1,) * 298
    empty = cx.empty((0, 1, 2**62, 4, 0), device="hip")
    assert getattr(empty, name)((1, 2, 3)).shape == (0, 0)
    if name == "max":
        with pytest.raises(ValueError):
            getattr(empty, name)(None)
    else:
        value = getattr(empty, name)(None).numpy()
        assert (value == 0) if name == "sum" else np.isnan(value)
    with pytest.raises(ValueError, match="overflow"):
        getattr(empty, name)((0, 4))
    # int32 through the same fold (mean rejects int32, as on the CPU path).
    xi = cx.tensor(np.arange(6, dtype=np.int32), device="hip").reshape((2,) + (1,) * 298 + (3,))
    if name == "mean":
        with pytest.raises(ValueError, match="float32"):
            xi.mean((299, 0))
    else:
        assert getattr(xi, name)((299, 0)).reshape(()).numpy() == {"sum": 15, "max": 5}[name]


def test_folded_selections_at_scale(cx):
    # Selections that fold into one long row (size-1 axes between the reduced
    # ones) take the tree path; alternating selections over more than eight
    # folded axes take the metadata kernel at its 40-axis capacity (at most
    # 64 elements per output: (0, 5, 8, 10)) or fold one run at a time.
    rng = np.random.default_rng(17)
    x = rng.standard_normal((300, 1, 1, 700)).astype(np.float32)
    h = cx.tensor(x, device="hip")
    for op in ("sum", "mean", "max", "min"):
        check_case(f"{op} long row", op, [x], {"axes": [0, 3]}, getattr(cx, op)(h, (0, 3)).numpy(),
                   getattr(oracle, op)(x, (0, 3)))
    shape = (3, 2, 4, 1, 3, 2, 5, 1, 2, 3, 2, 2)
    y = rng.standard_normal(shape).astype(np.float32)
    hy = cx.tensor(y, device="hip")
    for axes in ((0, 2, 5, 8, 10), (1, 4, 6, 9, 11), (0, 5, 8, 10)):
        for op in ("sum", "mean", "max", "min"):
            check_case(f"{op} {axes}", op, [y], {"axes": list(axes)}, getattr(cx, op)(hy, axes).numpy(),
                       getattr(oracle, op)(y, axes))
        assert_bits(cx.Tensor(cx._core._argmax_axes(hy._impl, list(axes))).numpy(),
                    oracle.argmax(y, axes), f"argmax {axes}")
    yi = rng.integers(-2**31, 2**31 - 1, shape, dtype=np.int64).astype(np.int32)
    hi = cx.tensor(yi, device="hip")
    assert_bits(cx.sum(hi, (0, 2, 5, 8, 10)).numpy(), oracle.sum(yi, (0, 2, 5, 8, 10)), "i32 sum")
    assert_bits(cx.max(hi, (1, 4, 6, 9, 11)).numpy(), oracle.max(yi, (1, 4, 6, 9, 11)), "i32 max")


def test_folded_broadcast_and_batches(cx):
    # Rank-12 broadcasts whose patterns alternate fold to 12 axes (past the
    # old 8-axis metadata), bit-exact against the oracle; a batched matmul
    # with 10 alternating batch axes walks its two leading axes on the host.
    rng = np.random.default_rng(18)
    ls, rs = (2, 1, 3, 1, 2, 1, 2, 1, 3, 1, 2, 2), (1, 2, 1, 3, 1, 2, 1, 2, 1, 3, 2, 1)
    a, b = rng.standard_normal(ls).astype(np.float32), rng.standard_normal(rs).astype(np.float32)
    ha, hb = cx.tensor(a, device="hip"), cx.tensor(b, device="hip")
    for op, fn in (("add", lambda p, q: p + q), ("subtract", lambda p, q: p - q),
                   ("multiply", lambda p, q: p * q), ("divide", lambda p, q: p / q)):
        assert_bits(fn(ha, hb).numpy(), oracle.binary(op, a, b), f"rank-12 {op}")
    ai = rng.integers(-2**31, 2**31 - 1, ls, dtype=np.int64).astype(np.int32)
    bi = rng.integers(-2**31, 2**31 - 1, rs, dtype=np.int64).astype(np.int32)
    assert_bits((cx.tensor(ai, device="hip") * cx.tensor(bi, device="hip")).numpy(),
                oracle.binary("multiply", ai, bi), "rank-12 int32 multiply")
    p = rng.standard_normal((2, 1, 2, 1, 2, 1, 2, 1, 2, 1, 33, 40)).astype(np.float32)
    q = rng.standard_normal((1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 40, 17)).astype(np.float32)
    actual = cx.matmul(cx.tensor(p, device="hip"), cx.tensor(q, device="hip")).numpy()
    assert_matmul(actual, oracle.matmul(p, q), p, q, "batch rank 10")


def test_empty_and_scalar(cx):
    z = cx.tensor(np.zeros((2, 0, 3), np.float32), device="hip")
    assert cx.sum(z, 1).numpy().tolist() == [[0, 0, 0], [0, 0, 0]]
    assert np.all(np.isnan(cx.mean(z, 1).numpy()))
    with pytest.raises(ValueError):
        cx.max(z, 1)
    with pytest.raises(ValueError):
        cx.argmax(z, 1)
    s = cx.tensor(np.float32(2.5), device="hip")
    assert cx.sum(s).numpy() == 2.5 and cx.max(s, 0).numpy() == 2.5
    assert cx.argmax(s).numpy() == 0


# ------------------------------------------------------------- row ops
# Widths cover each row kernel: rows of 1-1536 in lane groups (1 to 64
# lanes, 1 to 6 float4 per lane, any alignment, partial last groups), one
# 256-thread block per row (1537-3072
# floats, 4096 with a weight or bias: aligned full and masked, and
# unaligned), one 512-thread block per row holding 3073-16384
# floats in 4 or 8 float4 per thread (aligned and unaligned) and wider rows in
# 12 or 20, the re-reading block kernel, and strided rows.
@pytest.mark.parametrize("shape,axis", [((16, 4096), 1), ((5, 300), 1), ((7, 8192), 1), ((3, 20000), -1),
                                        ((3, 7), 0), ((2, 3, 70), 1), ((9, 1), 1), ((4, 1022), 1),
                                        ((4, 1024), 1), ((6, 1501), 1), ((4, 2048), 1), ((3, 3001), 1),
                                        ((5, 4100), 1), ((2, 12288), 1), ((3, 16384), 1), ((2, 16383), 1),
                                        ((1000, 1028), 1), ((3, 5001), 1), ((2, 9999), 1), ((9, 130), 1),
                                        ((17, 100), 1), ((33, 257), 1), ((5, 1536), 1), ((3, 1537), 1),
                                        ((1001, 65), 1), ((3, 30001), 1)])
def test_row_ops_random(cx, shape, axis):
    rng = np.random.default_rng(13)
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    h = cx.tensor(x, device="hip")
    assert_close(cx.softmax(h, axis).numpy(), oracle.softmax(x, axis), 1e-5, 1e-5, "softmax")
    assert_close(cx.rmsnorm(h, axis).numpy(), oracle.rmsnorm(x, axis), 1e-5, 1e-5, "rmsnorm")
    assert_close(cx.layernorm(h, axis).numpy(), oracle.layernorm(x, axis), 1e-5, 1e-5, "layernorm")
    n = shape[axis]
    g = rng.uniform(0.5, 1.5, size=n).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, size=n).astype(np.float32)
    gh, bh = cx.tensor(g, device="hip"), cx.tensor(b, device="hip")
    assert_close(cx.layernorm(h, axis, weight=gh, bias=bh).numpy(),
                 oracle.affine_norm(x, axis, 1e-5, g, b), 1e-5, 1e-5, "affine layernorm")
    assert_close(cx.rmsnorm(h, axis, weight=gh).numpy(),
                 oracle.affine_norm(x, axis, 1e-5, g, None, rms=True), 1e-5, 1e-5, "affine rmsnorm")


@pytest.fixture(scope="module")
def capi():
    require_gpu()
    import tensorcx_hip_capi
    return tensorcx_hip_capi


@pytest.mark.parametrize("width", [45000, 50257, 65536, 100003, 128256, 139008])
@pytest.mark.parametrize("off", [1, 2, 3])
def test_resident_lds_rows_at_every_base(capi, width, off):
    # Rows held in registers plus LDS (two 512-thread blocks per CU at 20 or,
    # for LayerNorm, 24 float4 per thread; 1024 threads of 24 float4 past
    # them), with input and output bases 1-3 floats past a 16-byte boundary:
    # the float4 body, its head and tail and the LDS chunks all shift. Held
    # to the row-op bar against float64 truth widened by the oracle's own
    # drift, and against the oracle within the same bar.
    rows = 5
    rng = np.random.default_rng(width + off)
    flat = rng.standard_normal(rows * width + off).astype(np.float32)
    x = flat[off:].reshape(rows, width)
    x[1, width // 3] = np.nan
    g = rng.uniform(0.5, 1.5, width).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, width).astype(np.float32)
    dx, dg, db = (capi.DeviceArray.from_numpy(t) for t in (flat, g, b))
    # Output with a sentinel before the base and 4 floats past the last row.
    out = capi.DeviceArray.from_numpy(np.full(rows * width + off + 4, 7.0, np.float32))
    xp, op_ = dx.ptr + 4 * off, out.ptr + 4 * off
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    mean = x64.mean(axis=1, keepdims=True)
    ln = (x64 - mean) / np.sqrt(((x64 - mean) ** 2).mean(axis=1, keepdims=True) + 1e-5)
    rms = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5)
    runs = {"softmax": (lambda: capi.softmax(xp, op_, rows, width, 1), oracle.softmax(x, 1),
                        e / e.sum(axis=1, keepdims=True)),
            "rmsnorm": (lambda: capi.rmsnorm(xp, None, op_, rows, width, 1, 1e-5), oracle.rmsnorm(x, 1), rms),
            "rmsnorm + weight": (lambda: capi.rmsnorm(xp, dg.ptr, op_, rows, width, 1, 1e-5),
                                 oracle.affine_norm(x, 1, 1e-5, g, None, rms=True), rms * g),
            "layernorm + weight/bias": (lambda: capi.layernorm(xp, dg.ptr, db.ptr, op_, rows, width, 1, 1e-5),
                                        oracle.affine_norm(x, 1, 1e-5, g, b), ln * g + b)}
    with np.errstate(all="ignore"):
        for name, (run, expected, truth) in runs.items():
            run()
            capi.synchronize()
            whole = out.numpy()
            assert np.all(whole[:off] == 7.0) and np.all(whole[off + rows * width:] == 7.0), \
                f"{name} wrote outside the rows, width {width} +{off}"
            got = whole[off:off + rows * width].reshape(rows, width)
            fin = np.isfinite(truth)
            assert np.array_equal(np.isnan(got), np.isnan(expected)), f"{name} NaN rows, width {width} +{off}"
            drift = float(np.max(np.abs(expected[fin] - truth[fin]) / np.maximum(np.abs(truth[fin]), 1e-30)))
            assert_close(got[fin].reshape(-1), truth[fin].reshape(-1), 1e-5 + drift, 1e-5,
                         f"{name} vs float64, width {width} +{off}")
            assert_close(got, expected, 1e-5 + drift, 1e-5, f"{name}, width {width} +{off}")


def test_row_ops_and_reductions_random_widths_and_bases(capi):
    # Seeded random contiguous rows through the C ABI: widths log-uniform
    # over 1-140000 (every width class of the row kernels, from lane groups
    # to rows held in registers and LDS), row counts, and bases 0-3 floats
    # past a 16-byte boundary (input and output alike, so rows start at every
    # alignment). Softmax, RMSNorm + weight and LayerNorm + weight/bias meet
    # the row-op bar, widened by the oracle's own distance from float64
    # truth, against both truth and the oracle: on N(0, 9) rows a few large
    # terms dominate the softmax denominator and the reference's sequential
    # float32 sum drifts from float64 by up to 1e-4 relative (the kernel's
    # tree sums measured within 1e-5 of truth here), as past 65536 elements
    # for the wide rows above; two nearly equal elements make x - mean
    # cancel in any float32 LayerNorm. Max and argmax are bit-exact, sums
    # within the sum bar.
    rng = np.random.default_rng(31)
    failures = []
    for case in range(48):
        width = int(np.exp(rng.uniform(0.0, np.log(140000.0))))
        rows = int(max(1, min(int(rng.integers(1, 400)), 2_000_000 // width)))
        off = int(rng.integers(0, 4))
        flat = (rng.standard_normal(rows * width + off) * 3).astype(np.float32)
        x = flat[off:].reshape(rows, width)
        g = rng.uniform(0.5, 1.5, width).astype(np.float32)
        b = rng.uniform(-0.1, 0.1, width).astype(np.float32)
        dx, dg, db = (capi.DeviceArray.from_numpy(t) for t in (flat, g, b))
        out = capi.DeviceArray((rows * width + off,))
        xp, op_ = dx.ptr + 4 * off, out.ptr + 4 * off
        context = f"case {case}: [{rows}, {width}] base +{off} floats"
        x64 = x.astype(np.float64)
        e = np.exp(x64 - x64.max(axis=1, keepdims=True))
        mean = x64.mean(axis=1, keepdims=True)
        ln = (x64 - mean) / np.sqrt(((x64 - mean) ** 2).mean(axis=1, keepdims=True) + 1e-5)
        rms = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5)
        runs = {"softmax": (lambda: capi.softmax(xp, op_, rows, width, 1), oracle.softmax(x, 1),
                            e / e.sum(axis=1, keepdims=True)),
                "rmsnorm + weight": (lambda: capi.rmsnorm(xp, dg.ptr, op_, rows, width, 1, 1e-5),
                                     oracle.affine_norm(x, 1, 1e-5, g, None, rms=True), rms * g),
                "layernorm + weight/bias": (lambda: capi.layernorm(xp, dg.ptr, db.ptr, op_, rows, width, 1, 1e-5),
                                            oracle.affine_norm(x, 1, 1e-5, g, b), ln * g + b)}
        try:
            for name, (run, expected, truth) in runs.items():
                run()
                capi.synchronize()
                got = out.numpy()[off:].reshape(rows, width)
                drift = float(np.max(np.abs(expected - truth) / np.maximum(np.abs(truth), 1e-30)))
                assert_close(got, truth, 1e-5 + drift, 1e-5, f"{name} vs float64 {context} (oracle drift {drift:.1e})")
                assert_close(got, expected, 1e-5 + drift, 1e-5, f"{name} {context} (oracle drift {drift:.1e})")
            res = capi.DeviceArray((rows,))
            for op in ("max", "argmax", "sum"):
                ws = capi.reduce_workspace(op, capi.TCX_FLOAT32, rows, width, 1)
                capi.reduce(op, capi.TCX_FLOAT32, xp, res.ptr, rows, width, 1, ws)
                capi.synchronize()
                got = res.numpy()
                if op == "max":
                    assert_bits(got, oracle.max(x, 1), f"max {context}")
                elif op == "argmax":
                    assert_bits(got.view(np.int32), oracle.argmax(x, 1), f"argmax {context}")
                else:
                    err = sum_error(got, oracle.sum(x, 1), x, rows, width, 1)
                    assert err <= 1e-5, f"sum {context}: {err:.3e}"
        except AssertionError as error:
            failures.append(str(error))
    assert not failures, "\n".join(failures[:10])


@pytest.mark.parametrize("width", [2, 3, 5, 8, 13, 16, 17, 31, 33, 50, 63, 64,
                                   65, 100, 127, 129, 130, 193, 200, 257, 385, 500, 513, 769, 1024, 1025, 1536, 1537,
                                   2048, 3001, 3073, 4095, 4096, 8191, 8192, 16383, 16384, 16385, 20003,
                                   24577, 32000, 40001, 40961, 50257, 61184, 61185, 65536, 69376, 69377, 70000,
                                   90113, 100003, 128256, 130816, 130817, 131000, 139008, 139009])
def test_row_ops_special_values_wide_rows(cx, width):
    # Non-finite values in rows of every width class (rows of 2-1536 in
    # groups of 1 to 64 lanes at 1 to 6 float4 per lane, any alignment, with
    # row 1's last float4 reading row 2's leading -inf; split rows at 2 and 4
    # float4 per thread, aligned and unaligned, rows of
    # 3073-16384 held at 4 or 8 float4 per thread by a 512-thread block
    # (without a weight or bias up to 4096), rows held in registers at 12 or
    # 20 float4 per thread (up to 24576 and 40960 floats), at 20 or (for
    # LayerNorm) 24 with up to 79 KB of LDS (to 61184 and 69376 floats),
    # softmax and RMSNorm at 24 float4 for 1024 threads plus LDS (to 139008),
    # LayerNorm at 44 (up to 90112) and then LDS (up to 130816), and re-read
    # beyond): a
    # NaN, +inf last, -inf first, a row of -inf, +inf with -inf, and a row
    # whose squares overflow to inf.
    rng = np.random.default_rng(23)
    x = rng.standard_normal((7, width)).astype(np.float32)
    x[0, width // 2] = np.nan
    x[1, width - 1] = np.inf
    x[2, 0] = -np.inf
    x[3] = -np.inf
    x[4, 1], x[4, width - 2] = np.inf, -np.inf
    x[5] *= np.float32(1e20)
    g = rng.uniform(0.5, 1.5, size=width).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, size=width).astype(np.float32)
    h, gh, bh = (cx.tensor(t, device="hip") for t in (x, g, b))
    # Float64 truth of the one row of ordinary values (row 6).
    r64 = x[6].astype(np.float64)
    e = np.exp(r64 - r64.max())
    mean = r64.mean()
    ln = (r64 - mean) / np.sqrt(((r64 - mean) ** 2).mean() + 1e-5)
    rms = r64 / np.sqrt((r64 * r64).mean() + 1e-5)
    truth = {"softmax": e / e.sum(), "rmsnorm": rms, "layernorm": ln, "affine layernorm": ln * g + b,
             "affine rmsnorm": rms * g}

    def check(actual, expected, context):
        if width <= 65536:
            assert_close(actual, expected, 1e-5, 1e-5, context)
            return
        # Past 65536 elements the reference's own sequential float32 sums can
        # miss float64 truth by more than the 1e-5 bar (2.4e-5 for the sum
        # of squares at 100003, giving outputs 1.2e-5 off): row 6 must then
        # meet the bar against truth, and against the oracle within the bar
        # widened by the oracle's own relative distance from truth.
        assert_close(actual[:6], expected[:6], 1e-5, 1e-5, context)
        t = truth[context]
        drift = float(np.max(np.abs(expected[6] - t) / np.abs(t)))
        assert_close(actual[6], t, 1e-5, 1e-5, context + " vs float64")
        assert_close(actual[6], expected[6], 1e-5 + drift, 1e-5, context)

    with np.errstate(all="ignore"):
        check(cx.softmax(h, 1).numpy(), oracle.softmax(x, 1), "softmax")
        check(cx.rmsnorm(h, 1).numpy(), oracle.rmsnorm(x, 1), "rmsnorm")
        check(cx.layernorm(h, 1).numpy(), oracle.layernorm(x, 1), "layernorm")
        check(cx.layernorm(h, 1, weight=gh, bias=bh).numpy(), oracle.affine_norm(x, 1, 1e-5, g, b), "affine layernorm")
        check(cx.rmsnorm(h, 1, weight=gh).numpy(), oracle.affine_norm(x, 1, 1e-5, g, None, rms=True), "affine rmsnorm")
        # The same rows through the reductions: extrema bit-exact; sums carry
        # NaN / inf as in any order (no finite overflow), the rest at the bar.
        for op in ("max", "min", "argmax"):
            assert_bits(getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1), f"{op} special {width}")
        for op in ("sum", "mean"):
            actual, expected = getattr(cx, op)(h, 1).numpy(), getattr(oracle, op)(x, 1)
            assert np.array_equal(np.isinf(actual), np.isinf(expected)), op
            assert np.array_equal(np.sign(actual[np.isinf(expected)]), np.sign(expected[np.isinf(expected)])), op
            assert np.array_equal(np.isnan(actual), np.isnan(expected)), op
            fin = np.isfinite(expected)
            scale = width if op == "mean" else 1
            assert sum_error(actual[fin] * scale, expected[fin] * scale, x[fin], int(fin.sum()), width, 1) <= 1e-5, op


@pytest.mark.parametrize("eps", [0.0, 1e-45, 1e-5, 1e30])
@pytest.mark.parametrize("width", [5, 33, 100, 130, 512, 1025, 1537, 4096, 3001, 8192, 16384, 20003, 32000, 100003])
def test_constant_rows(cx, eps, width):
    x = np.full((5, width), 2.5, np.float32)
    x[3] = -7.0
    x[4, width - 1] = 2.5000002  # equal except the last element
    h = cx.tensor(x, device="hip")
    for op in ("rmsnorm", "layernorm"):
        assert_close(getattr(cx, op)(h, 1, eps).numpy(), getattr(oracle, op)(x, 1, eps), 1e-5, 1e-5, op)


def test_row_op_errors(cx):
    h = cx.tensor(np.ones((2, 8), np.float32), device="hip")
    for eps in (-1.0, np.nan, np.inf, 1e100, 1e-100):
        with pytest.raises(ValueError):
            cx.layernorm(h, 1, eps)
    with pytest.raises(ValueError):
        cx.softmax(h, 2)
    with pytest.raises(ValueError):
        cx.softmax(cx.tensor(np.ones((2, 8), np.int32), device="hip"), 1)


# ------------------------------------------------------------- elementwise / linear
def test_unary_and_bias_act(cx):
    x = np.concatenate([np.linspace(-12, 12, 4001, dtype=np.float32),
                        np.array([0, -0.0, np.inf, -np.inf, np.nan, 100, -100, 1e-38], np.float32)])
    h = cx.tensor(x, device="hip")
    for op in ("exp", "gelu", "silu"):
        assert_close(getattr(cx, op)(h).numpy(), getattr(oracle, op)(x), 1e-6, 1e-6, op)
    rng = np.random.default_rng(2)
    y = rng.standard_normal((33, 64)).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    yh, bh = cx.tensor(y, device="hip"), cx.tensor(b, device="hip")
    assert_bits((yh + bh).numpy(), oracle.binary("add", y, b), "bias add")
    for act in ("silu", "gelu"):
        fused = cx.hip.bias_act(yh, bh, act).numpy()
        assert_close(fused, getattr(oracle, act)(oracle.binary("add", y, b)), 1e-6, 1e-6, act)


@pytest.mark.parametrize("rows,cols", [(3, 5), (7, 1001), (2048, 2052), (4096, 4096), (999, 512), (300, 8),
                                       (70000, 1024)])
def test_bias_act_special_values(cx, rows, cols):
    # The fused bias + activation kernel (rows of 1024+ 4-aligned floats: a
    # column tile per block striding over rows, 70000 rows past the grid's
    # row extent; narrower 4-aligned rows: a flat float4 stream whose bias
    # column steps with the grid stride; scalar path otherwise) with
    # non-finite and overflowing inputs in both operands, against the
    # reference's add-then-activation.
    rng = np.random.default_rng(29)
    y = rng.standard_normal((rows, cols)).astype(np.float32) * 4
    b = rng.standard_normal(cols).astype(np.float32)
    specials = np.array([np.nan, np.inf, -np.inf, 100., -100., 1e30, -1e30, 0., -0., 1e-38], np.float32)
    flat = y.reshape(-1)
    idx = rng.choice(flat.size, size=min(flat.size, 4 * specials.size), replace=False)
    flat[idx] = np.resize(specials, idx.size)
    b[rng.choice(cols, size=min(cols, 3), replace=False)] = np.array([np.inf, -np.inf, np.nan], np.float32)[:min(cols, 3)]
    yh, bh = cx.tensor(y, device="hip"), cx.tensor(b, device="hip")
    with np.errstate(all="ignore"):
        pre = oracle.binary("add", y, b)
        for act in ("silu", "gelu"):
            fused = cx.hip.bias_act(yh, bh, act).numpy()
            assert_close(fused, getattr(oracle, act)(pre), 1e-6, 1e-6, f"{act} {rows}x{cols}")


@pytest.mark.parametrize("shape", [(5, 48), (2, 3, 48), (48,), (257, 130)])
def test_linear(cx, shape):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(shape).astype(np.float32)
    w = rng.standard_normal((20, shape[-1])).astype(np.float32)
    b = rng.standard_normal(20).astype(np.float32)
    xh, wh, bh = (cx.tensor(v, device="hip") for v in (x, w, b))
    assert_matmul(cx.linear(xh, wh, bh).numpy(), oracle.linear(x, w, b), x, w.T, "linear")
    assert_matmul(cx.linear(xh, wh).numpy(), oracle.linear(x, w), x, w.T, "linear no bias")
    fused = cx.hip.linear_act(xh, wh, bh, "silu").numpy()
    expected = oracle.silu(oracle.linear(x, w, b))
    assert fused.shape == expected.shape
    # matmul-class error, propagated through silu (|silu'| <= 1.1)
    assert np.max(np.abs(fused - expected)) <= 1.1e-4 * np.sqrt(shape[-1]) * np.sqrt(np.mean(x * x)) * \
        np.sqrt(np.mean(w * w)) + 1e-6


@pytest.mark.parametrize("xs,ws", [((4096, 4096), (1024, 4096)), ((4, 1024, 256), (1024, 256)),
                                   ((2048, 2048), (2048, 2048))])
def test_linear_direct128(cx, xs, ws):
    # Linear layers with fewer than one round of 256x256 tiles but >= 256
    # full 128x128 ones (the MLP's second linear, a batched input, a square
    # 2048 layer) take the direct 128x128 kernel over the whole K rather than
    # a K split, with bias.
    rng = np.random.default_rng(33)
    x = rng.standard_normal(xs).astype(np.float32)
    w = rng.standard_normal(ws).astype(np.float32)
    b = rng.standard_normal(ws[0]).astype(np.float32)
    got = cx.linear(cx.tensor(x, device="hip"), cx.tensor(w, device="hip"), cx.tensor(b, device="hip")).numpy()
    truth = x.astype(np.float64) @ w.astype(np.float64).T + b
    x2 = x.reshape(-1, xs[-1])
    assert_matmul(got.reshape(-1, ws[0]) - b, truth.reshape(-1, ws[0]) - b, x2, w.T, f"linear {xs}x{ws}")


def test_linear_direct128_dyadic_exact_and_special(cx):
    # 16 x 16 tiles of 128x128 over K = 96 (three k-tiles): exact in any
    # order with dyadic inputs (pins the tile map and the fragment layout bit
    # for bit), then non-finite values in x rows and a W row.
    i = np.arange(2048 * 96)
    x = ((i % 13 - 6) / 8).astype(np.float32).reshape(2048, 96)
    j = np.arange(2048 * 96)
    w = ((j % 11 - 5) / 16).astype(np.float32).reshape(2048, 96)
    b = ((np.arange(2048) % 7 - 3) / 4).astype(np.float32)
    xh, wh, bh = (cx.tensor(t, device="hip") for t in (x, w, b))
    exact = (x.astype(np.float64) @ w.astype(np.float64).T + b).astype(np.float32)
    assert_bits(cx.linear(xh, wh, bh).numpy(), exact, "dyadic direct128")
    x[5, 3], x[700, 10], x[1500, 95] = np.inf, -np.inf, np.nan
    w[2047, 40] = np.inf
    got = cx.linear(cx.tensor(x, device="hip"), cx.tensor(w, device="hip"), bh).numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        truth = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.array_equal(np.isnan(got), np.isnan(truth))
    assert np.array_equal(np.isinf(got), np.isinf(truth))
    assert np.array_equal(np.sign(got[np.isinf(truth)]), np.sign(truth[np.isinf(truth)]))
    fin = np.isfinite(truth)
    assert np.array_equal(got[fin], truth[fin].astype(np.float32))


def test_linear_full_tiles(cx):
    # 4096 x 4096 outputs: the transposed-B direct-to-LDS kernel, with the bias
    # and SiLU epilogue; checked against float64.
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4096, 256)).astype(np.float32)
    w = rng.standard_normal((4096, 256)).astype(np.float32)
    b = rng.standard_normal(4096).astype(np.float32)
    xh, wh, bh = (cx.tensor(v, device="hip") for v in (x, w, b))
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert_matmul(cx.linear(xh, wh).numpy(), exact, x, w.T, "linear full tiles")
    assert_matmul(cx.linear(xh, wh, bh).numpy(), exact + b, x, w.T, "linear full tiles + bias")
    fused = cx.hip.linear_act(xh, wh, bh, "silu").numpy()
    z = exact + b
    expected = z / (1.0 + np.exp(-z))
    bound = 1.1e-4 * np.sqrt(256) * np.sqrt(np.mean(x * x)) * np.sqrt(np.mean(w * w)) + 1e-6
    assert np.max(np.abs(fused - expected)) <= bound


def test_concurrent_threads(cx):
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(8)
    a = rng.standard_normal((64, 96)).astype(np.float32)
    b = rng.standard_normal((96, 80)).astype(np.float32)
    expected = oracle.softmax(oracle.matmul(a, b), 1)

    def work(_):
        out = cx.softmax(cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")), 1)
        return out.numpy()

    with ThreadPoolExecutor(4) as pool:
        for result in pool.map(work, range(16)):
            assert_close(result, expected, 1e-5, 1e-5, "threaded chain")


def test_memory_pool_reuse(cx):
    with cx.memory_pool("hip", max_cached_bytes=64 << 20, max_cached_blocks=8) as pool:
        x = cx.tensor(np.ones((256, 256), np.float32), device="hip")
        for _ in range(3):
            y = cx.softmax(x, 1)
            del y
        stats = pool.stats()
    assert stats["hits"] >= 1 and stats["active"]


@pytest.mark.parametrize("ls,rs", [((300, 1028), (1028,)), ((300, 1028), (300, 1)), ((1, 1030), (257, 1)),
                                   ((4097,), (4097,)), ((), (5000,)), ((64, 8), (64, 8)), ((3, 7, 5), (7, 1))])
def test_binary_two_axis_streams(cx, ls, rs):
    # Broadcasts that fold to at most two axes (a same-shape stream, a row or
    # column operand, a scalar) take the row/column-strided kernel, 16-byte
    # where the inner strides are 0 or 1 on aligned rows; bit-exact against
    # the reference's one IEEE operation per element, int32 wrapping.
    rng = np.random.default_rng(len(ls) * 7 + len(rs))
    a = rng.standard_normal(ls).astype(np.float32)
    b = rng.standard_normal(rs).astype(np.float32)
    b.reshape(-1)[:1] = 0.0
    ha, hb = cx.tensor(a, device="hip"), cx.tensor(b, device="hip")
    for op, fn in (("add", lambda p, q: p + q), ("subtract", lambda p, q: p - q),
                   ("multiply", lambda p, q: p * q), ("divide", lambda p, q: p / q)):
        with np.errstate(all="ignore"):
            assert_bits(fn(ha, hb).numpy(), oracle.binary(op, a, b), f"{op} {ls} {rs}")
            assert_bits(fn(hb, ha).numpy(), oracle.binary(op, b, a), f"{op} {rs} {ls}")
    ai = rng.integers(-2**31, 2**31 - 1, ls, dtype=np.int64).astype(np.int32)
    bi = rng.integers(-2**31, 2**31 - 1, rs, dtype=np.int64).astype(np.int32)
    hai, hbi = cx.tensor(ai, device="hip"), cx.tensor(bi, device="hip")
    for op, fn in (("add", lambda p, q: p + q), ("multiply", lambda p, q: p * q)):
        assert_bits(fn(hai, hbi).numpy(), oracle.binary(op, ai, bi), f"i32 {op} {ls} {rs}")


@pytest.mark.parametrize("batch,m,n,k,trans", [(65536, 8, 8, 8, False), (300, 16, 16, 16, True), (64, 64, 64, 64, False),
                                               (100, 3, 5, 7, False), (77, 1, 64, 33, True), (129, 64, 1, 2, False),
                                               (64, 17, 29, 64, True), (1000, 5, 7, 3, False)])
def test_matmul_tiny_batched(cx, batch, m, n, k, trans):
    # Many small products (items up to 64 x 64 x 64, at least 64 of them)
    # stage whole items in LDS, several per block, and sum each output's k in
    # order: bit-exact against the reference's sequential float32 loop.
    rng = np.random.default_rng(batch + m + n + k)
    clean = rng.standard_normal((batch, m, k)).astype(np.float32)
    b = rng.standard_normal((batch, n, k) if trans else (batch, k, n)).astype(np.float32)
    a = clean.copy()
    a.reshape(-1)[5] = np.inf
    bt = np.ascontiguousarray(np.swapaxes(b, 1, 2)) if trans else b
    expected = oracle.matmul(a, bt)
    ha, hb = cx.tensor(a, device="hip"), cx.tensor(bt, device="hip")
    with np.errstate(all="ignore"):
        assert_bits(cx.matmul(ha, hb).numpy(), expected, f"tiny {batch}x{m}x{n}x{k}")
    if trans:
        # The transposed-B route: linear over batched rows (x @ W^T, W shared).
        w = rng.standard_normal((n, k)).astype(np.float32)
        bias = rng.standard_normal(n).astype(np.float32)
        hc = cx.tensor(clean, device="hip")
        got = cx.linear(hc, cx.tensor(w, device="hip"), cx.tensor(bias, device="hip")).numpy()
        assert_matmul(got, (clean.astype(np.float64) @ w.T.astype(np.float64)) + bias, clean.reshape(-1, k), w.T,
                      f"tiny linear {batch}x{m}x{n}x{k}")


def test_matmul_tiny_shared_a(cx):
    # One A shared by 300 items of a [k, n] B (A's batch stride 0; a shared
    # B would fold into one 2-D product instead): not a dense batch, so items
    # are staged one element at a time through their offsets, where dense
    # batches (the cases above without a transposed B) stage two contiguous
    # runs with 16-byte loads. Bit-exact against the sequential loop.
    rng = np.random.default_rng(91)
    a = rng.standard_normal((1, 5, 7)).astype(np.float32)
    b = rng.standard_normal((300, 7, 6)).astype(np.float32)
    assert_bits(cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy(), oracle.matmul(a, b),
                "tiny shared a")


@pytest.mark.parametrize("m,n,k,trans", [(4096, 4096, 4, False), (3000, 1028, 16, True), (20000, 16, 16, False),
                                         (70000, 4, 1, False), (999, 2052, 7, False), (513, 260, 13, True)])
def test_matmul_small_k(cx, m, n, k, trans):
    # K <= 16 (unbatched, at least 65536 outputs): B columns in registers and
    # the output streamed as float4 rows, each output's k summed in order:
    # bit-exact against the reference's sequential float32 loop, and fused
    # bias + activation through linear.
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if trans else (k, n)).astype(np.float32)
    a[3, 0] = np.inf
    bt = np.ascontiguousarray(b.T) if trans else b
    with np.errstate(all="ignore"):
        expected = oracle.matmul(a, bt)
        assert_bits(cx.matmul(cx.tensor(a, device="hip"), cx.tensor(bt, device="hip")).numpy(), expected,
                    f"small-k {m}x{n}x{k}")
    if trans:
        clean = rng.standard_normal((m, k)).astype(np.float32)
        bias = rng.standard_normal(n).astype(np.float32)
        got = cx.linear(cx.tensor(clean, device="hip"), cx.tensor(b, device="hip"), cx.tensor(bias, device="hip"))
        assert_matmul(got.numpy(), clean.astype(np.float64) @ b.T.astype(np.float64) + bias, clean, b.T,
                      f"small-k linear {m}x{n}x{k}")


@pytest.mark.parametrize("batch,n,k", [(200, 2048, 1024), (128, 1028, 333), (300, 516, 7), (1, 4096, 4096),
                                       (4, 2052, 3001)])
def test_matmul_batched_vector_matrix(cx, batch, n, k):
    # One row of A against a row-major B per batch item: 1024-column blocks,
    # K in four in-block groups added in order, and with too few blocks K
    # split over blocks (partials in the workspace the backend brings, added
    # in split order); at the matmul bar.
    rng = np.random.default_rng(batch + n + k)
    a = rng.standard_normal((batch, 1, k)).astype(np.float32)
    b = rng.standard_normal((batch, k, n)).astype(np.float32)
    got = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    assert_matmul(got, np.matmul(a.astype(np.float64), b.astype(np.float64)), a, b, f"vecmat {batch}x{n}x{k}")
    # Dyadic operands make every partial sum exact: any order matches bitwise.
    ad = rng.integers(-8, 9, (batch, 1, k)).astype(np.float32)
    bd = rng.integers(-8, 9, (batch, k, n)).astype(np.float32)
    got = cx.matmul(cx.tensor(ad, device="hip"), cx.tensor(bd, device="hip")).numpy()
    assert_bits(got, np.matmul(ad.astype(np.float64), bd.astype(np.float64)).astype(np.float32), "vecmat dyadic")


@pytest.mark.parametrize("m,n,k,trans", [(70000, 64, 64, False), (50000, 48, 32, True), (40000, 20, 60, False)])
def test_matmul_tall_short_k_narrow_n(cx, m, n, k, trans):
    # Many 64x64 tiles of a short K and a narrow N run the small kernel's
    # 32x32 tiles; at the matmul bar, fused bias + activation included.
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if trans else (k, n)).astype(np.float32)
    bt = b.T if trans else b
    got = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(np.ascontiguousarray(bt), device="hip")).numpy()
    assert_matmul(got, a.astype(np.float64) @ bt.astype(np.float64), a, bt, f"tall {m}x{n}x{k}")
    if trans:
        bias = rng.standard_normal(n).astype(np.float32)
        got = cx.linear(cx.tensor(a, device="hip"), cx.tensor(b, device="hip"), cx.tensor(bias, device="hip")).numpy()
        assert_matmul(got, a.astype(np.float64) @ b.T.astype(np.float64) + bias, a, b.T, f"tall linear {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k,trans", [(2048, 2049, 2048, False), (2049, 2051, 1027, True), (1025, 1025, 1025, False),
                                         (1000, 1001, 999, True)])
def test_matmul_padded_odd_shapes(cx, m, n, k, trans):
    # Unbatched products whose K or N is not a multiple of 4 and of at least
    # 2^32 multiply-adds run zero-padded copies through the 16-byte kernels
    # when a workspace is brought (the backend brings it); the output is
    # stripped with the bias and activation applied as the kernels' epilogue
    # applies them. Smaller odd shapes keep the scalar-load kernels.
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if trans else (k, n)).astype(np.float32)
    bt = b.T if trans else b
    truth = a.astype(np.float64) @ bt.astype(np.float64)
    got = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(np.ascontiguousarray(bt), device="hip")).numpy()
    assert_matmul(got, truth, a, bt, f"padded {m}x{n}x{k}")
    if trans:
        bias = rng.standard_normal(n).astype(np.float32)
        xa, wb, bb = cx.tensor(a, device="hip"), cx.tensor(b, device="hip"), cx.tensor(bias, device="hip")
        pre = cx.linear(xa, wb, bb).numpy()
        assert_matmul(pre, truth + bias, a, bt, f"padded linear {m}x{n}x{k}")
        for act in ("silu", "gelu"):
            # The same padded product, so the activation meets the same bits.
            fused = cx.hip.linear_act(xa, wb, bb, act).numpy()
            assert_close(fused, getattr(oracle, act)(pre), 1e-6, 1e-6, f"padded {act} {m}x{n}x{k}")
