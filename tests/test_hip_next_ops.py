"""GPU parity of the ops next to the hot path: log/sqrt/abs, clip, topk,
embedding and attention, on the hip device against the CPU oracle.

The cases follow the reference's device-generic suites
(tests/python/test_math_ops.py and test_inference_ops.py): same shapes, special
values, masks and error contracts, with the oracle in place of the reference's
CPU device. Bars are those of tests/hip_cases.py.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import require_gpu
from hip_cases import assert_bits, assert_close, assert_nan_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cx():
    require_gpu()
    import tensorcx
    return tensorcx


def f32(shape, seed=31):
    return np.random.default_rng(seed).normal(size=shape).astype(np.float32)


def hip(cx, a):
    return cx.tensor(a, device="hip")


# ------------------------------------------------------------- log / sqrt / abs
@pytest.mark.parametrize("name", ["log", "sqrt", "abs"])
@pytest.mark.parametrize("shape", [(), (0,), (2, 0, 3), (1,), (2, 3, 5), (513,), (4099,)])
def test_unary_math(cx, name, shape):
    a = np.random.default_rng(912).uniform(.01, 100, shape).astype(np.float32)
    x = hip(cx, a)
    y = getattr(cx, name)(x)
    expected = getattr(oracle, name)(a)
    assert y.device == "hip" and y.shape == expected.shape and y.dtype == "float32"
    if name == "log":
        assert_close(y.numpy(), expected, 1e-6, 0.0, name)
    else:
        assert_bits(y.numpy(), expected, name)
    assert_bits(getattr(x, name)().numpy(), y.numpy(), name + " method")
    assert not cx._core._shares_storage(x._impl, y._impl)
    assert_bits(x.numpy(), a, "input untouched")


@pytest.mark.parametrize("name", ["log", "sqrt", "abs"])
def test_unary_ieee_and_subnormal(cx, name):
    words = np.array([0, 0x80000000, 1, 2, 0x007fffff, 0x00800000, 0x80000001, 0x807fffff, 0x80800000,
                      0x3f800000, 0xbf800000, 0x7f7fffff, 0x7f800000, 0xff800000, 0x7fc01234], np.uint32)
    a = words.view(np.float32)
    y = getattr(cx, name)(hip(cx, a)).numpy()
    expected = getattr(oracle, name)(a)
    if name == "log":
        assert_close(y, expected, 1e-6, 0.0, name)
    else:
        assert_nan_bits(y, expected, name)
    if name == "abs":
        np.testing.assert_array_equal(y.view(np.uint32), words & 0x7fffffff)
    if name == "sqrt":
        assert y.view(np.uint32)[1] == 0x80000000  # sqrt(-0) = -0


def test_abs_int32_wraps(cx):
    a = np.array([-2**31, -2**31 + 1, -16777217, -1, 0, 1, 2**31 - 1], np.int32)
    assert_bits(cx.abs(hip(cx, a)).numpy(), oracle.abs(a), "abs int32")
    assert_bits(abs(hip(cx, a)).numpy(), oracle.abs(a), "builtin abs")
    with pytest.raises(ValueError):
        cx.log(hip(cx, a))


# ------------------------------------------------------------- clip
@pytest.mark.parametrize("dtype", ["float32", "int32"])
@pytest.mark.parametrize("bounds", [(-2, 3), (None, 3), (-2, None), (4, -4), (0, 0)])
@pytest.mark.parametrize("shape", [(), (0,), (2, 3, 4), (3, 1000)])
def test_clip_scalar(cx, dtype, bounds, shape):
    a = np.random.default_rng(75).integers(-10, 10, shape).astype(dtype)
    lim = (-np.inf, np.inf) if dtype == "float32" else (-2**31, 2**31 - 1)
    lo = lim[0] if bounds[0] is None else bounds[0]
    hi = lim[1] if bounds[1] is None else bounds[1]
    expected = oracle.clip(a, np.array(lo, dtype), np.array(hi, dtype))
    np.testing.assert_array_equal(expected, np.clip(a, *bounds).astype(dtype))
    assert_bits(hip(cx, a).clip(*bounds).numpy(), expected, "clip")


@pytest.mark.parametrize("dtype", ["float32", "int32"])
def test_clip_broadcast_bounds(cx, dtype):
    a = np.array([[[-4], [1], [9]]], dtype=dtype)
    lo = np.array([[-1, 2, 7, 8]], dtype=dtype)
    hi = np.array([[[3]], [[10]]], dtype=dtype)
    x = hip(cx, a)
    result = cx.clip(x, hip(cx, lo), hip(cx, hi))
    assert_bits(result.numpy(), oracle.clip(a, lo, hi), "clip broadcast")
    assert not cx._core._shares_storage(result._impl, x._impl)


def test_clip_ieee(cx):
    a = np.array([np.nan, -0., 0., 1e-40, -1e-40, np.inf, -np.inf, 1., 2.], np.float32)
    lo = np.array([-1., 0., -0., -2e-40, -2e-40, -1., -1., np.nan, -1.], np.float32)
    hi = np.array([1., 0., -0., 2e-40, 2e-40, 1., 1., 2., np.nan], np.float32)
    result = cx.clip(*[hip(cx, v) for v in (a, lo, hi)]).numpy()
    assert_bits(result, oracle.clip(a, lo, hi), "clip ieee")


def test_clip_contract(cx):
    x = hip(cx, np.zeros(3, np.float32))
    with pytest.raises(ValueError):
        cx.clip(x)
    with pytest.raises(TypeError):
        cx.clip(x, True)
    with pytest.raises(ValueError):
        cx.clip(x, hip(cx, np.zeros(3, np.int32)))
    with pytest.raises(ValueError):
        cx.clip(hip(cx, np.zeros(3, np.int32)), 0.5)


# ------------------------------------------------------------- topk
@pytest.mark.parametrize("dtype", ["float32", "int32"])
@pytest.mark.parametrize("shape,axis", [((3, 5, 6), 0), ((3, 5, 6), 1), ((3, 5, 6), -1), ((7,), 0),
                                        ((4, 300), 1), ((2, 2049), -1), ((300, 3), 0)])
@pytest.mark.parametrize("largest", [True, False])
@pytest.mark.parametrize("sort", [True, False])
def test_topk(cx, dtype, shape, axis, largest, sort):
    rng = np.random.default_rng(81)
    a = rng.integers(-4, 5, shape).astype(dtype)  # many ties
    if dtype == "float32":
        flat = a.reshape(-1)
        flat[rng.integers(0, flat.size, 3)] = np.nan
        flat[rng.integers(0, flat.size, 3)] = -0.0
    n = shape[axis]
    for k in sorted({0, 1, n // 3, n}):
        values, indices = cx.topk(hip(cx, a), k, axis, largest, sort)
        ev, ei = oracle.topk(a, k, axis, largest, sort)
        assert values.dtype == dtype and indices.dtype == "int32"
        assert_bits(values.numpy(), ev, f"topk values k={k}")
        assert_bits(indices.numpy(), ei, f"topk indices k={k}")


def test_topk_contract(cx):
    x = hip(cx, np.arange(6, dtype=np.float32).reshape(2, 3))
    for k in (-1, 4):
        with pytest.raises(ValueError):
            cx.topk(x, k)
    for k in (True, 1.5, "2"):
        with pytest.raises(TypeError):
            cx.topk(x, k)
    with pytest.raises(TypeError):
        cx.topk(x, 1, largest=1)
    with pytest.raises(ValueError):
        cx.topk(hip(cx, np.float32(3)), 1)
    with pytest.raises(ValueError):
        cx.topk(x, 1, axis=2)
    values, indices = x.topk(2)
    assert_bits(values.numpy(), np.array([[2, 1], [5, 4]], np.float32), "method")
    assert_bits(indices.numpy(), np.array([[2, 1], [2, 1]], np.int32), "method")


# ------------------------------------------------------------- embedding
@pytest.mark.parametrize("shape", [(), (4,), (2, 3), (2, 0, 3), (64, 65)])
@pytest.mark.parametrize("width", [0, 1, 7, 128])
def test_embedding(cx, shape, width):
    indices = np.random.default_rng(7).integers(0, 5, size=shape, dtype=np.int32)
    w = f32((5, width))
    ids, weight = hip(cx, indices), hip(cx, w)
    y = cx.embedding(ids, weight)
    assert_bits(y.numpy(), oracle.embedding(indices, w), "embedding")
    assert_bits(ids.embedding(weight).numpy(), oracle.embedding(indices, w), "method")
    assert not cx._core._shares_storage(y._impl, weight._impl)
    assert_bits(ids.numpy(), indices, "indices untouched")


def test_embedding_bits_and_errors(cx):
    words = np.array([[0, 0x80000000, 1, 0x7fc01234], [0x7f800000, 0xff800000, 0x80000001, 0x3f800000]],
                     np.uint32)
    ids = np.array([1, 0, 1], np.int32)
    out = cx.embedding(hip(cx, ids), hip(cx, words.view(np.float32))).numpy()
    np.testing.assert_array_equal(out.view(np.uint32), words[ids])
    for width in (0, 3):
        for bad, vocab in (([-1], 2), ([2], 2), ([0], 0), ([0, 1, 2147483647], 2)):
            with pytest.raises(ValueError):
                cx.embedding(hip(cx, np.array(bad, np.int32)), cx.zeros((vocab, width), device="hip"))
    with pytest.raises(ValueError):
        cx.embedding(cx.zeros((0,), device="hip"), cx.zeros((2, 3), device="hip"))
    with pytest.raises(ValueError):
        cx.embedding(cx.zeros((0,), dtype="int32", device="hip"), cx.zeros((3,), device="hip"))
    empty = cx.embedding(cx.empty((2, 0), dtype="int32", device="hip"), cx.empty((0, 4), device="hip"))
    assert empty.shape == (2, 0, 4)


# ------------------------------------------------------------- attention
ATTENTION_SHAPES = [((3, 4), (5, 4), (5, 2)), ((2, 3, 4), (2, 5, 4), (2, 5, 6)),
                    ((2, 1, 3, 4), (1, 3, 5, 4), (2, 3, 5, 2)), ((3, 4), (5, 4), (2, 1, 5, 2)),
                    ((0, 4), (5, 4), (5, 2)), ((3, 4), (0, 4), (0, 2)),
                    ((0, 3, 4), (1, 5, 4), (1, 5, 2)), ((3, 4), (5, 4), (5, 0)),
                    ((2, 8, 100, 64), (2, 8, 130, 64), (2, 8, 130, 64))]


def attention_check(cx, q, k, v, mask=None, causal=False, scale=None):
    expected = oracle.attention(q, k, v, mask, causal, scale)
    args = [hip(cx, t) for t in (q, k, v)]
    m = None if mask is None else hip(cx, mask)
    got = cx.attention(*args, m, is_causal=causal, scale=scale)
    assert got.device == "hip" and got.dtype == "float32" and got.shape == expected.shape
    assert_close(got.numpy(), expected, 2e-4, 2e-5, "attention")
    return got


@pytest.mark.parametrize("shapes", ATTENTION_SHAPES)
@pytest.mark.parametrize("mask_kind", ["none", "bool", "additive", "scalar_false"])
@pytest.mark.parametrize("causal", [False, True])
def test_attention(cx, shapes, mask_kind, causal):
    q, k, v = [f32(shape, i + 10) for i, shape in enumerate(shapes)]
    mshape = (q.shape[-2], k.shape[-2])
    rng = np.random.default_rng(41)
    mask = None
    if mask_kind == "bool":
        mask = rng.random(mshape) > .4
        if mask.shape[0]:
            mask[0] = False
    elif mask_kind == "additive":
        mask = f32(mshape)
        mask[rng.random(mshape) < .3] = -np.inf
        if mask.shape[0]:
            mask[0] = -np.inf
    elif mask_kind == "scalar_false":
        mask = np.array(False)
    attention_check(cx, q, k, v, mask, causal)


@pytest.mark.parametrize("scale", [0, -0.5, 2, np.float32(.3), 1e-39, -1e-40])
def test_attention_scale_and_batched_mask(cx, scale):
    q, k, v = f32((2, 3, 4)), f32((5, 4), 2), f32((5, 3), 3)
    mask = np.random.default_rng(4).random((2, 1, 5)) > .3
    attention_check(cx, q, k, v, mask, scale=float(scale))


def test_attention_causality(cx):
    q, k, v = f32((5, 4)), f32((5, 4), 2), f32((5, 3), 3)
    before = cx.attention(*[hip(cx, t) for t in (q, k, v)], is_causal=True).numpy()
    k[3:] += 100
    v[3:] -= 500
    after = cx.attention(*[hip(cx, t) for t in (q, k, v)], is_causal=True).numpy()
    np.testing.assert_array_equal(before[:3], after[:3])


@pytest.mark.parametrize("exceptional", [np.nan, np.inf, -np.inf])
@pytest.mark.parametrize("masked", [False, True])
def test_attention_nonfinite_scores(cx, exceptional, masked):
    q, k, v = np.ones((1, 2), np.float32), np.ones((2, 2), np.float32), f32((2, 3))
    k[0] = exceptional
    with np.errstate(all="ignore"):
        attention_check(cx, q, k, v, np.array([[not masked, True]]))


@pytest.mark.parametrize("bias", [np.nan, np.inf, -np.inf])
def test_attention_nonfinite_additive_mask(cx, bias):
    q, k, v = f32((2, 3)), f32((4, 3)), f32((4, 2))
    mask = np.array([[bias, 0, -np.inf, 0], [bias, bias, bias, bias]], np.float32)
    with np.errstate(all="ignore"):
        attention_check(cx, q, k, v, mask)


def test_attention_nan_value_under_zero_probability(cx):
    q = cx.ones((1, 1), device="hip")
    y = cx.attention(q, q, hip(cx, np.array([[np.nan]], np.float32)), hip(cx, np.array(False)))
    assert np.isnan(y.numpy()).all()


@pytest.mark.parametrize("scale", [np.nan, np.inf, -np.inf, 1e300, 1e-300, 10**400])
def test_attention_invalid_scale(cx, scale):
    q, k, v = [cx.zeros(s, device="hip") for s in ((0, 2), (3, 2), (3, 1))]
    with pytest.raises(ValueError):
        cx.attention(q, k, v, scale=scale)


def test_attention_contract(cx):
    def t(shape, dtype="float32"):
        return cx.zeros(shape, dtype=dtype, device="hip")
    for call in (lambda: cx.attention(t((3,)), t((2, 3)), t((2, 3))),
                 lambda: cx.attention(t((0, 3)), t((2, 4)), t((2, 3))),
                 lambda: cx.attention(t((0, 0)), t((2, 0)), t((2, 3))),
                 lambda: cx.attention(t((0, 3)), t((2, 3)), t((3, 3))),
                 lambda: cx.attention(t((2, 0, 3)), t((3, 2, 3)), t((3, 2, 3))),
                 lambda: cx.attention(t((0, 3)), t((2, 3)), t((2, 3)), t((0, 2), "int32")),
                 lambda: cx.attention(t((0, 3)), t((2, 3)), t((2, 3)), t((0, 3), "bool")),
                 lambda: cx.attention(t((0, 3)), t((2, 3)), t((2, 3)), t((1, 0, 2), "bool")),
                 lambda: cx.attention(t((0, 3), "int32"), t((2, 3)), t((2, 3)))):
        with pytest.raises(ValueError):
            call()
    x = cx.ones((2, 2), device="hip")
    for scale in (True, "2", 1j, [1]):
        with pytest.raises(TypeError):
            cx.attention(x, x, x, scale=scale)
    with pytest.raises(TypeError):
        cx.attention(x, x, x, is_causal=1)
    with pytest.raises(TypeError):
        cx.attention(x, x, x, [[True]])


def test_attention_shapes_at_the_edges(cx):
    q = cx.empty((0, 2**62, 4, 0, 2), device="hip")
    v = cx.empty((0, 2**62, 4, 0, 3), device="hip")
    assert cx.attention(q, q, v).shape == (0, 2**62, 4, 0, 3)
    shape = (1,) * 17
    attention_check(cx, f32(shape + (3, 4)), f32(shape + (2, 4), 2), f32(shape + (2, 3), 3))
    q, k, v = f32((257, 3)), f32((513, 3), 4), f32((513, 2), 5)
    tensors = [hip(cx, t) for t in (q, k, v)]
    result = attention_check(cx, q, k, v, causal=True)
    for source, array in zip(tensors, (q, k, v)):
        assert not cx._core._shares_storage(source._impl, result._impl)
        assert_bits(source.numpy(), array, "inputs untouched")


def test_inference_pipeline(cx):
    """embedding -> linear -> causal self-attention -> affine LayerNorm -> linear
    (test_inference_ops.py:259-280), every stage on the device."""
    ids_np = np.array([[0, 2, 1], [1, 3, 0]], np.int32)
    table, weight, bias, gain, shift = f32((4, 4)), f32((4, 4), 2), f32((4,), 3), f32((4,), 4), f32((4,), 5)
    ids = hip(cx, ids_np)
    ts = [hip(cx, t) for t in (table, weight, bias, gain, shift)]
    embedded = cx.embedding(ids, ts[0])
    projected = cx.linear(embedded, ts[1], ts[2])
    attended = cx.attention(projected, projected, projected, is_causal=True)
    normalized = cx.layernorm(attended, -1, weight=ts[3], bias=ts[4])
    output = cx.linear(normalized, ts[1])
    p = oracle.linear(oracle.embedding(ids_np, table), weight, bias)
    a = oracle.attention(p, p, p, None, True)
    expected = oracle.linear(oracle.affine_norm(a, -1, 1e-5, gain, shift), weight)
    assert_close(output.numpy(), expected, 2e-4, 2e-5, "pipeline")


def test_attention_masked_full_tiles(cx):
    # 8 x 2048 x 2048 scores over K = 64: 512 full 256x256 tiles, so the
    # score product (B transposed) takes the direct-to-LDS GEMM kernel.
    q, k, v = f32((8, 2048, 64), 21), f32((8, 2048, 64), 22), f32((8, 2048, 64), 23)
    mask = np.random.default_rng(24).random((2048, 2048)) > .2
    attention_check(cx, q, k, v, mask)


def test_attention_masked_direct128_scores(cx):
    # 8 x 1024 x 1024 scores over K = 64: 512 full 128x128 tiles but only 128
    # of 256x256, so the batched score product (B transposed) takes the
    # direct 128x128 kernel.
    q, k, v = f32((8, 1024, 64), 25), f32((8, 1024, 64), 26), f32((8, 1024, 64), 27)
    mask = np.random.default_rng(28).random((1024, 1024)) > .2
    attention_check(cx, q, k, v, mask)


# ------------------------------------------------------------- fused attention
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("rows,cols", [(1, 1), (64, 64), (65, 130), (200, 37), (5, 0), (3, 257), (300, 1000)])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_attention(cx, d, rows, cols, causal):
    # Unmasked attention over matching batches takes the fused kernel.
    q, k, v = f32((2, 3, rows, d), 1), f32((2, 3, cols, d), 2), f32((2, 3, cols, d), 3)
    attention_check(cx, q, k, v, None, causal)
    attention_check(cx, q, k, v, None, causal, scale=0.05)


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_attention_xcd_block_order(cx, d, causal):
    # 8 batch matrices x 3 query tiles: the unmasked kernel regroups its blocks
    # by batch matrix (launch count a multiple of 8).
    q, k, v = f32((2, 4, 300, d), 21), f32((2, 4, 700, d), 22), f32((2, 4, 700, d), 23)
    attention_check(cx, q, k, v, None, causal)


@pytest.mark.parametrize("causal", [False, True])
def test_fused_attention_bench_size(cx, causal):
    # The bench workload (16 x 2048 x 128): checked against float64 truth
    # (the sequential-dot oracle would take minutes at this size), with the
    # attention bar of the reference test.
    import tensorcx_workloads as wl
    q, k, v = wl.attention_inputs()
    got = cx.attention(*(hip(cx, t) for t in (q, k, v)), None, is_causal=causal).numpy()
    q64, k64, v64 = (t.astype(np.float64) for t in (q, k, v))
    s = (q64 @ np.swapaxes(k64, -1, -2)) / np.sqrt(q.shape[-1])
    if causal:
        s = np.where(np.tril(np.ones(s.shape[-2:], dtype=bool)), s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    expected = (p / p.sum(axis=-1, keepdims=True)) @ v64
    assert_close(got, expected, 2e-4, 2e-5, "attention bench size")


@pytest.mark.parametrize("causal", [False, True])
def test_fused_attention_many_batch_matrices(cx, causal):
    # More batch matrices than a grid dimension of 65535 blocks holds: the
    # fused kernel runs on a 1-D grid of (batch, query tile) items.
    q, k, v = f32((66000, 3, 32), 24), f32((66000, 5, 32), 25), f32((66000, 5, 32), 26)
    attention_check(cx, q, k, v, None, causal)


@pytest.mark.parametrize("d", [32, 64, 128])
def test_fused_attention_causal_value_scan(cx, d):
    # Non-finite values in V rows behind the causal mask of whole query tiles:
    # the tail scan (rows past a block's last run tile) must flag exactly their
    # columns, across its 8-deep unrolled passes and its remainder loop.
    q, k, v = f32((2, 700, d), 31), f32((2, 700, d), 32), f32((2, 700, d), 33)
    v[0, 650, 3] = np.nan
    v[0, 699, d - 1] = np.inf
    v[0, 130, 0] = -np.inf
    v[1, 64, d // 2] = np.inf     # the first row the first query tile's scan reads
    v[1, 520, 1] = np.nan
    with np.errstate(all="ignore"):
        attention_check(cx, q, k, v, None, True)


@pytest.mark.parametrize("d", [32, 64, 128])
def test_fused_attention_special_values(cx, d):
    q, k, v = f32((1, 70, d), 4), f32((1, 90, d), 5), f32((1, 90, d), 6)
    q[0, 3, 7] = np.nan            # a NaN query: its row is NaN
    k[0, 11] = np.inf              # an infinite key: +inf / NaN scores
    k[0, 12] = -np.inf
    v[0, 80, 5] = np.nan           # a NaN value behind the causal mask of early queries
    with np.errstate(all="ignore"):
        for causal in (False, True):
            attention_check(cx, q, k, v, None, causal)
    # All scores -inf for one query: 0 * V.
    q2, k2, v2 = np.ones((1, 2, d), np.float32), np.ones((1, 3, d), np.float32), f32((1, 3, d), 7)
    q2[0, 1] = -np.inf
    k2[0, :, :] = 1.0
    with np.errstate(all="ignore"):
        attention_check(cx, q2, k2, v2)


# Causal shapes with 256 or more batch matrices: at least two query tiles per
# CU, more blocks than fit on the device at once (heaviest first: 130 rows
# and more at D = 128, two blocks per CU) or all resident (the heavy/light
# block order: 64 rows, one query tile per matrix), with
# partial last tiles, key lengths other than the query length and empty keys.
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("rows,cols", [(64, 64), (130, 130), (257, 200), (200, 257), (300, 37), (65, 0)])
def test_fused_attention_causal_many_tiles(cx, d, rows, cols):
    q, k, v = f32((256, rows, d), 41), f32((256, cols, d), 42), f32((256, cols, d), 43)
    attention_check(cx, q, k, v, None, True)
    attention_check(cx, q, k, v, None, True, scale=0.05)


@pytest.mark.parametrize("d", [32, 128])
def test_fused_attention_causal_odd_tile_count(cx, d):
    # 3 query tiles per matrix: the heavy/light order pairs tiles of
    # different matrices on one CU.
    q, k, v = f32((512, 150, d), 44), f32((512, 150, d), 45), f32((512, 150, d), 46)
    attention_check(cx, q, k, v, None, True)


@pytest.mark.parametrize("d", [32, 64, 128])
def test_fused_attention_causal_many_value_scan(cx, d):
    # Non-finite V rows behind the causal masks of early query tiles (the
    # tail scan) and inside the key ranges the tiles run.
    q, k, v = f32((256, 300, d), 47), f32((256, 300, d), 48), f32((256, 300, d), 49)
    v[0, 290, 3] = np.nan      # inside the key range of the last query tile
    v[3, 70, d - 1] = np.inf   # behind the first query tile (queries 0..63)
    v[5, 20, 0] = -np.inf      # an early key, seen by every query tile
    v[7, 200, 1] = np.nan      # behind the first three query tiles
    v[9, 299, 2] = np.inf      # the last key
    with np.errstate(all="ignore"):
        attention_check(cx, q, k, v, None, True)


@pytest.mark.parametrize("d", [32, 128])
def test_fused_attention_causal_many_special_values(cx, d):
    q, k, v = f32((256, 200, d), 50), f32((256, 200, d), 51), f32((256, 200, d), 52)
    q[0, 3, 7] = np.nan          # a NaN query: its row is NaN
    q[1, 190, 0] = np.nan        # in the last query tile
    k[2, 11] = np.inf            # +inf / NaN scores for every query after key 11
    k[3, 150] = -np.inf
    q[4, 199] = -np.inf          # scores of -inf and +inf / NaN
    with np.errstate(all="ignore"):
        attention_check(cx, q, k, v, None, True)
