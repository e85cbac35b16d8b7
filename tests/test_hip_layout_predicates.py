"""GPU parity of layout, conversion and predicate ops on the hip device:
indexing / transpose / concat / stack / split, astype, scalar arithmetic,
comparisons, logical ops, where, any / all and masked_select.

Cases follow the reference's device-generic suites (tests/python/
test_indexing_joining.py, test_cast_broadcast.py, test_boolean_masks.py,
test_int32_primitives.py). These ops are exact (bit-preserving copies, IEEE
comparisons, wrapping int32), so NumPy's own result is the oracle, as in those
suites; every comparison is bit-exact (for float arithmetic, NaN payloads
aside: IEEE leaves the payload of an arithmetic NaN open, so there the NaN
positions must agree and every other bit must match).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import require_gpu
from hip_cases import assert_bits, assert_nan_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cx():
    require_gpu()
    import tensorcx
    return tensorcx


def hip(cx, a):
    return cx.tensor(a, device="hip")


# ------------------------------------------------------------- indexing and joining
@pytest.mark.parametrize("dtype", ["float32", "int32"])
@pytest.mark.parametrize("shape,key", [
    ((3, 4, 5), 1), ((3, 4, 5), -1), ((3, 4, 5), (1, -1, 2)),
    ((3, 4, 5), (slice(None), slice(1, 4, 2), slice(None, None, -1))),
    ((3, 4), (None, Ellipsis, -1, None)), ((3, 4), (Ellipsis, None)),
    ((3, 4), (slice(None, None, -1), slice(3, 0, -2))),
    ((3, 4), (slice(99), slice(-99, 99))), ((3, 4), (slice(2, 1),)),
    ((0, 3), (slice(None, None, -1), 1)), ((2, 0, 3), (1, Ellipsis, None)),
    ((3,), (slice(None, None, 10**100),)), ((3,), (slice(None, None, -(10**100)),)),
    ((3,), np.int64(1)), ((), ()), ((), Ellipsis), ((3, 4), (1, Ellipsis, 2)),
    ((2, 3, 4, 5, 6, 7, 8, 9, 2), (1, slice(None, None, 2), Ellipsis, slice(1, None)))])
def test_indexing(cx, dtype, shape, key):
    values = np.arange(np.prod(shape, dtype=int), dtype=dtype).reshape(shape)
    x = hip(cx, values)
    y = x[key]
    expected = values[key]
    assert y.shape == expected.shape and y.dtype == dtype
    assert not cx._core._shares_storage(x._impl, y._impl)
    assert_bits(y.numpy(), np.asarray(expected), f"x[{key!r}]")


def test_indexing_errors(cx):
    x = hip(cx, np.zeros((3, 4), np.float32))
    for key in ((0, 0, 0), 3, -4, (Ellipsis, Ellipsis), 1.5, (slice(True),)):
        with pytest.raises((IndexError, ValueError)):
            x[key]


@pytest.mark.parametrize("axis", [0, 1, -1, -2])
@pytest.mark.parametrize("dtype", ["float32", "int32", "bool"])
@pytest.mark.parametrize("sizes", [(2, 3, 1), (0, 3, 0), (5,)])
def test_concat(cx, dtype, axis, sizes):
    arrays = [(np.arange(4 * n).reshape((n, 4) if axis in (0, -2) else (4, n)) % 3).astype(dtype)
              for n in sizes]
    result = cx.concat(iter([hip(cx, a) for a in arrays]), axis)
    assert_bits(result.numpy(), np.concatenate(arrays, axis), "concat")


@pytest.mark.parametrize("shape", [(), (0,), (2, 3), (2, 0, 3)])
@pytest.mark.parametrize("axis", [0, -1])
def test_stack_and_split(cx, shape, axis):
    values = np.arange(np.prod(shape, dtype=int), dtype=np.float32).reshape(shape)
    x = hip(cx, values)
    stacked = cx.stack([x, x, x], axis)
    assert_bits(stacked.numpy(), np.stack([values] * 3, axis), "stack")
    parts = cx.split(stacked, 3, axis)
    for part, ref in zip(parts, np.split(np.stack([values] * 3, axis), 3, axis)):
        assert_bits(part.numpy(), ref, "split")
    assert not cx._core._shares_storage(x._impl, stacked._impl)


@pytest.mark.parametrize("perm", [None, (0, 1, 2), (2, 0, 1), (-1, -3, -2)])
def test_transpose(cx, perm):
    values = np.random.default_rng(2).normal(size=(3, 4, 5)).astype(np.float32)
    values[0, 0, :3] = [np.nan, -0.0, np.inf]
    y = cx.transpose(hip(cx, values), perm)
    assert_bits(y.numpy(), np.ascontiguousarray(np.transpose(values, perm)), "transpose")
    assert_bits(hip(cx, values).T.numpy(), np.ascontiguousarray(values.T), ".T")


def test_transpose_high_rank_and_squeeze(cx):
    values = np.arange(2 * 3 * 1 * 4 * 1 * 2 * 3 * 1 * 2 * 2, dtype=np.int32).reshape(2, 3, 1, 4, 1, 2, 3, 1, 2, 2)
    perm = (9, 0, 8, 1, 7, 2, 6, 3, 5, 4)
    assert_bits(cx.transpose(hip(cx, values), perm).numpy(), np.ascontiguousarray(values.transpose(perm)), "rank 10")
    x = hip(cx, values)
    assert cx.squeeze(x).shape == values.squeeze().shape
    assert cx.expand_dims(x, (0, -1)).shape == (1,) + values.shape + (1,)
    with pytest.raises(ValueError):
        cx.squeeze(x, 0)
    with pytest.raises(ValueError):
        cx.transpose(x, (0, 0, 1, 2, 3, 4, 5, 6, 7, 8))


# ------------------------------------------------------------- casts and scalar arithmetic
def test_astype(cx):
    f = np.array([0.0, -0.0, 1.9, -1.9, 2147483520.0, -2147483648.0, 1e-40, 3.5e6, np.nan], np.float32)
    i = np.array([0, 1, -1, 2**31 - 1, -2**31, 16777217, 7], np.int32)
    b = np.array([True, False, True])
    for name, arr in (("f", f[:-1]), ("i", i), ("b", b)):
        for dst in ("float32", "int32", "bool"):
            got = cx.astype(hip(cx, arr), dst).numpy()
            expected = (arr != 0).astype(dst) if dst == "bool" or arr.dtype == np.bool_ else arr.astype(dst)
            assert_bits(got, expected, f"{name}->{dst}")
    assert_bits(hip(cx, f).astype("bool").numpy(), f != 0, "NaN is true")
    for bad in (np.nan, np.inf, -np.inf, 2147483648.0):
        with pytest.raises(ValueError):
            cx.astype(hip(cx, np.array([1.0, bad], np.float32)), "int32")
    x = hip(cx, f)
    assert x.astype("float32", copy=False) is x
    assert not cx._core._shares_storage(x.astype("float32")._impl, x._impl)


@pytest.mark.parametrize("scalar", [0.1, -3, 1e30, 0.0, -0.0])
def test_scalar_arithmetic_f32(cx, scalar):
    a = np.random.default_rng(5).normal(size=(7, 300)).astype(np.float32) * 3
    a[0, :3] = [np.nan, np.inf, -0.0]
    x = hip(cx, a)
    s = np.float32(scalar)
    with np.errstate(all="ignore"):
        for got, expected in ((x + scalar, a + s), (scalar + x, s + a), (x - scalar, a - s), (scalar - x, s - a),
                              (x * scalar, a * s), (scalar * x, s * a), (x / scalar, a / s), (scalar / x, s / a),
                              (-x, -a)):
            assert_nan_bits(got.numpy(), np.asarray(expected, np.float32), f"scalar {scalar}")


def test_scalar_arithmetic_i32_wraps(cx):
    a = np.random.default_rng(6).integers(-2**31, 2**31 - 1, (5, 99), dtype=np.int64).astype(np.int32)
    a[0, :2] = [-2**31, 2**31 - 1]
    x, u = hip(cx, a), a.astype(np.uint32)
    for s in (1, -7, 2**31 - 1, -2**31):
        su = np.uint32(s & 0xFFFFFFFF)
        with np.errstate(all="ignore"):
            assert_bits((x + s).numpy(), (u + su).view(np.int32), "add")
            assert_bits((s - x).numpy(), (su - u).view(np.int32), "rsub")
            assert_bits((x * s).numpy(), (u * su).view(np.int32), "mul")
    assert_bits((-x).numpy(), (np.uint32(0) - u).view(np.int32), "negate wraps")
    with pytest.raises(ValueError):
        x / 2
    with pytest.raises(ValueError):
        x + 0.5
    with pytest.raises(ValueError):
        x + 2**31
    with pytest.raises(TypeError):
        x + True


# ------------------------------------------------------------- predicates
@pytest.mark.parametrize("name,op", [("equal", np.equal), ("not_equal", np.not_equal), ("less", np.less),
                                     ("less_equal", np.less_equal), ("greater", np.greater),
                                     ("greater_equal", np.greater_equal)])
@pytest.mark.parametrize("dtype", ["float32", "int32", "bool"])
def test_comparisons(cx, name, op, dtype):
    rng = np.random.default_rng(9)
    if dtype == "float32":
        a = np.array([[0.0, -0.0, np.nan, 1.0, -np.inf, 2.5]], np.float32)
        b = np.array([[0.0], [np.nan], [2.5]], np.float32)
    elif dtype == "int32":
        a, b = rng.integers(-3, 4, (4, 1, 6)).astype(np.int32), rng.integers(-3, 4, (5, 6)).astype(np.int32)
    else:
        a, b = rng.random((3, 1)) > .5, rng.random((1, 4)) > .5
    with np.errstate(invalid="ignore"):
        expected = op(a, b)
    got = getattr(cx, name)(hip(cx, a), hip(cx, b))
    assert got.dtype == "bool"
    assert_bits(got.numpy(), expected, name)


def test_operators_and_scalars(cx):
    a = np.arange(-3, 5, dtype=np.int32)
    x = hip(cx, a)
    assert_bits((x == 2).numpy(), a == 2, "==")
    assert_bits((x != 2).numpy(), a != 2, "!=")
    assert_bits((x < 1).numpy(), a < 1, "<")
    assert_bits((3 >= x).numpy(), 3 >= a, "reflected >=")
    m1, m2 = x > 0, x < 3
    assert_bits((m1 & m2).numpy(), (a > 0) & (a < 3), "&")
    assert_bits((m1 | m2).numpy(), (a > 0) | (a < 3), "|")
    assert_bits((m1 ^ m2).numpy(), (a > 0) ^ (a < 3), "^")
    assert_bits((~m1).numpy(), ~(a > 0), "~")
    assert_bits((m1 & True).numpy(), a > 0, "& scalar")
    with pytest.raises(TypeError):
        m1 & 1
    with pytest.raises(ValueError):
        x == 0.5
    with pytest.raises(ValueError):
        cx.logical_and(x, x)
    assert bool(hip(cx, np.array([True])))
    with pytest.raises(ValueError):
        bool(m1)


@pytest.mark.parametrize("dtype", ["float32", "int32", "bool"])
def test_where(cx, dtype):
    rng = np.random.default_rng(11)
    cond = rng.random((3, 1, 6)) > .5
    a = (rng.normal(size=(1, 5, 6)) * 3).astype(dtype)
    b = (rng.normal(size=(3, 5, 1)) * 3).astype(dtype)
    got = cx.where(hip(cx, cond), hip(cx, a), hip(cx, b))
    assert_bits(got.numpy(), np.where(cond, a, b), "where")
    if dtype != "bool":
        scalar = 2 if dtype == "int32" else 2.5
        got = cx.where(hip(cx, cond), hip(cx, a), scalar)
        assert_bits(got.numpy(), np.where(cond, a, np.asarray(scalar, dtype)), "where scalar")
    with pytest.raises(TypeError):
        cx.where(hip(cx, a.astype(np.float32)), hip(cx, a), hip(cx, b))


@pytest.mark.parametrize("name", ["any", "all"])
@pytest.mark.parametrize("axis", [None, 0, 1, -1, (0, 2), (), (2, 0)])
@pytest.mark.parametrize("keepdims", [False, True])
def test_any_all(cx, name, axis, keepdims):
    values = np.random.default_rng(12).random((3, 4, 5)) > .7
    got = getattr(cx, name)(hip(cx, values), axis, keepdims)
    expected = getattr(np, name)(values, axis=axis, keepdims=keepdims)
    assert_bits(got.numpy(), np.asarray(expected), f"{name} {axis}")
    empty = np.zeros((2, 0), bool)
    assert_bits(getattr(cx, name)(hip(cx, empty), 1).numpy(), getattr(np, name)(empty, axis=1), "empty")
    with pytest.raises(ValueError):
        getattr(cx, name)(hip(cx, values.astype(np.float32)))


@pytest.mark.parametrize("dtype", ["float32", "int32", "bool"])
@pytest.mark.parametrize("mask_shape", [(4,), (4, 5), (4, 5, 3), (0,)])
def test_masked_select(cx, dtype, mask_shape):
    rng = np.random.default_rng(13)
    shape = (0, 5, 3) if mask_shape == (0,) else (4, 5, 3)
    values = (rng.normal(size=shape) * 4).astype(dtype)
    mask = rng.random(mask_shape) > .5
    x, m = hip(cx, values), hip(cx, mask)
    got = cx.masked_select(x, m)
    expected = values.reshape((int(np.prod(mask_shape)),) + shape[len(mask_shape):])[mask.reshape(-1)]
    assert_bits(got.numpy(), np.ascontiguousarray(expected), "masked_select")
    assert_bits(x[m].numpy(), np.ascontiguousarray(expected), "x[mask]")
    with pytest.raises(ValueError):
        cx.masked_select(x, hip(cx, np.ones((5,), bool)))


def test_masked_select_many_chunks(cx):
    rng = np.random.default_rng(14)
    values = rng.normal(size=(100003, 3)).astype(np.float32)
    mask = rng.random(100003) > .3
    got = cx.masked_select(hip(cx, values), hip(cx, mask))
    assert_bits(got.numpy(), values[mask], "100k mask")
