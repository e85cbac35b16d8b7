"""Pins the CPU oracle: golden vectors from the reference, the reference library
itself when built, and closed forms that a plausible mistake would break."""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from oracle import ref
from conftest import assert_bits_equal


def run_oracle(op, inputs, kw):
    axis = kw.get("axis", 0)
    if op == "matmul":
        return oracle.matmul(*inputs)
    if op in ("sum", "max", "mean"):
        if "axes" in kw:
            return getattr(oracle, op)(inputs[0], tuple(kw["axes"]))
        return getattr(oracle, op)(inputs[0], axis)
    if op in ("min", "argmax"):
        return getattr(oracle, op)(inputs[0], tuple(kw["axes"]))
    if op == "softmax":
        return oracle.softmax(inputs[0], axis)
    if op in ("rmsnorm", "layernorm"):
        return getattr(oracle, op)(inputs[0], axis, kw.get("eps", 1e-5))
    if op in ("exp", "gelu", "silu"):
        return getattr(oracle, op)(inputs[0])
    if op in ("add", "subtract", "multiply", "divide"):
        return oracle.binary(op, *inputs)
    if op == "linear":
        return oracle.linear(*inputs)
    if op in ("affine_layernorm", "affine_rmsnorm"):
        rms = op == "affine_rmsnorm"
        weight = inputs[1] if kw.get("has_weight") else None
        bias = inputs[-1] if kw.get("has_bias") else None
        return oracle.affine_norm(inputs[0], axis, kw.get("eps", 1e-5), weight, bias, rms=rms)
    if op in ("log", "sqrt", "abs"):
        return getattr(oracle, op)(inputs[0])
    if op == "clip":
        return oracle.clip(*inputs)
    if op == "topk":
        return oracle.topk(inputs[0], kw["k"], axis, kw.get("largest", True), kw.get("sorted", True))
    if op == "embedding":
        return oracle.embedding(*inputs)
    if op == "attention":
        mask = inputs[3] if len(inputs) == 4 else None
        return oracle.attention(*inputs[:3], mask, kw.get("causal", False), kw.get("scale"))
    if op in ("negative", "add_scalar", "subtract_scalar", "multiply_scalar", "divide_scalar"):
        return oracle.scalar_op(op, inputs[0], kw.get("scalar", 0.0), kw.get("scalar_left", False))
    if op == "astype":
        return oracle.astype(inputs[0], kw["target_dtype"])
    if op == "transpose":
        return oracle.transpose(inputs[0], kw["perm"])
    if op == "slice":
        return oracle.slice_(inputs[0], kw["starts"], kw["steps"], kw["lengths"])
    if op == "concat":
        return oracle.concat(inputs, axis)
    if op in ("any", "all"):
        return oracle.bool_reduce(op, inputs[0], kw["axes"])
    if op == "masked_select":
        return oracle.masked_select(*inputs)
    if op in ("equal", "not_equal", "less", "less_equal", "greater", "greater_equal", "logical_and",
              "logical_or", "logical_xor", "logical_not", "where"):
        return oracle.predicate(op, *inputs)
    raise AssertionError(op)


def expected_outputs(entry, arrays):
    if "outputs" in entry:
        return tuple(arrays[k] for k in entry["outputs"])
    return arrays[entry["output"]]


def test_golden_vectors_bit_exact(golden):
    manifest, arrays = golden
    assert len(manifest) > 600
    for entry in manifest:
        inputs = [arrays[k] for k in entry["inputs"]]
        if "error" in entry:
            with pytest.raises(ValueError):
                run_oracle(entry["op"], inputs, entry["kwargs"])
            continue
        actual = run_oracle(entry["op"], inputs, entry["kwargs"])
        expected = expected_outputs(entry, arrays)
        if isinstance(expected, tuple):
            for n, (a, e) in enumerate(zip(actual, expected)):
                assert_bits_equal(a, e, f"{entry['name']} output {n}")
        else:
            assert_bits_equal(actual, expected, entry["name"])


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_against_reference_library_random(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((9, 515)) * 3).astype(np.float32)
    for op in ("sum", "max", "mean", "softmax", "rmsnorm", "layernorm"):
        for axis in (0, 1):
            assert_bits_equal(run_oracle(op, [x], {"axis": axis}),
                              ref.execute(op, [x], axis=axis), f"{op} axis {axis}")
    for op in ("min", "argmax"):
        assert_bits_equal(oracle.__dict__[op](x, (1,)), ref.execute(op, [x], axes=[1]), op)
    a = rng.standard_normal((2, 31, 77)).astype(np.float32)
    b = rng.standard_normal((77, 45)).astype(np.float32)
    assert_bits_equal(oracle.matmul(a, b), ref.execute("matmul", [a, b]), "matmul")


# ---------------------------------------------------------------- closed forms
def test_matmul_dyadic_exact_and_kat():
    # Dyadic inputs make every product and partial sum exact in float32
    # (tests/cpp/batched_matmul_contract.h:25-26), so any order gives float64 truth.
    i = np.arange(3 * 20 * 30)
    a = ((i % 11 - 5) / 8).astype(np.float32).reshape(3, 20, 30)
    j = np.arange(30 * 12)
    b = ((j % 7 - 3) / 8).astype(np.float32).reshape(30, 12)
    expected = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    assert_bits_equal(oracle.matmul(a, b), expected, "dyadic")
    kat = oracle.matmul(np.array([[1, 2], [3, 4]], np.float32), np.array([[5, 6], [7, 8]], np.float32))
    assert kat.tolist() == [[19, 22], [43, 50]]


def test_matmul_is_sequential_k_order():
    # A transposed operand or a reordered k loop changes these bits: with
    # a = [1e8, 1, -1e8] and b = ones, sequential order gives (1e8+1)-1e8 = 0.
    a = np.array([[1e8, 1.0, -1e8]], np.float32)
    b = np.ones((3, 1), np.float32)
    assert oracle.matmul(a, b)[0, 0] == 0.0
    a = np.array([[1.0, 1e8, -1e8]], np.float32)
    assert oracle.matmul(a, b)[0, 0] == 0.0  # (1+1e8) rounds to 1e8
    a = np.array([[1e8, -1e8, 1.0]], np.float32)
    assert oracle.matmul(a, b)[0, 0] == 1.0


def test_reductions_against_numpy_exact_cases():
    rng = np.random.default_rng(5)
    xi = rng.integers(-1000, 1001, size=(17, 300)).astype(np.float32)  # integer-valued: exact
    np.testing.assert_array_equal(oracle.sum(xi, 1), xi.sum(axis=1, dtype=np.float64).astype(np.float32))
    np.testing.assert_array_equal(oracle.sum(xi, 0), xi.sum(axis=0, dtype=np.float64).astype(np.float32))
    np.testing.assert_array_equal(oracle.max(xi, 1), xi.max(axis=1))
    np.testing.assert_array_equal(oracle.min(xi, 1), xi.min(axis=1))
    np.testing.assert_array_equal(oracle.argmax(xi, 1), xi.argmax(axis=1).astype(np.int32))
    ii = rng.integers(-2**31, 2**31 - 1, size=(5, 1000), dtype=np.int64).astype(np.int32)
    np.testing.assert_array_equal(oracle.sum(ii, 1), ii.sum(axis=1, dtype=np.int32))
    np.testing.assert_array_equal(oracle.max(ii, 1), ii.max(axis=1))
    full = oracle.sum(xi, None)
    assert full.shape == () and full == xi.astype(np.float64).sum()


def test_sum_sequential_order_pins():
    # test_multi_axis_reductions.py:114-130: one pass in row-major order.
    assert oracle.sum(np.array([[1e20, 1], [-1e20, 3]], np.float32), None) == 3.0
    assert np.isposinf(oracle.mean(np.array([[3e38, 3e38], [-3e38, -3e38]], np.float32), None))
    s = oracle.sum(np.array([[-0.0, -0.0]], np.float32), 1)
    assert s[0] == 0 and not np.signbit(s[0])  # accumulator starts at +0


def test_argext_rules():
    x = np.array([[1, 5, 5, 2], [0.0, -0.0, 0.0, -1], [1, np.nan, 7, np.nan], [np.nan, 1, 2, 3]],
                 np.float32)
    np.testing.assert_array_equal(oracle.argmax(x, 1), np.array([1, 0, 1, 0], np.int32))
    m = oracle.min(x, 1)
    assert m[0] == 1 and m[1] == -1 and np.isnan(m[2]) and np.isnan(m[3])
    ties = np.array([[-0.0, 0.0, 1.0]], np.float32)
    assert np.signbit(oracle.min(ties, 1)[0])  # first of the equal zeros
    assert np.signbit(oracle.max(ties[:, :2], 1)[0])  # std::max keeps the earlier zero


def test_rowwise_closed_forms():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((8, 513)) * 3).astype(np.float32)
    x64 = x.astype(np.float64)
    sm = oracle.softmax(x, 1)
    ref64 = np.exp(x64 - x64.max(1, keepdims=True))
    ref64 /= ref64.sum(1, keepdims=True)
    np.testing.assert_allclose(sm, ref64, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(sm.sum(1), 1.0, rtol=1e-5)
    ln = oracle.layernorm(x, 1, 1e-5)
    mu = x64.mean(1, keepdims=True)
    np.testing.assert_allclose(ln, (x64 - mu) / np.sqrt(x64.var(1, keepdims=True) + 1e-5),
                               rtol=1e-4, atol=1e-5)
    rms = oracle.rmsnorm(x, 1, 1e-5)
    np.testing.assert_allclose(rms, x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-5),
                               rtol=1e-5, atol=1e-6)
    const = np.full((1, 8), 3.0, np.float32)
    assert np.all(oracle.layernorm(const, 1, 1e-5) == 0)
    assert np.all(np.isnan(oracle.layernorm(const, 1, 0.0)))


def test_elementwise_closed_forms():
    x = np.linspace(-8, 8, 101, dtype=np.float32)
    x64 = x.astype(np.float64)
    np.testing.assert_allclose(oracle.silu(x), x64 / (1 + np.exp(-x64)), rtol=1e-6, atol=1e-7)
    g = 0.5 * x64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (x64 + 0.044715 * x64 ** 3)))
    np.testing.assert_allclose(oracle.gelu(x), g, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(oracle.exp(x), np.exp(x64), rtol=1e-6)
    b = np.arange(10, dtype=np.float32)
    y = np.ones((3, 10), np.float32)
    np.testing.assert_array_equal(oracle.binary("add", y, b), y + b)
    np.testing.assert_array_equal(oracle.linear(y, np.eye(10, dtype=np.float32), b), y + b)


def test_plans_match_numpy_broadcasting():
    for a, b in [((2, 1, 5, 7), (3, 7, 4)), ((7,), (7, 3)), ((3, 7), (7,)), ((1, 4, 5), (6, 5, 2))]:
        out_shape = oracle.make_matmul_plan(a, b)[0]
        assert out_shape == np.matmul(np.zeros(a), np.zeros(b)).shape
    with pytest.raises(ValueError):
        oracle.make_matmul_plan((2, 3), (4, 5))
    shape, meta, size = oracle.make_reduction_plan((3, 4, 5), (2, 0))
    assert shape == (4,) and size == 15 and meta == [4, 5, 3, 20, 5, 1]


def test_math_clip_topk_closed_forms():
    rng = np.random.default_rng(11)
    squares = (np.arange(1, 300, dtype=np.float32)) ** 2
    np.testing.assert_array_equal(oracle.sqrt(squares), np.arange(1, 300, dtype=np.float32))
    powers = np.float32(2.0) ** np.arange(-20, 20, dtype=np.float32)
    np.testing.assert_allclose(oracle.log(powers), np.arange(-20, 20) * np.log(2.0), rtol=1e-6, atol=1e-6)
    x = rng.standard_normal(1000).astype(np.float32)
    assert_bits_equal(oracle.abs(x), np.abs(x), "abs")
    assert oracle.abs(np.array([-2**31], np.int32))[0] == -2**31  # uint32 negation wraps
    lo, hi = np.float32(-0.5), np.float32(0.7)
    np.testing.assert_array_equal(oracle.clip(x, np.array(lo), np.array(hi)), np.clip(x, lo, hi))
    # topk equals a stable sort by (-value, index); unsorted lists the same set by index.
    xi = rng.integers(-5, 6, (4, 50)).astype(np.int32)
    values, indices = oracle.topk(xi, 9, 1, True, True)
    order = np.argsort(-xi.astype(np.int64), axis=1, kind="stable")[:, :9]
    np.testing.assert_array_equal(indices, order)
    np.testing.assert_array_equal(values, np.take_along_axis(xi, order, 1))
    _, unsorted = oracle.topk(xi, 9, 1, True, False)
    np.testing.assert_array_equal(unsorted, np.sort(order, axis=1))
    low_values, _ = oracle.topk(xi, 9, 1, False, True)
    np.testing.assert_array_equal(low_values, np.sort(xi, axis=1)[:, :9])


def test_embedding_and_attention_closed_forms():
    rng = np.random.default_rng(12)
    table = rng.standard_normal((7, 5)).astype(np.float32)
    ids = rng.integers(0, 7, (3, 4)).astype(np.int32)
    assert_bits_equal(oracle.embedding(ids, table), table[ids], "embedding")
    with pytest.raises(ValueError):
        oracle.embedding(np.array([7], np.int32), table)
    q, k, v = [rng.standard_normal(s).astype(np.float32) for s in ((2, 6, 8), (2, 9, 8), (2, 9, 3))]
    mask = rng.random((6, 9)) > 0.3
    mask[:, 0] = True
    s = (q.astype(np.float64) @ np.swapaxes(k, -1, -2)) / np.sqrt(8.0)
    s = np.where(mask & (np.arange(9) <= np.arange(6)[:, None]), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    expected = (p / p.sum(-1, keepdims=True)) @ v
    np.testing.assert_allclose(oracle.attention(q, k, v, mask, True), expected, rtol=2e-5, atol=2e-6)
    # A row with every key masked is all zeros, not NaN (cpu_inference.cpp:36-39).
    none = np.zeros((6, 9), bool)
    assert not oracle.attention(q, k, v, none).any()
    # Causality: keys after the query do not change the output.
    k2, v2 = k.copy(), v.copy()
    k2[:, 4:] += 100
    v2[:, 4:] -= 500
    a = oracle.attention(q, k, v, None, True)
    b = oracle.attention(q, k2, v2, None, True)
    assert_bits_equal(a[:, :4], b[:, :4], "causal prefix")
