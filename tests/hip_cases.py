"""Parity metrics and golden-case runners shared by the GPU tests.

Bars (stated once, used everywhere):
  * bit-exact: max, min, argmax, every int32 result, broadcast arithmetic, and
    float32 sum/mean on the exact-order paths (reductions of at most
    SEQUENTIAL_MAX elements, and selections of several reduced runs);
  * matmul / linear: max|dC| / (sqrt(K) * rms(A) * rms(B)) <= 1e-4;
  * float32 sum/mean over more than SEQUENTIAL_MAX elements of one reduced
    run (tree order along rows, a fixed interleaved order down columns):
    max|d| / sum|x| <= 1e-5 per output, a mean's error taken times its count;
  * softmax, LayerNorm, RMSNorm, affine norms, MLP output:
    allclose(rtol=1e-5, atol=1e-5), the reference's reduction class;
  * exp / gelu / silu: allclose(rtol=1e-6, atol=1e-6), the elementwise class;
  * abs, clip, topk, embedding, sqrt: bit-exact (sqrt is correctly rounded on
    both sides; NaNs compare as NaN, whatever their payload);
  * scalar arithmetic, casts, transpose / slice / concat, comparisons, logical
    ops, where, any / all, masked_select: bit-exact;
  * log: allclose(rtol=1e-6, atol=0), the bar of test_math_ops.py:15-21;
  * attention: allclose(rtol=2e-4, atol=2e-5), the bar of
    test_inference_ops.py:20-25.
"""

from __future__ import annotations

import numpy as np

import oracle

SEQUENTIAL_MAX = 64
MATMUL_BAR = 1e-4
SUM_BAR = 1e-5


def bits(x):
    x = np.asarray(x)
    return x.view(np.uint32) if x.dtype == np.float32 else x


def assert_bits(actual, expected, context=""):
    actual, expected = np.asarray(actual), np.asarray(expected)
    assert actual.shape == expected.shape, f"{context}: shape {actual.shape} != {expected.shape}"
    assert actual.dtype == expected.dtype, f"{context}: dtype {actual.dtype} != {expected.dtype}"
    diff = np.flatnonzero(bits(actual).reshape(-1) != bits(expected).reshape(-1))
    if diff.size:
        i = diff[0]
        raise AssertionError(f"{context}: {diff.size}/{actual.size} differ; first at {i}: "
                             f"{actual.reshape(-1)[i]!r} vs {expected.reshape(-1)[i]!r}")


def matmul_error(actual, expected, a, b) -> float:
    k = a.shape[-1] if a.ndim else 1
    if actual.size == 0 or k == 0:
        return 0.0 if np.array_equal(actual, expected) else np.inf
    scale = np.sqrt(k) * np.sqrt(np.mean(np.square(a, dtype=np.float64))) * \
        np.sqrt(np.mean(np.square(b, dtype=np.float64)))
    return float(np.max(np.abs(actual.astype(np.float64) - expected)) / max(scale, 1e-30))


def assert_matmul(actual, expected, a, b, context=""):
    assert actual.shape == expected.shape, f"{context}: shape {actual.shape} != {expected.shape}"
    err = matmul_error(actual, expected, a, b)
    assert err <= MATMUL_BAR, f"{context}: scaled matmul error {err:.3e} > {MATMUL_BAR}"
    return err


def sum_error(actual, expected, x, outer, reduce_, inner) -> float:
    """max |d| / sum|x| over outputs of an (outer, reduce, inner) reduction."""
    if actual.size == 0:
        return 0.0
    mag = np.abs(x.reshape(outer, reduce_, inner).astype(np.float64)).sum(axis=1).reshape(-1)
    d = np.abs(actual.reshape(-1).astype(np.float64) - expected.reshape(-1).astype(np.float64))
    finite = np.isfinite(expected.reshape(-1))
    assert np.array_equal(np.isnan(actual.reshape(-1)), np.isnan(expected.reshape(-1)))
    # Outputs whose expected value is NaN or infinite are checked above (NaN
    # positions) or not at all; their magnitude may itself be NaN.
    with np.errstate(invalid="ignore"):
        ratio = np.where(finite, d / np.maximum(mag, 1e-30), 0.0)
    return float(np.max(ratio))


def assert_close(actual, expected, rtol, atol, context=""):
    actual, expected = np.asarray(actual), np.asarray(expected)
    assert actual.shape == expected.shape, f"{context}: shape {actual.shape} != {expected.shape}"
    np.testing.assert_allclose(actual, expected, rtol=rtol, atol=atol, equal_nan=True, err_msg=context)


def selected_axes(shape, kw):
    """The normalized set of axes a reduction case selects."""
    rank = len(shape)
    if "axes" in kw:
        return {a % rank for a in kw["axes"]} if rank else set()
    return {oracle.normalize_axis(kw.get("axis", 0), rank)} if rank else set()


def selection_error(actual, expected, x, axes) -> float:
    """max |d| / sum|x| over the outputs of a reduction over `axes` of x."""
    if actual.size == 0:
        return 0.0
    mag = np.abs(x.astype(np.float64)).sum(axis=tuple(sorted(axes))).reshape(-1)
    d = np.abs(actual.reshape(-1).astype(np.float64) - expected.reshape(-1).astype(np.float64))
    finite = np.isfinite(expected.reshape(-1))
    assert np.array_equal(np.isnan(actual.reshape(-1)), np.isnan(expected.reshape(-1)))
    with np.errstate(invalid="ignore"):
        ratio = np.where(finite, d / np.maximum(mag, 1e-30), 0.0)
    return float(np.max(ratio))


def reduction_run(shape, kw):
    """(outer, reduce, inner, exact) for a golden reduction case, folded as the
    hip backend folds a selection: size-1 axes dropped, neighbouring axes of
    one kind merged. One run of reduced axes is an (outer, reduce, inner)
    reduction; several runs report (1, count, 1). Either is exact in order
    when at most SEQUENTIAL_MAX elements are reduced per output (a single run
    in a lane per output, several runs through the metadata kernel); more
    take the tree, blocked or run-by-run order, held to the sum bar."""
    rank = len(shape)
    axes = selected_axes(shape, kw)
    folded = []  # [extent, reduced]
    for i, extent in enumerate(shape):
        if extent == 1:
            continue
        if folded and folded[-1][1] == (i in axes):
            folded[-1][0] *= extent
        else:
            folded.append([extent, i in axes])
    runs = [i for i, (_, reduced) in enumerate(folded) if reduced]
    if len(runs) > 1:
        count = int(np.prod([e for e, reduced in folded if reduced], dtype=np.int64))
        return 1, count, 1, count <= SEQUENTIAL_MAX
    if not runs:
        return 1, 1, 1, True
    r = runs[0]
    outer = int(np.prod([e for e, _ in folded[:r]], dtype=np.int64))
    inner = int(np.prod([e for e, _ in folded[r + 1:]], dtype=np.int64))
    red = folded[r][0]
    return outer, red, inner, red <= SEQUENTIAL_MAX


def run_hip(cx, op, inputs, kw):
    """Runs one golden case through the tensorcx API on the hip device."""
    t = [cx.tensor(x, device="hip") for x in inputs]
    axis = kw.get("axis", 0)
    if op == "matmul":
        return cx.matmul(*t)
    if op in ("sum", "max", "mean"):
        return getattr(cx, op)(t[0], tuple(kw["axes"]) if "axes" in kw else axis)
    if op == "min":
        return cx.min(t[0], tuple(kw["axes"]))
    if op == "argmax":
        return cx.Tensor(cx._core._argmax_axes(t[0]._impl, list(kw["axes"])))
    if op == "softmax":
        return cx.softmax(t[0], axis)
    if op in ("rmsnorm", "layernorm"):
        return getattr(cx, op)(t[0], axis, kw.get("eps", 1e-5))
    if op in ("exp", "gelu", "silu"):
        return getattr(cx, op)(t[0])
    if op == "add":
        return t[0] + t[1]
    if op == "subtract":
        return t[0] - t[1]
    if op == "multiply":
        return t[0] * t[1]
    if op == "divide":
        return t[0] / t[1]
    if op == "linear":
        return cx.linear(*t)
    if op in ("affine_layernorm", "affine_rmsnorm"):
        weight = t[1] if kw.get("has_weight") else None
        bias = t[-1] if kw.get("has_bias") else None
        if op == "affine_rmsnorm":
            return cx.rmsnorm(t[0], axis, kw.get("eps", 1e-5), weight=weight)
        return cx.layernorm(t[0], axis, kw.get("eps", 1e-5), weight=weight, bias=bias)
    if op in ("log", "sqrt", "abs"):
        return getattr(cx, op)(t[0])
    if op == "clip":
        return cx.clip(*t)
    if op == "topk":
        return cx.topk(t[0], kw["k"], axis, kw.get("largest", True), kw.get("sorted", True))
    if op == "embedding":
        return cx.embedding(*t)
    if op == "attention":
        mask = t[3] if len(t) == 4 else None
        return cx.attention(*t[:3], mask, is_causal=kw.get("causal", False), scale=kw.get("scale"))
    if op == "negative":
        return -t[0]
    if op in ("add_scalar", "subtract_scalar", "multiply_scalar", "divide_scalar"):
        core = getattr(cx._core, op)
        return cx.Tensor(core(t[0]._impl, kw.get("scalar", 0.0), scalar_left=kw.get("scalar_left", False)))
    if op == "astype":
        return cx.astype(t[0], kw["target_dtype"])
    if op == "transpose":
        return cx.Tensor(cx._core.transpose(t[0]._impl, list(kw["perm"])))
    if op == "slice":
        return cx.Tensor(cx._core._slice(t[0]._impl, kw["starts"], kw["steps"], kw["lengths"]))
    if op == "concat":
        return cx.Tensor(cx._core._concat(t[0]._impl, [x._impl for x in t[1:]], axis))
    if op in ("any", "all"):
        return cx.Tensor(getattr(cx._core, f"_{op}_axes")(t[0]._impl, list(kw["axes"])))
    if op == "masked_select":
        return cx.masked_select(*t)
    if op in ("equal", "not_equal", "less", "less_equal", "greater", "greater_equal", "logical_and",
              "logical_or", "logical_xor", "logical_not", "where"):
        return cx.Tensor(getattr(cx._core, op)(*[x._impl for x in t]))
    raise AssertionError(op)


def host(result):
    """numpy value(s) of a run_hip result (a tensor or a tuple of tensors)."""
    if isinstance(result, tuple):
        return tuple(r.numpy() for r in result)
    return result.numpy()


def assert_nan_bits(actual, expected, context=""):
    """Bit-exact except that any NaN matches any NaN."""
    actual, expected = np.asarray(actual), np.asarray(expected)
    assert actual.shape == expected.shape and actual.dtype == expected.dtype, context
    nan_a, nan_e = np.isnan(actual), np.isnan(expected)
    assert np.array_equal(nan_a, nan_e), f"{context}: NaN positions differ"
    assert_bits(np.where(nan_a, 0, actual).astype(actual.dtype), np.where(nan_e, 0, expected).astype(expected.dtype),
                context)


def check_case(name, op, inputs, kw, actual, expected):
    """Applies the bar for `op` to one result (or tuple of results)."""
    if isinstance(expected, tuple):
        for n, (a, e) in enumerate(zip(actual, expected)):
            check_case(f"{name} output {n}", op, inputs, kw, a, e)
        return
    if op in ("max", "min", "argmax", "add", "subtract", "multiply", "divide", "abs", "clip", "topk",
              "embedding", "negative", "astype", "transpose", "slice", "concat", "equal", "not_equal", "less", "less_equal", "greater",
              "greater_equal", "logical_and", "logical_or", "logical_xor", "logical_not", "where", "any",
              "all", "masked_select") or expected.dtype in (np.int32, np.bool_):
        assert_bits(actual, expected, name)
    elif op in ("sqrt", "add_scalar", "subtract_scalar", "multiply_scalar", "divide_scalar"):
        # IEEE 754 leaves the payload of an arithmetic NaN open: NaN positions
        # must agree, every other bit must match.
        assert_nan_bits(actual, expected, name)
    elif op == "log":
        assert_close(actual, expected, 1e-6, 0.0, name)
    elif op == "attention":
        assert_close(actual, expected, 2e-4, 2e-5, name)
    elif op in ("sum", "mean"):
        outer, red, inner, exact = reduction_run(inputs[0].shape, kw)
        if exact:
            assert_bits(actual, expected, name)
        else:
            scale = np.float64(red if op == "mean" else 1)
            err = selection_error(actual * scale, expected * scale, inputs[0], selected_axes(inputs[0].shape, kw))
            assert err <= SUM_BAR, f"{name}: sum error {err:.3e}"
    elif op in ("matmul", "linear"):
        if op == "linear":
            a, b = inputs[0], inputs[1].T
        else:
            a, b = inputs[0], inputs[1]
        assert_matmul(actual, expected, a, b, name)
    elif op in ("exp", "gelu", "silu"):
        assert_close(actual, expected, 1e-6, 1e-6, name)
    else:
        assert_close(actual, expected, 1e-5, 1e-5, name)
