"""CPU ORACLE: test infrastructure only, never product code.

NumPy-level restatement of the tensor.cx CPU reference path for the hip hot
path. Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, and only as the checker. The arithmetic runs in
``liboracle.so`` (oracle.cpp, bit-identical restatement of the reference loops);
the shape plans below restate ``cpp/tensorcx/core/shape.cpp``.

Pinning: tests/test_oracle.py checks every function against golden vectors
written by the reference CPU backend itself (tests/golden/*.npz, made by
tests/golden/make_golden.py through oracle/_ref), against the reference
library directly when oracle/_ref is built, and against closed forms.
"""

from __future__ import annotations

import builtins
import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
_LIB = None

# Reference enum values (cpp/tensorcx/core/operation.h:12-53).
OPKIND = {
    "fill": 0, "add": 1, "multiply": 2, "matmul": 3, "sum": 4, "max": 5, "mean": 6,
    "exp": 7, "gelu": 8, "silu": 9, "softmax": 10, "rmsnorm": 11, "layernorm": 12,
    "subtract": 13, "divide": 14, "transpose": 21, "log": 38, "sqrt": 39, "abs": 40, "min": 41,
    "argmax": 42, "clip": 43, "topk": 44, "linear": 45, "affine_rmsnorm": 46,
    "affine_layernorm": 47, "embedding": 48, "attention": 49, "attention_softmax": 50,
}
DTYPE = {"float32": 0, "int32": 1, "bool": 2}


def default_threads() -> int:
    return builtins.max(1, builtins.min(16, os.cpu_count() or 1))


def build() -> None:
    """Compiles liboracle.so (and oracle/_ref when /root/reference is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "oracle"], check=True)
    if pathlib.Path("/root/reference/cpp/tensorcx").is_dir():
        subprocess.run(["make", "-s", "-j8", "-C", str(HERE), "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built; run `make -C oracle`")
        _LIB = ctypes.CDLL(str(path))
    return _LIB


def _p(array: np.ndarray):
    return array.ctypes.data_as(ctypes.c_void_p)


def _c(x) -> np.ndarray:
    """C-contiguous view or copy that keeps rank 0 (np.ascontiguousarray makes it rank 1)."""
    return np.asarray(x, order="C")


def _dims(values) -> np.ndarray:
    return np.asarray(np.asarray(values, dtype=np.int64).reshape(-1), order="C")


# ---------------------------------------------------------------- shape plans
def contiguous_strides(shape) -> list[int]:
    """shape.cpp:38-47."""
    strides, stride = [1] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        if shape[i] < 0:
            raise ValueError("shape dimensions must be non-negative")
        strides[i] = stride
        stride *= shape[i]
    return strides


def normalize_axis(axis: int, rank: int) -> int:
    """cpu_backend.cpp:79-91."""
    if rank == 0:
        if axis in (0, -1):
            return 0
        raise ValueError("reduction axis is out of range")
    if axis < 0:
        axis += rank
    if axis < 0 or axis >= rank:
        raise ValueError("reduction axis is out of range")
    return axis


def reduction_dims(shape, axis: int):
    """cpu_backend.cpp:93-123: (output_shape, outer, reduce, inner)."""
    axis = normalize_axis(axis, len(shape))
    if len(shape) == 0:
        return (), 1, 1, 1
    outer = int(np.prod(shape[:axis], dtype=np.int64))
    inner = contiguous_strides(shape)[axis]
    out_shape = tuple(d for i, d in enumerate(shape) if i != axis)
    return out_shape, outer, int(shape[axis]), inner


def make_matmul_plan(lhs, rhs):
    """shape.cpp:49-76: numpy matmul broadcasting over leading batch axes."""
    if len(lhs) == 0 or len(rhs) == 0:
        raise ValueError("matmul requires rank >= 1 tensors")
    ls, rs = contiguous_strides(lhs), contiguous_strides(rhs)
    lv, rv = len(lhs) == 1, len(rhs) == 1
    m = 1 if lv else lhs[-2]
    k = lhs[-1]
    rk = rhs[0] if rv else rhs[-2]
    n = 1 if rv else rhs[-1]
    if k != rk:
        raise ValueError("matmul shape mismatch: contracting dimensions differ")
    lb = 0 if lv else len(lhs) - 2
    rb = 0 if rv else len(rhs) - 2
    rank = builtins.max(lb, rb)
    batch, lstr, rstr = [1] * rank, [0] * rank, [0] * rank
    for axis in range(rank):
        has_l, has_r = axis >= rank - lb, axis >= rank - rb
        li, ri = axis - (rank - lb), axis - (rank - rb)
        left = lhs[li] if has_l else 1
        right = rhs[ri] if has_r else 1
        if left != right and left != 1 and right != 1:
            raise ValueError("matmul batch dimensions cannot broadcast")
        batch[axis] = right if left == 1 else left
        if has_l and left != 1:
            lstr[axis] = ls[li]
        if has_r and right != 1:
            rstr[axis] = rs[ri]
    out = list(batch)
    if not lv:
        out.append(m)
    if not rv:
        out.append(n)
    return tuple(out), batch, lstr, rstr, m, k, n


def matmul_batch_offset(batch: int, shape, strides) -> int:
    """shape.cpp:78-85."""
    offset = 0
    for axis in range(len(shape) - 1, -1, -1):
        offset += (batch % shape[axis]) * strides[axis]
        batch //= shape[axis]
    return offset


def make_reduction_plan(shape, axes):
    """shape.cpp:140-173: (output_shape, index_metadata, reduction_size)."""
    strides = contiguous_strides(shape)
    rank = len(shape)
    selected = [False] * rank
    for axis in axes:
        if axis < 0:
            axis += rank
        if axis < 0 or axis >= rank:
            raise ValueError("reduction axis is out of range")
        if selected[axis]:
            raise ValueError("reduction axes must not repeat")
        selected[axis] = True
    out_shape, meta, reduced = [], [], []
    for axis in range(rank):
        if selected[axis]:
            reduced.append(shape[axis])
        else:
            out_shape.append(shape[axis])
            meta += [shape[axis], strides[axis]]
    for axis in range(rank):
        if selected[axis]:
            meta += [shape[axis], strides[axis]]
    count = int(np.prod(out_shape, dtype=np.int64))
    if 0 in reduced:
        size = 0
    elif count != 0:
        size = int(np.prod(reduced, dtype=np.int64))
    else:
        size = 1
    return tuple(out_shape), meta, size


def make_broadcast_plan(lhs, rhs):
    """shape.cpp:202-229: (output_shape, lhs_strides, rhs_strides)."""
    lc, rc = contiguous_strides(lhs), contiguous_strides(rhs)
    rank = builtins.max(len(lhs), len(rhs))
    lp, rp = rank - len(lhs), rank - len(rhs)
    out, ls, rs = [0] * rank, [0] * rank, [0] * rank
    for axis in range(rank):
        left = 1 if axis < lp else lhs[axis - lp]
        right = 1 if axis < rp else rhs[axis - rp]
        if left != right and left != 1 and right != 1:
            raise ValueError("shape mismatch: tensor shapes are not broadcastable")
        out[axis] = right if left == 1 else left
        if axis >= lp and left != 1:
            ls[axis] = lc[axis - lp]
        if axis >= rp and right != 1:
            rs[axis] = rc[axis - rp]
    return tuple(out), ls, rs


def checked_epsilon(eps: float) -> np.float32:
    """cpu_backend.cpp:30-42."""
    if not np.isfinite(eps) or eps < 0 or eps > float(np.finfo(np.float32).max):
        raise ValueError("epsilon must be finite and non-negative and representable as float32")
    rounded = np.float32(eps)
    if eps > 0 and rounded == 0:
        raise ValueError("epsilon must be finite and non-negative and representable as float32")
    return rounded


# ------------------------------------------------------------------ operations
def _f32(x) -> np.ndarray:
    x = _c(x)
    if x.dtype != np.float32:
        raise ValueError("expected float32 input")
    return x


def matmul(a, b, threads: int | None = None) -> np.ndarray:
    """cpu_backend.cpp:1251-1276."""
    a, b = _f32(a), _f32(b)
    out_shape, batch, lstr, rstr, m, k, n = make_matmul_plan(a.shape, b.shape)
    out = np.empty(out_shape, dtype=np.float32)
    batches = int(np.prod(batch, dtype=np.int64)) if batch else 1
    if out.size == 0:
        return out
    lo = _dims([matmul_batch_offset(i, batch, lstr) for i in range(batches)])
    ro = _dims([matmul_batch_offset(i, batch, rstr) for i in range(batches)])
    lib().oracle_matmul_f32(_p(a), _p(b), _p(out), ctypes.c_int64(batches), ctypes.c_int64(m),
                            ctypes.c_int64(n), ctypes.c_int64(k), _p(lo), _p(ro),
                            ctypes.c_int(threads or default_threads()))
    return out


def _reduce_single(op: int, x: np.ndarray, axis: int, threads) -> np.ndarray:
    x = _c(x)
    out_shape, outer, reduce, inner = reduction_dims(x.shape, axis)
    if op == 1 and reduce == 0:
        raise ValueError("max reduction requires a non-empty axis")
    if op == 2 and x.dtype != np.float32:
        raise ValueError("mean only supports float32 tensors")
    out = np.empty(out_shape, dtype=x.dtype)
    if out.size == 0:
        return out
    t = ctypes.c_int(threads or default_threads())
    if x.dtype == np.float32:
        lib().oracle_reduce_f32(op, _p(x), _p(out), ctypes.c_int64(outer), ctypes.c_int64(reduce),
                                ctypes.c_int64(inner), t)
    elif x.dtype == np.int32:
        lib().oracle_reduce_i32(op, _p(x), _p(out), ctypes.c_int64(outer), ctypes.c_int64(reduce),
                                ctypes.c_int64(inner), t)
    else:
        raise ValueError("numeric reductions do not support bool tensors")
    return out


def _reduce_axes(op: int, x: np.ndarray, axes, threads) -> np.ndarray:
    x = _c(x)
    if op == 2 and x.dtype != np.float32:
        raise ValueError("mean only supports float32 tensors")
    out_shape, meta, size = make_reduction_plan(x.shape, tuple(axes))
    if op == 1 and size == 0:
        raise ValueError("max reduction requires non-empty axes")
    if len(axes) == 0:
        return x.copy()
    out = np.empty(out_shape, dtype=x.dtype)
    if out.size == 0:
        return out
    m = _dims(meta)
    lib().oracle_reduce_axes(op, DTYPE[str(x.dtype)], _p(x), _p(out), _p(m), len(out_shape),
                             x.ndim, ctypes.c_int64(out.size), ctypes.c_int64(size),
                             ctypes.c_int(threads or default_threads()))
    return out


def _reduce(op: int, x, axis, threads):
    """tensor.py:508-529 routing: None -> all axes; one axis -> single-axis path."""
    x = np.asarray(x)
    if axis is None:
        axes = tuple(range(x.ndim))
        if x.ndim == 0:
            return _reduce_single(op, x, 0, threads)
        return _reduce_axes(op, x, axes, threads)
    if isinstance(axis, (tuple, list)):
        if len(axis) == 1:
            return _reduce_single(op, x, axis[0], threads)
        return _reduce_axes(op, x, tuple(axis), threads)
    return _reduce_single(op, x, int(axis), threads)


def sum(x, axis=None, threads=None):  # noqa: A001
    return _reduce(0, x, axis, threads)


def max(x, axis=None, threads=None):  # noqa: A001
    return _reduce(1, x, axis, threads)


def mean(x, axis=None, threads=None):
    return _reduce(2, x, axis, threads)


def _argext(code: int, x, axis, threads) -> np.ndarray:
    """math.cpp:39-56 plan + cpu_math.cpp:48-54."""
    x = _c(x)
    if x.dtype not in (np.float32, np.int32):
        raise ValueError("math operations require float32 or int32 tensors")
    if axis is None:
        axes = tuple(range(x.ndim))
    elif isinstance(axis, (tuple, list)):
        axes = tuple(axis)
    else:
        axes = () if x.ndim == 0 and axis in (0, -1) else (int(axis),)
    out_shape, meta, size = make_reduction_plan(x.shape, axes)
    if size == 0:
        raise ValueError("min/argmax require a non-empty reduction")
    out = np.empty(out_shape, dtype=np.int32 if code == 4 else x.dtype)
    if out.size == 0:
        return out
    lib().oracle_argext(code, DTYPE[str(x.dtype)], _p(x), _p(out), _p(_dims(meta)), x.ndim,
                        ctypes.c_int64(out.size), ctypes.c_int64(size),
                        ctypes.c_int(threads or default_threads()))
    return out


def min(x, axis=None, threads=None):  # noqa: A001
    return _argext(3, x, axis, threads)


def argmax(x, axis=None, threads=None):
    return _argext(4, x, axis, threads)


def _rowwise(fn: str, x, axis: int, eps, threads) -> np.ndarray:
    x = _f32(x)
    _, outer, reduce, inner = reduction_dims(x.shape, axis)
    args = []
    if eps is not None:
        args = [ctypes.c_float(checked_epsilon(eps))]
    out = np.empty_like(x)
    if x.size == 0:
        return out
    getattr(lib(), fn)(_p(x), _p(out), ctypes.c_int64(outer), ctypes.c_int64(reduce),
                       ctypes.c_int64(inner), *args, ctypes.c_int(threads or default_threads()))
    return out


def softmax(x, axis=-1, threads=None):
    """cpu_backend.cpp:125-155."""
    return _rowwise("oracle_softmax", x, axis, None, threads)


def rmsnorm(x, axis=-1, eps=1e-5, threads=None):
    """cpu_backend.cpp:157-183."""
    return _rowwise("oracle_rmsnorm", x, axis, eps, threads)


def layernorm(x, axis=-1, eps=1e-5, threads=None):
    """cpu_backend.cpp:185-240."""
    return _rowwise("oracle_layernorm", x, axis, eps, threads)


def _unary(op: int, x, threads) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    if x.size:
        lib().oracle_unary(op, _p(x), _p(out), ctypes.c_int64(x.size),
                           ctypes.c_int(threads or default_threads()))
    return out


def exp(x, threads=None):
    return _unary(0, x, threads)


def gelu(x, threads=None):
    return _unary(1, x, threads)


def silu(x, threads=None):
    return _unary(2, x, threads)


_BINARY = {"add": 0, "subtract": 1, "multiply": 2, "divide": 3}


def binary(name: str, lhs, rhs, threads=None) -> np.ndarray:
    """cpu_backend.cpp:1014-1097."""
    lhs, rhs = _c(lhs), _c(rhs)
    if lhs.dtype != rhs.dtype:
        raise ValueError("dtype mismatch for binary operation")
    if name == "divide" and lhs.dtype != np.float32:
        raise ValueError("division only supports float32 tensors")
    shape, ls, rs = make_broadcast_plan(lhs.shape, rhs.shape)
    out = np.empty(shape, dtype=lhs.dtype)
    if out.size == 0:
        return out
    lib().oracle_binary(_BINARY[name], DTYPE[str(lhs.dtype)], _p(lhs), _p(rhs), _p(out),
                        _p(_dims(shape)), _p(_dims(ls)), _p(_dims(rs)), len(shape),
                        ctypes.c_int64(out.size), ctypes.c_int(threads or default_threads()))
    return out


def linear(x, weight, bias=None, threads=None) -> np.ndarray:
    """inference.cpp:89-102: transpose(W) copy, matmul, then broadcast add."""
    weight = _f32(weight)
    out = matmul(x, _c(weight.T), threads)
    if bias is not None:
        out = binary("add", out, bias, threads)
    return out


def affine_norm(x, axis, eps, weight=None, bias=None, rms=False, threads=None) -> np.ndarray:
    """inference.cpp:103-122: norm, then multiply by weight, then add bias."""
    x = _f32(x)
    out = (rmsnorm if rms else layernorm)(x, axis, eps, threads)
    view = [1] * x.ndim
    if x.ndim:
        view[normalize_axis(axis, x.ndim)] = x.shape[normalize_axis(axis, x.ndim)]
    if weight is not None:
        out = binary("multiply", out, np.asarray(weight).reshape(view), threads)
    if bias is not None:
        out = binary("add", out, np.asarray(bias).reshape(view), threads)
    return out


def mlp_forward(x, w1, b1, w2, b2, threads=None) -> np.ndarray:
    """The MLP chain linear -> silu -> linear -> softmax(axis=-1)."""
    h = silu(linear(x, w1, b1, threads), threads)
    return softmax(linear(h, w2, b2, threads), -1, threads)


# ------------------------------------------------------- ops next to the path
def _math_input(x) -> np.ndarray:
    x = _c(x)
    if x.dtype not in (np.float32, np.int32):
        raise ValueError("math operations require float32 or int32 tensors")
    return x


def _math_unary(code: int, x, threads) -> np.ndarray:
    """cpu_math.cpp:40-44 under math.cpp:29-31 (log/sqrt float32 only)."""
    x = _math_input(x)
    if code < 2 and x.dtype != np.float32:
        raise ValueError("log/sqrt only support float32 tensors")
    out = np.empty_like(x)
    if x.size:
        lib().oracle_math_unary(code, DTYPE[str(x.dtype)], _p(x), _p(out), ctypes.c_int64(x.size),
                                ctypes.c_int(threads or default_threads()))
    return out


def log(x, threads=None):
    return _math_unary(0, x, threads)


def sqrt(x, threads=None):
    return _math_unary(1, x, threads)


def abs(x, threads=None):  # noqa: A001
    return _math_unary(2, x, threads)


def clip(x, lower, upper, threads=None) -> np.ndarray:
    """cpu_math.cpp:45-50 over the three-way broadcast plan of math.cpp:32-38."""
    arrays = [_math_input(a) for a in (x, lower, upper)]
    if builtins.any(a.dtype != arrays[0].dtype for a in arrays):
        raise ValueError("math input dtypes must match")
    shape = tuple(arrays[0].shape)
    for a in arrays:
        shape = tuple(make_broadcast_plan(shape, a.shape)[0])
    strides = [d for a in arrays for d in make_broadcast_plan(a.shape, shape)[1]]
    out = np.empty(shape, dtype=arrays[0].dtype)
    if out.size:
        lib().oracle_clip(DTYPE[str(out.dtype)], _p(arrays[0]), _p(arrays[1]), _p(arrays[2]), _p(out),
                          _p(_dims(shape)), _p(_dims(strides)), len(shape), ctypes.c_int64(out.size),
                          ctypes.c_int(threads or default_threads()))
    return out


def topk(x, k: int, axis: int = -1, largest: bool = True, sorted: bool = True,  # noqa: A002
         threads=None):
    """cpu_math.cpp:57-67 under the plan of math.cpp:56-66: (values, int32 indices)."""
    x = _math_input(x)
    if x.ndim == 0:
        raise ValueError("topk requires rank >= 1")
    a = axis + x.ndim if axis < 0 else axis
    if a < 0 or a >= x.ndim:
        raise ValueError("topk axis out of range")
    reduce = x.shape[a]
    if k < 0 or k > reduce:
        raise ValueError("topk k must be between zero and the axis size")
    shape = list(x.shape)
    shape[a] = k
    values = np.empty(shape, dtype=x.dtype)
    indices = np.empty(shape, dtype=np.int32)
    if values.size:
        outer = int(np.prod(x.shape[:a], dtype=np.int64))
        inner = int(np.prod(x.shape[a + 1:], dtype=np.int64))
        lib().oracle_topk(DTYPE[str(x.dtype)], int(largest), int(sorted), _p(x), _p(values), _p(indices),
                          ctypes.c_int64(outer), ctypes.c_int64(reduce), ctypes.c_int64(inner),
                          ctypes.c_int64(k), ctypes.c_int(threads or default_threads()))
    return values, indices


def embedding(indices, weight) -> np.ndarray:
    """cpu_inference.cpp:12-21 under make_embedding_plan (inference.cpp:47-57)."""
    indices, weight = _c(indices), _c(weight)
    if indices.dtype != np.int32:
        raise ValueError("embedding indices must be int32")
    if weight.dtype != np.float32:
        raise ValueError("inference values require float32 tensors")
    if weight.ndim != 2:
        raise ValueError("embedding weight must have rank 2")
    if indices.size and (indices.min() < 0 or indices.max() >= weight.shape[0]):
        raise ValueError("embedding index out of range")
    out = np.empty(indices.shape + (weight.shape[1],), dtype=np.float32)
    if out.size:
        rows = out.reshape(-1, weight.shape[1])
        for i, index in enumerate(indices.reshape(-1)):  # row copies, bits preserved
            rows[i] = weight[index]
    return out


def checked_scale(scale: float) -> np.float32:
    """inference.cpp:15-20."""
    with np.errstate(over="ignore"):
        narrowed = np.float32(scale)
    if not np.isfinite(scale) or not np.isfinite(narrowed) or (scale != 0 and narrowed == 0):
        raise ValueError("attention scale must be finite and representable as float32")
    return narrowed


def make_attention_softmax_plan(scores_shape, mask, shape, scale):
    """inference.cpp:59-84: (metadata strides, rows, columns, float scale, mask kind)."""
    if len(scores_shape) < 2 or len(shape) < 2:
        raise ValueError("attention scores must have rank >= 2")
    shape = tuple(shape)
    if tuple(make_broadcast_plan(scores_shape, shape)[0]) != shape:
        raise ValueError("attention scores cannot broadcast to target")
    kind = 0
    if mask is not None:
        if mask.dtype not in (np.bool_, np.float32):
            raise ValueError("attention mask must be bool or float32")
        if tuple(make_broadcast_plan(mask.shape, shape)[0]) != shape:
            raise ValueError("attention mask cannot broadcast to scores")
        kind = 1 if mask.dtype == np.bool_ else 2
    count = int(np.prod(shape, dtype=np.int64))
    strides = list(make_broadcast_plan(scores_shape, shape)[1])
    strides += list(make_broadcast_plan(mask.shape, shape)[1]) if mask is not None else [0] * len(shape)
    columns = shape[-1]
    return strides, (count // columns if columns else 0), columns, checked_scale(scale), kind


def attention_softmax(scores, mask, shape, scale: float, causal: bool, threads=None) -> np.ndarray:
    """cpu_inference.cpp:22-47."""
    scores = _f32(scores)
    mask = None if mask is None else _c(mask)
    strides, rows, columns, fscale, kind = make_attention_softmax_plan(scores.shape, mask, shape, scale)
    out = np.empty(tuple(shape), dtype=np.float32)
    if rows:
        m = mask if mask is not None else np.zeros(1, np.float32)
        lib().oracle_attention_softmax(_p(scores), _p(m), kind, _p(out), _p(_dims(shape)),
                                       _p(_dims(strides)), len(shape), ctypes.c_int64(rows),
                                       ctypes.c_int64(columns), ctypes.c_float(fscale), int(causal),
                                       ctypes.c_int(threads or default_threads()))
    return out


def attention(q, k, v, mask=None, causal: bool = False, scale: float | None = None, threads=None):
    """inference.cpp:123-161: Q @ transpose(K), attention softmax, then @ V."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    for t in (q, k, v):
        if t.ndim < 2:
            raise ValueError("attention tensors require rank >= 2")
    features, rows, columns = q.shape[-1], q.shape[-2], k.shape[-2]
    if features <= 0 or features != k.shape[-1] or columns != v.shape[-2]:
        raise ValueError("attention query/key features and key/value sequence sizes must match")
    batch: tuple = ()
    for t in (q, k, v):
        rank = builtins.max(len(batch), t.ndim - 2)
        left = (1,) * (rank - len(batch)) + tuple(batch)
        right = (1,) * (rank - (t.ndim - 2)) + tuple(t.shape[:-2])
        merged = []
        for a, b in zip(left, right):
            if a != b and a != 1 and b != 1:
                raise ValueError("attention batch dimensions cannot broadcast")
            merged.append(b if a == 1 else a)
        batch = tuple(merged)
    scores_shape = batch + (rows, columns)
    s = checked_scale(1.0 / np.sqrt(float(features)) if scale is None else scale)
    mask = None if mask is None else _c(mask)
    make_attention_softmax_plan(scores_shape, mask, scores_shape, float(s))
    product = matmul(q, _c(np.swapaxes(k, -1, -2)), threads)
    probabilities = attention_softmax(product, mask, scores_shape, float(s), causal, threads)
    return matmul(probabilities, v, threads)


# ------------------------------------------------- layout, casts and predicates
OPKIND.update({"negative": 15, "add_scalar": 16, "subtract_scalar": 17, "multiply_scalar": 18,
               "divide_scalar": 19, "astype": 20, "slice": 22, "concat": 23, "equal": 24, "not_equal": 25,
               "less": 26, "less_equal": 27, "greater": 28, "greater_equal": 29, "logical_and": 30,
               "logical_or": 31, "logical_xor": 32, "logical_not": 33, "where": 34, "any": 35, "all": 36,
               "masked_select": 37})
_NP_OF = {"float32": np.float32, "int32": np.int32, "bool": np.bool_}


def scalar_op(name: str, x, scalar: float = 0.0, scalar_left: bool = False) -> np.ndarray:
    """cpu_backend.cpp:878-930: negate and scalar arithmetic; float32 rounds the
    scalar once, int32 wraps in uint32 (no division, integer scalars only)."""
    x = _c(x)
    if x.dtype == np.bool_:
        raise ValueError("numeric operations do not support bool")
    if x.dtype == np.int32 and name != "negative":
        if name == "divide_scalar":
            raise ValueError("division only supports float32 tensors")
        if not (float(scalar).is_integer() and -2**31 <= scalar <= 2**31 - 1):
            raise ValueError("arithmetic scalar must be an integer in int32 range")
    if x.dtype == np.float32:
        with np.errstate(all="ignore"):
            s = np.float32(scalar)
            lhs, rhs = (s, x) if scalar_left else (x, s)
            out = {"negative": lambda: -x, "add_scalar": lambda: lhs + rhs,
                   "subtract_scalar": lambda: lhs - rhs, "multiply_scalar": lambda: lhs * rhs,
                   "divide_scalar": lambda: lhs / rhs}[name]()
        return np.asarray(out, dtype=np.float32)
    v = x.astype(np.uint32)
    s = np.uint32(int(scalar) & 0xFFFFFFFF) if name != "negative" else np.uint32(0)
    lhs, rhs = (s, v) if scalar_left else (v, s)
    with np.errstate(all="ignore"):
        out = {"negative": lambda: np.uint32(0) - v, "add_scalar": lambda: lhs + rhs,
               "subtract_scalar": lambda: lhs - rhs, "multiply_scalar": lambda: lhs * rhs}[name]()
    return np.asarray(out, dtype=np.uint32).view(np.int32)


def astype(x, dtype: str) -> np.ndarray:
    """cpu_backend.cpp:834-876: bool conversions test != 0; float32 -> int32
    truncates after every value was checked finite and in [-2^31, 2^31)."""
    x = _c(x)
    if dtype not in _NP_OF:
        raise ValueError("unsupported cast target dtype")
    if dtype == "bool" or x.dtype == np.bool_:
        return (x != 0).astype(_NP_OF[dtype])
    if x.dtype == _NP_OF[dtype]:
        return x.copy()
    if dtype == "int32":
        if x.size and (not np.isfinite(x).all() or x.min() < -2147483648.0 or x.max() >= 2147483648.0):
            raise ValueError("float32 value is out of range for int32 cast")
        return x.astype(np.int32)
    return x.astype(np.float32)


def make_transpose_plan(shape, axes):
    """shape.cpp:175-200: a full permutation, negative axes allowed."""
    rank = len(shape)
    if len(axes) != rank:
        raise ValueError("transpose axes must be a full permutation")
    seen = set()
    out = []
    for a in axes:
        a = a + rank if a < 0 else a
        if a < 0 or a >= rank:
            raise ValueError("transpose axis is out of range")
        if a in seen:
            raise ValueError("transpose axes must not repeat")
        seen.add(a)
        out.append(a)
    return tuple(out)


def transpose(x, axes) -> np.ndarray:
    x = _c(x)
    return np.ascontiguousarray(np.transpose(x, make_transpose_plan(x.shape, tuple(axes)))).reshape(
        tuple(x.shape[a] for a in make_transpose_plan(x.shape, tuple(axes))))


def slice_(x, starts, steps, lengths) -> np.ndarray:
    """make_slice_plan (shape.cpp:87-114): every visited index in bounds."""
    x = _c(x)
    if not (len(starts) == len(steps) == len(lengths) == x.ndim):
        raise ValueError("slice metadata must match input rank")
    index = []
    for extent, start, step, length in zip(x.shape, starts, steps, lengths):
        if step == 0:
            raise ValueError("slice step cannot be zero")
        if length < 0:
            raise ValueError("shape dimensions must be non-negative")
        if length == 0:
            index.append(np.zeros(0, np.int64))
            continue
        if start < 0 or start >= extent:
            raise ValueError("slice start is out of bounds")
        last = start + step * (length - 1)
        if last < 0 or last >= extent:
            raise ValueError("slice endpoint is out of bounds")
        index.append(start + step * np.arange(length, dtype=np.int64))
    if not index:
        return x.copy()
    return np.ascontiguousarray(x[np.ix_(*index)])


def concat(arrays, axis: int) -> np.ndarray:
    """make_concat_plan (shape.cpp:116-138)."""
    arrays = [_c(a) for a in arrays]
    if not arrays:
        raise ValueError("concat requires at least one tensor")
    if builtins.any(a.dtype != arrays[0].dtype for a in arrays):
        raise ValueError("concat dtypes must match")
    rank = arrays[0].ndim
    a = axis + rank if axis < 0 else axis
    if a < 0 or a >= rank:
        raise ValueError("concat axis is out of range")
    for arr in arrays:
        if arr.ndim != rank:
            raise ValueError("concat ranks must match")
        if builtins.any(arr.shape[i] != arrays[0].shape[i] for i in range(rank) if i != a):
            raise ValueError("concat non-axis dimensions must match")
    return np.ascontiguousarray(np.concatenate(arrays, axis=a))


_COMPARE = {"equal": np.equal, "not_equal": np.not_equal, "less": np.less, "less_equal": np.less_equal,
            "greater": np.greater, "greater_equal": np.greater_equal}
_LOGICAL = {"logical_and": np.logical_and, "logical_or": np.logical_or, "logical_xor": np.logical_xor}


def predicate(name: str, *inputs) -> np.ndarray:
    """make_predicate_plan (predicate.cpp:23-44), cpu_predicate.cpp:22-50."""
    inputs = [_c(a) for a in inputs]
    arity = 3 if name == "where" else 1 if name == "logical_not" else 2
    if len(inputs) != arity:
        raise ValueError("invalid predicate operation or input count")
    if name == "where":
        if inputs[0].dtype != np.bool_:
            raise ValueError("where condition must be bool")
        if inputs[1].dtype != inputs[2].dtype:
            raise ValueError("where branch dtypes must match")
    else:
        for a in inputs:
            if a.dtype != inputs[0].dtype:
                raise ValueError("comparison dtypes must match")
            if name.startswith("logical") and a.dtype != np.bool_:
                raise ValueError("logical operations require bool tensors")
    shape: tuple = ()
    for a in inputs:
        shape = tuple(make_broadcast_plan(shape, a.shape)[0])
    b = [np.broadcast_to(a, shape) for a in inputs]
    if name == "where":
        return np.ascontiguousarray(np.where(b[0], b[1], b[2]))
    if name == "logical_not":
        return np.ascontiguousarray(np.logical_not(b[0]))
    if name in _LOGICAL:
        return np.ascontiguousarray(_LOGICAL[name](b[0], b[1]))
    with np.errstate(invalid="ignore"):
        return np.ascontiguousarray(_COMPARE[name](b[0], b[1]))


def bool_reduce(name: str, x, axes) -> np.ndarray:
    """make_boolean_reduction_plan (predicate.cpp:46-55), cpu_predicate.cpp:52-70."""
    x = _c(x)
    if x.dtype != np.bool_:
        raise ValueError("any/all require bool tensors")
    out_shape, _, _ = make_reduction_plan(x.shape, tuple(axes))
    rank = x.ndim
    norm = tuple(a + rank if a < 0 else a for a in axes)
    fn = np.all if name == "all" else np.any
    return np.ascontiguousarray(fn(x, axis=norm)).reshape(out_shape)


def masked_select(x, mask) -> np.ndarray:
    """make_masked_select_plan (predicate.cpp:57-72), cpu_predicate.cpp:72-96."""
    x, mask = _c(x), _c(mask)
    if mask.dtype != np.bool_:
        raise ValueError("mask must be bool")
    if mask.ndim > x.ndim:
        raise ValueError("mask rank exceeds input rank")
    if tuple(x.shape[:mask.ndim]) != tuple(mask.shape):
        raise ValueError("mask must match leading input dimensions")
    tail = x.shape[mask.ndim:]
    flat = x.reshape((int(np.prod(mask.shape, dtype=np.int64)),) + tail)
    return np.ascontiguousarray(flat[mask.reshape(-1)])
