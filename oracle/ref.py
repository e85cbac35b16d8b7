"""CPU ORACLE (reference build): test infrastructure only.

ctypes access to oracle/_ref/libtcxref.so, the reference CPU backend compiled
from /root/reference sources by oracle/Makefile (target ``ref``). Used to write
golden vectors (tests/golden/make_golden.py), to check the restatement in this
package when the library is present, and as bench.py's CPU baseline. The
library is built in the container that holds /root/reference; a GPU box only
loads the prebuilt file when it travelled with the tree.
"""

from __future__ import annotations

import ctypes
import pathlib

import numpy as np

from . import DTYPE, OPKIND

PATH = pathlib.Path(__file__).resolve().parent / "_ref" / "libtcxref.so"
_LIB = None
_NP = {0: np.float32, 1: np.int32, 2: np.bool_}


class ReferenceError(Exception):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def available() -> bool:
    return PATH.exists()


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = ctypes.CDLL(str(PATH))
        _LIB.tcxref_message.restype = ctypes.c_char_p
    return _LIB


def execute(kind: str, inputs, *, axis: int = 0, eps: float = 1e-5, axes=None,
            has_weight: bool = False, has_bias: bool = False, n_outputs: int = 1,
            causal: bool = False, scale: float | None = None, attention_shape=(),
            k: int = 0, largest: bool = True, sorted: bool = True,  # noqa: A002
            scalar: float = 0.0, scalar_left: bool = False, target_dtype: str | None = None,
            perm=None, starts=None, steps=None, lengths=None):
    """Runs one primitive through the reference CpuBackend::execute."""
    arrays = [np.asarray(a, order="C") for a in inputs]  # keeps rank 0
    att = (ctypes.c_int64 * max(1, len(attention_shape)))(*attention_shape)
    lib().tcxref_set_attributes(int(causal), int(scale is not None), ctypes.c_double(scale or 0.0),
                                len(attention_shape), att, ctypes.c_int64(k), int(largest), int(sorted),
                                ctypes.c_double(scalar))
    if perm is not None or starts is not None or target_dtype is not None or scalar_left:
        def arr(v):
            return (ctypes.c_int64 * max(1, len(v or ())))(*(v or ()))
        lib().tcxref_set_layout(len(perm or ()), arr(perm), len(starts or ()), arr(starts), arr(steps),
                                arr(lengths), DTYPE[target_dtype or "float32"], int(scalar_left))
    dtypes = (ctypes.c_int * max(1, len(arrays)))(*[DTYPE[str(a.dtype)] for a in arrays])
    ranks = (ctypes.c_int * max(1, len(arrays)))(*[a.ndim for a in arrays])
    dims = [d for a in arrays for d in a.shape]
    shapes = (ctypes.c_int64 * max(1, len(dims)))(*dims)
    datas = (ctypes.c_void_p * max(1, len(arrays)))(*[a.ctypes.data for a in arrays])
    axes_arr = (ctypes.c_int64 * max(1, len(axes or ())))(*(axes or ()))
    code = lib().tcxref_execute(
        OPKIND[kind], ctypes.c_int64(axis), ctypes.c_double(eps), int(axes is not None),
        axes_arr, len(axes or ()), int(has_weight), int(has_bias), len(arrays), dtypes, ranks,
        shapes, datas, n_outputs)
    if code != 0:
        raise ReferenceError(code, lib().tcxref_message().decode())
    results = []
    for index in range(n_outputs):
        dtype, rank = ctypes.c_int(), ctypes.c_int()
        shape = (ctypes.c_int64 * 512)()
        if lib().tcxref_result_info(index, ctypes.byref(dtype), ctypes.byref(rank), shape) != 0:
            raise ReferenceError(3, "missing reference output")
        out = np.empty(tuple(shape[i] for i in range(rank.value)), dtype=_NP[dtype.value])
        if lib().tcxref_result_copy(index, ctypes.c_void_p(out.ctypes.data), out.nbytes) != 0:
            raise ReferenceError(3, "reference output copy failed")
        results.append(out)
    return results[0] if n_outputs == 1 else tuple(results)


def matmul_rows(a: np.ndarray, b: np.ndarray, rows: int) -> np.ndarray:
    """Reference matmul of the first `rows` rows of a (timing a bounded slab)."""
    a = np.ascontiguousarray(a[:rows], dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty((rows, b.shape[1]), dtype=np.float32)
    code = lib().tcxref_matmul_rows(
        ctypes.c_void_p(a.ctypes.data), ctypes.c_void_p(b.ctypes.data),
        ctypes.c_void_p(out.ctypes.data), ctypes.c_int64(rows), ctypes.c_int64(b.shape[1]),
        ctypes.c_int64(a.shape[1]))
    if code != 0:
        raise ReferenceError(code, lib().tcxref_message().decode())
    return out
