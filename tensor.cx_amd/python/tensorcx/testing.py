"""Dtype-aware comparisons with the reference's tolerance classes.

Same table as reference python/tensorcx/testing.py:17-21: elementwise
(1e-6, 1e-6), reduction (1e-5, 1e-5), matmul (1e-4, 1e-4); integer results are
compared exactly.
"""

from __future__ import annotations

import numpy as np

_FLOAT_TOLERANCES = {"elementwise": (1e-6, 1e-6), "reduction": (1e-5, 1e-5), "matmul": (1e-4, 1e-4)}


def _as_array(value):
    return np.asarray(value.numpy()) if hasattr(value, "numpy") else np.asarray(value)


def assert_allclose(actual, expected, *, kind="elementwise", rtol=None, atol=None, equal_nan=True):
    if kind not in _FLOAT_TOLERANCES:
        raise ValueError(f"unknown tolerance kind {kind!r}; expected one of {sorted(_FLOAT_TOLERANCES)}")
    a, e = _as_array(actual), _as_array(expected)
    if a.shape != e.shape:
        raise AssertionError(f"shape mismatch: {a.shape} != {e.shape}")
    if a.dtype.kind in "iub" or e.dtype.kind in "iub":
        np.testing.assert_array_equal(a, e)
        return
    r, t = _FLOAT_TOLERANCES[kind]
    np.testing.assert_allclose(a, e, rtol=r if rtol is None else rtol, atol=t if atol is None else atol,
                               equal_nan=equal_nan)
