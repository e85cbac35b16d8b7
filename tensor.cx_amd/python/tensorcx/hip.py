"""Fused hip kernels reached through BackendOpClass::kKernel.

These run the built-in static-library kernels of HipBackend (entry points
"linear_bias_act" and "bias_act"): act(x @ weight^T + bias) in one GEMM
epilogue, and act(x + bias) in one pass. activation is "none", "silu" or
"gelu"; results equal linear() followed by silu()/gelu() up to the exp/tanh
implementation.
"""

from __future__ import annotations

_ACT = {"none": 0, "silu": 1, "gelu": 2}


def _act(name: str) -> int:
    if name not in _ACT:
        raise ValueError(f"unknown activation {name!r}")
    return _ACT[name]


def linear_act(input, weight, bias, activation: str = "silu"):
    from . import Tensor, _core, _hip
    x, w, b = _hip(input, weight, bias, name="linear_act")
    return Tensor(_core.linear_act(x, w, b, _act(activation)))


def bias_act(input, bias, activation: str = "silu"):
    from . import Tensor, _core, _hip
    x, b = _hip(input, bias, name="bias_act")
    return Tensor(_core.bias_act(x, b, _act(activation)))
