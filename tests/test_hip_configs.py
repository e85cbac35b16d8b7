"""GPU parity at the full BASELINE.json configs (C1-C5), against the oracle on
identical seeded inputs, plus size-independent properties at those sizes."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
import tensorcx_workloads as wl
from conftest import require_gpu
from hip_cases import assert_bits, assert_close, assert_matmul, sum_error

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cx():
    require_gpu()
    import tensorcx
    return tensorcx


@pytest.mark.parametrize("name", ["c1_512", "c2_edge", "c2_batched", "c2_4096"])
def test_gemm_configs(cx, name):
    a, b = wl.gemm_inputs(name)
    actual = cx.matmul(cx.tensor(a, device="hip"), cx.tensor(b, device="hip")).numpy()
    err = assert_matmul(actual, oracle.matmul(a, b), a, b, name)
    print(f"{name}: scaled error {err:.3e}")


def test_reduce_f32_config(cx):
    x = wl.reduce_f32_input()
    h = cx.tensor(x, device="hip")
    for op in ("max", "min", "argmax"):
        assert_bits(getattr(cx, op)(h, -1).numpy(), getattr(oracle, op)(x, -1), op)
    s = cx.sum(h, -1).numpy()
    err = sum_error(s, oracle.sum(x, -1), x, 8192, 8192, 1)
    assert err <= 1e-5, f"sum {err:.3e}"
    m = cx.mean(h, -1).numpy()
    err_m = sum_error(m * 8192, oracle.mean(x, -1) * 8192, x, 8192, 8192, 1)
    assert err_m <= 1e-5, f"mean {err_m:.3e}"
    full = cx.sum(h).numpy()
    err_f = sum_error(full.reshape(1), oracle.sum(x, None).reshape(1), x, 1, x.size, 1)
    assert err_f <= 1e-5, f"full sum {err_f:.3e}"
    print(f"sum {err:.2e} mean {err_m:.2e} full {err_f:.2e}")


def test_reduce_i32_config(cx):
    x = wl.reduce_i32_input()
    h = cx.tensor(x, device="hip")
    assert_bits(cx.sum(h, -1).numpy(), oracle.sum(x, -1), "i32 sum")
    assert_bits(cx.max(h, -1).numpy(), oracle.max(x, -1), "i32 max")


def test_rownorm_config(cx):
    x, g, b = wl.rownorm_inputs()
    h = cx.tensor(x, device="hip")
    sm = cx.softmax(h, -1).numpy()
    assert_close(sm, oracle.softmax(x, -1), 1e-5, 1e-5, "softmax")
    np.testing.assert_allclose(sm.sum(axis=1, dtype=np.float64), 1.0, rtol=1e-5)
    assert_close(cx.rmsnorm(h, -1, 1e-5).numpy(), oracle.rmsnorm(x, -1, 1e-5), 1e-5, 1e-5, "rmsnorm")
    gh, bh = cx.tensor(g, device="hip"), cx.tensor(b, device="hip")
    assert_close(cx.layernorm(h, -1, 1e-5, weight=gh, bias=bh).numpy(),
                 oracle.affine_norm(x, -1, 1e-5, g, b), 1e-5, 1e-5, "layernorm")


def test_mlp_config(cx):
    x, w1, b1, w2, b2 = wl.mlp_inputs()
    xh, w1h, b1h, w2h, b2h = (cx.tensor(v, device="hip") for v in (x, w1, b1, w2, b2))
    hidden = cx.hip.linear_act(xh, w1h, b1h, "silu")
    out = cx.softmax(cx.linear(hidden, w2h, b2h), -1).numpy()
    assert_close(out, oracle.mlp_forward(x, w1, b1, w2, b2), 1e-5, 1e-5, "mlp")
    # The unfused chain through the reference op sequence agrees too.
    chain = cx.softmax(cx.linear(cx.silu(cx.linear(xh, w1h, b1h)), w2h, b2h), -1).numpy()
    assert_close(chain, out, 1e-5, 1e-5, "mlp fused vs unfused")
