"""DLPack on the hip device (kDLROCM, device 0): zero-copy exchange, copies,
storage relations, the ROCm stream contract, borrow validation, the pool
boundary, and exchange with PyTorch-ROCm.

Cases follow the reference's tests/python/test_dlpack.py for its CUDA device
(roundtrip over dtypes/shapes/versions with ops on borrowed storage, copy
contract, independent wrappers, negotiation, stream rules), with the ROCm
stream values. Borrowed storage may start at any element-aligned address, so
kernels that load 16 bytes at a time must take their scalar routes there;
those results are checked against the same ops on an aligned copy.
"""

from __future__ import annotations

import gc
import os
import pathlib
import subprocess
import sys

import numpy as np
import pytest

from conftest import require_gpu
from dlpack_fixtures import ROCM, Fixture, address, describe, versioned
from hip_cases import SUM_BAR, assert_bits, assert_matmul, sum_error

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def cx():
    require_gpu()
    import tensorcx
    return tensorcx


@pytest.mark.parametrize("dtype", ["float32", "int32", "bool"])
@pytest.mark.parametrize("shape", [(), (6,), (2, 3), (2, 0, 3), (1, 2, 1)])
@pytest.mark.parametrize("version", [None, (0, 8), (1, 0), (2, 0)])
def test_roundtrip(cx, dtype, shape, version):
    values = (np.arange(np.prod(shape, dtype=int)).reshape(shape) % 2).astype(dtype)
    source = cx.tensor(values, device="hip")
    capsule = source.__dlpack__(max_version=version)
    d = describe(capsule)
    assert (d.device.device_type, d.device.device_id) == (ROCM, 0)
    imported = cx.from_dlpack(capsule, copy=False)
    assert (imported.device, imported.dtype, imported.shape) == ("hip", dtype, shape)
    np.testing.assert_array_equal(imported.numpy(), values)
    if values.size:
        assert cx._core._shares_storage(source._impl, imported._impl)
    # Borrowed buffers are ordinary kernel inputs.
    np.testing.assert_array_equal(imported.transpose().numpy(), values.transpose())
    if dtype == "float32":
        np.testing.assert_array_equal((imported + imported).numpy(), values + values)
    with pytest.raises(BufferError, match="unconsumed"):
        cx.from_dlpack(capsule)
    del source, capsule
    gc.collect()
    np.testing.assert_array_equal(imported.reshape((-1,)).numpy(), values.reshape(-1))


@pytest.mark.parametrize("copy", [None, False, True])
def test_copy_contract(cx, copy):
    source = cx.tensor([1.0, 2.0, 3.0], device="hip")
    shared = cx.from_dlpack(source, copy=copy)
    a, b = source.__dlpack__(), shared.__dlpack__()
    assert (describe(a).data == describe(b).data) is (copy is not True)
    np.testing.assert_array_equal(shared.numpy(), source.numpy())
    capsule = source.__dlpack__(max_version=(1, 0), copy=True)
    managed = versioned(capsule)
    assert managed.flags & 2 and managed.dl_tensor.data != describe(a).data
    np.testing.assert_array_equal(cx.from_dlpack(capsule).numpy(), source.numpy())


def test_independent_wrappers_storage_relation(cx):
    source = cx.tensor(np.arange(7, dtype=np.float32), device="hip")
    a, b = cx.from_dlpack(source), cx.from_dlpack(source)
    assert cx._core._shares_storage(a._impl, b._impl)
    assert cx._core._shares_storage(source._impl, a._impl)
    left, right = source.__dlpack__(), source.__dlpack__()
    describe(left).shape[0] = 6
    describe(right).shape[0] = 6
    describe(right).byte_offset = 4
    a, b = cx.from_dlpack(left), cx.from_dlpack(right)
    np.testing.assert_array_equal(a.numpy(), np.arange(6, dtype=np.float32))
    np.testing.assert_array_equal(b.numpy(), np.arange(1, 7, dtype=np.float32))
    with pytest.raises(ValueError, match="overlap"):
        cx._core._shares_storage(a._impl, b._impl)
    assert not cx._core._shares_storage(a._impl, cx.from_dlpack(b, copy=True)._impl)


def _offset_view(cx, values):
    """A hip tensor over `values` placed 4 bytes past a 256-byte aligned base."""
    flat = values.reshape(-1)
    padded = cx.tensor(np.concatenate([np.zeros(1, values.dtype), flat]), device="hip")
    capsule = padded.__dlpack__()
    d = describe(capsule)
    assert d.data % 16 == 0
    d.ndim = 1
    d.shape[0] = flat.size
    d.byte_offset = 4
    view = cx.from_dlpack(capsule).reshape(values.shape)
    assert address(view.__dlpack__()) % 16 == 4
    return view


def test_unaligned_borrowed_storage_through_kernels(cx):
    rng = np.random.default_rng(21)
    x = rng.normal(size=(64, 4096)).astype(np.float32)
    view, aligned = _offset_view(cx, x), cx.tensor(x, device="hip")
    # The scalar routes add in another order than the 16-byte ones: sums are
    # held to the sum bar against float64, exact ops stay bit-exact.
    err = sum_error(cx.sum(view, axis=-1).numpy(), x.astype(np.float64).sum(-1), x, 64, 4096, 1)
    assert err <= SUM_BAR, f"sum of an offset view: {err:.3e}"
    for name, op in (("max", lambda t: cx.max(t, axis=-1)), ("exp", cx.exp)):
        assert_bits(op(view).numpy(), op(aligned).numpy(), name)
    for name, op in (("softmax", lambda t: cx.softmax(t, -1)), ("rmsnorm", lambda t: cx.rmsnorm(t, -1)),
                     ("layernorm", lambda t: cx.layernorm(t, -1))):
        np.testing.assert_allclose(op(view).numpy(), op(aligned).numpy(), rtol=1e-5, atol=1e-6, err_msg=name)
    w = rng.normal(size=(4096, 128)).astype(np.float32)
    got = cx.matmul(view, _offset_view(cx, w)).numpy()
    assert_matmul(got, x.astype(np.float64) @ w.astype(np.float64), x, w, "matmul of offset views")
    q = rng.normal(size=(2, 64, 64)).astype(np.float32)
    k = rng.normal(size=(2, 64, 64)).astype(np.float32)
    v = rng.normal(size=(2, 64, 64)).astype(np.float32)
    fused = cx.attention(cx.tensor(q, device="hip"), cx.tensor(k, device="hip"), cx.tensor(v, device="hip"))
    routed = cx.attention(_offset_view(cx, q), _offset_view(cx, k), _offset_view(cx, v))
    np.testing.assert_allclose(routed.numpy(), fused.numpy(), rtol=2e-4, atol=2e-5)
    assert_bits(cx.transpose(view).numpy(), np.ascontiguousarray(x.T), "transpose of an offset view")


def test_protocol_negotiation(cx):
    x = cx.ones((2, 3), device="hip")
    calls = []

    class Producer:
        def __dlpack_device__(self):
            return x.__dlpack_device__()

        def __dlpack__(self, *, stream=None, max_version=None):
            calls.append((stream, max_version))
            return x.__dlpack__(stream=stream, max_version=max_version)

    np.testing.assert_array_equal(cx.from_dlpack(Producer()).numpy(), x.numpy())
    assert calls == [(0, (1, 0))]

    class LegacyProducer:
        def __dlpack_device__(self):
            return x.__dlpack_device__()

        def __dlpack__(self, stream=None):
            return x.__dlpack__(stream=stream)

    np.testing.assert_array_equal(cx.from_dlpack(LegacyProducer()).numpy(), x.numpy())


def test_stream_contract(cx):
    x = cx.ones((1,), device="hip")
    assert x.__dlpack_device__() == (ROCM, 0)
    for stream in (None, -1, 0, 123456):
        assert cx.from_dlpack(x.__dlpack__(stream=stream)).device == "hip"
    with pytest.raises(BufferError, match="synchronization"):
        x.__dlpack__(stream=-1, copy=True)
    for stream in (0, None):
        assert cx.from_dlpack(x.__dlpack__(stream=stream, copy=True)).device == "hip"
    with pytest.raises(BufferError, match="default stream"):
        x.__dlpack__(stream=123456, copy=True)
    for stream in (1, 2, -2):
        with pytest.raises(ValueError):
            x.__dlpack__(stream=stream)
    with pytest.raises(TypeError):
        x.__dlpack__(stream=True)
    with pytest.raises(BufferError):
        x.__dlpack__(dl_device=(1, 0))


def test_borrow_rejects_host_memory(cx):
    fixture = Fixture(device=ROCM)
    with pytest.raises(BufferError, match="device"):
        cx.from_dlpack(fixture.capsule)
    assert fixture.deleted == 1


def test_borrow_rejects_range_past_allocation(cx):
    source = cx.tensor(np.zeros(16, np.float32), device="hip")
    capsule = source.__dlpack__()
    describe(capsule).shape[0] = 1 << 30  # 4 GiB claimed over a 64-byte allocation
    with pytest.raises(BufferError, match="allocation"):
        cx.from_dlpack(capsule)
    np.testing.assert_array_equal(source.numpy(), np.zeros(16, np.float32))


def test_exported_storage_bypasses_pool_cache(cx):
    pool = cx.memory_pool("hip", max_cached_bytes=8 << 20, max_cached_blocks=8)
    with pool:
        kept = cx.tensor(np.ones((64, 64), np.float32), device="hip")
        plain = cx.exp(kept)
        del plain
        before = pool.stats()
        assert before["cached_blocks"] == 1
        shared = cx.exp(kept)
        capsule = shared.__dlpack__()
        borrowed = cx.from_dlpack(capsule)
        del shared, capsule
        gc.collect()
        np.testing.assert_allclose(borrowed.numpy(), np.full((64, 64), np.e, np.float32), rtol=1e-6)
        del borrowed
        gc.collect()
        after = pool.stats()
        assert after["uncached_returns"] == before["uncached_returns"] + 1
        assert after["cached_blocks"] == 0  # the hit took the cached block; the export did not return it


TORCH_EXCHANGE = r"""
import gc, sys
import torch  # first: one HIP runtime per process, as the reference's bridge orders it
if not torch.cuda.is_available():
    print("TORCH-NO-GPU"); sys.exit(0)
import numpy as np
sys.path[:0] = sys.argv[1:3]
import tensorcx as cx
from dlpack_fixtures import address

dev = "cuda"
t = torch.arange(12, dtype=torch.float32, device=dev).reshape(3, 4)
x = cx.from_dlpack(t)
assert x.device == "hip" and x.shape == (3, 4)
assert address(x.__dlpack__()) == t.data_ptr(), "import must share torch's storage"
np.testing.assert_array_equal(x.numpy(), t.cpu().numpy())
t.add_(1); torch.cuda.synchronize()
np.testing.assert_array_equal(x.numpy(), t.cpu().numpy())
print("torch -> hip shared", flush=True)

a = torch.randn(64, 96, device=dev); b = torch.randn(96, 32, device=dev)
got = cx.matmul(cx.from_dlpack(a), cx.from_dlpack(b)).numpy()
ref = a.cpu().double().numpy() @ b.cpu().double().numpy()
assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-4
print("matmul on torch storage", flush=True)

off = torch.arange(33, dtype=torch.float32, device=dev)[1:].reshape(4, 8)
assert off.data_ptr() % 16 == 4
np.testing.assert_allclose(cx.sum(cx.from_dlpack(off), axis=-1).numpy(), off.sum(-1).cpu().numpy(), rtol=1e-6)
for dtype in (torch.int32, torch.bool):
    s = (torch.arange(10, device=dev) % 3 == 0).to(dtype)
    np.testing.assert_array_equal(cx.from_dlpack(s).numpy(), s.cpu().numpy())
try:
    cx.from_dlpack(t.T)
    raise AssertionError("a transposed torch view must be rejected")
except BufferError as error:
    assert "contiguous" in str(error)
print("offset, int32, bool, layout", flush=True)

y = cx.tensor(np.arange(6, dtype=np.float32).reshape(2, 3), device="hip")
ty = torch.from_dlpack(y)
assert ty.device.type == "cuda" and ty.data_ptr() == address(y.__dlpack__())
np.testing.assert_array_equal(ty.cpu().numpy(), y.numpy())
ty.mul_(2); torch.cuda.synchronize()
np.testing.assert_array_equal(y.numpy(), np.arange(6, dtype=np.float32).reshape(2, 3) * 2)
del y; gc.collect()
assert float(ty.sum().item()) == 30.0
del ty; gc.collect(); torch.cuda.synchronize()
print("hip -> torch shared", flush=True)
print("DLPACK-TORCH-OK")
"""


def test_exchange_with_torch(cx):
    """Runs in a child process that imports torch before tensorcx."""
    pytest.importorskip("torch")
    paths = [str(ROOT / "tensor.cx_amd" / "python"), str(ROOT / "tests")]
    env = dict(os.environ)
    print("torch exchange child starting", flush=True)
    result = subprocess.run([sys.executable, "-c", TORCH_EXCHANGE, *paths], capture_output=True, text=True,
                            timeout=240, env=env)
    print(result.stdout[-2000:], result.stderr[-2000:], flush=True)
    if "TORCH-NO-GPU" in result.stdout:
        pytest.skip("torch sees no GPU")
    assert result.returncode == 0 and "DLPACK-TORCH-OK" in result.stdout
