"""DLPack protocol on host tensors: negotiation, ownership, validation.

The contract follows the reference's tests/python/test_dlpack.py (shared
storage for copy=None/False, explicit copies, consume-once capsules, the
producer's deleter exactly once even for rejected descriptors, read-only and
is-copied flags, contiguity, offsets) on host tensors. Host tensors here are
data placement only (compute is on hip), so checks read values back rather
than running ops on them. The hip device's side is tests/test_hip_dlpack.py.
"""

from __future__ import annotations

import gc
import weakref

import numpy as np
import pytest

from dlpack_fixtures import CPU, ROCM, Fixture, describe, versioned

cx = pytest.importorskip("tensorcx")


@pytest.mark.parametrize("dtype", ["float32", "int32", "bool"])
@pytest.mark.parametrize("shape", [(), (6,), (2, 3), (2, 0, 3), (1, 2, 1)])
@pytest.mark.parametrize("version", [None, (0, 8), (1, 0), (2, 0)])
def test_host_roundtrip(dtype, shape, version):
    values = (np.arange(np.prod(shape, dtype=int)).reshape(shape) % 2).astype(dtype)
    source = cx.tensor(values)
    capsule = source.__dlpack__(max_version=version)
    imported = cx.from_dlpack(capsule, copy=False)
    assert (imported.device, imported.dtype, imported.shape) == ("cpu", dtype, shape)
    np.testing.assert_array_equal(imported.numpy(), values)
    with pytest.raises(BufferError, match="unconsumed"):
        cx.from_dlpack(capsule)
    del source, capsule
    gc.collect()
    np.testing.assert_array_equal(imported.reshape((-1,)).numpy(), values.reshape(-1))


@pytest.mark.parametrize("dtype", ["float32", "int32", "bool"])
@pytest.mark.parametrize("shape", [(), (5,), (2, 3), (0, 3), (1, 2, 1)])
def test_numpy_zero_copy_and_lifetime(dtype, shape):
    source = np.ones(shape, dtype=dtype)
    alive = weakref.ref(source)
    tensor = cx.from_dlpack(source, copy=False)
    exported = np.from_dlpack(tensor)
    if source.size:
        assert exported.ctypes.data == source.ctypes.data
        source.flat[0] = 0
        np.testing.assert_array_equal(tensor.numpy(), source)
    view = tensor.reshape((-1,))
    del source, tensor, exported
    gc.collect()
    assert alive() is not None
    final = np.from_dlpack(view)
    del view
    gc.collect()
    assert alive() is not None
    del final
    gc.collect()
    assert alive() is None


@pytest.mark.parametrize("copy", [None, False, True])
def test_copy_contract(copy):
    source = cx.tensor([1.0, 2.0, 3.0])
    shared = cx.from_dlpack(source, copy=copy)
    a, b = source.__dlpack__(), shared.__dlpack__()
    assert (describe(a).data == describe(b).data) is (copy is not True)
    np.testing.assert_array_equal(shared.numpy(), source.numpy())
    capsule = source.__dlpack__(max_version=(1, 0), copy=True)
    managed = versioned(capsule)
    assert managed.flags & 2
    assert managed.dl_tensor.data != describe(a).data
    np.testing.assert_array_equal(cx.from_dlpack(capsule).numpy(), source.numpy())


@pytest.mark.parametrize("copy", [0, 1, "yes", [], np.bool_(True)])
def test_bad_copy_argument(copy):
    source = cx.ones((2,))
    with pytest.raises(TypeError):
        source.__dlpack__(copy=copy)
    with pytest.raises(TypeError):
        cx.from_dlpack(source, copy=copy)


def test_discarded_export_releases_owner():
    source = np.ones(3, np.float32)
    alive = weakref.ref(source)
    tensor = cx.from_dlpack(source)
    capsule = tensor.__dlpack__(max_version=(1, 0))
    del tensor, source
    gc.collect()
    assert alive() is not None
    del capsule
    gc.collect()
    assert alive() is None


@pytest.mark.parametrize("as_versioned", [False, True])
def test_offset_and_single_release(as_versioned):
    fixture = Fixture(versioned=as_versioned, offset=4, shape=(2, 1, 3), strides=(3, 99, 1))
    tensor = cx.from_dlpack(fixture.capsule)
    assert fixture.deleted == 0
    np.testing.assert_array_equal(tensor.numpy(), np.arange(1, 7, dtype=np.float32).reshape(2, 1, 3))
    reexport = tensor.__dlpack__()
    view = tensor.reshape((6,))
    del tensor, view
    gc.collect()
    assert fixture.deleted == 0
    del reexport
    gc.collect()
    assert fixture.deleted == 1


def _break(fixture, case):
    t = fixture.tensor
    if case == "version":
        fixture.managed.version.major = 2
    elif case == "flags":
        fixture.managed.flags = 4
    elif case == "device":
        t.device.device_type = 8
    elif case == "cuda_device":
        t.device.device_type = 2
    elif case == "index":
        t.device.device_id = 1
    elif case == "dtype":
        t.dtype.bits = 64
    elif case == "lanes":
        t.dtype.lanes = 2
    elif case == "negative_shape":
        fixture.shape[0] = -1
    elif case == "negative_rank":
        t.ndim = -1
    elif case == "null_shape":
        t.shape = None
    elif case == "null_data":
        t.data = None
    elif case == "alignment":
        t.byte_offset = 1
    elif case == "offset_overflow":
        t.byte_offset = 2**64 - 1
    elif case == "strides":
        import ctypes
        fixture.strides = (ctypes.c_int64 * 2)(1, 2)
        t.strides = fixture.strides


@pytest.mark.parametrize("case", ["version", "flags", "device", "cuda_device", "index", "dtype", "lanes",
                                  "negative_shape", "negative_rank", "null_shape", "null_data", "alignment",
                                  "offset_overflow", "strides"])
def test_invalid_descriptor_released_once(case):
    fixture = Fixture()
    _break(fixture, case)
    with pytest.raises((BufferError, ValueError)):
        cx.from_dlpack(fixture.capsule)
    assert fixture.deleted == 1
    with pytest.raises(BufferError):
        cx.from_dlpack(fixture.capsule)
    assert fixture.deleted == 1


@pytest.mark.parametrize("copy", [None, False, True])
def test_read_only_policy(copy):
    fixture = Fixture(flags=1)
    if copy is True:
        tensor = cx.from_dlpack(fixture.capsule, copy=True)
        assert fixture.deleted == 1
        np.testing.assert_array_equal(tensor.numpy(), fixture.data[:6].reshape(2, 3))
        fixture.data[0] = -10
        assert tensor.numpy()[0, 0] == 0
    else:
        with pytest.raises(BufferError, match="read-only"):
            cx.from_dlpack(fixture.capsule, copy=copy)
        assert fixture.deleted == 1


def test_copy_false_rejects_producer_copy():
    fixture = Fixture(flags=2)
    with pytest.raises(BufferError, match="copied"):
        cx.from_dlpack(fixture.capsule, copy=False)
    assert fixture.deleted == 1


def test_protocol_negotiation():
    x = cx.ones((2, 3))
    calls = []

    class Producer:
        def __dlpack_device__(self):
            return x.__dlpack_device__()

        def __dlpack__(self, *, stream=None, max_version=None):
            calls.append((stream, max_version))
            return x.__dlpack__(stream=stream, max_version=max_version)

    np.testing.assert_array_equal(cx.from_dlpack(Producer()).numpy(), x.numpy())
    assert calls == [(None, (1, 0))]

    class LegacyProducer:
        def __dlpack_device__(self):
            return x.__dlpack_device__()

        def __dlpack__(self, stream=None):
            return x.__dlpack__(stream=stream)

    np.testing.assert_array_equal(cx.from_dlpack(LegacyProducer()).numpy(), x.numpy())

    class Broken(Producer):
        def __dlpack__(self, **kwargs):
            calls.append("broken")
            raise TypeError("producer internal error")

    with pytest.raises(TypeError, match="internal"):
        cx.from_dlpack(Broken())
    assert calls.count("broken") == 1


def test_device_mismatch():
    fixture = Fixture()

    class Liar:
        def __dlpack_device__(self):
            return (ROCM, 0)

        def __dlpack__(self, **kwargs):
            return fixture.capsule

    with pytest.raises(BufferError, match="differs"):
        cx.from_dlpack(Liar())
    assert fixture.deleted == 1


def test_unsupported_producer_device():
    class Cuda:
        def __dlpack_device__(self):
            return (2, 0)

        def __dlpack__(self, **kwargs):
            raise AssertionError("must not be asked for a capsule")

    with pytest.raises(BufferError, match="ROCm"):
        cx.from_dlpack(Cuda())


def test_empty_noncanonical_strides():
    fixture = Fixture(shape=(2, 0, 3), strides=(3, 3, 1))
    result = cx.from_dlpack(fixture.capsule)
    assert result.shape == (2, 0, 3)
    assert result.numpy().size == 0


@pytest.mark.parametrize("stream", [-1, 0, 1, 2, True, "stream"])
def test_host_export_rejects_stream(stream):
    with pytest.raises(BufferError):
        cx.ones((1,)).__dlpack__(stream=stream)


def test_no_implicit_copy_for_layout():
    x = np.arange(12, dtype=np.float32).reshape(3, 4).T
    for copy in (None, False, True):
        with pytest.raises(BufferError, match="contiguous"):
            cx.from_dlpack(x, copy=copy)


def test_export_does_not_transfer_devices():
    with pytest.raises(BufferError):
        cx.ones((2,)).__dlpack__(dl_device=(ROCM, 0))
    assert cx.ones((2,)).__dlpack_device__() == (CPU, 0)
    with pytest.raises(BufferError):
        cx.tensor(np.zeros(2, np.float64)).__dlpack__(dl_device=(2, 0))


TORCH_HOST_EXCHANGE = r"""
import sys
import torch  # first, as the reference's bridge orders the imports
import numpy as np
sys.path[:0] = sys.argv[1:3]
import tensorcx as cx
from dlpack_fixtures import address

t = torch.arange(12, dtype=torch.float32).reshape(3, 4)
x = cx.from_dlpack(t)
assert x.device == "cpu" and address(x.__dlpack__()) == t.data_ptr()
t.add_(1)
np.testing.assert_array_equal(x.numpy(), t.numpy())
y = cx.tensor(np.arange(6, dtype=np.int32).reshape(2, 3))
ty = torch.from_dlpack(y)
assert ty.dtype == torch.int32 and ty.data_ptr() == address(y.__dlpack__())
ty.mul_(2)
np.testing.assert_array_equal(y.numpy(), np.arange(6, dtype=np.int32).reshape(2, 3) * 2)
b = torch.tensor([True, False, True])
np.testing.assert_array_equal(cx.from_dlpack(b).numpy(), [True, False, True])
try:
    cx.from_dlpack(t.T)
    raise AssertionError("a transposed torch view must be rejected")
except BufferError as error:
    assert "contiguous" in str(error)
print("DLPACK-TORCH-HOST-OK")
"""


def test_exchange_with_torch_host_tensors():
    """Zero-copy both ways with torch CPU tensors, in a child that imports torch first."""
    import pathlib
    import subprocess
    import sys

    pytest.importorskip("torch")
    root = pathlib.Path(__file__).resolve().parents[1]
    paths = [str(root / "tensor.cx_amd" / "python"), str(root / "tests")]
    result = subprocess.run([sys.executable, "-c", TORCH_HOST_EXCHANGE, *paths], capture_output=True, text=True,
                            timeout=300)
    assert result.returncode == 0 and "DLPACK-TORCH-HOST-OK" in result.stdout, result.stderr[-2000:]
