"""DLPack exchange for contiguous hip (kDLROCM) and host float32, int32 and bool tensors.

The contract of the reference's python/tensorcx/dlpack.py (docs/DLPACK.md),
with the hip device in place of CUDA: the device is (10, 0) (kDLROCM, device
0), and the stream rules are the DLPack / Array API ones for ROCm, where 0
names the default stream and 1 and 2 are not valid stream values.

* ``Tensor.__dlpack__(stream=None, max_version=None, dl_device=None, copy=None)``
  exports a legacy capsule unless ``max_version >= (1, 0)``; a versioned
  copy carries the is-copied flag. ``dl_device`` may only name the tensor's
  own device.
* ``from_dlpack(source, copy=None)`` accepts a producer with ``__dlpack__``
  and ``__dlpack_device__`` or an unconsumed capsule. ``copy=None``/``False``
  share storage, ``copy=True`` makes an independent copy on the same device,
  and read-only input requires ``copy=True``.

Every hip operation finishes before it returns, so export needs no stream
work. Import waits for all work on the device before the shared memory is
read, which also covers a producer that handed over a bare capsule. Writes
another framework makes later must be synchronised by the caller before
tensorcx reads the buffer again.
"""

from __future__ import annotations

import inspect
import operator

from . import _core

CPU = (1, 0)
ROCM = (10, 0)


def _copy_option(copy):
    if copy is not None and type(copy) is not bool:
        raise TypeError("copy must be True, False or None")
    return copy


def _device_tuple(value):
    if not isinstance(value, tuple) or len(value) != 2:
        raise TypeError("DLPack device must be a (device_type, device_id) tuple")
    result = []
    for item in value:
        if isinstance(item, bool):
            raise TypeError("DLPack device fields must be integers")
        result.append(operator.index(item))
    return tuple(result)


def device_of(tensor):
    """(device_type, device_id) of a tensor: (1, 0) host, (10, 0) hip."""
    return CPU if tensor.device == "cpu" else ROCM


def _check_stream(stream, copy):
    """Stream argument of a hip export (DLPack Python specification, ROCm)."""
    if stream is None:
        return
    if isinstance(stream, bool):
        raise TypeError("ROCm stream must be an integer or None")
    stream = operator.index(stream)
    if stream in (1, 2) or stream < -1:
        raise ValueError("ROCm stream must be -1, 0 or a stream pointer")
    if stream == -1 and copy is True:
        raise BufferError("ROCm copy=True requires synchronization; stream=-1 forbids it")
    if stream != 0 and copy is True:
        raise BufferError("ROCm copy=True supports only the default stream")


def export(tensor, *, stream=None, max_version=None, dl_device=None, copy=None):
    _copy_option(copy)
    device = device_of(tensor)
    if dl_device is not None and _device_tuple(dl_device) != device:
        raise BufferError("DLPack export does not transfer devices; use Tensor.to explicitly")
    if device == CPU:
        if stream is not None:
            raise BufferError("CPU DLPack export requires stream=None")
    else:
        _check_stream(stream, copy)
    versioned = False
    if max_version is not None:
        major, minor = _device_tuple(max_version)
        if major < 0 or minor < 0:
            raise ValueError("max_version must contain nonnegative integers")
        versioned = (major, minor) >= (1, 0)
    if device == CPU:
        return _core._to_dlpack_host(tensor._impl, versioned, copy is True)
    return _core._to_dlpack(tensor._impl, versioned, copy is True)


def from_dlpack(source, *, copy=None):
    """Share supported contiguous storage, or make an explicit same-device copy.

    Writes through any sharing tensor are visible to all of them. Read-only
    versioned storage requires copy=True. A capsule can be consumed once.
    """
    from . import Tensor

    _copy_option(copy)
    device = (-1, -1)
    if hasattr(source, "__dlpack__"):
        if not hasattr(source, "__dlpack_device__"):
            raise TypeError("DLPack producer must define __dlpack_device__")
        device = _device_tuple(source.__dlpack_device__())
        if device not in (CPU, ROCM):
            raise BufferError("DLPack import supports CPU and ROCm device 0 only")
        method = source.__dlpack__
        # The consumer reads on the default stream (0 for ROCm); the import
        # also waits for the whole device.
        kwargs = {"stream": 0} if device == ROCM else {}
        # A Python producer exposes its signature, so a TypeError raised
        # inside it is never mistaken for a missing keyword. Builtins are
        # negotiated by the unexpected-keyword error.
        try:
            signature = inspect.signature(method)
        except (TypeError, ValueError):
            signature = None
        if signature is not None:
            parameters = signature.parameters.values()
            if "max_version" in signature.parameters or any(p.kind == p.VAR_KEYWORD for p in parameters):
                kwargs["max_version"] = (1, 0)
            capsule = method(**kwargs)
        else:
            try:
                capsule = method(**kwargs, max_version=(1, 0))
            except TypeError as error:
                text = str(error)
                if "max_version" not in text or not any(s in text for s in ("unexpected keyword", "invalid keyword")):
                    raise
                capsule = method(**kwargs)
    else:
        capsule = source
    return Tensor(_core._from_dlpack(capsule, copy is True, copy is False, *device))
