"""Hand-built DLPack capsules for protocol tests.

ctypes mirrors of the DLPack 1.0 structs (field order fixed by the DLPack
specification), a capsule factory over memory the test owns, and a reader
for a capsule's descriptor. The factory counts deleter calls, so tests can
check that a consumer releases a capsule exactly once, including when it
rejects the descriptor.
"""

from __future__ import annotations

import ctypes as C

import numpy as np


class DLDevice(C.Structure):
    _fields_ = [("device_type", C.c_int32), ("device_id", C.c_int32)]


class DLDataType(C.Structure):
    _fields_ = [("code", C.c_uint8), ("bits", C.c_uint8), ("lanes", C.c_uint16)]


class DLTensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("device", DLDevice), ("ndim", C.c_int32), ("dtype", DLDataType),
                ("shape", C.POINTER(C.c_int64)), ("strides", C.POINTER(C.c_int64)), ("byte_offset", C.c_uint64)]


DELETER = C.CFUNCTYPE(None, C.c_void_p)


class DLManagedTensor(C.Structure):
    _fields_ = [("dl_tensor", DLTensor), ("manager_ctx", C.c_void_p), ("deleter", DELETER)]


class DLPackVersion(C.Structure):
    _fields_ = [("major", C.c_uint32), ("minor", C.c_uint32)]


class DLManagedTensorVersioned(C.Structure):
    _fields_ = [("version", DLPackVersion), ("manager_ctx", C.c_void_p), ("deleter", DELETER),
                ("flags", C.c_uint64), ("dl_tensor", DLTensor)]


_new_capsule = C.pythonapi.PyCapsule_New
_new_capsule.restype = C.py_object
_new_capsule.argtypes = [C.c_void_p, C.c_char_p, C.c_void_p]
_capsule_pointer = C.pythonapi.PyCapsule_GetPointer
_capsule_pointer.restype = C.c_void_p
_capsule_pointer.argtypes = [C.py_object, C.c_char_p]

CPU, ROCM = 1, 10


class Fixture:
    """A capsule over `data` (a NumPy array, or a raw address with `device`).

    The Fixture object keeps every native piece alive; `deleted` counts the
    deleter calls. The capsule has no destructor of its own, so dropping it
    unconsumed releases nothing.
    """

    def __init__(self, data=None, *, address=None, device=CPU, versioned=True, shape=(2, 3), strides=None,
                 offset=0, flags=0, code=2, bits=32):
        self.deleted = 0
        self.data = np.arange(64, dtype=np.float32) if data is None and address is None else data
        pointer = address if address is not None else self.data.ctypes.data
        self.shape = (C.c_int64 * max(len(shape), 1))(*shape)
        self.strides = None if strides is None else (C.c_int64 * len(strides))(*strides)

        def delete(_):
            self.deleted += 1

        self.deleter = DELETER(delete)
        tensor = DLTensor(pointer, DLDevice(device, 0), len(shape), DLDataType(code, bits, 1),
                          self.shape, self.strides, offset)
        if versioned:
            self.managed = DLManagedTensorVersioned(DLPackVersion(1, 0), None, self.deleter, flags, tensor)
        else:
            self.managed = DLManagedTensor(tensor, None, self.deleter)
        name = b"dltensor_versioned" if versioned else b"dltensor"
        self.capsule = _new_capsule(C.addressof(self.managed), name, None)

    @property
    def tensor(self) -> DLTensor:
        return self.managed.dl_tensor


def describe(capsule) -> DLTensor:
    """The DLTensor of an unconsumed legacy or versioned capsule.

    The result is a view into memory the capsule owns: keep the capsule
    referenced while the view is used (address() reads a temporary's).
    """
    try:
        return C.cast(_capsule_pointer(capsule, b"dltensor"), C.POINTER(DLManagedTensor)).contents.dl_tensor
    except ValueError:
        pass
    return versioned(capsule).dl_tensor


def address(capsule) -> int:
    """Data address of a capsule, read while the capsule is still referenced."""
    return describe(capsule).data


def versioned(capsule) -> DLManagedTensorVersioned:
    return C.cast(_capsule_pointer(capsule, b"dltensor_versioned"), C.POINTER(DLManagedTensorVersioned)).contents
