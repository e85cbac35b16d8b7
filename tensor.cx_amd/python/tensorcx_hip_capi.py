"""ctypes binding of the hip device's C ABI (include/tensorcx_hip.h).

This is the thin layer bench.py and the kernel-level tests use to drive the
kernels directly: device buffers, the per-thread stream, HIP events and every
kernel launcher. Loading it never needs a GPU; the calls that touch the device
report TCX_UNAVAILABLE without one. The library is built by
``python tensor.cx_amd/build.py``; nothing here falls back to CPU code.
"""

from __future__ import annotations

import ctypes
import pathlib

import numpy as np

PKG = pathlib.Path(__file__).resolve().parents[1]
LIB_PATH = PKG / "lib" / "libtensorcx_hip.so"

TCX_OK, TCX_INVALID_ARGUMENT, TCX_UNAVAILABLE, TCX_INTERNAL = 0, 1, 2, 3
TCX_FLOAT32, TCX_INT32 = 0, 1
TCX_POOL_OOM = 102
REDUCE_NOALLOC_MAX_WORKSPACE = 4194304
ACT = {"none": 0, "silu": 1, "gelu": 2}
REDUCE = {"sum": 0, "max": 1, "mean": 2, "min": 3, "argmax": 4}
UNARY = {"exp": 0, "gelu": 1, "silu": 2}
BINARY = {"add": 0, "subtract": 1, "multiply": 2, "divide": 3}
MAX_BATCH_RANK = 8

# Every entry point include/tensorcx_hip.h declares.
EXPORTS = [
    "tcx_hip_last_error", "tcx_hip_init", "tcx_hip_device_count", "tcx_hip_device_info",
    "tcx_hip_stream", "tcx_hip_stream_synchronize", "tcx_hip_allocate", "tcx_hip_release",
    "tcx_hip_release_uncached", "tcx_hip_borrow_check", "tcx_hip_memcpy_h2d", "tcx_hip_memcpy_d2h", "tcx_hip_memcpy_d2d", "tcx_hip_pool_create",
    "tcx_hip_pool_enter", "tcx_hip_pool_exit", "tcx_hip_pool_trim", "tcx_hip_pool_stats",
    "tcx_hip_pool_destroy", "tcx_hip_event_create", "tcx_hip_event_record",
    "tcx_hip_event_synchronize", "tcx_hip_event_elapsed_ms", "tcx_hip_event_destroy",
    "tcx_hip_gemm_f32", "tcx_hip_gemm_workspace_bytes", "tcx_hip_gemm_f32_ws",
    "tcx_hip_reduce_workspace_bytes", "tcx_hip_reduce", "tcx_hip_reduce_noalloc",
    "tcx_hip_reduce_axes", "tcx_hip_softmax_f32", "tcx_hip_rmsnorm_f32", "tcx_hip_layernorm_f32",
    "tcx_hip_rownorm_workspace_bytes", "tcx_hip_softmax_f32_ws", "tcx_hip_rmsnorm_f32_ws",
    "tcx_hip_layernorm_f32_ws",
    "tcx_hip_bias_act_f32", "tcx_hip_unary_f32", "tcx_hip_binary", "tcx_hip_fill",
    "tcx_hip_math_unary", "tcx_hip_clip", "tcx_hip_topk", "tcx_hip_embedding_f32",
    "tcx_hip_attention_softmax_f32", "tcx_hip_flash_attention_supported", "tcx_hip_flash_attention_f32",
    "tcx_hip_gather_strided", "tcx_hip_copy_blocks", "tcx_hip_cast", "tcx_hip_scalar_op", "tcx_hip_predicate",
    "tcx_hip_bool_reduce", "tcx_hip_mask_chunks", "tcx_hip_mask_count", "tcx_hip_masked_select",
]


class HipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64),
                ("compute_units", ctypes.c_int), ("clock_khz", ctypes.c_int),
                ("memory_clock_khz", ctypes.c_int), ("memory_bus_width", ctypes.c_int),
                ("l2_bytes", ctypes.c_int), ("runtime_version", ctypes.c_int),
                ("driver_version", ctypes.c_int), ("total_bytes", ctypes.c_size_t),
                ("free_bytes", ctypes.c_size_t)]


class GemmDesc(ctypes.Structure):
    _fields_ = [("m", ctypes.c_int64), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
                ("batch_count", ctypes.c_int64), ("batch_rank", ctypes.c_int32),
                ("rhs_transposed", ctypes.c_int32),
                ("batch_shape", ctypes.c_int64 * MAX_BATCH_RANK),
                ("lhs_batch_strides", ctypes.c_int64 * MAX_BATCH_RANK),
                ("rhs_batch_strides", ctypes.c_int64 * MAX_BATCH_RANK),
                ("bias", ctypes.c_void_p), ("activation", ctypes.c_int32)]


ALLOCATE_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t)
FREE_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)
CLEAR_FN = ctypes.CFUNCTYPE(ctypes.c_int)


class PoolRuntime(ctypes.Structure):
    _fields_ = [("allocate", ALLOCATE_FN), ("free", FREE_FN), ("clear_error", CLEAR_FN)]


class PoolStats(ctypes.Structure):
    _fields_ = [(name, ctypes.c_size_t) for name in (
        "max_cached_bytes", "max_cached_blocks", "cached_bytes", "cached_blocks", "in_use_bytes",
        "peak_in_use_bytes", "peak_cached_bytes")] + [(name, ctypes.c_uint64) for name in (
        "hits", "misses", "allocation_calls", "free_calls", "allocation_failures", "oom_retries",
        "uncached_returns", "readiness_failures", "free_failures", "failed_free_bytes")] + [
        ("active", ctypes.c_int)]


_LIB = None


def lib() -> ctypes.CDLL:
    """Loads libtensorcx_hip.so; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python tensor.cx_amd/build.py`")
        L = ctypes.CDLL(str(LIB_PATH))
        L.tcx_hip_last_error.restype = ctypes.c_char_p
        vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
        L.tcx_hip_stream.argtypes = [ctypes.POINTER(vp)]
        L.tcx_hip_stream_synchronize.argtypes = [vp]
        L.tcx_hip_allocate.argtypes = [sz, ctypes.POINTER(vp), ctypes.POINTER(vp)]
        L.tcx_hip_release.argtypes = [vp, sz, vp]
        L.tcx_hip_release.restype = None
        for name in ("tcx_hip_memcpy_h2d", "tcx_hip_memcpy_d2h", "tcx_hip_memcpy_d2d"):
            getattr(L, name).argtypes = [vp, vp, sz, vp]
        L.tcx_hip_pool_create.argtypes = [sz, sz, ctypes.POINTER(PoolRuntime), ctypes.POINTER(vp)]
        for name in ("tcx_hip_pool_enter", "tcx_hip_pool_exit", "tcx_hip_pool_trim"):
            getattr(L, name).argtypes = [vp]
        L.tcx_hip_pool_stats.argtypes = [vp, ctypes.POINTER(PoolStats)]
        L.tcx_hip_pool_destroy.argtypes = [vp]
        L.tcx_hip_pool_destroy.restype = None
        L.tcx_hip_event_create.argtypes = [ctypes.POINTER(vp)]
        L.tcx_hip_event_record.argtypes = [vp, vp]
        L.tcx_hip_event_synchronize.argtypes = [vp]
        L.tcx_hip_event_elapsed_ms.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_float)]
        L.tcx_hip_event_destroy.argtypes = [vp]
        L.tcx_hip_gemm_f32.argtypes = [vp, vp, vp, ctypes.POINTER(GemmDesc), vp]
        L.tcx_hip_gemm_workspace_bytes.argtypes = [ctypes.POINTER(GemmDesc)]
        L.tcx_hip_gemm_workspace_bytes.restype = sz
        L.tcx_hip_gemm_f32_ws.argtypes = [vp, vp, vp, ctypes.POINTER(GemmDesc), vp, sz, vp]
        L.tcx_hip_reduce_workspace_bytes.argtypes = [ctypes.c_int, ctypes.c_int, i64, i64, i64]
        L.tcx_hip_reduce_workspace_bytes.restype = sz
        L.tcx_hip_reduce.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, i64, i64, i64, vp, sz, vp]
        L.tcx_hip_reduce_noalloc.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, i64, i64, i64, vp]
        L.tcx_hip_reduce_axes.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_int32,
                                          ctypes.c_int32, i64, i64, vp]
        L.tcx_hip_softmax_f32.argtypes = [vp, vp, i64, i64, i64, vp]
        L.tcx_hip_rmsnorm_f32.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.c_float, vp]
        L.tcx_hip_layernorm_f32.argtypes = [vp, vp, vp, vp, i64, i64, i64, ctypes.c_float, vp]
        L.tcx_hip_rownorm_workspace_bytes.argtypes = [i64, i64, i64]
        L.tcx_hip_rownorm_workspace_bytes.restype = sz
        L.tcx_hip_softmax_f32_ws.argtypes = [vp, vp, i64, i64, i64, vp, sz, vp]
        L.tcx_hip_rmsnorm_f32_ws.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.c_float, vp, sz, vp]
        L.tcx_hip_layernorm_f32_ws.argtypes = [vp, vp, vp, vp, i64, i64, i64, ctypes.c_float, vp, sz, vp]
        L.tcx_hip_bias_act_f32.argtypes = [vp, vp, vp, i64, i64, ctypes.c_int, vp]
        L.tcx_hip_unary_f32.argtypes = [ctypes.c_int, vp, vp, i64, vp]
        L.tcx_hip_binary.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_int32, vp, vp,
                                     vp, vp]
        L.tcx_hip_fill.argtypes = [ctypes.c_int, vp, i64, ctypes.c_double, vp]
        L.tcx_hip_flash_attention_supported.argtypes = [i64, i64]
        L.tcx_hip_flash_attention_f32.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, ctypes.c_float,
                                                  ctypes.c_int, vp]
        _LIB = L
    return _LIB


def last_error() -> str:
    return (lib().tcx_hip_last_error() or b"").decode()


def check(code: int, what: str = "") -> None:
    if code != TCX_OK:
        raise HipError(code, f"{what}: {last_error()}")


def available() -> bool:
    return lib().tcx_hip_init() == TCX_OK


def device_info() -> dict:
    info = DeviceInfo()
    check(lib().tcx_hip_device_info(0, ctypes.byref(info)), "device_info")
    return {name: (getattr(info, name).decode() if isinstance(getattr(info, name), bytes)
                   else getattr(info, name)) for name, _ in DeviceInfo._fields_}


def stream() -> int:
    s = ctypes.c_void_p()
    check(lib().tcx_hip_stream(ctypes.byref(s)), "stream")
    return s.value


def synchronize() -> None:
    check(lib().tcx_hip_stream_synchronize(stream()), "synchronize")


class DeviceBuffer:
    """Device memory from tcx_hip_allocate, released on close()/garbage collection."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        self.owner = ctypes.c_void_p()
        check(lib().tcx_hip_allocate(self.nbytes, ctypes.byref(self.ptr), ctypes.byref(self.owner)),
              "allocate")

    @property
    def address(self) -> int:
        return self.ptr.value or 0

    def close(self) -> None:
        if self.ptr.value:
            lib().tcx_hip_release(self.ptr, self.nbytes, self.owner)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass


class DeviceArray:
    """A typed device buffer with a shape, for driving the kernels directly."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        self.size = int(np.prod(self.shape, dtype=np.int64))
        self.buffer = DeviceBuffer(self.size * self.dtype.itemsize)

    @classmethod
    def from_numpy(cls, array: np.ndarray) -> "DeviceArray":
        array = np.ascontiguousarray(array)
        out = cls(array.shape, array.dtype)
        if out.buffer.nbytes:
            check(lib().tcx_hip_memcpy_h2d(out.buffer.ptr, array.ctypes.data, array.nbytes, stream()),
                  "h2d")
        return out

    @property
    def ptr(self) -> int:
        return self.buffer.address

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if out.nbytes:
            check(lib().tcx_hip_memcpy_d2h(out.ctypes.data, self.buffer.ptr, out.nbytes, stream()),
                  "d2h")
        return out


class Event:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(lib().tcx_hip_event_create(ctypes.byref(self.handle)), "event_create")

    def record(self, s: int | None = None) -> None:
        check(lib().tcx_hip_event_record(self.handle, s if s is not None else stream()), "event_record")

    def synchronize(self) -> None:
        check(lib().tcx_hip_event_synchronize(self.handle), "event_synchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().tcx_hip_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)), "elapsed")
        return ms.value

    def __del__(self):
        try:
            if self.handle.value:
                lib().tcx_hip_event_destroy(self.handle)
        except Exception:  # noqa: BLE001
            pass


# ------------------------------------------------------------------ kernels
def gemm_desc(m, n, k, *, batch_shape=(), lhs_batch_strides=(), rhs_batch_strides=(),
              rhs_transposed=False, bias: int | None = None, activation="none") -> GemmDesc:
    d = GemmDesc()
    d.m, d.n, d.k = m, n, k
    d.batch_rank = len(batch_shape)
    d.batch_count = int(np.prod(batch_shape, dtype=np.int64)) if batch_shape else 1
    for i, (e, ls, rs) in enumerate(zip(batch_shape, lhs_batch_strides, rhs_batch_strides)):
        d.batch_shape[i], d.lhs_batch_strides[i], d.rhs_batch_strides[i] = e, ls, rs
    d.rhs_transposed = int(rhs_transposed)
    d.bias = bias
    d.activation = ACT[activation]
    return d


def gemm(lhs: int, rhs: int, out: int, desc: GemmDesc, s: int | None = None,
         workspace: DeviceBuffer | None = None) -> None:
    """tcx_hip_gemm_f32, or tcx_hip_gemm_f32_ws with a workspace (gemm_workspace)."""
    if workspace is None:
        check(lib().tcx_hip_gemm_f32(lhs, rhs, out, ctypes.byref(desc), s or stream()), "gemm")
    else:
        check(lib().tcx_hip_gemm_f32_ws(lhs, rhs, out, ctypes.byref(desc), workspace.address, workspace.nbytes,
                                        s or stream()), "gemm")


def gemm_workspace(desc: GemmDesc) -> DeviceBuffer | None:
    """The workspace tcx_hip_gemm_f32_ws can use for desc (None when it needs none)."""
    nbytes = lib().tcx_hip_gemm_workspace_bytes(ctypes.byref(desc))
    return DeviceBuffer(nbytes) if nbytes else None


def reduce(op: str, dtype: int, x: int, out: int, outer: int, reduce_: int, inner: int,
           workspace: DeviceBuffer | None = None, s: int | None = None) -> None:
    ws_ptr = workspace.address if workspace is not None else None
    ws_bytes = workspace.nbytes if workspace is not None else 0
    check(lib().tcx_hip_reduce(REDUCE[op], dtype, x, out, outer, reduce_, inner, ws_ptr, ws_bytes,
                               s or stream()), f"reduce {op}")


def reduce_noalloc(op: str, dtype: int, x: int, out: int, outer: int, reduce_: int, inner: int,
                   s: int | None = None) -> None:
    """tcx_hip_reduce_noalloc: no workspace, the library's static scratch."""
    check(lib().tcx_hip_reduce_noalloc(REDUCE[op], dtype, x, out, outer, reduce_, inner, s or stream()),
          f"reduce_noalloc {op}")


def reduce_workspace(op: str, dtype: int, outer: int, reduce_: int, inner: int) -> DeviceBuffer | None:
    nbytes = lib().tcx_hip_reduce_workspace_bytes(REDUCE[op], dtype, outer, reduce_, inner)
    return DeviceBuffer(nbytes) if nbytes else None


def softmax(x: int, out: int, outer: int, reduce_: int, inner: int, s: int | None = None) -> None:
    check(lib().tcx_hip_softmax_f32(x, out, outer, reduce_, inner, s or stream()), "softmax")


def rmsnorm(x: int, gamma: int | None, out: int, outer, reduce_, inner, eps=1e-5, s=None) -> None:
    check(lib().tcx_hip_rmsnorm_f32(x, gamma, out, outer, reduce_, inner, eps, s or stream()), "rmsnorm")


def layernorm(x: int, gamma: int | None, beta: int | None, out: int, outer, reduce_, inner, eps=1e-5,
              s=None) -> None:
    check(lib().tcx_hip_layernorm_f32(x, gamma, beta, out, outer, reduce_, inner, eps, s or stream()),
          "layernorm")


def rownorm_workspace(outer: int, reduce_: int, inner: int) -> DeviceBuffer | None:
    """A workspace for the *_ws row ops of this shape, or None when none is needed."""
    nbytes = lib().tcx_hip_rownorm_workspace_bytes(outer, reduce_, inner)
    return DeviceBuffer(nbytes) if nbytes else None


def _ws_args(workspace):
    return (workspace.address, workspace.nbytes) if workspace is not None else (None, 0)


def softmax_ws(x: int, out: int, outer: int, reduce_: int, inner: int, workspace=None, s=None) -> None:
    check(lib().tcx_hip_softmax_f32_ws(x, out, outer, reduce_, inner, *_ws_args(workspace), s or stream()),
          "softmax_ws")


def rmsnorm_ws(x: int, gamma: int | None, out: int, outer, reduce_, inner, eps=1e-5, workspace=None,
               s=None) -> None:
    check(lib().tcx_hip_rmsnorm_f32_ws(x, gamma, out, outer, reduce_, inner, eps, *_ws_args(workspace),
                                       s or stream()), "rmsnorm_ws")


def layernorm_ws(x: int, gamma: int | None, beta: int | None, out: int, outer, reduce_, inner, eps=1e-5,
                 workspace=None, s=None) -> None:
    check(lib().tcx_hip_layernorm_f32_ws(x, gamma, beta, out, outer, reduce_, inner, eps,
                                         *_ws_args(workspace), s or stream()), "layernorm_ws")


def bias_act(x: int, bias: int | None, out: int, rows: int, cols: int, activation="none", s=None) -> None:
    check(lib().tcx_hip_bias_act_f32(x, bias, out, rows, cols, ACT[activation], s or stream()), "bias_act")


def flash_attention(q, k, v, out, batch: int, rows: int, cols: int, features: int, scale: float,
                    causal: bool, stream_=None):
    """Fused attention on device pointers (tcx_hip_flash_attention_f32)."""
    check(lib().tcx_hip_flash_attention_f32(q, k, v, out, batch, rows, cols, features, scale, int(causal),
                                            stream_ or stream()), "flash_attention")
