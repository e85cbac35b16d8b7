"""Host-only checks of the C ABI library and the HipBackend boundary.

No kernel runs here: the library must load and export every entry point the
header declares; the bounded pool's logic is driven through its injectable
allocator seam (the reference's PoolRuntime idea, cuda_memory_pool.h:20-27);
device entry points must fail cleanly when no device is visible; and
hip_backend.cpp must compile against the reference's own core headers, which
is what makes it a drop-in backend.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import re
import subprocess

import pytest

import tensorcx_hip_capi as capi

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tensorcx_hip.h"
REFERENCE_CPP = pathlib.Path("/root/reference/cpp")


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(tcx_hip_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(capi.EXPORTS)


def test_library_exports_every_declared_symbol():
    if not capi.LIB_PATH.exists():
        pytest.fail("libtensorcx_hip.so is not built: run `python tensor.cx_amd/build.py`")
    out = subprocess.run(["nm", "-D", "--defined-only", str(capi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (tcx_hip_\w+)$", out, re.M))
    missing = [name for name in declared_functions() if name not in exported]
    assert not missing, f"missing exports: {missing}"
    lib = capi.lib()
    for name in declared_functions():
        assert getattr(lib, name) is not None


@pytest.mark.parametrize("m,n,k,batch,trans,expect", [
    (4096, 1024, 4096, (), True, 0),                      # the MLP's second linear: 256 128x128 tiles
    (4096, 1024, 4096, (), False, 0),                     # the same with a [k, n] B
    (2048, 1024, 4096, (), True, 4 * 2048 * 1024 * 4),   # 128 tiles of 128x128: 4 splits
    (1024, 1024, 8192, (), False, 8 * 1024 * 1024 * 4),   # 64 tiles: 8 splits of 1024
    (512, 512, 8192, (4,), False, 8 * 4 * 512 * 512 * 4),  # batched: 64 tiles
    (4096, 4096, 4096, (), False, 0),                     # four full rounds of 256 tiles
    (3072, 3072, 3072, (), False, 4 * 3072 * 3072 * 4),   # 576 tiles: the third round 1/4 full
    (4096, 3072, 1024, (), True, 0),                      # 768 tiles: three full rounds
    (1000, 1000, 1000, (), False, 0),                     # partial tiles
    (1024, 1024, 1024, (), False, 0),                     # splits would keep < 512 of K
    (512, 512, 16384, (), False, 16 * 512 * 512 * 4),     # 16 tiles: the 16-split cap
    (512, 512, 512, (), False, 0),
    # K or N not a multiple of 4, at least 2^32 multiply-adds, unbatched:
    # zero-padded copies of A [M][K4], B [K4][N4] and the output [M][N4],
    # each rounded up to 64 floats.
    (2048, 2049, 2048, (), False, (4194304 + 4202496 + 4202496) * 4),
    (2048, 2049, 2048, (), True, (4194304 + 4202496 + 4202496) * 4),
    (2048, 2049, 2048, (2,), False, 0),                   # batched: not padded
    (1025, 1025, 1025, (), False, 0),                     # too small to pay
    # One row against a row-major B with too few 1024-column blocks: K split
    # (4 blocks x 32 splits of 128 rows), partials [splits][N].
    (1, 4096, 4096, (), False, 32 * 4096 * 4),
    (1, 4096, 4096, (), True, 0),                         # the GEMV route
])
def test_gemm_workspace_query(m, n, k, batch, trans, expect):
    if not capi.LIB_PATH.exists():
        pytest.fail("libtensorcx_hip.so is not built: run `python tensor.cx_amd/build.py`")
    strides = tuple(m * k for _ in batch), tuple(k * n for _ in batch)
    d = capi.gemm_desc(m, n, k, batch_shape=batch, lhs_batch_strides=strides[0], rhs_batch_strides=strides[1],
                       rhs_transposed=trans)
    assert capi.lib().tcx_hip_gemm_workspace_bytes(ctypes.byref(d)) == expect


def test_reduce_workspace_fits_the_noalloc_scratch():
    # tcx_hip_reduce_noalloc accepts every plan whose workspace query is at
    # most TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE; the query stays under it for
    # every float32 tensor that fits in 288 GB of HBM (at most 2^36
    # elements): fewer than 448 rows of 32768+ elements are split into about
    # 448 items in all, so rows x items stays below 896 partials of 16 bytes,
    # and rows longer than 2^32 elements add at most 16 items per row. A sweep of row counts and row lengths
    # around the segmenting thresholds shows it.
    if not capi.LIB_PATH.exists():
        pytest.fail("libtensorcx_hip.so is not built: run `python tensor.cx_amd/build.py`")
    query = capi.lib().tcx_hip_reduce_workspace_bytes
    largest = 0
    for rows in (1, 2, 3, 5, 63, 64, 1000, 4095, 4097, 8000, 8191, 8192, 16384):
        for cols in (65, 8192, 8193, 16384, 100_000, 2**20 + 3, 2**26, 2**31 + 5, 2**33):
            if rows * cols > 2**36:
                continue
            for op in ("sum", "max", "argmax"):
                largest = max(largest, query(capi.REDUCE[op], capi.TCX_FLOAT32, rows, cols, 1))
    assert 0 < largest <= capi.REDUCE_NOALLOC_MAX_WORKSPACE
    # The full-tensor sum: 443 block items of four 37888-element (37 x 1024)
    # wave segments.
    assert query(0, capi.TCX_FLOAT32, 1, 8192 * 8192, 1) == 443 * 16
    # Rows of 8192+ elements with enough rows to fill the grid: no partials.
    assert query(0, capi.TCX_FLOAT32, 448, 1 << 20, 1) == 0
    assert query(0, capi.TCX_FLOAT32, 447, 1 << 20, 1) == 447 * 2 * 16


def test_column_reduce_workspace_query():
    # Strided reductions (inner > 1) of more than 64 rows: column tiles of
    # 256 columns (inner a multiple of 4) or 64, or the power of two at or
    # above a narrower inner, whose waves then step G = 256 / W (or 64 / W)
    # rows at a time. Rows split by doubling while tiles x splits < 512,
    # each split keeps at least 64 x G rows and the 16-byte partials fit the
    # no-allocation scratch.
    if not capi.LIB_PATH.exists():
        pytest.fail("libtensorcx_hip.so is not built: run `python tensor.cx_amd/build.py`")
    query = capi.lib().tcx_hip_reduce_workspace_bytes
    assert query(0, capi.TCX_FLOAT32, 1, 8192, 64) == 32 * 64 * 16          # G 4: 32 splits of 256 rows
    assert query(1, capi.TCX_FLOAT32, 1, 4096, 4096) == 32 * 4096 * 16      # 16 tiles x 32 splits
    assert query(4, capi.TCX_FLOAT32, 1, 100_000, 3) == 64 * 3 * 16         # G 16: 64 splits of 1563 rows
    assert query(0, capi.TCX_FLOAT32, 2, 1000, 1030) == 8 * 2 * 1030 * 16   # 34 tiles of 64, 8 splits
    assert query(0, capi.TCX_FLOAT32, 5, 3001, 7) == 4 * 5 * 7 * 16         # G 8: 4 splits
    assert query(0, capi.TCX_FLOAT32, 16, 512, 8192) == 0                   # 512 tiles: no split
    assert query(0, capi.TCX_FLOAT32, 1, 65, 600) == 0                      # 65 rows: too few to split
    assert query(0, capi.TCX_FLOAT32, 1, 64, 600) == 0                      # exact-order lanes
    largest = 0
    for outer in (1, 2, 7, 64, 1000):
        for rows in (65, 300, 4096, 65536, 2**24):
            for inner in (2, 3, 64, 65, 256, 4100, 2**20):
                if outer * rows * inner <= 2**36:
                    largest = max(largest, query(0, capi.TCX_FLOAT32, outer, rows, inner))
    assert 0 < largest <= capi.REDUCE_NOALLOC_MAX_WORKSPACE


def test_rownorm_workspace_query():
    # Strided row ops split the rows of few column tiles (256 columns when
    # inner is a multiple of 4, else 64, or the power of two at or above a
    # narrower inner, whose waves step 256 / W or 64 / W rows): doubling
    # while tiles x splits < 512 and each split keeps 64 x G rows; the
    # workspace holds the split statistics and one parameter record per
    # column, 16 bytes each. Contiguous rows and unsplit plans need none.
    if not capi.LIB_PATH.exists():
        pytest.fail("libtensorcx_hip.so is not built: run `python tensor.cx_amd/build.py`")
    query = capi.lib().tcx_hip_rownorm_workspace_bytes
    assert query(8192, 8192, 1) == 0
    assert query(64, 64, 4096) == 0
    assert query(1, 8192, 64) == (32 + 1) * 64 * 16
    assert query(1, 100_000, 3) == (64 + 1) * 3 * 16
    assert query(1, 8192, 8192) == (16 + 1) * 8192 * 16
    assert query(0, 8192, 64) == 0 and query(1, 0, 64) == 0
    largest = max(query(o, r, i) for o in (1, 3, 64) for r in (65, 1000, 2**20) for i in (2, 7, 64, 4096, 2**16))
    assert 0 < largest <= 16 << 20


CONTRACT = ROOT / "tests" / "cpp" / "_bin" / "hip_backend_contract"


def test_backend_contract_rejects_malformed_requests_without_a_device():
    # tests/cpp/hip_backend_contract.cpp part 1: every malformed request is
    # kInvalidArgument before any allocation (a host-backed pool counts
    # none), with its output slots untouched; a well-formed one is stopped
    # only by the missing device. Exit 77 = passed without a device.
    if not CONTRACT.exists():
        pytest.fail(f"{CONTRACT} is not built: run `python tensor.cx_amd/build.py`")
    from conftest import gpu_present
    if gpu_present():
        pytest.skip("a device is present: tests/test_hip_contract.py runs the whole contract")
    env = {k: v for k, v in os.environ.items() if k != "TENSORCX_REQUIRE_HIP"}
    result = subprocess.run([str(CONTRACT)], capture_output=True, text=True, timeout=120, env=env)
    assert result.returncode == 77, result.stdout + result.stderr
    assert "malformed requests rejected before allocation" in result.stdout
    assert "metadata validation passed" in result.stdout


def test_header_compiles_as_c():
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-x", "c", str(HEADER)],
                   check=True)


class FakeDevice:
    """Host allocator standing in for hipMalloc/hipFree, with forced OOM."""

    def __init__(self, capacity: int):
        self.capacity = capacity
        self.used = 0
        self.blocks: dict[int, int] = {}
        self.next = 0x1000
        self.fail_free = False
        self.pending = capi.TCX_OK
        self.allocate = capi.ALLOCATE_FN(self._allocate)
        self.free = capi.FREE_FN(self._free)
        self.clear = capi.CLEAR_FN(self._clear)

    def _allocate(self, out, nbytes):
        if self.used + nbytes > self.capacity:
            self.pending = capi.TCX_POOL_OOM
            return capi.TCX_POOL_OOM
        self.next += 0x100000
        self.blocks[self.next] = nbytes
        self.used += nbytes
        out[0] = self.next
        return capi.TCX_OK

    def _free(self, ptr):
        if self.fail_free:
            return capi.TCX_INTERNAL
        self.used -= self.blocks.pop(ptr)
        return capi.TCX_OK

    def _clear(self):
        code, self.pending = self.pending, capi.TCX_OK
        return code

    def runtime(self):
        return capi.PoolRuntime(self.allocate, self.free, self.clear)


def make_pool(device: FakeDevice, max_bytes=1 << 20, max_blocks=4):
    lib = capi.lib()
    pool = ctypes.c_void_p()
    rt = device.runtime()
    capi.check(lib.tcx_hip_pool_create(max_bytes, max_blocks, ctypes.byref(rt), ctypes.byref(pool)))
    return pool, rt


def stats(pool) -> capi.PoolStats:
    s = capi.PoolStats()
    capi.check(capi.lib().tcx_hip_pool_stats(pool, ctypes.byref(s)))
    return s


def alloc(nbytes):
    ptr, owner = ctypes.c_void_p(), ctypes.c_void_p()
    code = capi.lib().tcx_hip_allocate(nbytes, ctypes.byref(ptr), ctypes.byref(owner))
    return code, ptr, owner


def test_pool_reuses_exact_sizes_and_bounds_the_cache():
    lib = capi.lib()
    dev = FakeDevice(1 << 30)
    pool, rt = make_pool(dev, max_bytes=3000, max_blocks=2)
    capi.check(lib.tcx_hip_pool_enter(pool))
    try:
        code, p1, o1 = alloc(1000)
        assert code == capi.TCX_OK and o1.value == pool.value
        lib.tcx_hip_release(p1, 1000, o1)
        code, p2, o2 = alloc(1000)
        assert p2.value == p1.value, "exact-size block must be reused"
        code, p3, o3 = alloc(999)
        assert p3.value != p1.value, "only exact sizes are reused"
        s = stats(pool)
        assert (s.hits, s.misses, s.in_use_bytes) == (1, 2, 1999)
        # Cache bounds: 2 blocks / 3000 bytes.
        _, p4, o4 = alloc(2500)
        for ptr, n, owner in ((p2, 1000, o2), (p3, 999, o3), (p4, 2500, o4)):
            lib.tcx_hip_release(ptr, n, owner)
        s = stats(pool)
        assert s.cached_blocks == 2 and s.cached_bytes == 1999 and s.uncached_returns == 1
    finally:
        capi.check(lib.tcx_hip_pool_exit(pool))
    assert stats(pool).cached_blocks == 0 and dev.used == 0
    lib.tcx_hip_pool_destroy(pool)


def test_pool_drains_cache_and_retries_once_on_oom():
    lib = capi.lib()
    dev = FakeDevice(3000)
    pool, rt = make_pool(dev, max_bytes=1 << 20, max_blocks=8)
    capi.check(lib.tcx_hip_pool_enter(pool))
    _, p1, o1 = alloc(2000)
    lib.tcx_hip_release(p1, 2000, o1)         # cached, still holding 2000 device bytes
    code, p2, o2 = alloc(2500)                # OOM -> drain -> retry succeeds
    assert code == capi.TCX_OK
    s = stats(pool)
    assert s.oom_retries == 1 and s.cached_blocks == 0 and s.allocation_calls == 3
    code, p3, _ = alloc(2000)                 # nothing cached to drain: a plain failure
    assert code == capi.TCX_INTERNAL and "out of memory" in capi.last_error()
    assert stats(pool).allocation_failures == 1
    lib.tcx_hip_release(p2, 2500, o2)
    capi.check(lib.tcx_hip_pool_exit(pool))
    lib.tcx_hip_pool_destroy(pool)
    assert dev.used == 0


def test_pool_scope_rules():
    lib = capi.lib()
    dev = FakeDevice(1 << 20)
    a, rta = make_pool(dev)
    b, rtb = make_pool(dev)
    capi.check(lib.tcx_hip_pool_enter(a))
    assert lib.tcx_hip_pool_enter(b) == capi.TCX_INVALID_ARGUMENT
    assert "nested" in capi.last_error()
    assert lib.tcx_hip_pool_exit(b) == capi.TCX_INVALID_ARGUMENT
    capi.check(lib.tcx_hip_pool_exit(a))
    assert lib.tcx_hip_pool_enter(a) == capi.TCX_INVALID_ARGUMENT   # single use
    assert "single-use" in capi.last_error()
    bad = ctypes.c_void_p()
    assert lib.tcx_hip_pool_create(1, 0, None, ctypes.byref(bad)) == capi.TCX_INVALID_ARGUMENT
    lib.tcx_hip_pool_destroy(a)
    lib.tcx_hip_pool_destroy(b)


def test_pool_outlives_destroy_until_blocks_return():
    lib = capi.lib()
    dev = FakeDevice(1 << 20)
    pool, rt = make_pool(dev)
    capi.check(lib.tcx_hip_pool_enter(pool))
    _, p, o = alloc(4096)
    capi.check(lib.tcx_hip_pool_exit(pool))
    lib.tcx_hip_pool_destroy(pool)            # a block is still out
    assert dev.used == 4096
    lib.tcx_hip_release(p, 4096, o)           # returns to the device, pool goes away
    assert dev.used == 0


def test_pool_free_failures_are_counted():
    lib = capi.lib()
    dev = FakeDevice(1 << 20)
    pool, rt = make_pool(dev)
    capi.check(lib.tcx_hip_pool_enter(pool))
    _, p, o = alloc(64)
    lib.tcx_hip_release(p, 64, o)
    dev.fail_free = True
    assert lib.tcx_hip_pool_trim(pool) == capi.TCX_INTERNAL
    s = stats(pool)
    assert s.free_failures == 1 and s.failed_free_bytes == 64 and s.cached_blocks == 0
    dev.fail_free = False
    capi.check(lib.tcx_hip_pool_exit(pool))
    lib.tcx_hip_pool_destroy(pool)


@pytest.mark.skipif(capi.available(), reason="a HIP device is visible")
def test_device_calls_fail_cleanly_without_a_device():
    lib = capi.lib()
    assert lib.tcx_hip_init() == capi.TCX_UNAVAILABLE
    s = ctypes.c_void_p()
    assert lib.tcx_hip_stream(ctypes.byref(s)) == capi.TCX_UNAVAILABLE
    code, _, _ = alloc(16)
    assert code == capi.TCX_UNAVAILABLE
    d = capi.gemm_desc(4, 4, 4)
    assert lib.tcx_hip_gemm_f32(None, None, None, ctypes.byref(d), None) == capi.TCX_INVALID_ARGUMENT
    assert lib.tcx_hip_reduce(9, 0, None, None, 1, 1, 1, None, 0, None) == capi.TCX_INVALID_ARGUMENT
    assert lib.tcx_hip_reduce(2, 1, None, None, 1, 1, 1, None, 0, None) == capi.TCX_INVALID_ARGUMENT
    assert "float32" in capi.last_error()


def test_validation_happens_before_device_use():
    # Malformed descriptors are rejected with INVALID_ARGUMENT whether or not
    # a device exists (cf. test_cuda_backend_contract.cpp:416-443).
    lib = capi.lib()
    d = capi.gemm_desc(4, 4, 4)
    d.batch_rank = 9
    assert lib.tcx_hip_gemm_f32(None, None, None, ctypes.byref(d), None) == capi.TCX_INVALID_ARGUMENT
    d = capi.gemm_desc(-1, 4, 4)
    assert lib.tcx_hip_gemm_f32(None, None, None, ctypes.byref(d), None) == capi.TCX_INVALID_ARGUMENT
    d = capi.gemm_desc(4, 4, 4, activation="none")
    d.activation = 7
    assert lib.tcx_hip_gemm_f32(None, None, None, ctypes.byref(d), None) == capi.TCX_INVALID_ARGUMENT
    assert lib.tcx_hip_reduce(1, 0, None, None, 3, 0, 1, None, 0, None) == capi.TCX_INVALID_ARGUMENT
    assert "non-empty" in capi.last_error()
    shape = (ctypes.c_int64 * 9)(*([1] * 9))
    assert lib.tcx_hip_binary(0, 0, None, None, None, 9, shape, shape, shape, None) == \
        capi.TCX_INVALID_ARGUMENT
    assert lib.tcx_hip_binary(3, 1, None, None, None, 1, shape, shape, shape, None) == \
        capi.TCX_INVALID_ARGUMENT
    assert lib.tcx_hip_layernorm_f32(None, None, None, None, 1, 4, 1, ctypes.c_float(-1.0), None) == \
        capi.TCX_INVALID_ARGUMENT


@pytest.mark.skipif(not REFERENCE_CPP.is_dir(), reason="reference sources not mounted")
def test_hip_backend_compiles_against_reference_core_headers():
    """Drop-in conformance: the backend source builds unchanged against the
    reference's cpp/tensorcx/core headers (the repository's own restatement of
    those headers is not on the include path)."""
    src = ROOT / "tensor.cx_amd" / "cpp" / "tensorcx" / "backends" / "hip" / "hip_backend.cpp"
    shadow = ROOT / "tensor.cx_amd" / "_build" / "conformance"
    (shadow / "tensorcx" / "backends" / "hip").mkdir(parents=True, exist_ok=True)
    for name in ("hip_backend.h", "hip_device_interval.h"):
        (shadow / "tensorcx" / "backends" / "hip" / name).write_text((src.parent / name).read_text())
    subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", f"-I{shadow}",
                    f"-I{REFERENCE_CPP}", f"-I{ROOT / 'include'}", str(src)], check=True)


def test_backend_library_has_no_cpu_compute_fallback():
    """The native module links the HIP library and calls no oracle code."""
    core = list((ROOT / "tensor.cx_amd" / "python" / "tensorcx").glob("_core*.so"))
    if not core:
        pytest.fail("tensorcx/_core is not built")
    deps = subprocess.run(["ldd", str(core[0])], capture_output=True, text=True,
                          env={**os.environ, "LD_LIBRARY_PATH": ""}).stdout
    assert "libtensorcx_hip.so" in deps
    assert "oracle" not in deps and "tcxref" not in deps


def test_launch_grids_fit_hip_work_item_count(tmp_path):
    """The grid-stride launchers' grid arithmetic (launch_grid.hpp), compiled
    on the host: no launch exceeds HIP's 32-bit work-item count for item counts
    up to 2^62, and shapes below the cap keep a single pass."""
    src = ROOT / "tests" / "cpp" / "launch_grid_test.cpp"
    exe = tmp_path / "launch_grid_test"
    subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'tensor.cx_amd' / 'csrc'}",
                    "-o", str(exe), str(src)], check=True)
    done = subprocess.run([str(exe)], capture_output=True, text=True)
    assert done.returncode == 0, done.stdout + done.stderr


def test_forked_child_is_refused_before_any_hip_call():
    """A process forked from the one that loaded the library gets
    TCX_UNAVAILABLE from every entry point that reaches the HIP runtime, with
    the reference's message and before any HIP call (cf. the reference's
    cuda_context.cpp:16-20): init, device queries, stream and event calls."""
    lib = capi.lib()
    read_end, write_end = os.pipe()
    pid = os.fork()
    if pid == 0:  # child: report the codes through the pipe, then leave at once
        try:
            os.close(read_end)
            count = ctypes.c_int(-1)
            codes = [lib.tcx_hip_init(), lib.tcx_hip_device_count(ctypes.byref(count)),
                     lib.tcx_hip_stream_synchronize(None), lib.tcx_hip_event_destroy(None)]
            os.write(write_end, (",".join(map(str, codes)) + "|" + capi.last_error()).encode())
        finally:
            os._exit(0)
    os.close(write_end)
    with os.fdopen(read_end) as pipe:
        report = pipe.read()
    os.waitpid(pid, 0)
    codes, message = report.split("|", 1)
    assert [int(c) for c in codes.split(",")] == [capi.TCX_UNAVAILABLE] * 4
    assert message == "HIP requires a fresh process after fork"


def test_device_interval_event_seam(tmp_path):
    """HipBackend's device intervals through their event seam: a scripted
    event API fails at every step in turn (the reference's fake-Events test of
    DeviceTimer, test_cuda_profile.cpp:22-59), checked against the profile
    session's device event and the event bookkeeping."""
    obj = ROOT / "tensor.cx_amd" / "_build" / "cxx_cpp_tensorcx_core_profiling.o"
    assert obj.exists(), "build() compiles the core objects first"
    exe = tmp_path / "device_interval_test"
    subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'tensor.cx_amd' / 'cpp'}",
                    f"-I{ROOT / 'include'}", "-o", str(exe), str(ROOT / "tests" / "cpp" / "device_interval_test.cpp"),
                    str(obj), "-pthread"], check=True)
    done = subprocess.run([str(exe)], capture_output=True, text=True)
    assert done.returncode == 0, done.stdout + done.stderr
