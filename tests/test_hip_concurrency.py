"""Concurrency of the hip device's shared state, and device discovery with the
GPU hidden.

HipBackend::execute runs with the GIL released, so calls from several Python
threads overlap inside the C++ layer, as the reference's concurrency suite
assumes (tests/python/test_concurrency.py:28-80). What those calls share here:

* the per-device static scratch of tcx_hip_reduce_noalloc, which full-tensor
  sums and reductions over a few long rows use when no other call holds it
  (a call that finds it taken runs on a workspace of its own);
* the split-K GEMM workspace and the split-row statistics workspace, taken
  from the calling thread's memory pool when one is entered, else allocated;
* memory_pool scopes entered on several threads at once.

Workers align on a barrier right before their first device call, so the
shared paths are hit under real contention, and joins have a timeout, so a
deadlock fails the test instead of hanging it. Every result must equal the
single-thread result bit for bit (the kernels are deterministic and the
scratch and workspace paths run the same kernels with the same splits).
"""

from __future__ import annotations

import os
import subprocess
import sys
import threading

import numpy as np
import pytest

import oracle
import tensorcx_hip_capi as capi
from conftest import ROOT, gpu_present, require_gpu
from hip_cases import assert_bits

THREADS = 8
ITERATIONS = 4
JOIN_TIMEOUT_SECONDS = 90.0

# Shapes chosen for the shared paths (checked by test_shapes_take_the_shared_paths):
FULL_SUM = (2048, 3072)       # axis=None: one long segmented row, the static scratch
LONG_ROWS = (3, 1 << 20)      # few long rows, segmented: the static scratch
SPLIT_K = (1024, 8192, 1024)  # m, k, n: fewer than 256 128x128 tiles, long K: K split
MIDDLE_AXIS = (2, 65536, 8)   # softmax over axis 1: few columns, long axis: split rows


def _run_in_threads(worker):
    """Runs worker(index, barrier) on THREADS threads and re-raises the first
    failure (reference tests/python/test_concurrency.py:49-80)."""
    barrier = threading.Barrier(THREADS)
    errors = []

    def wrapped(index):
        try:
            worker(index, barrier)
        except Exception as error:  # noqa: BLE001 - re-raised on the main thread
            barrier.abort()
            errors.append((index, error))

    threads = [threading.Thread(target=wrapped, args=(i,), daemon=True) for i in range(THREADS)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=JOIN_TIMEOUT_SECONDS)
    stuck = [t for t in threads if t.is_alive()]
    if stuck:
        raise AssertionError(f"{len(stuck)} worker thread(s) did not finish within "
                             f"{JOIN_TIMEOUT_SECONDS}s: possible deadlock in the native layer")
    if errors:
        index, error = errors[0]
        raise AssertionError(f"worker thread {index} failed: {error!r}") from error


def test_shapes_take_the_shared_paths():
    """The shapes above reach the scratch and workspace paths (host-side
    workspace queries, no device needed)."""
    lib = capi.lib()
    f32 = 0
    assert 0 < lib.tcx_hip_reduce_workspace_bytes(capi.REDUCE["sum"], f32, 1, FULL_SUM[0] * FULL_SUM[1], 1) \
        <= capi.REDUCE_NOALLOC_MAX_WORKSPACE
    assert 0 < lib.tcx_hip_reduce_workspace_bytes(capi.REDUCE["max"], f32, LONG_ROWS[0], LONG_ROWS[1], 1) \
        <= capi.REDUCE_NOALLOC_MAX_WORKSPACE
    m, k, n = SPLIT_K
    assert lib.tcx_hip_gemm_workspace_bytes(capi.gemm_desc(m, n, k)) > 0
    assert lib.tcx_hip_rownorm_workspace_bytes(*MIDDLE_AXIS) > 0


def _hidden_device_child(env_overrides):
    env = {**os.environ, **env_overrides}
    code = """
import sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import tensorcx as cx
import tensorcx_hip_capi as capi
assert not capi.available(), 'a HIP device is still visible'
assert not cx.is_available('hip')
assert cx.devices() == ['cpu'], cx.devices()
assert cx.ones((3,)).numpy().tolist() == [1, 1, 1]
assert cx.tensor([1.0, 2.0]).device == 'cpu'
for make in (lambda: cx.ones((1,), device='hip'), lambda: cx.tensor([1.0], device='hip'),
             lambda: cx.zeros((2,), device='hip'), lambda: cx.ones((1,)).to('hip')):
    try:
        make()
    except ValueError as error:
        assert 'device is not available: hip' in str(error), str(error)
    else:
        raise AssertionError('an unavailable hip device was accepted')
print('hidden-device child ok')
"""
    result = subprocess.run([sys.executable, "-c", code, str(ROOT), str(ROOT / "tensor.cx_amd" / "python")],
                            env=env, capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "hidden-device child ok" in result.stdout


@pytest.mark.skipif(gpu_present(), reason="a HIP device is visible (the gpu suite hides it instead)")
def test_no_device_discovery_keeps_cpu():
    """Reference tests/python/test_cuda.py:13-31 on a host without a GPU."""
    _hidden_device_child({})


@pytest.mark.gpu
def test_hidden_device_discovery_keeps_cpu():
    """Reference tests/python/test_cuda.py:13-31 on the GPU host: a fresh
    process with the device hidden drops hip from devices() and refuses hip
    placement with ValueError, while the CPU keeps working."""
    require_gpu()
    # An invalid ordinal hides every device from the HIP runtime (an empty
    # HIP_VISIBLE_DEVICES means "no restriction" to it).
    _hidden_device_child({"HIP_VISIBLE_DEVICES": "-1", "ROCR_VISIBLE_DEVICES": "-1"})


# ------------------------------------------------------------------ GPU side
@pytest.fixture(scope="module")
def cx():
    require_gpu()
    import tensorcx
    return tensorcx


def _inputs(index):
    rng = np.random.default_rng(100 + index)
    m, k, n = SPLIT_K
    return {
        "full": rng.standard_normal(FULL_SUM).astype(np.float32),
        "rows": rng.standard_normal(LONG_ROWS).astype(np.float32),
        "a": rng.standard_normal((m, k)).astype(np.float32),
        "b": rng.standard_normal((k, n)).astype(np.float32),
        "mid": (3.0 * rng.standard_normal(MIDDLE_AXIS)).astype(np.float32),
    }


def _work(cx, t):
    """The shared-state calls of one iteration, on device tensors t."""
    return {
        "full": cx.sum(t["full"]).numpy(),
        "mean": cx.mean(t["full"]).numpy(),
        "rows": cx.max(t["rows"], axis=-1).numpy(),
        "rowsum": cx.sum(t["rows"], axis=1).numpy(),
        "gemm": cx.matmul(t["a"], t["b"]).numpy(),
        "mid": cx.softmax(t["mid"], 1).numpy(),
        "midln": cx.layernorm(t["mid"], 1).numpy(),
    }


@pytest.mark.gpu
def test_barrier_aligned_shared_state(cx):
    inputs = [_inputs(i) for i in range(THREADS)]
    device = [{k: cx.tensor(v, device="hip") for k, v in inp.items()} for inp in inputs]
    # Single-thread results first: the bits every concurrent call must give.
    expected = [_work(cx, t) for t in device]

    def worker(index, barrier):
        t = device[index]
        barrier.wait()
        for it in range(ITERATIONS):
            if (it + index) % 2 == 0:
                with cx.memory_pool("hip", max_cached_bytes=256 << 20):
                    got = _work(cx, t)
            else:
                got = _work(cx, t)
            for name, value in got.items():
                assert_bits(value, expected[index][name], f"thread {index} iteration {it} {name}")

    _run_in_threads(worker)


@pytest.mark.gpu
def test_barrier_aligned_first_wide_rows(cx):
    """Each worker's first device calls are rows held in registers plus LDS,
    on both wide routes (two 512-thread blocks per CU at 50257 floats, 1024
    threads at 100003): every thread sets those kernels' LDS limit on its
    first call and launches them at once. Results equal the single-thread
    bits."""
    rng = np.random.default_rng(23)
    shapes = ((16, 50257), (16, 100003))
    xs = [(2.0 * rng.standard_normal(sh)).astype(np.float32) for sh in shapes]
    gs = [rng.uniform(0.5, 1.5, sh[1]).astype(np.float32) for sh in shapes]
    bs = [rng.uniform(-0.1, 0.1, sh[1]).astype(np.float32) for sh in shapes]
    device = [(cx.tensor(x, device="hip"), cx.tensor(g, device="hip"), cx.tensor(b, device="hip"))
              for x, g, b in zip(xs, gs, bs)]

    def work():
        out = {}
        for i, (x, g, b) in enumerate(device):
            out[f"softmax {i}"] = cx.softmax(x, 1).numpy()
            out[f"rmsnorm {i}"] = cx.rmsnorm(x, 1, weight=g).numpy()
            out[f"layernorm {i}"] = cx.layernorm(x, 1, weight=g, bias=b).numpy()
        return out

    expected = work()

    def worker(index, barrier):
        barrier.wait()
        for it in range(ITERATIONS):
            for name, value in work().items():
                assert_bits(value, expected[name], f"thread {index} iteration {it} {name}")

    _run_in_threads(worker)


@pytest.mark.gpu
def test_barrier_aligned_pool_scopes(cx):
    """Pools entered on every thread at once, each serving its own thread's
    output and workspace allocations, then trimmed and closed."""
    inputs = [_inputs(i) for i in range(THREADS)]
    device = [{k: cx.tensor(v, device="hip") for k, v in inp.items() if k in ("a", "b", "full")}
              for inp in inputs]
    expected = [(cx.matmul(t["a"], t["b"]).numpy(), cx.sum(t["full"]).numpy()) for t in device]

    def worker(index, barrier):
        t = device[index]
        with cx.memory_pool("hip", max_cached_bytes=128 << 20, max_cached_blocks=4) as pool:
            barrier.wait()
            for it in range(ITERATIONS):
                c = cx.matmul(t["a"], t["b"])
                s = cx.sum(t["full"])
                assert_bits(c.numpy(), expected[index][0], f"thread {index} iteration {it} gemm")
                assert_bits(s.numpy(), expected[index][1], f"thread {index} iteration {it} sum")
                del c, s
            stats = pool.stats()
            assert stats["hits"] > 0, stats
            pool.trim()

    _run_in_threads(worker)


@pytest.mark.gpu
def test_concurrent_inference_chain(cx):
    """Reference tests/python/test_cuda_primitives.py:90-101 with the same
    chain of primitives, four workers, twelve calls."""
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(19)
    x = rng.normal(size=(7, 17)).astype(np.float32)
    w1 = rng.normal(size=(17, 31)).astype(np.float32)
    w2 = rng.normal(size=(31, 5)).astype(np.float32)

    def forward(a, b, c):
        return cx.softmax(cx.matmul(cx.gelu(cx.layernorm(cx.matmul(a, b), axis=-1)), c), axis=-1)

    gx, g1, g2 = (cx.tensor(v, device="hip") for v in (x, w1, w2))
    expected = forward(gx, g1, g2).numpy()
    reference = oracle.softmax(oracle.matmul(oracle.gelu(oracle.layernorm(oracle.matmul(x, w1), -1)), w2), -1)
    np.testing.assert_allclose(expected, reference, rtol=1e-4, atol=1e-5)
    with ThreadPoolExecutor(max_workers=4) as pool:
        futures = [pool.submit(forward, gx, g1, g2) for _ in range(12)]
        for f in futures:
            assert_bits(f.result().numpy(), expected, "threaded inference chain")
