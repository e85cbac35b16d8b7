"""Benchmark of the hip hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME]

Headline (the JSON `value`): fp32 matmul TFLOP/s at 4096^3 (config C2, the
second entry of BASELINE.json's configs), inputs resident in HBM. Every line
is timed the same way on this thread's HIP stream: W warm-up launches, then
more untimed launches until 20 ms of GPU time has passed (the clock ramps up
under sustained load), then K launches between two HIP events (the average,
which the roofline uses) and K more with an event pair around each launch
(the median). Operands rotate through enough copies that no launch finds its
inputs in the 256 MB Infinity Cache from an earlier one.

The JSON line carries `roofline` for the headline kernel, `cpu_baseline` (the
oracle's single-thread restatement of the reference CPU matmul on a bounded
row slab, extrapolated), and `secondary`: the other configs' kernels
(batched/edge GEMM, reductions, softmax/norms, MLP, fused attention), each as
GB/s or TFLOP/s with its roofline fraction and its own single-thread CPU
baseline on a bounded sample of the same workload.

Peaks: fp32 MFMA 157.3 TFLOP/s, HBM 8.0 TB/s (MI355X published figures).
"""

from __future__ import annotations

import argparse
import contextlib
import json
import os
import pathlib
import statistics
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tensor.cx_amd" / "python"))
sys.path.insert(0, str(ROOT))

import tensorcx_hip_capi as capi  # noqa: E402
import tensorcx_workloads as wl  # noqa: E402

PEAK_FP32_MFMA = 157.3e12
PEAK_HBM = 8.0e12
PROFILES = ROOT / "profiles"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# Every line warms up for at least this much GPU time: the GPU clock ramps up
# over the first milliseconds of sustained load, and each line starts after
# host-side input generation has let it idle. A 4096x4096x1024 GEMM measured
# 283 us after 3 warm-up launches and 256 us after 300.
WARM_MS = 20.0
# Operand copies rotate until they exceed the 256 MB Infinity Cache.
ROTATE_BYTES = 320 * 1024 * 1024
# The per-launch median is taken over at least this many launches.
MEDIAN_REPS = 31


def _roctx():
    """The ROCTx library of rocprofiler-sdk, if present: every bench line runs
    inside a range named for it, so that a `rocprofv3 --kernel-trace
    --marker-trace` run attributes each dispatch to its line. Outside a
    profiler the ranges cost a call each and record nothing."""
    import ctypes
    for name in ("librocprofiler-sdk-roctx.so.1", "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1"):
        try:
            lib = ctypes.CDLL(name)
        except OSError:
            continue
        lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
        return lib
    return None


ROCTX = _roctx()


@contextlib.contextmanager
def marked(name: str):
    if ROCTX is not None:
        ROCTX.roctxRangePushA(name.encode())
    try:
        yield
    finally:
        if ROCTX is not None:
            ROCTX.roctxRangePop()


def timed(launch, steps: int, warmup: int, warm_ms: float = WARM_MS, name: str = "launches"):
    """Runs `launch` warmup times, then (untimed) until warm_ms of GPU time has
    passed; then K = steps launches between two HIP events on the launch
    stream (total), then max(K, MEDIAN_REPS) more with an event pair around
    each (per launch). The timed launches, not the warm-up, run inside a
    ROCTx range called name, so a kernel trace's per-line average covers the
    launches the HIP events time (warm-up launches at a rising clock had
    lifted it 3 % above them at 4096^3).
    The stream is idle on both sides of each pass. Returns (total_ms,
    per_launch_ms list, warm-up launches)."""
    return _timed(launch, steps, warmup, warm_ms, name)


def _timed(launch, steps: int, warmup: int, warm_ms: float, name: str):
    s = capi.stream()
    launches = 0
    for _ in range(warmup):
        launch(s)
        launches += 1
    if warm_ms > 0:
        begin, now = capi.Event(), capi.Event()
        begin.record(s)
        while launches < 20000:
            for _ in range(8):
                launch(s)
            launches += 8
            now.record(s)
            now.synchronize()
            if begin.elapsed_ms(now) >= warm_ms:
                break
    capi.synchronize()
    with marked(name):
        start, stop = capi.Event(), capi.Event()
        start.record(s)
        for _ in range(steps):
            launch(s)
        stop.record(s)
        stop.synchronize()
        total = start.elapsed_ms(stop)
        reps = max(steps, MEDIAN_REPS)
        marks = [capi.Event() for _ in range(reps + 1)]
        marks[0].record(s)
        for i in range(reps):
            launch(s)
            marks[i + 1].record(s)
        marks[-1].synchronize()
        capi.synchronize()
    per = [marks[i].elapsed_ms(marks[i + 1]) for i in range(reps)]
    return total, per, launches


def rotate(copies):
    """Cycles through input copies, one per call."""
    state = {"i": 0}

    def nxt():
        state["i"] = (state["i"] + 1) % len(copies)
        return copies[state["i"]]
    return nxt


def copies_for(nbytes: int, cap: int = 160) -> int:
    """Copies of an nbytes operand set that together exceed ROTATE_BYTES."""
    return int(min(cap, max(2, -(-ROTATE_BYTES // max(nbytes, 1)))))


def bench_gemm(name: str, steps: int, warmup: int):
    a, b = wl.gemm_inputs(name)
    sets = [(capi.DeviceArray.from_numpy(a), capi.DeviceArray.from_numpy(b))
            for _ in range(copies_for(a.nbytes + b.nbytes))]
    if a.ndim == 3:
        batch = a.shape[0]
        m, k, n = a.shape[1], a.shape[2], b.shape[2]
        desc = capi.gemm_desc(m, n, k, batch_shape=(batch,), lhs_batch_strides=(m * k,),
                              rhs_batch_strides=(k * n,))
        out = capi.DeviceArray((batch, m, n))
    else:
        m, k, n = a.shape[0], a.shape[1], b.shape[1]
        desc = capi.gemm_desc(m, n, k)
        out = capi.DeviceArray((m, n))
    ws = capi.gemm_workspace(desc)  # None unless the shape runs with K split
    nxt = rotate(sets)

    def launch(s):
        da, db = nxt()
        capi.gemm(da.ptr, db.ptr, out.ptr, desc, s, ws)

    total, per, warm = timed(launch, steps, warmup, name=f"gemm_{name}")
    flops = wl.gemm_flops(name)
    avg = total / steps
    return {"name": f"gemm_{name}", "unit": "TFLOP/s", "value": flops / (avg * 1e-3) / 1e12,
            "kernel_avg_ms": avg, "kernel_median_ms": statistics.median(per),
            "achieved": flops / (avg * 1e-3) / 1e12, "peak": PEAK_FP32_MFMA / 1e12,
            "frac": flops / (avg * 1e-3) / PEAK_FP32_MFMA, "flop_per_launch": flops,
            "ms_per_step": avg, "operand_copies": len(sets), "warmup_launches": warm}


def api_wall(steps: int, warmup: int) -> dict:
    """Wall time of tensorcx.matmul at 4096^3 through the whole drop-in path
    (Python binding, HipBackend::execute, an output allocation from a
    memory_pool scope, the kernel, the stream synchronisation that makes the
    call complete on return), per call, after warm-up calls."""
    import tensorcx as cx
    a, b = wl.gemm_inputs("c2_4096")
    ta, tb = cx.tensor(a, device="hip"), cx.tensor(b, device="hip")
    calls = max(steps, MEDIAN_REPS)
    with cx.memory_pool("hip", max_cached_bytes=256 << 20):
        for _ in range(max(warmup, 5)):
            out = cx.matmul(ta, tb)
        times = []
        for _ in range(calls):
            t = time.perf_counter()
            out = cx.matmul(ta, tb)
            times.append(time.perf_counter() - t)
        del out
    return {"path": "tensorcx.matmul -> HipBackend::execute (pooled output, synchronous)",
            "calls": calls, "ms_per_call_median": statistics.median(times) * 1e3,
            "ms_per_call_mean": statistics.mean(times) * 1e3}


def bench_hbm(name: str, launch_for, nbytes: int, steps: int, warmup: int):
    total, per, warm = timed(launch_for, steps, warmup, name=name)
    avg = total / steps
    return {"name": name, "unit": "GB/s", "value": nbytes / (avg * 1e-3) / 1e9,
            "kernel_avg_ms": avg, "kernel_median_ms": statistics.median(per),
            "achieved": nbytes / (avg * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9,
            "frac": nbytes / (avg * 1e-3) / PEAK_HBM, "bytes_per_launch": nbytes, "warmup_launches": warm}


# ---------------------------------------------------------------- CPU baselines
# The oracle restates the reference CPU path loop for loop (bit-identical, see
# oracle/__init__.py); here it runs on one thread, as the reference's CPU
# backend does, on a bounded sample of each workload, and the rate is
# extrapolated to the whole workload.
CPU_LINE_SECONDS = 1.0


def host_cpu() -> str:
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_sample(run_rows, total_rows: int, budget_s: float):
    """Times run_rows(r) on growing row counts until one run takes a quarter
    of budget_s, then on the row count expected to take about budget_s (so a
    fixed per-call cost does not dominate the sample). Returns (rows, s)."""
    rows = 1
    while True:
        t = time.perf_counter()
        run_rows(rows)
        dt = time.perf_counter() - t
        if dt >= budget_s / 4 or rows >= total_rows:
            break
        rows = min(total_rows, rows * 4)
    target = int(min(total_rows, max(rows, rows * budget_s / max(dt, 1e-9))))
    if target != rows:
        rows = target
        t = time.perf_counter()
        run_rows(rows)
        dt = time.perf_counter() - t
    return rows, dt


def cpu_line(run_rows, total_rows: int, work: float, unit: str, scale: float, what: str,
             budget_s: float = CPU_LINE_SECONDS) -> dict:
    """The single-thread oracle rate for a workload of `work` units (FLOP or
    bytes, `scale` per reported unit) spread evenly over total_rows rows."""
    rows, dt = cpu_sample(run_rows, total_rows, budget_s)
    full = dt * total_rows / rows
    return {"value": work / full / scale, "unit": unit, "cores": 1, "kind": "port",
            "sample": f"{what}: rows 0..{rows} of {total_rows}, {dt:.2f} s on one thread, "
                      f"extrapolated to {full:.1f} s for the whole workload"}


def naive_matmul_rows(a2: np.ndarray, b2: np.ndarray):
    """rows -> the oracle's cpu::matmul loop over the first `rows` rows of a2 @ b2."""
    import ctypes

    import oracle
    m, k = a2.shape
    n = b2.shape[1]
    out = np.empty((m, n), np.float32)

    def run(rows):
        oracle.lib().oracle_matmul_f32_naive(
            ctypes.c_void_p(a2.ctypes.data), ctypes.c_void_p(b2.ctypes.data), ctypes.c_void_p(out.ctypes.data),
            ctypes.c_int64(m), ctypes.c_int64(n), ctypes.c_int64(k), ctypes.c_int64(0), ctypes.c_int64(rows))
    return run


def cpu_gemm(name: str, budget_s: float = CPU_LINE_SECONDS) -> dict:
    a, b = wl.gemm_inputs(name)
    a2, b2 = (a[0], b[0]) if a.ndim == 3 else (a, b)
    batches = a.shape[0] if a.ndim == 3 else 1
    return cpu_line(naive_matmul_rows(np.ascontiguousarray(a2), np.ascontiguousarray(b2)), batches * a2.shape[0],
                    wl.gemm_flops(name), "TFLOP/s", 1e12, f"cpu::matmul loop, {'x'.join(map(str, a.shape))} operand",
                    budget_s)


def secondary_benches(steps: int, warmup: int, only: str | None, cpu: bool):
    import oracle
    out = []

    def want(n):
        return only is None or only in n

    def add(line, cpu_leg=None):
        if cpu and cpu_leg is not None:
            line["cpu_baseline"] = cpu_leg()
        out.append(line)
        unit = line["unit"]
        fmt = f"{line['achieved']:.1f} {unit}" if unit == "TFLOP/s" else f"{line['achieved']:.0f} {unit}"
        log(f"{line['name']}: {fmt} ({line['frac']:.1%})"
            + (f", cpu {line['cpu_baseline']['value']:.3g} {line['cpu_baseline']['unit']}" if "cpu_baseline" in line else ""))

    for name in ("c2_batched", "c2_edge", "c1_512"):
        if want(name):
            add(bench_gemm(name, steps, warmup), lambda name=name: cpu_gemm(name))

    if want("reduce") or want("sum") or want("max") or want("argmax"):
        x = wl.reduce_f32_input()
        copies = [capi.DeviceArray.from_numpy(x) for _ in range(2)]
        rows, cols = 8192, 8192
        res = capi.DeviceArray((rows,), np.float32)
        nbytes = rows * cols * 4 + rows * 4
        for op in ("sum", "max", "mean", "min", "argmax"):
            nxt = rotate(copies)
            fn = getattr(oracle, op)
            add(bench_hbm(f"reduce_{op}_f32_8192x8192", lambda s, op=op: capi.reduce(
                op, capi.TCX_FLOAT32, nxt().ptr, res.ptr, rows, cols, 1, None, s), nbytes, steps, warmup),
                lambda fn=fn, op=op: cpu_line(lambda r: fn(x[:r], -1, threads=1), rows, nbytes, "GB/s", 1e9,
                                              f"{op} over the last axis of [8192, 8192]"))
        full = capi.DeviceArray((1,), np.float32)
        flat = x.reshape(-1)
        full_cpu = (lambda: cpu_line(lambda r: oracle.sum(flat[:r * cols], 0, threads=1), rows, rows * cols * 4 + 4,
                                     "GB/s", 1e9, "sequential sum of the flattened [8192, 8192]"))
        nxt = rotate(copies)
        # The backend's call: segment partials in the library's static
        # scratch, then the combine launch (two kernels, no allocation).
        add(bench_hbm("reduce_full_sum_f32_8192x8192", lambda s: capi.reduce_noalloc(
            "sum", capi.TCX_FLOAT32, nxt().ptr, full.ptr, 1, rows * cols, 1, s), rows * cols * 4 + 4, steps, warmup),
            full_cpu)
        # Over the first axis (a strided reduction: 32 column tiles x 16 row
        # splits, the split partials in the static scratch).
        for op in ("sum", "max"):
            nxt = rotate(copies)
            fn = getattr(oracle, op)
            add(bench_hbm(f"reduce_col{op}_f32_8192x8192", lambda s, op=op: capi.reduce_noalloc(
                op, capi.TCX_FLOAT32, nxt().ptr, res.ptr, 1, rows, cols, s), nbytes, steps, warmup),
                lambda fn=fn, op=op: cpu_line(lambda r: fn(x[:r], 0, threads=1), rows, nbytes, "GB/s", 1e9,
                                              f"{op} over the first axis of [8192, 8192] (a sample of its rows)"))
        del copies, x, flat

    if want("i32"):
        xi = wl.reduce_i32_input()
        copies = [capi.DeviceArray.from_numpy(xi)]
        rows, cols = 65536, 4096
        res = capi.DeviceArray((rows,), np.int32)
        nbytes = rows * cols * 4 + rows * 4
        for op in ("sum", "max"):
            fn = getattr(oracle, op)
            add(bench_hbm(f"reduce_{op}_i32_65536x4096", lambda s, op=op: capi.reduce(
                op, capi.TCX_INT32, copies[0].ptr, res.ptr, rows, cols, 1, None, s), nbytes, steps, warmup),
                lambda fn=fn, op=op: cpu_line(lambda r: fn(xi[:r], -1, threads=1), rows, nbytes, "GB/s", 1e9,
                                              f"int32 {op} over the last axis of [65536, 4096]"))
        del copies, xi

    if want("softmax") or want("norm"):
        x, g, b = wl.rownorm_inputs()
        copies = [capi.DeviceArray.from_numpy(x) for _ in range(2)]
        gd, bd = capi.DeviceArray.from_numpy(g), capi.DeviceArray.from_numpy(b)
        rows, cols = 16384, 4096
        y = capi.DeviceArray((rows, cols))
        nbytes = 2 * rows * cols * 4
        nxt = rotate(copies)
        add(bench_hbm("softmax_16384x4096", lambda s: capi.softmax(nxt().ptr, y.ptr, rows, cols, 1, s),
                      nbytes, steps, warmup),
            lambda: cpu_line(lambda r: oracle.softmax(x[:r], -1, threads=1), rows, nbytes, "GB/s", 1e9,
                             "softmax over the last axis of [16384, 4096]"))
        add(bench_hbm("rmsnorm_16384x4096", lambda s: capi.rmsnorm(
            nxt().ptr, None, y.ptr, rows, cols, 1, 1e-5, s), nbytes, steps, warmup),
            lambda: cpu_line(lambda r: oracle.rmsnorm(x[:r], -1, 1e-5, threads=1), rows, nbytes, "GB/s", 1e9,
                             "rmsnorm over the last axis of [16384, 4096]"))
        add(bench_hbm("layernorm_affine_16384x4096", lambda s: capi.layernorm(
            nxt().ptr, gd.ptr, bd.ptr, y.ptr, rows, cols, 1, 1e-5, s), nbytes + 2 * cols * 4, steps, warmup),
            lambda: cpu_line(lambda r: oracle.affine_norm(x[:r], -1, 1e-5, g, b, rms=False, threads=1), rows,
                             nbytes + 2 * cols * 4, "GB/s", 1e9,
                             "layernorm then weight then bias (the affine composite) over [16384, 4096]"))
        del copies, x

    # Rows as wide as a vocabulary: one block per row holds the whole row in
    # registers and LDS ([512, 128256]), or stages it in LDS ([4096, 32000]).
    for rows, cols, ops in ((512, 128256, ("softmax", "rmsnorm", "layernorm_affine")), (4096, 32000, ("softmax",))):
        if not any(want(f"{op}_{rows}x{cols}") for op in ops):
            continue
        x, g, b = wl.long_row_inputs(rows, cols)
        copies = [capi.DeviceArray.from_numpy(x) for _ in range(2)]
        gd, bd = capi.DeviceArray.from_numpy(g), capi.DeviceArray.from_numpy(b)
        y = capi.DeviceArray((rows, cols))
        nbytes = 2 * rows * cols * 4
        nxt = rotate(copies)
        shape = f"[{rows}, {cols}]"
        launches = {
            "softmax": (lambda s: capi.softmax(nxt().ptr, y.ptr, rows, cols, 1, s), nbytes,
                        lambda r: oracle.softmax(x[:r], -1, threads=1), f"softmax over the last axis of {shape}"),
            "rmsnorm": (lambda s: capi.rmsnorm(nxt().ptr, None, y.ptr, rows, cols, 1, 1e-5, s), nbytes,
                        lambda r: oracle.rmsnorm(x[:r], -1, 1e-5, threads=1), f"rmsnorm over the last axis of {shape}"),
            "layernorm_affine": (
                lambda s: capi.layernorm(nxt().ptr, gd.ptr, bd.ptr, y.ptr, rows, cols, 1, 1e-5, s), nbytes + 2 * cols * 4,
                lambda r: oracle.affine_norm(x[:r], -1, 1e-5, g, b, rms=False, threads=1),
                f"layernorm then weight then bias (the affine composite) over {shape}"),
        }
        for op in ops:
            if not want(f"{op}_{rows}x{cols}"):
                continue
            launch, nb, cpu_rows, what = launches[op]
            add(bench_hbm(f"{op}_{rows}x{cols}", launch, nb, steps, warmup),
                lambda cpu_rows=cpu_rows, nb=nb, what=what: cpu_line(cpu_rows, rows, nb, "GB/s", 1e9, what))
        del copies, x

    if want("mlp"):
        x, w1, b1, w2, b2 = wl.mlp_inputs()
        dx, dw1, db1, dw2, db2 = (capi.DeviceArray.from_numpy(v) for v in (x, w1, b1, w2, b2))
        h = capi.DeviceArray((4096, 4096))
        logits = capi.DeviceArray((4096, 1024))
        prob = capi.DeviceArray((4096, 1024))
        d1 = capi.gemm_desc(4096, 4096, 1024, rhs_transposed=True, bias=db1.ptr, activation="silu")
        d2 = capi.gemm_desc(4096, 1024, 4096, rhs_transposed=True, bias=db2.ptr)
        ws1, ws2 = capi.gemm_workspace(d1), capi.gemm_workspace(d2)

        def mlp(s):
            capi.gemm(dx.ptr, dw1.ptr, h.ptr, d1, s, ws1)
            capi.gemm(h.ptr, dw2.ptr, logits.ptr, d2, s, ws2)
            capi.softmax(logits.ptr, prob.ptr, 4096, 1024, 1, s)

        total, per, warm = timed(mlp, steps, warmup, name="mlp_forward_4096x1024x4096")
        flops = 2 * 2 * 4096 * 4096 * 1024
        avg = total / steps
        add({"name": "mlp_forward_4096x1024x4096", "unit": "TFLOP/s", "value": flops / (avg * 1e-3) / 1e12,
             "step_avg_ms": avg, "step_median_ms": statistics.median(per),
             "achieved": flops / (avg * 1e-3) / 1e12, "peak": PEAK_FP32_MFMA / 1e12,
             "frac": flops / (avg * 1e-3) / PEAK_FP32_MFMA, "tokens_per_s": 4096 / (avg * 1e-3),
             "warmup_launches": warm},
            lambda: cpu_line(lambda r: oracle.mlp_forward(x[:r], w1, b1, w2, b2, threads=1), 4096, flops, "TFLOP/s",
                             1e12, "linear, silu, linear, softmax composites (two weight transposes per call)",
                             budget_s=2.0))

    if want("attention"):
        q, k, v = wl.attention_inputs()
        bh, seq, d = q.shape
        dq, dk, dv = (capi.DeviceArray.from_numpy(t) for t in (q, k, v))
        o = capi.DeviceArray((bh, seq, d))
        for causal in (False, True):
            flops = wl.attention_flops(causal)
            total, per, warm = timed(lambda s, c=causal: capi.flash_attention(
                dq.ptr, dk.ptr, dv.ptr, o.ptr, bh, seq, seq, d, 1.0 / np.sqrt(d), c, s), steps, warmup,
                name=f"attention_fused_{bh}x{seq}x{d}" + ("_causal" if causal else ""))
            avg = total / steps
            # The reference composite computes every score and masks it, so
            # its time does not shrink with the causal mask; the rate counts
            # the kept pairs like the GPU line.
            add({"name": f"attention_fused_{bh}x{seq}x{d}" + ("_causal" if causal else ""),
                 "unit": "TFLOP/s", "value": flops / (avg * 1e-3) / 1e12,
                 "kernel_avg_ms": avg, "kernel_median_ms": statistics.median(per),
                 "achieved": flops / (avg * 1e-3) / 1e12, "peak": PEAK_FP32_MFMA / 1e12,
                 "frac": flops / (avg * 1e-3) / PEAK_FP32_MFMA, "flop_per_launch": flops, "warmup_launches": warm},
                lambda c=causal, flops=flops: cpu_line(
                    lambda r: oracle.attention(q[:1, :r], k[:1], v[:1], None, c, None, threads=1), bh * seq, flops,
                    "TFLOP/s", 1e12, "attention composite (transpose, matmul, softmax, matmul) of one head's queries"))
    return out


def extra_benches(steps: int, warmup: int):
    """Shapes off the bench lines that route to other kernels (rows that are
    short, unaligned, staged in LDS or resident in registers; the matrix-vector,
    streaming, vector-matrix, short-K and tiny-item GEMM routes), timed like
    the secondary lines against HBM (algorithmic bytes: each input read once
    plus the output), and the 32x64-tile GEMM against the fp32 MFMA peak, for
    the kernel traces of the profiles. No CPU legs."""
    out = []
    rng = np.random.default_rng(13)

    def operands(*shapes):
        arrays = [rng.standard_normal(sh, dtype=np.float32) for sh in shapes]
        nbytes = sum(a.nbytes for a in arrays)
        sets = [[capi.DeviceArray.from_numpy(a) for a in arrays] for _ in range(copies_for(nbytes))]
        return rotate(sets), nbytes

    def add(name, launch, nbytes):
        line = bench_hbm(name, launch, nbytes, steps, warmup)
        out.append(line)
        log(f"{name}: {line['achieved']:.0f} GB/s ({line['frac']:.1%})")

    for rows, cols in ((100000, 130), (16384, 1023), (8192, 8191)):
        nxt, nbytes = operands((rows, cols))
        res = capi.DeviceArray((rows,), np.float32)
        for op in ("sum", "max"):
            add(f"reduce_{op}_f32_{rows}x{cols}", lambda s, op=op, rows=rows, cols=cols, nxt=nxt, res=res: capi.reduce(
                op, capi.TCX_FLOAT32, nxt()[0].ptr, res.ptr, rows, cols, 1, None, s), nbytes + rows * 4)
    for rows, cols in ((8192, 8191), (4096, 20001), (1000, 100003), (100000, 130), (8192, 1500), (2048, 50257)):
        nxt, nbytes = operands((rows, cols))
        g = capi.DeviceArray.from_numpy(rng.uniform(0.5, 1.5, cols).astype(np.float32))
        b = capi.DeviceArray.from_numpy(rng.uniform(-0.1, 0.1, cols).astype(np.float32))
        y = capi.DeviceArray((rows, cols))
        add(f"softmax_{rows}x{cols}", lambda s, rows=rows, cols=cols, nxt=nxt, y=y: capi.softmax(
            nxt()[0].ptr, y.ptr, rows, cols, 1, s), 2 * nbytes)
        add(f"layernorm_affine_{rows}x{cols}", lambda s, rows=rows, cols=cols, nxt=nxt, y=y, g=g, b=b: capi.layernorm(
            nxt()[0].ptr, g.ptr, b.ptr, y.ptr, rows, cols, 1, 1e-5, s), 2 * nbytes + 2 * cols * 4)
    # RMSNorm with a weight on rows held at 20 float4 per thread (the
    # two-phase weighted write).
    rows, cols = 4096, 32000
    nxt, nbytes = operands((rows, cols))
    g = capi.DeviceArray.from_numpy(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    y = capi.DeviceArray((rows, cols))
    add(f"rmsnorm_weight_{rows}x{cols}", lambda s, rows=rows, cols=cols, nxt=nxt, y=y, g=g: capi.rmsnorm(
        nxt()[0].ptr, g.ptr, y.ptr, rows, cols, 1, 1e-5, s), 2 * nbytes + cols * 4)
    # GEMM routes: (name, m, n, k, batch, B transposed)
    for name, m, n, k, batch, trans in (("gemv_1x4096x4096_linear", 1, 4096, 4096, 1, True),
                                        ("stream_16x4096x4096_linear", 16, 4096, 4096, 1, True),
                                        ("vecmat_16x1x4096x4096", 1, 4096, 4096, 16, False),
                                        ("smallk_4096x4096x4", 4096, 4096, 4, 1, False),
                                        ("tiny_65536x8x8x8", 8, 8, 8, 65536, False)):
        a_shape = (batch, m, k) if batch > 1 else (m, k)
        b_shape = ((batch,) if batch > 1 else ()) + ((n, k) if trans else (k, n))
        nxt, nbytes = operands(a_shape, b_shape)
        desc = capi.gemm_desc(m, n, k, batch_shape=(batch,) if batch > 1 else (),
                              lhs_batch_strides=(m * k,) if batch > 1 else (),
                              rhs_batch_strides=(k * n,) if batch > 1 else (), rhs_transposed=trans)
        c = capi.DeviceArray((batch * m, n))
        ws = capi.gemm_workspace(desc)

        def launch(s, nxt=nxt, c=c, desc=desc, ws=ws):
            da, db = nxt()
            capi.gemm(da.ptr, db.ptr, c.ptr, desc, s, ws)
        add(f"gemm_{name}", launch, nbytes + batch * m * n * 4)
    # The 32x64-tile route (more than 256 tiles of 64x64 whose last round
    # holds at most 128): 1100^3, 324 such tiles, rated in TFLOP/s.
    m = n = k = 1100
    nxt, _ = operands((m, k), (k, n))
    desc = capi.gemm_desc(m, n, k)
    c = capi.DeviceArray((m, n))

    def launch_half(s, nxt=nxt, c=c, desc=desc):
        da, db = nxt()
        capi.gemm(da.ptr, db.ptr, c.ptr, desc, s)
    name = "gemm_half_1100x1100x1100"
    total, per, warm = timed(launch_half, steps, warmup, name=name)
    avg, flops = total / steps, 2 * m * n * k
    out.append({"name": name, "unit": "TFLOP/s", "value": flops / (avg * 1e-3) / 1e12, "kernel_avg_ms": avg,
                "kernel_median_ms": statistics.median(per), "achieved": flops / (avg * 1e-3) / 1e12,
                "peak": PEAK_FP32_MFMA / 1e12, "frac": flops / (avg * 1e-3) / PEAK_FP32_MFMA,
                "flop_per_launch": flops, "warmup_launches": warm})
    log(f"{name}: {out[-1]['achieved']:.1f} TFLOP/s ({out[-1]['frac']:.1%})")
    return out


def cpu_baseline(budget_s: float) -> dict:
    """The headline's CPU leg: the oracle's cpu::matmul loop (bit-identical
    restatement of the reference's, single thread) on a bounded row slab of
    the 4096^3 product, extrapolated."""
    line = cpu_gemm("c2_4096", budget_s)
    line["host_cpu"] = host_cpu()
    line["host_cpus"] = os.cpu_count()
    return line


def read_traffic(kernel: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    path = PROFILES / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(kernel)
    except (ValueError, OSError):
        return None


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=30)
    # 20 untimed steps (about 20 ms for the 1 ms headline) let the GPU clock
    # settle before the timed steps.
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--cpu-seconds", type=float, default=12.0)
    parser.add_argument("--only", default=None, help="run only secondary benches whose name contains this")
    parser.add_argument("--headline-only", action="store_true")
    parser.add_argument("--no-headline", action="store_true",
                        help="skip the 4096^3 GEMM (profiling runs of the secondary kernels)")
    parser.add_argument("--extra-shapes", action="store_true",
                        help="only time the shapes off the bench lines that route to other kernels (profiling)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run 1 GiB device-to-device copies (PMC byte-counter calibration)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs every kernel on one MI355X and has no "
              f"multi-GPU path, so --gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    if not capi.available():
        print(f"no usable HIP device: {capi.last_error()}", file=sys.stderr)
        return 1
    info = capi.device_info()
    log(f"device: {info['name']} {info['arch']} CUs={info['compute_units']} clock={info['clock_khz']} kHz")

    if args.copy_calibration:
        src, dst = capi.DeviceBuffer(1 << 30), capi.DeviceBuffer(1 << 30)
        s = capi.stream()
        ev = [capi.Event() for _ in range(4)]
        ev[0].record(s)
        for i in range(3):
            capi.check(capi.lib().tcx_hip_memcpy_d2d(dst.ptr, src.ptr, 1 << 30, s), "copy")
            ev[i + 1].record(s)
        ev[-1].synchronize()
        ms = [ev[i].elapsed_ms(ev[i + 1]) for i in range(3)]
        # read + write of 1 GiB each: HIP's own copy kernel as a stream reference
        log("copy calibration: 3 x 1 GiB device-to-device copies, "
            + ", ".join(f"{2 * (1 << 30) / m / 1e6:.0f} GB/s" for m in ms) + " (read + write)")
        return 0
    if args.extra_shapes:
        for r in extra_benches(args.steps, args.warmup):
            print(json.dumps(r), flush=True)
        return 0
    if args.no_headline:
        for r in secondary_benches(args.steps, args.warmup, args.only, not args.no_cpu):
            print(json.dumps(r), flush=True)
        return 0
    headline = bench_gemm("c2_4096", args.steps, args.warmup)
    log(f"gemm 4096^3: {headline['achieved']:.1f} TFLOP/s ({headline['frac']:.1%} of fp32 MFMA peak), "
        f"median launch {headline['kernel_median_ms']:.4f} ms")
    with marked("api_wall_gemm_c2_4096"):
        api = api_wall(args.steps, args.warmup)
    log(f"gemm 4096^3 through tensorcx.matmul: {api['ms_per_call_median']:.4f} ms per call (median)")
    secondary = [] if args.headline_only else secondary_benches(args.steps, args.warmup, args.only,
                                                                  not args.no_cpu)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    if cpu is not None:
        log(f"cpu baseline: {cpu['value'] * 1e3:.3f} GFLOP/s on one thread of {cpu['host_cpu']}")

    traffic = read_traffic("gemm_f32_kernel_4096")
    line = {
        "metric": "fp32 matmul TFLOP/s (4096^3) + softmax/reduction GB/s, % of roofline, 1 GPU",
        "value": round(headline["value"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(headline["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic (NumPy PCG64 seed 1, N(0,1) float32), resident in HBM, "
                f"{headline['operand_copies']} rotated operand copies",
        "config": {"workload": "fp32 matmul C=A@B, 4096x4096x4096, row-major (BASELINE config C2)",
                   "m": 4096, "n": 4096, "k": 4096, "seed": 1},
        "roofline": {"bound": "mfma", "achieved": round(headline["achieved"], 3),
                     "peak": 157.3, "unit": "TFLOP/s", "frac": round(headline["frac"], 4),
                     "traffic": traffic, "kernel_avg_ms": round(headline["kernel_avg_ms"], 4),
                     "kernel_median_ms": round(headline["kernel_median_ms"], 4),
                     "flop_per_launch": headline["flop_per_launch"],
                     "warmup_launches": headline["warmup_launches"]},
        "api_wall": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in api.items()},
        "cpu_baseline": cpu,
        "secondary": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
                      for r in secondary],
        "host": {"cpu": host_cpu(), "cpus": os.cpu_count()},
        "device": {"name": info["name"], "arch": info["arch"], "cus": info["compute_units"],
                   "clock_khz": info["clock_khz"]},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
