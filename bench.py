"""Benchmark of the hip hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME]

Headline (the JSON `value`): fp32 matmul TFLOP/s at 4096^3 (config C2, the
second entry of BASELINE.json's configs), inputs resident in HBM, K timed GEMM launches bracketed by stream
synchronisation, timed with HIP events on the launch stream. The same JSON line
carries `roofline` for that kernel, `cpu_baseline` (the reference CPU matmul,
single thread, on a bounded row slab), and `secondary`: the other configs'
kernels (batched/edge GEMM, reductions, softmax/norms, MLP, fused attention)
each as GB/s or TFLOP/s with its roofline fraction.

Peaks: fp32 MFMA 157.3 TFLOP/s, HBM 8.0 TB/s (MI355X published figures).
"""

from __future__ import annotations

import argparse
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


# Secondary benches warm up for at least this much GPU time: the GPU clock
# ramps up over the first milliseconds of sustained load, and each secondary
# starts after host-side input generation has let it idle. A 4096x4096x1024
# GEMM measured 283 us after 3 warm-up launches and 256 us after 300; the
# 4096^3 headline (1 ms per launch) measured the same either way.
SECONDARY_WARM_MS = 20.0


def timed(launch, steps: int, warmup: int, warm_ms: float = 0.0):
    """Runs `launch` warmup times, then (untimed) until warm_ms of GPU time has
    passed, then K = steps timed times on this thread's stream, and returns
    (total_ms, per_launch_ms, warm-up launches): two HIP events bracket the K
    timed launches on the launch stream, with the stream idle on both sides."""
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
    start, stop = capi.Event(), capi.Event()
    start.record(s)
    for _ in range(steps):
        launch(s)
    stop.record(s)
    stop.synchronize()
    capi.synchronize()
    total = start.elapsed_ms(stop)
    return total, [total / steps] * steps, launches


def rotate(arrays_per_copy):
    """Index helper: cycle through input copies so 256 MB operands are not
    served from the 256 MB Infinity Cache on the next launch."""
    state = {"i": 0}

    def nxt():
        state["i"] = (state["i"] + 1) % len(arrays_per_copy)
        return arrays_per_copy[state["i"]]
    return nxt


def bench_gemm(name: str, steps: int, warmup: int, transposed=False, warm_ms: float = 0.0):
    a, b = wl.gemm_inputs(name)
    da, db = capi.DeviceArray.from_numpy(a), capi.DeviceArray.from_numpy(b)
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
    total, per, warm = timed(lambda s: capi.gemm(da.ptr, db.ptr, out.ptr, desc, s, ws), steps, warmup, warm_ms)
    flops = wl.gemm_flops(name)
    avg = statistics.mean(per)
    return {"name": f"gemm_{name}", "unit": "TFLOP/s", "value": flops / (total / steps * 1e-3) / 1e12,
            "kernel_avg_ms": avg, "kernel_median_ms": statistics.median(per),
            "achieved": flops / (avg * 1e-3) / 1e12, "peak": PEAK_FP32_MFMA / 1e12,
            "frac": flops / (avg * 1e-3) / PEAK_FP32_MFMA, "flop_per_launch": flops,
            "ms_per_step": total / steps, "warmup_launches": warm}


def bench_hbm(name: str, launch_for, nbytes: int, steps: int, warmup: int):
    total, per, warm = timed(launch_for, steps, warmup, SECONDARY_WARM_MS)
    avg = statistics.mean(per)
    return {"name": name, "unit": "GB/s", "value": nbytes / (total / steps * 1e-3) / 1e9,
            "kernel_avg_ms": avg, "kernel_median_ms": statistics.median(per),
            "achieved": nbytes / (avg * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9,
            "frac": nbytes / (avg * 1e-3) / PEAK_HBM, "bytes_per_launch": nbytes, "warmup_launches": warm}


def secondary_benches(steps: int, warmup: int, only: str | None):
    out = []

    def want(n):
        return only is None or only in n

    for name in ("c2_batched", "c2_edge", "c1_512"):
        if want(name):
            out.append(bench_gemm(name, steps, warmup, warm_ms=SECONDARY_WARM_MS))
            log(f"{out[-1]['name']}: {out[-1]['achieved']:.1f} TFLOP/s ({out[-1]['frac']:.1%})")

    if want("reduce") or want("sum") or want("max") or want("argmax"):
        x = wl.reduce_f32_input()
        copies = [capi.DeviceArray.from_numpy(x) for _ in range(2)]
        del x
        rows, cols = 8192, 8192
        res = capi.DeviceArray((rows,), np.float32)
        nbytes = rows * cols * 4 + rows * 4
        for op in ("sum", "max", "mean", "min", "argmax"):
            nxt = rotate(copies)
            out.append(bench_hbm(f"reduce_{op}_f32_8192x8192", lambda s, op=op: capi.reduce(
                op, capi.TCX_FLOAT32, nxt().ptr, res.ptr, rows, cols, 1, None, s), nbytes, steps, warmup))
            log(f"{out[-1]['name']}: {out[-1]['achieved']:.0f} GB/s ({out[-1]['frac']:.1%})")
        ws = capi.reduce_workspace("sum", capi.TCX_FLOAT32, 1, rows * cols, 1)
        full = capi.DeviceArray((1,), np.float32)
        nxt = rotate(copies)
        out.append(bench_hbm("reduce_full_sum_f32_8192x8192", lambda s: capi.reduce(
            "sum", capi.TCX_FLOAT32, nxt().ptr, full.ptr, 1, rows * cols, 1, ws, s),
            rows * cols * 4 + 4, steps, warmup))
        log(f"{out[-1]['name']}: {out[-1]['achieved']:.0f} GB/s ({out[-1]['frac']:.1%})")
        del copies

    if want("i32"):
        xi = wl.reduce_i32_input()
        copies = [capi.DeviceArray.from_numpy(xi)]
        del xi
        rows, cols = 65536, 4096
        res = capi.DeviceArray((rows,), np.int32)
        nbytes = rows * cols * 4 + rows * 4
        for op in ("sum", "max"):
            out.append(bench_hbm(f"reduce_{op}_i32_65536x4096", lambda s, op=op: capi.reduce(
                op, capi.TCX_INT32, copies[0].ptr, res.ptr, rows, cols, 1, None, s), nbytes, steps, warmup))
            log(f"{out[-1]['name']}: {out[-1]['achieved']:.0f} GB/s ({out[-1]['frac']:.1%})")
        del copies

    if want("softmax") or want("norm"):
        x, g, b = wl.rownorm_inputs()
        copies = [capi.DeviceArray.from_numpy(x) for _ in range(2)]
        del x
        gd, bd = capi.DeviceArray.from_numpy(g), capi.DeviceArray.from_numpy(b)
        rows, cols = 16384, 4096
        y = capi.DeviceArray((rows, cols))
        nbytes = 2 * rows * cols * 4
        nxt = rotate(copies)
        out.append(bench_hbm("softmax_16384x4096", lambda s: capi.softmax(nxt().ptr, y.ptr, rows, cols, 1, s),
                             nbytes, steps, warmup))
        log(f"{out[-1]['name']}: {out[-1]['achieved']:.0f} GB/s ({out[-1]['frac']:.1%})")
        out.append(bench_hbm("rmsnorm_16384x4096", lambda s: capi.rmsnorm(
            nxt().ptr, None, y.ptr, rows, cols, 1, 1e-5, s), nbytes, steps, warmup))
        log(f"{out[-1]['name']}: {out[-1]['achieved']:.0f} GB/s ({out[-1]['frac']:.1%})")
        out.append(bench_hbm("layernorm_affine_16384x4096", lambda s: capi.layernorm(
            nxt().ptr, gd.ptr, bd.ptr, y.ptr, rows, cols, 1, 1e-5, s), nbytes + 2 * cols * 4, steps, warmup))
        log(f"{out[-1]['name']}: {out[-1]['achieved']:.0f} GB/s ({out[-1]['frac']:.1%})")
        del copies

    if want("mlp"):
        x, w1, b1, w2, b2 = wl.mlp_inputs()
        dx, dw1, db1, dw2, db2 = (capi.DeviceArray.from_numpy(v) for v in (x, w1, b1, w2, b2))
        h = capi.DeviceArray((4096, 4096))
        logits = capi.DeviceArray((4096, 1024))
        prob = capi.DeviceArray((4096, 1024))
        d1 = capi.gemm_desc(4096, 4096, 1024, rhs_transposed=True, bias=db1.ptr, activation="silu")
        d2 = capi.gemm_desc(4096, 1024, 4096, rhs_transposed=True, bias=db2.ptr)

        ws1, ws2 = capi.gemm_workspace(d1), capi.gemm_workspace(d2)  # the second linear splits K

        def mlp(s):
            capi.gemm(dx.ptr, dw1.ptr, h.ptr, d1, s, ws1)
            capi.gemm(h.ptr, dw2.ptr, logits.ptr, d2, s, ws2)
            capi.softmax(logits.ptr, prob.ptr, 4096, 1024, 1, s)

        total, per, warm = timed(mlp, steps, warmup, SECONDARY_WARM_MS)
        flops = 2 * 2 * 4096 * 4096 * 1024
        avg = statistics.mean(per)
        out.append({"name": "mlp_forward_4096x1024x4096", "unit": "TFLOP/s",
                    "value": flops / (total / steps * 1e-3) / 1e12, "step_avg_ms": avg,
                    "achieved": flops / (avg * 1e-3) / 1e12, "peak": PEAK_FP32_MFMA / 1e12,
                    "frac": flops / (avg * 1e-3) / PEAK_FP32_MFMA,
                    "tokens_per_s": 4096 / (avg * 1e-3), "warmup_launches": warm})
        log(f"{out[-1]['name']}: {out[-1]['achieved']:.1f} TFLOP/s ({out[-1]['frac']:.1%})")

    if want("attention"):
        q, k, v = wl.attention_inputs()
        bh, seq, d = q.shape
        dq, dk, dv = (capi.DeviceArray.from_numpy(t) for t in (q, k, v))
        o = capi.DeviceArray((bh, seq, d))
        for causal in (False, True):
            flops = wl.attention_flops(causal)
            total, per, warm = timed(lambda s, c=causal: capi.flash_attention(
                dq.ptr, dk.ptr, dv.ptr, o.ptr, bh, seq, seq, d, 1.0 / np.sqrt(d), c, s), steps, warmup,
                SECONDARY_WARM_MS)
            avg = statistics.mean(per)
            out.append({"name": f"attention_fused_{bh}x{seq}x{d}" + ("_causal" if causal else ""),
                        "unit": "TFLOP/s", "value": flops / (total / steps * 1e-3) / 1e12,
                        "kernel_avg_ms": avg, "achieved": flops / (avg * 1e-3) / 1e12,
                        "peak": PEAK_FP32_MFMA / 1e12, "frac": flops / (avg * 1e-3) / PEAK_FP32_MFMA,
                        "flop_per_launch": flops, "warmup_launches": warm})
            log(f"{out[-1]['name']}: {out[-1]['achieved']:.1f} TFLOP/s ({out[-1]['frac']:.1%})")
    return out


def cpu_baseline(budget_s: float):
    """Reference CPU matmul (oracle/_ref, the reference's own cpu::matmul,
    single thread) on a bounded row slab of the 4096^3 product; falls back to
    the oracle restatement when the reference build is absent."""
    a, b = wl.gemm_inputs("c2_4096")
    try:
        from oracle import ref
        if not ref.available():
            raise ImportError
        kind = "reference"

        def run(rows):
            ref.matmul_rows(a, b, rows)
    except ImportError:
        import ctypes

        import oracle
        kind = "port"
        out = np.empty((4096, 4096), np.float32)

        def run(rows):
            oracle.lib().oracle_matmul_f32_naive(
                ctypes.c_void_p(a.ctypes.data), ctypes.c_void_p(b.ctypes.data),
                ctypes.c_void_p(out.ctypes.data), ctypes.c_int64(4096), ctypes.c_int64(4096),
                ctypes.c_int64(4096), ctypes.c_int64(0), ctypes.c_int64(rows))
    t = time.perf_counter()
    run(2)
    per_row = (time.perf_counter() - t) / 2
    rows = int(max(2, min(4096, budget_s / max(per_row, 1e-6))))
    t = time.perf_counter()
    run(rows)
    dt = time.perf_counter() - t
    flops = 2.0 * rows * 4096 * 4096
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": kind,
            "sample": f"rows 0..{rows} of the 4096x4096x4096 fp32 matmul (C2 inputs, seed 1), "
                      f"{dt:.1f} s, single thread, extrapolates to {dt * 4096 / rows:.0f} s for the full product",
            "host_cpus": os.cpu_count()}


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
    if args.no_headline:
        for r in secondary_benches(args.steps, args.warmup, args.only):
            print(json.dumps(r), flush=True)
        return 0
    headline = bench_gemm("c2_4096", args.steps, args.warmup)
    log(f"gemm 4096^3: {headline['achieved']:.1f} TFLOP/s ({headline['frac']:.1%} of fp32 MFMA peak)")
    secondary = [] if args.headline_only else secondary_benches(args.steps, args.warmup, args.only)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

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
        "data": "synthetic (NumPy PCG64 seed 1, N(0,1) float32), resident in HBM",
        "config": {"workload": "fp32 matmul C=A@B, 4096x4096x4096, row-major (BASELINE config C2)",
                   "m": 4096, "n": 4096, "k": 4096, "seed": 1},
        "roofline": {"bound": "mfma", "achieved": round(headline["achieved"], 3),
                     "peak": 157.3, "unit": "TFLOP/s", "frac": round(headline["frac"], 4),
                     "traffic": traffic, "kernel_avg_ms": round(headline["kernel_avg_ms"], 4),
                     "flop_per_launch": headline["flop_per_launch"]},
        "cpu_baseline": cpu,
        "secondary": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
                      for r in secondary],
        "device": {"name": info["name"], "arch": info["arch"], "cus": info["compute_units"],
                   "clock_khz": info["clock_khz"]},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
