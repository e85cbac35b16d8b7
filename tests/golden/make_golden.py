"""Writes tests/golden/golden.npz + golden.json from the reference CPU backend.

Run in the container that holds /root/reference after `make -C oracle ref`:

    python tests/golden/make_golden.py

Every expected output comes from oracle/_ref/libtcxref.so, i.e. the reference's
own CpuBackend::execute compiled from its sources; inputs are small and seeded
(NumPy PCG64, float64 draws cast to float32, the reference idiom of
python/tensorcx/tensor.py:496). The case list also carries the reference's own
known-answer tests: the 2x2 matmul KAT (cpu_backend.cpp:593-621), the [[1..6]]
row sums (cpu_backend.cpp:566-591), the canonical-order special values of
tests/python/test_multi_axis_reductions.py:114-130 and the dyadic batched matmul
inputs of tests/cpp/batched_matmul_contract.h:25-26.
"""

from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ref  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent


def f32(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def cases():
    rng = np.random.default_rng(20260101)
    c = []

    def add(name, op, inputs, **kw):
        c.append((name, op, inputs, kw))

    # ---- matmul (cpu_backend.cpp:1251-1276; shape.cpp:49-85)
    add("matmul_kat_2x2", "matmul", [np.array([[1, 2], [3, 4]], np.float32),
                                     np.array([[5, 6], [7, 8]], np.float32)])
    for m, k, n in [(1, 1, 1), (2, 3, 4), (15, 17, 31), (17, 16, 15), (32, 33, 16),
                    (65, 129, 67), (0, 3, 4), (3, 0, 4), (3, 4, 0), (130, 260, 70)]:
        add(f"matmul_{m}x{k}x{n}", "matmul", [f32(rng, (m, k)), f32(rng, (k, n))])
    add("matmul_batch_broadcast", "matmul", [f32(rng, (2, 1, 5, 7)), f32(rng, (3, 7, 4))])
    add("matmul_vec_mat", "matmul", [f32(rng, (7,)), f32(rng, (7, 3))])
    add("matmul_mat_vec", "matmul", [f32(rng, (3, 7)), f32(rng, (7,))])
    add("matmul_vec_vec", "matmul", [f32(rng, (9,)), f32(rng, (9,))])
    i = np.arange(4 * 9 * 11)
    a = ((i % 11 - 5) / 8).astype(np.float32).reshape(4, 9, 11)
    j = np.arange(4 * 11 * 6)
    b = ((j % 7 - 3) / 8).astype(np.float32).reshape(4, 11, 6)
    add("matmul_dyadic_batched", "matmul", [a, b])

    # ---- single-axis reductions (cpu_backend.cpp:1154-1249)
    six = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    add("sum_kat_rows", "sum", [six], axis=1)
    for shape in [(), (1,), (7,), (2, 3, 5), (2, 0, 3), (0, 2, 3), (3, 257), (2, 4097), (5, 1000)]:
        x = f32(rng, shape)
        rank = max(1, len(shape))
        for op in ("sum", "max", "mean"):
            for axis in range(-rank, rank):
                add(f"{op}_{'x'.join(map(str, shape)) or 'scalar'}_axis{axis}", op, [x], axis=axis)
    xi = rng.integers(-2**31, 2**31 - 1, size=(6, 300), dtype=np.int64).astype(np.int32)
    for op in ("sum", "max"):
        add(f"{op}_i32_wrap_rows", op, [xi], axis=1)
        add(f"{op}_i32_wrap_cols", op, [xi], axis=0)
    for row in ([0., -0., 1e-38, -1e-38], [1., np.nan, 2., 3.], [np.inf, 1., 2., -np.inf],
                [1e20] * 4, [-0., -0., -0., -0.], [np.nan, np.inf, -np.inf, 0.]):
        x = np.array([row, row[::-1]], np.float32)
        for op in ("sum", "max", "mean", "softmax", "rmsnorm", "layernorm"):
            add(f"{op}_special_{len(c)}", op, [x], axis=1)

    # ---- multi-axis reductions (cpu_backend.cpp:1102-1153; shape.cpp:140-173)
    x = f32(rng, (3, 4, 5))
    for op in ("sum", "max", "mean"):
        for axes in ([0, 1, 2], [0, 2], [2, 0], [1], [], [-1, -2]):
            add(f"{op}_axes_{'_'.join(map(str, axes)) or 'none'}", op, [x], axes=axes)
    for values in ([[0., -0.], [-0., 0.]], [[np.inf, 2], [-np.inf, 4]], [[1, np.nan], [3, 4]],
                   [[3e38, 3e38], [-3e38, -3e38]], [[1e20, 1], [-1e20, 3]]):
        x = np.array(values, np.float32)
        for op in ("sum", "max", "mean"):
            add(f"{op}_canonical_{len(c)}", op, [x], axes=[0, 1])
    xi = np.array([[2**31 - 1, 2**31 - 1], [-2**31, -17]], np.int32)
    for op in ("sum", "max"):
        add(f"{op}_i32_axes_wrap", op, [xi], axes=[0, 1])

    # ---- min / argmax (cpu_math.cpp:27-76; math.cpp:39-56)
    x = f32(rng, (4, 33))
    x[1, 7] = x[1, 20] = x[1].max() + 1   # tie: lowest index wins
    x[2, 3], x[2, 9] = np.nan, -np.nan  # first NaN wins
    x[3, :] = 0.0
    x[3, 5] = -0.0                       # +0 / -0 compare equal
    for op in ("min", "argmax"):
        add(f"{op}_rows", op, [x], axes=[1])
        add(f"{op}_cols", op, [x], axes=[0])
        add(f"{op}_all", op, [x], axes=[0, 1])
    xi = rng.integers(-5, 5, size=(5, 40)).astype(np.int32)
    for op in ("min", "argmax"):
        add(f"{op}_i32_rows", op, [xi], axes=[1])

    # ---- softmax / rmsnorm / layernorm (cpu_backend.cpp:125-240)
    for shape, axis in [((4, 300), 1), ((3, 5), 0), ((2, 3, 70), -1), ((1, 4096), 1), ((0, 4), 1)]:
        x = f32(rng, shape, 3.0)
        for op in ("softmax", "rmsnorm", "layernorm"):
            add(f"{op}_{'x'.join(map(str, shape))}_axis{axis}", op, [x], axis=axis)
    const = np.full((2, 16), 2.5, np.float32)
    for eps in (0.0, 1e-45, 1e-5, 1e30):
        for op in ("rmsnorm", "layernorm"):
            add(f"{op}_const_eps{eps}", op, [const], axis=1, eps=eps)

    # ---- elementwise (cpu_backend.cpp:1000-1010, 1014-1097)
    x = np.linspace(-8, 8, num=257, dtype=np.float32)
    sp = np.array([0., -0., np.inf, -np.inf, np.nan, 100, -100, 1e-38], np.float32)
    for op in ("exp", "gelu", "silu"):
        add(f"{op}_linspace", op, [x])
        add(f"{op}_special", op, [sp])
    for op in ("add", "subtract", "multiply", "divide"):
        add(f"{op}_bias_broadcast", op, [f32(rng, (6, 10)), f32(rng, (10,))])
        add(f"{op}_col_broadcast", op, [f32(rng, (6, 1)), f32(rng, (2, 1, 10))])
    xi = rng.integers(-2**31, 2**31 - 1, size=(4, 8), dtype=np.int64).astype(np.int32)
    yi = rng.integers(-2**31, 2**31 - 1, size=(8,), dtype=np.int64).astype(np.int32)
    for op in ("add", "subtract", "multiply"):
        add(f"{op}_i32_wrap", op, [xi, yi])

    # ---- inference composites (inference.cpp:86-122)
    x, w, b = f32(rng, (5, 48)), f32(rng, (20, 48)), f32(rng, (20,))
    add("linear_bias", "linear", [x, w, b])
    add("linear_nobias", "linear", [x, w])
    add("linear_3d", "linear", [f32(rng, (2, 3, 48)), w, b])
    x = f32(rng, (6, 64), 3.0)
    g = rng.uniform(0.5, 1.5, size=64).astype(np.float32)
    be = rng.uniform(-0.1, 0.1, size=64).astype(np.float32)
    add("affine_layernorm_gb", "affine_layernorm", [x, g, be], axis=-1, has_weight=True, has_bias=True)
    add("affine_layernorm_g", "affine_layernorm", [x, g], axis=-1, has_weight=True)
    add("affine_rmsnorm_g", "affine_rmsnorm", [x, g], axis=-1, has_weight=True)
    return c


def main() -> None:
    if not ref.available():
        raise SystemExit("oracle/_ref/libtcxref.so is missing: run `make -C oracle ref`")
    arrays, manifest = {}, []
    for index, (name, op, inputs, kw) in enumerate(cases()):
        entry = {"name": name, "op": op, "kwargs": kw, "inputs": []}
        for n, x in enumerate(inputs):
            key = f"c{index}_in{n}"
            arrays[key] = x
            entry["inputs"].append(key)
        try:
            out = ref.execute(op, inputs, **kw)
            arrays[f"c{index}_out"] = out
            entry["output"] = f"c{index}_out"
        except ref.ReferenceError as error:
            entry["error"] = {"code": error.code, "message": str(error)}
        manifest.append(entry)
    np.savez_compressed(OUT / "golden.npz", **arrays)
    (OUT / "golden.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(f"wrote {len(manifest)} cases")


if __name__ == "__main__":
    main()
