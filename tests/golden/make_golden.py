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

    # ---- log / sqrt / abs (cpu_math.cpp:40-44; cases of test_math_ops.py:26-60)
    bits = np.array([0, 0x80000000, 1, 2, 0x007fffff, 0x00800000, 0x80000001, 0x807fffff, 0x80800000,
                     0x3f800000, 0xbf800000, 0x7f7fffff, 0x7f800000, 0xff800000, 0x7fc01234], np.uint32)
    for op in ("log", "sqrt", "abs"):
        for shape in [(2, 3, 5), (513,), (0,), ()]:
            add(f"{op}_{'x'.join(map(str, shape)) or 'scalar'}", op,
                [rng.uniform(.01, 100, shape).astype(np.float32)])
        add(f"{op}_ieee", op, [bits.view(np.float32)])
    add("abs_i32_wrap", "abs", [np.array([-2**31, -2**31 + 1, -16777217, -1, 0, 1, 2**31 - 1], np.int32)])
    add("log_i32_rejected", "log", [np.array([1, 2], np.int32)])

    # ---- clip (cpu_math.cpp:45-50; test_math_ops.py:94-120)
    lim = {"float32": (-np.inf, np.inf), "int32": (-2**31, 2**31 - 1)}
    for dtype in ("float32", "int32"):
        xi = rng.integers(-10, 10, (2, 3, 4)).astype(dtype)
        for lo, hi in [(-2, 3), (None, 3), (-2, None), (4, -4), (0, 0)]:
            lo = lim[dtype][0] if lo is None else lo
            hi = lim[dtype][1] if hi is None else hi
            add(f"clip_{dtype}_{lo}_{hi}", "clip", [xi, np.array(lo, dtype), np.array(hi, dtype)])
        add(f"clip_{dtype}_broadcast", "clip", [np.array([[[-4], [1], [9]]], dtype),
                                               np.array([[-1, 2, 7, 8]], dtype), np.array([[[3]], [[10]]], dtype)])
    add("clip_ieee", "clip", [np.array([np.nan, -0., 0., 1e-40, -1e-40, np.inf, -np.inf, 1., 2.], np.float32),
                              np.array([-1., 0., -0., -2e-40, -2e-40, -1., -1., np.nan, -1.], np.float32),
                              np.array([1., 0., -0., 2e-40, 2e-40, 1., 1., 2., np.nan], np.float32)])
    add("clip_random_f32", "clip", [f32(rng, (7, 130)), f32(rng, (130,), .5) - 1, f32(rng, (7, 1), .5) + 1])

    # ---- topk (cpu_math.cpp:57-67; test_math_ops.py:123-180)
    tx = rng.integers(-3, 4, (3, 5, 6)).astype(np.float32)
    tx[0, 1, 2] = np.nan
    tx[2, 3, 1] = np.nan
    tx[1, 2, 3] = -0.0
    for dtype in ("float32", "int32"):
        x = tx if dtype == "float32" else np.nan_to_num(tx).astype(np.int32)
        for axis in (0, 1, 2, -1):
            n = x.shape[axis]
            for k in sorted({0, 1, n // 2, n}):
                for largest in (True, False):
                    for srt in (True, False):
                        add(f"topk_{dtype}_a{axis}_k{k}_{int(largest)}{int(srt)}", "topk", [x], axis=axis, k=k,
                            largest=largest, sorted=srt, n_outputs=2)
    add("topk_wide", "topk", [f32(rng, (4, 3000))], axis=1, k=37, n_outputs=2)
    add("topk_k_too_large", "topk", [f32(rng, (2, 3))], axis=1, k=4, n_outputs=2)

    # ---- embedding (cpu_inference.cpp:12-21; test_inference_ops.py:100-130)
    for shape in [(), (4,), (2, 3), (2, 0, 3)]:
        for width in (0, 1, 7):
            add(f"embedding_{'x'.join(map(str, shape)) or 'scalar'}_w{width}", "embedding",
                [rng.integers(0, 5, size=shape, dtype=np.int32), f32(rng, (5, width))])
    ebits = np.array([[0, 0x80000000, 1, 0x7fc01234], [0x7f800000, 0xff800000, 0x80000001, 0x3f800000]],
                     np.uint32).view(np.float32)
    add("embedding_bits", "embedding", [np.array([1, 0, 1], np.int32), ebits])
    add("embedding_index_negative", "embedding", [np.array([-1], np.int32), f32(rng, (2, 3))])
    add("embedding_index_past_end", "embedding", [np.array([0, 1, 2], np.int32), f32(rng, (2, 3))])
    add("embedding_big_table", "embedding", [rng.integers(0, 1000, (3, 17), dtype=np.int32), f32(rng, (1000, 96))])

    # ---- attention (inference.cpp:123-161 over cpu_inference.cpp:22-47;
    #      cases of test_inference_ops.py:133-343)
    shapes = [((3, 4), (5, 4), (5, 2)), ((2, 3, 4), (2, 5, 4), (2, 5, 6)),
              ((2, 1, 3, 4), (1, 3, 5, 4), (2, 3, 5, 2)), ((3, 4), (5, 4), (2, 1, 5, 2)),
              ((0, 4), (5, 4), (5, 2)), ((3, 4), (0, 4), (0, 2)), ((3, 4), (5, 4), (5, 0))]
    for si, (qs, ks, vs) in enumerate(shapes):
        q, k, v = f32(rng, qs), f32(rng, ks), f32(rng, vs)
        ms = (qs[-2], ks[-2])
        bmask = rng.random(ms) > .4
        if ms[0]:
            bmask[0] = False
        amask = f32(rng, ms)
        amask[rng.random(ms) < .3] = -np.inf
        if ms[0]:
            amask[0] = -np.inf
        for mname, mask in (("none", None), ("bool", bmask), ("additive", amask), ("false", np.array(False))):
            for causal in (False, True):
                ins = [q, k, v] + ([] if mask is None else [mask])
                add(f"attention_s{si}_{mname}_c{int(causal)}", "attention", ins, causal=causal)
    q, k, v = f32(rng, (2, 3, 4)), f32(rng, (5, 4)), f32(rng, (5, 3))
    bm = rng.random((2, 1, 5)) > .3
    for scale in (0.0, -0.5, 2.0, float(np.float32(.3)), 1e-39, -1e-40):
        add(f"attention_scale_{scale}", "attention", [q, k, v, bm], scale=scale)
    for exceptional in (np.nan, np.inf, -np.inf):
        kk = np.ones((2, 2), np.float32)
        kk[0] = exceptional
        for masked in (False, True):
            add(f"attention_nonfinite_{exceptional}_{masked}", "attention",
                [np.ones((1, 2), np.float32), kk, f32(rng, (2, 3)), np.array([[not masked, True]])])
    for bias in (np.nan, np.inf, -np.inf):
        add(f"attention_bias_{bias}", "attention", [f32(rng, (2, 3)), f32(rng, (4, 3)), f32(rng, (4, 2)),
                np.array([[bias, 0, -np.inf, 0], [bias, bias, bias, bias]], np.float32)])
    add("attention_high_rank", "attention", [f32(rng, (1,) * 6 + (3, 4)), f32(rng, (1,) * 6 + (2, 4)),
                                             f32(rng, (1,) * 6 + (2, 3))])
    add("attention_long_causal", "attention", [f32(rng, (257, 3)), f32(rng, (513, 3)), f32(rng, (513, 2))],
        causal=True)
    add("attention_heads_64", "attention", [f32(rng, (2, 4, 33, 64)), f32(rng, (2, 4, 70, 64)),
                                            f32(rng, (2, 4, 70, 64))], causal=True)
    for scale in (float("nan"), float("inf"), 1e300, 1e-300):
        add(f"attention_bad_scale_{scale}", "attention", [np.zeros((0, 2), np.float32),
            np.zeros((3, 2), np.float32), np.zeros((3, 1), np.float32)], scale=scale)
    add("attention_bad_features", "attention", [f32(rng, (2, 3)), f32(rng, (2, 4)), f32(rng, (2, 3))])
    add("attention_bad_batch", "attention", [f32(rng, (2, 0, 3)), f32(rng, (3, 2, 3)), f32(rng, (3, 2, 3))])
    add("attention_bad_mask", "attention", [f32(rng, (2, 3)), f32(rng, (2, 3)), f32(rng, (2, 3)),
                                            np.zeros((2, 3), bool)])

    # ---- scalar arithmetic and negate (cpu_backend.cpp:878-930)
    xs = f32(rng, (4, 33), 3.0)
    xs[0, :4] = [np.nan, np.inf, -0.0, 1e-40]
    xi = rng.integers(-2**31, 2**31 - 1, (5, 7), dtype=np.int64).astype(np.int32)
    xi[0, :3] = [-2**31, 2**31 - 1, 0]
    add("negative_f32", "negative", [xs])
    add("negative_i32_wrap", "negative", [xi])
    for name in ("add_scalar", "subtract_scalar", "multiply_scalar", "divide_scalar"):
        for left in (False, True):
            add(f"{name}_f32_{int(left)}", name, [xs], scalar=0.1, scalar_left=left)
        add(f"{name}_f32_inf", name, [xs], scalar=float("inf"))
        if name != "divide_scalar":
            add(f"{name}_i32_{int(left)}", name, [xi], scalar=-123457, scalar_left=True)
            add(f"{name}_i32_wrap", name, [xi], scalar=2**31 - 1)
    add("divide_scalar_i32_rejected", "divide_scalar", [xi], scalar=2.0)
    add("add_scalar_i32_fraction_rejected", "add_scalar", [xi], scalar=0.5)
    add("negative_bool_rejected", "negative", [np.array([True, False])])

    # ---- casts (cpu_backend.cpp:834-876)
    cf = np.array([0.0, -0.0, 1.9, -1.9, 2147483520.0, -2147483648.0, 1e-40, 3.5e6], np.float32)
    ci = np.array([0, 1, -1, 2**31 - 1, -2**31, 16777217, 7], np.int32)
    cb = np.array([True, False, True])
    for src, arr in (("f32", cf), ("i32", ci), ("bool", cb)):
        for dst in ("float32", "int32", "bool"):
            add(f"astype_{src}_{dst}", "astype", [arr], target_dtype=dst)
    for bad in (np.nan, np.inf, -np.inf, 2147483648.0, -2147483904.0):
        add(f"astype_f32_i32_bad_{bad}", "astype", [np.array([1.0, bad], np.float32)], target_dtype="int32")
    add("astype_empty", "astype", [np.zeros((0, 3), np.float32)], target_dtype="int32")

    # ---- transpose / slice / concat (shape.cpp:87-200; cpu_backend.cpp:808-833, 317-339)
    xt = f32(rng, (2, 3, 4, 5))
    for perm in ((0, 1, 2, 3), (3, 2, 1, 0), (1, 3, 0, 2), (-1, 0, -3, 2)):
        add(f"transpose_{'_'.join(map(str, perm))}", "transpose", [xt], perm=list(perm))
    add("transpose_bool", "transpose", [rng.random((3, 5)) > .5], perm=[1, 0])
    add("transpose_i32", "transpose", [xi], perm=[1, 0])
    add("transpose_scalar", "transpose", [np.float32(3.5)], perm=[])
    add("transpose_repeat_rejected", "transpose", [xt], perm=[0, 0, 1, 2])
    for si, (starts, steps, lengths) in enumerate((([0, 0, 0, 0], [1, 1, 1, 1], [2, 3, 4, 5]),
                                                  ([1, 2, 3, 4], [-1, -1, -1, -1], [2, 3, 4, 5]),
                                                  ([0, 1, 0, 4], [1, 1, 2, -2], [2, 2, 2, 3]),
                                                  ([1, 0, 2, 0], [1, 1, 1, 1], [1, 0, 1, 5]))):
        add(f"slice_{si}", "slice", [xt], starts=starts, steps=steps, lengths=lengths)
    add("slice_oob_rejected", "slice", [xt], starts=[0, 0, 0, 3], steps=[1, 1, 1, 1], lengths=[2, 3, 4, 3])
    a1, a2, a3 = f32(rng, (2, 3, 4)), f32(rng, (2, 1, 4)), f32(rng, (2, 0, 4))
    add("concat_axis1", "concat", [a1, a2, a3], axis=1)
    add("concat_axis0", "concat", [a1, f32(rng, (3, 3, 4))], axis=0)
    add("concat_axis_neg", "concat", [a1, f32(rng, (2, 3, 2))], axis=-1)
    add("concat_bool", "concat", [rng.random((2, 3)) > .5, rng.random((2, 2)) > .5], axis=1)
    add("concat_mismatch_rejected", "concat", [a1, f32(rng, (2, 3, 5))], axis=1)

    # ---- predicates (cpu_predicate.cpp:22-50)
    pa = np.array([[0.0, -0.0, np.nan, 1.0, -np.inf, 2.5]], np.float32)
    pb = np.array([[0.0], [np.nan], [2.5]], np.float32)
    pia = rng.integers(-3, 4, (4, 1, 6)).astype(np.int32)
    pib = rng.integers(-3, 4, (5, 6)).astype(np.int32)
    pba, pbb = rng.random((3, 1)) > .5, rng.random((1, 4)) > .5
    for name in ("equal", "not_equal", "less", "less_equal", "greater", "greater_equal"):
        add(f"{name}_f32", name, [pa, pb])
        add(f"{name}_i32", name, [pia, pib])
        add(f"{name}_bool", name, [pba, pbb])
    for name in ("logical_and", "logical_or", "logical_xor"):
        add(f"{name}", name, [pba, pbb])
    add("logical_not", "logical_not", [pba])
    add("logical_and_f32_rejected", "logical_and", [pa, pa])
    add("equal_mixed_rejected", "equal", [pa, pia])
    cond = rng.random((3, 1, 6)) > .5
    add("where_f32", "where", [cond, pa, pb[:, :1]])
    add("where_i32", "where", [cond, pib[:1], np.int32(-9) * np.ones((), np.int32)])
    add("where_bool", "where", [cond, pba[:, :1], ~pba[:, :1]])
    add("where_cond_rejected", "where", [pa, pa, pa])

    # ---- any / all (cpu_predicate.cpp:52-70)
    xb = rng.random((3, 4, 5)) > .7
    for name in ("any", "all"):
        for axes in ([0], [1], [2], [0, 2], [], [0, 1, 2], [-1]):
            add(f"{name}_axes_{'_'.join(map(str, axes)) or 'none'}", name, [xb], axes=axes)
        add(f"{name}_empty", name, [np.zeros((2, 0), bool)], axes=[1])
        add(f"{name}_f32_rejected", name, [pa], axes=[1])

    # ---- masked_select (cpu_predicate.cpp:72-96)
    mx = f32(rng, (4, 5, 3))
    add("masked_select_leading", "masked_select", [mx, rng.random((4,)) > .5])
    add("masked_select_two", "masked_select", [mx, rng.random((4, 5)) > .5])
    add("masked_select_full", "masked_select", [mx, rng.random((4, 5, 3)) > .5])
    add("masked_select_none", "masked_select", [mx, np.zeros((4, 5), bool)])
    add("masked_select_i32", "masked_select", [pib, pib > 0])
    add("masked_select_bool", "masked_select", [xb, xb[:, :, 0]])
    add("masked_select_shape_rejected", "masked_select", [mx, np.ones((5,), bool)])
    big = f32(rng, (3000, 2))
    add("masked_select_chunks", "masked_select", [big, rng.random((3000,)) > .4])
    suite_tables(add)
    folded_shapes(add)
    return c


def python_route(shape, axis):
    """The backend request the reference's Python layer makes for
    x.sum/max/mean(axis) (python/tensorcx/tensor.py:508-529): one axis (or a
    scalar's 0/-1) goes to the single-axis op, anything else to the axes op."""
    rank = len(shape)
    if axis is None:
        axes, scalar = tuple(range(rank)), rank == 0
    else:
        single = isinstance(axis, int)
        axes = (axis,) if single else tuple(axis)
        scalar = rank == 0 and single and axis in (0, -1)
        if scalar:
            axes = ()
    if scalar or len(axes) == 1:
        return {"axis": axes[0] if axes else 0}
    return {"axes": list(axes)}


def label(shape, axis):
    dims = "x".join(map(str, shape)) or "scalar"
    if axis is None:
        return f"{dims}_all"
    if isinstance(axis, int):
        return f"{dims}_a{axis}"
    return f"{dims}_axes{'_'.join(map(str, axis)) or 'none'}"


def suite_tables(add):
    """Case tables of the reference's device-generic suites, with their own
    inputs: tests/python/test_multi_axis_reductions.py:19-27 (values
    np.resize([-5, -1, 0, 2, 7]) in float32 and int32),
    test_int32_primitives.py:24,95-98 (the int32 EDGES), test_batched_matmul.py:
    14-28 (U(-1, 1) from seed 741 per case) and test_inference_ops.py:15-16,
    55-101 (normal draws from seeds 31, 4/5 and 9/6)."""
    multi_axis = [
        ((2, 3, 4), None), ((2, 3, 4), ()), ((2, 3, 4), (0, 2)),
        ((2, 3, 4), (2, 0)), ((2, 3, 4), (-1, 0)), ((2, 3, 4), (0, 1, 2)),
        ((2, 3, 4), (0, 1)), ((2, 3, 4), (1, 2)), ((2, 3, 4), (1,)),
        ((2, 3, 4), -1), ((1, 1, 1), (0, 2)), ((257, 2, 3), (1, 2)),
        ((2, 3, 257), (0, 2)), ((0, 2, 3), (1, 2)), ((2, 0, 3), (0, 2)),
        ((2, 0, 3), (1, 2)), ((2, 0, 3), None), ((2, 0, 3), ()),
        ((0, 2, 0), (0, 2)), ((0,), None), ((), None), ((), ()), ((), 0), ((), -1),
    ]
    for shape, axis in multi_axis:
        for dtype in (np.float32, np.int32):
            values = np.resize(np.array([-5, -1, 0, 2, 7], dtype=dtype), shape)
            for op in ("sum", "max", "mean"):
                add(f"suite_multi_axis_{op}_{np.dtype(dtype).name}_{label(shape, axis)}", op, [values],
                    **python_route(shape, axis))
    edges = np.array([-2**31, 2**31 - 1, -16777217, 16777217, -1, 0, 1, 65537], dtype=np.int32)
    int32_tables = [((2, 3, 257), 0), ((2, 3, 257), 1), ((3, 257), -1),
                    ((2, 3, 257), (0, 2)), ((2, 3, 257), (2, 0)), ((3, 257), None),
                    ((2, 3), ()), ((2, 0, 3), 1), ((0, 2, 3), (1, 2)),
                    ((0, 2, 3), (0, 2)), ((2, 0, 3), None), ((), 0), ((), -1), ((), None)]
    for shape, axis in int32_tables:
        for op in ("sum", "max"):
            add(f"suite_int32_{op}_{label(shape, axis)}", op, [np.resize(edges, shape)], **python_route(shape, axis))
    batched = [
        ((3,), (3,)), ((2, 3), (3,)), ((3,), (3, 4)),
        ((2, 3, 4), (2, 4, 5)), ((2, 3, 4), (4, 5)),
        ((3, 4), (2, 4, 5)), ((4,), (2, 4, 5)), ((2, 3, 4), (4,)),
        ((2, 1, 3, 4), (1, 5, 4, 6)), ((1, 2, 3, 4), (3, 1, 4, 5)),
        ((2, 1, 1, 3, 4), (1, 5, 1, 4, 2)),
        ((2, 17, 19), (1, 19, 33)), ((2, 33, 17), (2, 17, 1)),
        ((0,), (0,)), ((2, 0), (0,)), ((0,), (0, 3)),
        ((2, 3, 0), (1, 0, 4)), ((0, 3, 4), (1, 4, 2)),
        ((1, 3, 4), (0, 4, 2)), ((2, 0, 4), (2, 4, 3)),
        ((2, 3, 4), (2, 4, 0)), ((0, 2, 3, 0), (1, 2, 0, 4)),
        ((2, 1, 0, 3), (1, 5, 3, 4)), ((3,), (0, 3, 4)),
        ((0, 2, 3), (3,)), ((2, 1, 3, 4), (5, 4, 2)),
    ]
    for shapes in batched:
        rng = np.random.default_rng(741)
        a, b = (rng.uniform(-1, 1, s).astype(np.float32) for s in shapes)
        add(f"suite_batched_matmul_{label(shapes[0], None)}_{label(shapes[1], None)}", "matmul", [a, b])

    def normal(shape, seed=31):
        return np.random.default_rng(seed).normal(size=shape).astype(np.float32)

    for shape, out in [((3,), 4), ((2, 3), 5), ((2, 1, 4, 3), 2), ((0, 3), 2), ((2, 0), 3), ((2, 3), 0),
                       ((0,), 2)]:
        a, w, b = normal(shape), normal((out, shape[-1]), 4), normal((out,), 9)
        add(f"suite_linear_{label(shape, None)}_out{out}", "linear", [a, w])
        add(f"suite_linear_bias_{label(shape, None)}_out{out}", "linear", [a, w, b])
    for shape, axis in [((2, 3, 4), -1), ((2, 3, 4), 1), ((2, 3, 4), 0), ((3,), -1), ((), 0), ((), -1),
                        ((0, 3), 1), ((2, 0, 3), 1)]:
        a = normal(shape)
        pshape = (shape[axis],) if shape else ()
        w, b = normal(pshape, 5), normal(pshape, 6)
        add(f"suite_affine_rmsnorm_w_{label(shape, axis)}", "affine_rmsnorm", [a, w], axis=axis, has_weight=True)
        add(f"suite_affine_layernorm_w_{label(shape, axis)}", "affine_layernorm", [a, w], axis=axis,
            has_weight=True)
        add(f"suite_affine_layernorm_wb_{label(shape, axis)}", "affine_layernorm", [a, w, b], axis=axis,
            has_weight=True, has_bias=True)
        add(f"suite_affine_layernorm_b_{label(shape, axis)}", "affine_layernorm", [a, b], axis=axis,
            has_bias=True)


def folded_shapes(add):
    """High-rank requests that the hip device folds before launching (size-1
    axes dropped, neighbouring axes of one kind merged): the selection of
    tests/python/test_multi_axis_reductions.py:143-149 at rank 64, selections that fold
    into one long row or into more axes than 8, a rank-12 broadcast, and a
    batched matmul whose batch axes alternate between the operands."""
    rng = np.random.default_rng(20261202)
    # NumPy arrays stop at 64 axes; the rank-300 case itself runs in the GPU
    # tests through reshape.
    high = np.arange(6, dtype=np.float32).reshape((2,) + (1,) * 62 + (3,))
    for op in ("sum", "max", "mean"):
        add(f"fold_rank64_{op}", op, [high], axes=[63, 0])
    add("fold_rank64_sum_i32", "sum", [high.astype(np.int32)], axes=[63, 0])
    add("fold_rank64_min", "min", [high], axes=[63, 0])
    add("fold_rank64_argmax", "argmax", [high], axes=[0, 63])
    long_row = f32(rng, (70, 1, 1, 90))
    for op in ("sum", "mean", "max"):
        add(f"fold_long_row_{op}", op, [long_row], axes=[0, 3])
    add("fold_long_row_argmax", "argmax", [long_row], axes=[0, 3])
    alternating = f32(rng, (2, 3, 1, 2, 3, 2, 1, 3, 2, 3, 2))
    for op in ("sum", "max", "mean"):
        add(f"fold_alternating_{op}", op, [alternating], axes=[0, 3, 5, 8, 10])
    add("fold_alternating_min", "min", [alternating], axes=[1, 4, 7, 9])
    add("fold_alternating_argmax", "argmax", [alternating], axes=[1, 4, 7, 9])
    add("fold_alternating_sum_i32", "sum",
        [rng.integers(-2**31, 2**31 - 1, (2, 3, 1, 2, 3, 2, 1, 3, 2, 3, 2), dtype=np.int64).astype(np.int32)],
        axes=[0, 3, 5, 8, 10])
    lhs_shape = (2, 1, 3, 1, 2, 1, 2, 1, 3, 1, 2, 2)
    rhs_shape = (1, 2, 1, 3, 1, 2, 1, 2, 1, 3, 2, 1)
    for op in ("add", "subtract", "multiply", "divide"):
        add(f"fold_rank12_{op}", op, [f32(rng, lhs_shape), f32(rng, rhs_shape)])
    add("fold_rank12_add_i32", "add",
        [rng.integers(-2**31, 2**31 - 1, lhs_shape, dtype=np.int64).astype(np.int32),
         rng.integers(-2**31, 2**31 - 1, rhs_shape, dtype=np.int64).astype(np.int32)])
    add("fold_batch10_matmul", "matmul", [f32(rng, (2, 1, 2, 1, 2, 1, 2, 1, 2, 1, 3, 4)),
                                          f32(rng, (1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 4, 5))])
    add("fold_batch_size1_matmul", "matmul", [f32(rng, (1, 3, 1, 1, 2, 1, 5, 6)), f32(rng, (3, 1, 1, 2, 1, 6, 4))])


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
            if isinstance(out, tuple):
                for n, o in enumerate(out):
                    arrays[f"c{index}_out{n}"] = o
                entry["outputs"] = [f"c{index}_out{n}" for n in range(len(out))]
            else:
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
