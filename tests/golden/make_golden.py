"""Write the golden fixtures under tests/golden/ from the compiled reference.

Run in a container that holds the reference tree:

    make -C oracle            # builds oracle/_ref/tensor_ops.so from tensor_ops.c
    python tests/golden/make_golden.py [--codecs]

Every expected output is produced by the reference library itself
(``oracle/_ref/tensor_ops.so``, compiled from ``tensor_ops/tensor_ops.c`` with the
reference makefile flags), driven through its C ABI with the operands
pre-broadcast as its Python layer does (``nn/__init__.py:210-279``).  Inputs are
seeded; dtype combinations follow the 45 plans of ``numerical_correctness.py:432-567``
plus BASELINE-config-shaped cases at reduced sizes and the edge-value tables.

Outputs:
  cases.json / cases.npz   operator cases (inputs + reference outputs)
  codecs.npz               exhaustive decoder tables and 2^32 encoder digests (--codecs)
"""
from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def mixed_floats(rng, shape):
    """numerical_correctness.py:123-131: 50% U(-10,10), 25% U(-1e3,1e3), 25% U(-0.01,0.01)."""
    n = int(np.prod(shape))
    parts = [rng.uniform(-10, 10, n), rng.uniform(-1000, 1000, n), rng.uniform(-0.01, 0.01, n)]
    pick = rng.choice(3, size=n, p=[0.5, 0.25, 0.25])
    return np.select([pick == 0, pick == 1, pick == 2], parts).reshape(shape)


def bf16_bits(x):
    """Round-to-nearest-even f32 -> bf16 bits (used only to make inputs)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def gen(rng, shape, dt):
    """Inputs per numerical_correctness.py:110-138, in storage form."""
    shape = tuple(shape)
    if dt == "int4":
        return rng.integers(-7, 7, shape).astype(np.int8)
    if dt == "int8":
        return rng.integers(-120, 120, shape).astype(np.int8)
    if dt in ("int16", "int32", "int64", "uint8"):
        return rng.integers(-1000, 1000, shape).astype(O.STORAGE[O.NAMES[dt]])
    if dt.startswith("float8"):
        return rng.integers(0, 256, shape).astype(np.uint8)
    raw = mixed_floats(rng, shape)
    if dt == "bfloat16":
        return bf16_bits(raw)
    if dt == "float16":
        return raw.astype(np.float16).view(np.uint16)
    if dt == "float64":
        return raw
    return raw.astype(np.float32)


class Writer:
    def __init__(self):
        self.cases = []
        self.arrays = {}

    def add(self, name, op, ins, dts, out_dt, out, **params):
        assert name not in {c["name"] for c in self.cases}, name
        keys = []
        for i, a in enumerate(ins):
            if a is None:
                keys.append(None)
                continue
            k = f"{name}__in{i}"
            self.arrays[k] = np.asarray(a)
            keys.append(k)
        if isinstance(out, (tuple, list)):          # several outputs (DynamicQuantizeLinear)
            outk = [f"{name}__out{i}" for i in range(len(out))]
            for k, a in zip(outk, out):
                self.arrays[k] = np.asarray(a)
        else:
            outk = f"{name}__out"
            self.arrays[outk] = out
        self.cases.append({"name": name, "op": op, "inputs": keys, "dtypes": dts,
                           "out_dtype": out_dt, "out": outk, "params": params})

    def save(self):
        with open(os.path.join(HERE, "cases.json"), "w") as f:
            json.dump(self.cases, f, indent=1)
        np.savez_compressed(os.path.join(HERE, "cases.npz"), **self.arrays)


def run_case(ref, w, name, op, shapes, dts, out_dt, params, rng):
    ins = [gen(rng, s, d) if s is not None else None for s, d in zip(shapes, dts)]
    if op in ("quantize_linear", "dequantize_linear"):
        # numerical_correctness.py:278-282: scale = |s| + 1e-4, zero point rounded (and clipped).
        s = np.abs(ins[1].astype(np.float64)) + 1e-4
        ins[1] = s.astype(O.STORAGE[O.NAMES[dts[1]]])
        z = np.round(ins[2].astype(np.float64))
        if op == "quantize_linear":
            z = np.clip(z, -128, 127)
        ins[2] = z.astype(O.STORAGE[O.NAMES[dts[2]]])
    out = call(ref, op, ins, dts, out_dt, params)
    w.add(name, op, ins, dts, out_dt, out, **params)


def call(lib, op, ins, dts, out_dt, params):
    if op in ("relu", "abs", "cos"):
        return lib.unary(op, ins[0], dts[0], out_dt)
    if op in ("add", "sub", "mul", "div"):
        return lib.binary(op, ins[0], dts[0], ins[1], dts[1], out_dt)
    if op in ("quantize_linear", "dequantize_linear"):
        s, z = ins[1], ins[2]
        if "axis" in params and s.ndim == 1 and ins[0].ndim > 1:   # nn/Operators.py:439-445
            shp = [1] * ins[0].ndim
            shp[params["axis"]] = s.size
            s, z = s.reshape(shp), z.reshape(shp)
        return lib.qdq(op.split("_")[0], ins[0], dts[0], s, dts[1], z, dts[2], out_dt)
    if op == "conv2d":
        return lib.conv(ins[0], dts[0], ins[1], dts[1], ins[2], dts[2], out_dt,
                        params["pads"], params["strides"], params["dilations"], params["group"])
    if op == "max_pool":
        return lib.maxpool(ins[0], dts[0], out_dt, params["kernel_shape"], params["pads"],
                           params["strides"], params.get("dilations", [1, 1]))
    if op == "gemm":
        return lib.gemm(ins[0], dts[0], ins[1], dts[1], ins[2], dts[2], out_dt,
                        params["alpha"], params["beta"], params["transA"], params["transB"])
    if op == "softmax":
        return lib.softmax(ins[0], dts[0], out_dt, params["axis"])
    if op in ("flatten", "reshape"):
        return lib.flatten(ins[0], dts[0], tuple(params["shape"]), out_dt, name=op)
    if op == "global_average_pool":
        return lib.gap(ins[0], dts[0], out_dt)
    if op == "dynamic_quantize_linear":
        return lib.dql(ins[0], dts[0], params.get("zp_dtype", "uint8"))
    raise ValueError(op)


# numerical_correctness.py:432-567 (shapes, dtypes, output dtype, attributes).
PLANS = [
    ("add", [(64, 64), (64, 64)], ["float32", "float32"], "float32", {}),
    ("sub", [(64, 64), (64, 64)], ["float16", "float16"], "float16", {}),
    ("mul", [(64, 64), (64, 64)], ["bfloat16", "bfloat16"], "bfloat16", {}),
    ("div", [(64, 64), (64, 64)], ["float32", "float32"], "float32", {}),
    ("div", [(64, 64), (64, 64)], ["float16", "float32"], "float16", {}),
    ("mul", [(64, 64), (64, 64)], ["int8", "int8"], "int32", {}),
    ("add", [(64, 64), (64, 64)], ["int8", "int32"], "int32", {}),
    ("mul", [(64, 64), (64, 64)], ["int4", "int4"], "int16", {}),
    ("mul", [(64, 64), (64, 64)], ["float32", "int4"], "float32", {}),
    ("add", [(64, 64), (64, 64)], ["float32", "int4"], "float32", {}),
    ("mul", [(64, 64), (64, 64)], ["float16", "int8"], "float16", {}),
    ("add", [(64, 64), (64, 64)], ["float16", "int8"], "float16", {}),
    ("mul", [(64, 64), (64, 64)], ["float32", "int8"], "float32", {}),
    ("add", [(64, 64), (64, 64)], ["float32", "int8"], "float32", {}),
    ("add", [(64, 64), (64, 64)], ["float16", "float32"], "float32", {}),
    ("mul", [(64, 64), (64, 64)], ["bfloat16", "float32"], "float32", {}),
    ("div", [(64, 64), (64, 64)], ["float32", "float16"], "float16", {}),
    ("mul", [(64, 64), (64, 64)], ["float8_e4m3", "float8_e4m3"], "float16", {}),
    ("add", [(64, 64), (64, 64)], ["float8_e5m2", "float16"], "float16", {}),
    ("mul", [(64, 64), (64, 64)], ["float8_e4m3", "float8_e5m2"], "float32", {}),
    ("mul", [(64, 64), (64, 64)], ["bfloat16", "bfloat16"], "bfloat16", {}),
    ("add", [(64, 64), (64, 64)], ["float8_e4m3", "float16"], "float16", {}),
    ("div", [(10, 10, 10), (10, 1)], ["float32", "float32"], "float32", {}),
    ("sub", [(4, 1, 16), (16,)], ["float32", "float32"], "float32", {}),
    ("abs", [(100,)], ["float8_e4m3"], "float8_e4m3", {}),
    ("cos", [(100,)], ["float32"], "float32", {}),
    ("cos", [(100,)], ["float16"], "float16", {}),
    ("relu", [(100, 100)], ["float32"], "float32", {}),
    ("relu", [(100, 100)], ["float16"], "float16", {}),
    ("relu", [(100, 100)], ["int8"], "int8", {}),
    ("quantize_linear", [(64, 64), (1,), (1,)], ["float32", "float32", "float32"], "int8", {}),
    ("quantize_linear", [(2, 16, 4, 4), (1, 16, 1, 1), (1, 16, 1, 1)],
     ["float32", "float32", "float32"], "int8", {}),
    ("dequantize_linear", [(64, 64), (1,), (1,)], ["int8", "float32", "float32"], "float32", {}),
    ("conv2d", [(1, 1, 5, 5), (1, 1, 3, 3), (1,)], ["float32", "float32", "float32"], "float32",
     {"pads": [0, 0, 0, 0], "strides": [1, 1], "dilations": [1, 1], "group": 1}),
    ("max_pool", [(1, 1, 4, 4)], ["float32"], "float32",
     {"kernel_shape": [2, 2], "pads": [0, 0, 0, 0], "strides": [2, 2]}),
    ("gemm", [(2, 3), (3, 4), (4,)], ["float32", "float32", "float32"], "float32",
     {"alpha": 1.0, "beta": 1.0, "transA": 0, "transB": 0}),
    ("softmax", [(2, 5)], ["float32"], "float32", {"axis": 1}),
    ("conv2d", [(1, 2, 7, 7), (4, 2, 3, 3), (4,)], ["float16", "float16", "float32"], "float32",
     {"pads": [1, 1, 1, 1], "strides": [1, 1], "dilations": [1, 1], "group": 1}),
    ("conv2d", [(1, 4, 8, 8), (8, 4, 3, 3), (8,)], ["float8_e4m3", "float8_e4m3", "float16"],
     "float16", {"pads": [0, 0, 0, 0], "strides": [2, 2], "dilations": [1, 1], "group": 1}),
    ("conv2d", [(1, 8, 6, 6), (8, 1, 3, 3), None], ["bfloat16", "bfloat16", "float32"], "bfloat16",
     {"pads": [1, 1, 1, 1], "strides": [1, 1], "dilations": [1, 1], "group": 8}),
    ("gemm", [(16, 32), (32, 8), (8,)], ["float16", "float16", "float32"], "float32",
     {"alpha": 1.0, "beta": 1.0, "transA": 0, "transB": 0}),
    ("gemm", [(8, 16), (8, 16), None], ["float8_e5m2", "float8_e4m3", "float32"], "bfloat16",
     {"alpha": 0.5, "beta": 0.0, "transA": 0, "transB": 1}),
    ("max_pool", [(1, 2, 16, 16)], ["bfloat16"], "bfloat16",
     {"kernel_shape": [2, 2], "pads": [0, 0, 0, 0], "strides": [2, 2]}),
    ("softmax", [(4, 64)], ["float16"], "float16", {"axis": -1}),
    ("softmax", [(2, 10)], ["float8_e4m3"], "float8_e4m3", {"axis": 1}),
]


def edge_cases(ref, w):
    """Known-answer inputs at the codecs' rounding and saturation boundaries
    (ties, the e4m3 / e5m2 extremes, NaN and infinities), answered by the reference."""
    f32 = np.float32
    xq = np.array([0.3, 0.5, 1.5, 2.5, -2.5, 3.5, 17, 18, 19, 448, 464, 480, 1000, 57344, 61439,
                   61440, 65536, np.inf, -np.inf, np.nan, -0.0], dtype=f32)
    one, zero = np.ones(1, f32), np.zeros(1, f32)
    for dt in ("float8_e4m3", "float8_e5m2", "int8", "uint8", "int4", "int16", "int32", "int64"):
        zdt = "float32"
        out = ref.qdq("quantize", xq, "float32", one, "float32", zero, zdt, dt)
        w.add(f"kat_quant_{dt}", "quantize_linear", [xq, one, zero], ["float32", "float32", zdt],
              dt, out)
    xs = np.array([0.01, 2.0 ** -7, 2.0 ** -9, 2.0 ** -6, 1e-5, 2.0 ** -14, 2.0 ** -16,
                   2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 65504, 65519, 65520, 1e9, -1e9,
                   -0.0, np.inf, np.nan], dtype=f32)
    for dt in ("float8_e4m3", "float8_e5m2", "float16", "bfloat16", "int8", "uint8", "int64"):
        out = ref.binary("sub", xs, "float32", zero, "float32", dt)
        w.add(f"kat_sub0_{dt}", "sub", [xs, zero], ["float32", "float32"], dt, out)
    xr = np.array([np.nan, -0.0, -1.0, 0.0, 1.0, -np.inf, np.inf, 1e-45, -1e-45], dtype=f32)
    for op in ("relu", "abs"):
        out = ref.unary(op, xr, "float32", "float32")
        w.add(f"kat_{op}_f32", op, [xr], ["float32"], "float32", out)
    xi = np.array([-(2 ** 63), 2 ** 63 - 1, -5, 0, 7, -(2 ** 31), 2 ** 40], dtype=np.int64)
    for op in ("relu", "abs"):
        for dt in ("int64", "int32", "int8", "float32", "float16"):
            out = ref.unary(op, xi, "int64", dt)
            w.add(f"kat_{op}_i64_{dt}", op, [xi], ["int64"], dt, out)
    # Integer division corner cases and wrap-around (tensor_ops.c:610-684).
    a = np.array([7, -7, 7, -7, 5, -5, 0, 2 ** 62, -(2 ** 62), 9, 2 ** 40], dtype=np.int64)
    b = np.array([2, 2, -2, -2, 0, 0, 0, 4, 4, 3, 2 ** 30], dtype=np.int64)
    for op in ("add", "sub", "mul", "div"):
        for dt in ("int64", "int32", "int8", "uint8", "int4", "int16"):
            out = ref.binary(op, a, "int64", b, "int64", dt)
            w.add(f"kat_int_{op}_{dt}", op, [a, b], ["int64", "int64"], dt, out)
    # float inputs into the integer path: rintf then the x86 cast.
    fa = np.array([2.5, 3.5, -2.5, 1e10, -1e10, 1e19, -1e19, np.inf, np.nan, 0.49999997],
                  dtype=f32)
    fz = np.zeros_like(fa)
    for dt in ("int32", "int64", "int8", "uint8"):
        out = ref.binary("add", fa, "float32", fz, "float32", dt)
        w.add(f"kat_fint_add_{dt}", "add", [fa, fz], ["float32", "float32"], dt, out)
    # MaxPool: NaN never wins, +-0 order, an all-padding window gives -inf.
    xp = np.array([[[[np.nan, -0.0, 0.0, -1.0], [0.0, -0.0, np.nan, np.nan],
                     [-np.inf, -np.inf, 3.0, 2.0], [np.nan, np.nan, np.nan, np.nan]]]], dtype=f32)
    out = ref.maxpool(xp, "float32", "float32", [2, 2], [0, 0, 0, 0], [2, 2])
    w.add("kat_maxpool_specials", "max_pool", [xp], ["float32"], "float32", out,
          kernel_shape=[2, 2], pads=[0, 0, 0, 0], strides=[2, 2])
    out = ref.maxpool(xp, "float32", "float32", [1, 1], [2, 2, 2, 2], [1, 1])
    w.add("kat_maxpool_padonly", "max_pool", [xp], ["float32"], "float32", out,
          kernel_shape=[1, 1], pads=[2, 2, 2, 2], strides=[1, 1])
    # Cos over a wide range (LUT replica must be bit-exact), incl. multiples of pi/2.
    rng = np.random.default_rng(11)
    xc = np.concatenate([rng.uniform(-40, 40, 4000), rng.uniform(-1e5, 1e5, 500),
                         np.arange(-64, 65) * (np.pi / 4), [0.0, -0.0, 2 * np.pi, 1e-30, 3e38]])
    xc = xc.astype(f32)
    for dt in ("float32", "float16", "float64", "bfloat16"):
        out = ref.unary("cos", xc, "float32", dt)
        w.add(f"cos_range_{dt}", "cos", [xc], ["float32"], dt, out)
    xc64 = rng.uniform(-50, 50, 2000)
    out = ref.unary("cos", xc64, "float64", "float64")
    w.add("cos_range_f64in", "cos", [xc64], ["float64"], "float64", out)


def config_cases(ref, w):
    """BASELINE configs at reduced sizes (same distributions and dtype paths)."""
    rng = np.random.default_rng(0)
    # Config 1: chain Add -> Mul -> Sub -> Div -> Relu -> Abs -> Cos with B [64,1,1].
    A = rng.uniform(-4, 4, (2, 64, 7, 7)).astype(np.float32)
    B = rng.uniform(-4, 4, (64, 1, 1)).astype(np.float32)
    Bd = (np.sign(B) * np.maximum(np.abs(B), 0.1)).astype(np.float32)
    t = ref.binary("add", A, "float32", B, "float32", "float32")
    w.add("c1_add", "add", [A, B], ["float32", "float32"], "float32", t)
    t2 = ref.binary("mul", t, "float32", B, "float32", "float32")
    w.add("c1_mul", "mul", [t, B], ["float32", "float32"], "float32", t2)
    t3 = ref.binary("sub", t2, "float32", B, "float32", "float32")
    w.add("c1_sub", "sub", [t2, B], ["float32", "float32"], "float32", t3)
    t4 = ref.binary("div", t3, "float32", Bd, "float32", "float32")
    w.add("c1_div", "div", [t3, Bd], ["float32", "float32"], "float32", t4)
    t5 = ref.unary("relu", t4, "float32", "float32")
    w.add("c1_relu", "relu", [t4], ["float32"], "float32", t5)
    t6 = ref.unary("abs", t5, "float32", "float32")
    w.add("c1_abs", "abs", [t5], ["float32"], "float32", t6)
    t7 = ref.unary("cos", t6, "float32", "float32")
    w.add("c1_cos", "cos", [t6], ["float32"], "float32", t7)
    I = rng.integers(-(2 ** 31), 2 ** 31 - 1, (2, 64, 7, 7), dtype=np.int64).astype(np.int32)
    for dt in ("float64", "float32"):
        out = ref.binary("add", I, "int32", B, "float32", dt)
        w.add(f"c1_i32add_{dt}", "add", [I, B], ["int32", "float32"], dt, out)
    I2 = rng.integers(-(2 ** 20), 2 ** 20, (2, 64, 7, 7)).astype(np.int32)
    out = ref.binary("add", I2, "int32", B, "float32", "float32")
    w.add("c1_i32small_f32", "add", [I2, B], ["int32", "float32"], "float32", out)

    # Config 2: Q/DQ round trips on [4,16,64] with outliers.
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1.5, (4, 16, 64))
    x[rng.random(x.shape) < 0.01] *= 20
    x = x.astype(np.float32)
    mn, mx = float(x.min()), float(x.max())
    s_u8 = np.array([(mx - mn) / 255], np.float32)
    z_u8 = np.array([np.clip(np.round(-mn / float(s_u8[0])), 0, 255)], np.uint8)
    s_ax = (np.abs(x).max(axis=(0, 2)) / 127).astype(np.float32)
    z_ax = np.zeros(16, np.int8)
    amax = float(np.abs(x).max())
    variants = [
        ("u8", s_u8, "float32", z_u8, "uint8", "uint8", None),
        ("i8axis", s_ax, "float32", z_ax, "int8", "int8", 1),
        ("e4m3", np.array([amax / 448], np.float32), "float32", np.zeros(1, np.uint8),
         "float8_e4m3", "float8_e4m3", None),
        ("e5m2", np.array([amax / 57344], np.float32), "float32", np.zeros(1, np.uint8),
         "float8_e5m2", "float8_e5m2", None),
        ("e4m3_stress", np.array([amax / 448 / 16], np.float32), "float32",
         np.zeros(1, np.uint8), "float8_e4m3", "float8_e4m3", None),
        ("e5m2_stress", np.array([amax / 57344 / 16], np.float32), "float32",
         np.zeros(1, np.uint8), "float8_e5m2", "float8_e5m2", None),
    ]
    for tag, s, sdt, z, zdt, ydt, axis in variants:
        params = {"axis": axis} if axis is not None else {}
        y = call(ref, "quantize_linear", [x, s, z], ["float32", sdt, zdt], ydt, params)
        w.add(f"c2_q_{tag}", "quantize_linear", [x, s, z], ["float32", sdt, zdt], ydt, y, **params)
        xr = call(ref, "dequantize_linear", [y, s, z], [ydt, sdt, zdt], "float32", params)
        w.add(f"c2_dq_{tag}", "dequantize_linear", [y, s, z], [ydt, sdt, zdt], "float32", xr,
              **params)

    # Config 3: Gemm with bias (f32 and f16), transB=1, plus WOQ int8 DQ -> Gemm.
    rng = np.random.default_rng(2)
    for (M, N, K) in ((64, 48, 96), (33, 17, 70)):
        a = rng.normal(0, 1 / np.sqrt(K), (M, K)).astype(np.float32)
        b = rng.normal(0, 1 / np.sqrt(K), (N, K)).astype(np.float32)
        c = rng.normal(0, 1 / 64, (N,)).astype(np.float32)
        for dt in ("float32", "float16"):
            aa, bb = (a, b) if dt == "float32" else (a.astype(np.float16).view(np.uint16),
                                                      b.astype(np.float16).view(np.uint16))
            out = ref.gemm(aa, dt, bb, dt, c, "float32", dt, 1.0, 1.0, 0, 1)
            w.add(f"c3_gemm_{dt}_{M}x{N}x{K}", "gemm", [aa, bb, c], [dt, dt, "float32"], dt, out,
                  alpha=1.0, beta=1.0, transA=0, transB=1)
    for ta in (0, 1):
        for tb in (0, 1):
            a = rng.normal(0, 1, (40, 24) if not ta else (24, 40)).astype(np.float32)
            b = rng.normal(0, 1, (24, 36) if not tb else (36, 24)).astype(np.float32)
            c = rng.normal(0, 1, (40, 1)).astype(np.float32)
            out = ref.gemm(a, "float32", b, "float32", c, "float32", "float32", 0.75, -1.5, ta, tb)
            w.add(f"c3_gemm_t{ta}{tb}", "gemm", [a, b, c], ["float32"] * 3, "float32", out,
                  alpha=0.75, beta=-1.5, transA=ta, transB=tb)
    bw = rng.normal(0, 1 / 64, (48, 96))
    sw = (np.abs(bw).max(axis=1) / 127).astype(np.float32)
    bq = np.clip(np.rint(bw / sw[:, None]), -127, 127).astype(np.int8)
    deq = call(ref, "dequantize_linear", [bq, sw, np.zeros(48, np.int8)],
               ["int8", "float32", "int8"], "float32", {"axis": 0})
    w.add("c3_woq_dq", "dequantize_linear", [bq, sw, np.zeros(48, np.int8)],
          ["int8", "float32", "int8"], "float32", deq, axis=0)
    a = rng.normal(0, 1 / 64, (16, 96)).astype(np.float32)
    cb = rng.normal(0, 1 / 64, (48,)).astype(np.float32)
    out = ref.gemm(a, "float32", deq, "float32", cb, "float32", "float32", 1.0, 1.0, 0, 1)
    w.add("c3_woq_gemm", "gemm", [a, deq, cb], ["float32"] * 3, "float32", out,
          alpha=1.0, beta=1.0, transA=0, transB=1)

    # Config 4: conv stem / 3x3 / 1x1 / maxpool at reduced batch and spatial size.
    rng = np.random.default_rng(3)
    convs = [("stem", (2, 3, 32, 32), (16, 3, 7, 7), [3, 3, 3, 3], [2, 2]),
             ("3x3", (2, 16, 14, 14), (16, 16, 3, 3), [1, 1, 1, 1], [1, 1]),
             ("1x1", (2, 16, 14, 14), (32, 16, 1, 1), [0, 0, 0, 0], [1, 1]),
             ("dil", (1, 4, 11, 13), (6, 2, 3, 3), [2, 1, 0, 2], [2, 1])]
    for tag, xs, ws, pads, strides in convs:
        x = rng.normal(0, 1, xs).astype(np.float32)
        fan = ws[1] * ws[2] * ws[3]
        wt = rng.normal(0, np.sqrt(2 / fan), ws).astype(np.float32)
        bias = rng.normal(0, 1 / 64, (ws[0],)).astype(np.float32)
        dil = [2, 1] if tag == "dil" else [1, 1]
        group = 2 if tag == "dil" else 1
        out = ref.conv(x, "float32", wt, "float32", bias, "float32", "float32", pads, strides,
                       dil, group)
        w.add(f"c4_conv_{tag}", "conv2d", [x, wt, bias], ["float32"] * 3, "float32", out,
              pads=pads, strides=strides, dilations=dil, group=group)
    x = rng.normal(0, 1, (2, 8, 24, 24)).astype(np.float32)
    out = ref.maxpool(x, "float32", "float32", [3, 3], [1, 1, 1, 1], [2, 2])
    w.add("c4_maxpool", "max_pool", [x], ["float32"], "float32", out,
          kernel_shape=[3, 3], pads=[1, 1, 1, 1], strides=[2, 2])
    x = rng.normal(0, 1, (1, 3, 13, 11)).astype(np.float32)
    out = ref.maxpool(x, "float32", "float32", [3, 2], [1, 0, 2, 1], [2, 1], [2, 1])
    w.add("c4_maxpool_dil", "max_pool", [x], ["float32"], "float32", out,
          kernel_shape=[3, 2], pads=[1, 0, 2, 1], strides=[2, 1], dilations=[2, 1])

    # Config 5: softmax rows (N(0,3) logits) and a non-last axis.
    rng = np.random.default_rng(4)
    x = rng.normal(0, 3, (4, 3000)).astype(np.float32)
    out = ref.softmax(x, "float32", "float32", 1)
    w.add("c5_softmax_rows", "softmax", [x], ["float32"], "float32", out, axis=1)
    x = rng.normal(0, 3, (3, 50, 7)).astype(np.float32)
    out = ref.softmax(x, "float32", "float32", 1)
    w.add("c5_softmax_mid", "softmax", [x], ["float32"], "float32", out, axis=1)
    x = rng.normal(0, 3, (2, 1000)).astype(np.float32)
    out = ref.softmax(x, "float32", "float64", -1)
    w.add("c5_softmax_f64out", "softmax", [x], ["float32"], "float64", out, axis=-1)


def next_row_cases(ref, w):
    """Operators next to the hot path: GlobalAveragePool, Flatten / Reshape and
    DynamicQuantizeLinear (tensor_ops.c:1289-1299, 2844-2868, 3760-3809)."""
    rng = np.random.default_rng(5)
    for tag, shape, dt, ydt in (("f32_7x7", (2, 8, 7, 7), "float32", "float32"),
                                ("f32_odd", (2, 3, 13, 11), "float32", "float32"),
                                ("f32_56x56", (1, 4, 56, 56), "float32", "float32"),
                                ("f16", (2, 4, 5, 6), "float16", "float16"),
                                ("i8_to_f32", (2, 3, 4, 4), "int8", "float32"),
                                ("f32_to_f64", (1, 5, 9, 9), "float32", "float64")):
        x = gen(rng, shape, dt)
        w.add(f"gap_{tag}", "global_average_pool", [x], [dt], ydt, ref.gap(x, dt, ydt))
    for tag, shape, oshape, dt in (("f32", (2, 3, 4, 5), (2, 60), "float32"),
                                   ("i8", (4, 6), (24,), "int8"),
                                   ("f16_4d", (2, 8, 1, 1), (2, 8), "float16")):
        x = gen(rng, shape, dt)
        for op in ("flatten", "reshape"):
            w.add(f"{op}_{tag}", op, [x], [dt], dt, ref.flatten(x, dt, oshape, dt, name=op),
                  shape=list(oshape))
    x = rng.normal(0, 1.5, (4, 16, 64))
    x[rng.random(x.shape) < 0.01] *= 20
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0], np.float32)
    dql_inputs = [("normal", x.astype(np.float32), "float32"),
                  ("positive", np.abs(x).astype(np.float32) + 0.5, "float32"),
                  ("negative", -np.abs(x).astype(np.float32) - 0.5, "float32"),
                  ("zeros", np.zeros((3, 5), np.float32), "float32"),
                  ("ties", (np.arange(-300, 300) * 0.5).astype(np.float32), "float32"),
                  ("nan", np.concatenate([x.reshape(-1)[:200].astype(np.float32), specials[:1]]), "float32"),
                  ("inf", np.concatenate([x.reshape(-1)[:200].astype(np.float32), specials[1:3]]), "float32"),
                  ("f16", x.astype(np.float16).view(np.uint16), "float16"),
                  ("i32", rng.integers(-1000, 3000, (40, 9)).astype(np.int32), "int32")]
    for tag, xin, dt in dql_inputs:
        w.add(f"dql_{tag}", "dynamic_quantize_linear", [xin], [dt], "uint8", ref.dql(xin, dt))


def make_cases(ref):
    w = Writer()
    rng = np.random.default_rng(12345)
    for i, (op, shapes, dts, out_dt, params) in enumerate(PLANS):
        run_case(ref, w, f"plan{i:02d}_{op}", op, shapes, dts, out_dt, params, rng)
    edge_cases(ref, w)
    config_cases(ref, w)
    next_row_cases(ref, w)
    w.save()
    print(f"wrote {len(w.cases)} cases")


CHUNK = 1 << 24


def make_codecs(ref):
    """Decoder tables (exhaustive) and per-chunk digests of the 2^32 encoder sweep."""
    out = {}
    z = np.zeros(1, np.float32)
    codes16 = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    for name, dt in (("f16", "float16"), ("bf16", "bfloat16")):
        out[f"dec_{name}"] = ref.binary("sub", codes16, dt, z, "float32", "float32").view(np.uint32)
    codes8 = np.arange(256, dtype=np.uint16).astype(np.uint8)
    for name, dt in (("e4m3", "float8_e4m3"), ("e5m2", "float8_e5m2")):
        out[f"dec_{name}"] = ref.binary("sub", codes8, dt, z, "float32", "float32").view(np.uint32)
    o = O.oracle()   # only for its checksum helper (a plain weighted sum)
    for name, dt in (("f16", "float16"), ("bf16", "bfloat16"), ("e4m3", "float8_e4m3"),
                     ("e5m2", "float8_e5m2"), ("i64", "int64")):
        sums = np.zeros(256, np.uint64)
        for c in range(256):
            x = (np.arange(CHUNK, dtype=np.uint64) + c * CHUNK).astype(np.uint32).view(np.float32)
            y = ref.binary("sub", x, "float32", z, "float32", dt)
            sums[c] = o.checksum(y, c * CHUNK)
        out[f"enc_{name}_digest"] = sums
        print("digest", name, flush=True)
    np.savez_compressed(os.path.join(HERE, "codecs.npz"), **out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--codecs", action="store_true", help="also write codecs.npz (slow: ~10 min)")
    args = ap.parse_args()
    ref = O.reference()
    if ref is None:
        raise SystemExit("oracle/_ref/tensor_ops.so missing: run `make -C oracle` where the "
                         "reference tree is present")
    make_cases(ref)
    if args.codecs:
        make_codecs(ref)


if __name__ == "__main__":
    main()
