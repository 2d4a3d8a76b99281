"""Benchmark of the tensor_ops hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-suite]

Headline: QuantizeLinear -> DequantizeLinear round trips
on x f32 [32,512,1024] (seed 1, N(0,1.5) with 0.1% outliers x20) for the four
variants (a) per-tensor uint8, (b) per-axis int8 on axis 1, (c) e4m3 and
e5m2.  One step = 4 quantize + 4 dequantize launches; every launch reads and
writes buffers that are not cache-resident (8 rotating input sets and 8
rotating code sets, > 1 GB in total, so the 256 MB Infinity Cache cannot hold
them).  value = algorithmic bytes per step / time per step, inputs already in
HBM.  Algorithmic bytes per launch: 4 B in + 1 B out per element (quantize),
1 B in + 4 B out (dequantize) = 83,886,080 B.

The JSON line also carries:
  roofline      the dominant kernel's algorithmic bytes / average duration,
                measured with HIP events around each launch (a second pass of
                the same steps, so the headline timing carries no event
                overhead), against 8 TB/s;
  cpu_baseline  the reference tensor_ops.c (oracle/_ref, compiled from source)
                or the restatement, on this host's cores, on a bounded sample;
  ops           per-operator results for the other configurations
                (elementwise chain, Gemm, Conv, MaxPool, Softmax) with their
                roofline fractions.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12           # B/s
MFMA_F32 = 157.3e12         # FLOP/s dense
MFMA_F16 = 2516.6e12

E4M3, E5M2, F16, BF16, F32, F64, I4, I8, U8, I16, I32, I64 = range(12)
NP = {E4M3: np.uint8, E5M2: np.uint8, F16: np.float16, F32: np.float32, I8: np.int8, U8: np.uint8,
      I32: np.int32, F64: np.float64}


class CT(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("shape", ctypes.POINTER(ctypes.c_int)), ("ndim", ctypes.c_int),
                ("size", ctypes.c_size_t), ("dtype", ctypes.c_int)]


PT = ctypes.POINTER(CT)


class CStep(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int), ("operand", ctypes.c_int), ("reversed", ctypes.c_int)]


class Params(ctypes.Structure):
    _fields_ = [("a", ctypes.POINTER(ctypes.c_int)), ("b", ctypes.POINTER(ctypes.c_int)),
                ("c", ctypes.POINTER(ctypes.c_int)), ("d", ctypes.POINTER(ctypes.c_int))]


class ConvP(ctypes.Structure):
    _fields_ = [("pads", ctypes.POINTER(ctypes.c_int)), ("strides", ctypes.POINTER(ctypes.c_int)),
                ("dilations", ctypes.POINTER(ctypes.c_int)), ("group", ctypes.c_int)]


def ints(v):
    return (ctypes.c_int * len(v))(*v)


class Lib:
    def __init__(self, path):
        self.lib = L = ctypes.CDLL(path)
        L.create_tensor_device.restype = PT
        L.create_tensor_device.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        L.create_tensor.restype = PT
        L.create_tensor.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        L.tensor_from_host.argtypes = [PT, ctypes.c_void_p]
        L.tensor_from_host.restype = ctypes.c_int
        L.tensor_ops_hip_last_error.restype = ctypes.c_char_p
        L.tensor_ops_hip_set_stream.argtypes = [ctypes.c_void_p]
        L.free_tensor.argtypes = [PT]
        for n in ("quantize_linear_forward", "dequantize_linear_forward"):
            getattr(L, n).argtypes = [PT, PT, PT, PT]
        for n in ("add_forward", "sub_forward", "mul_forward", "div_forward"):
            getattr(L, n).argtypes = [PT, PT, PT]
        for n in ("relu_forward", "abs_forward", "cos_forward"):
            getattr(L, n).argtypes = [PT, PT]
        L.gemm_forward.argtypes = [PT, PT, PT, PT, ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.conv2d_forward.argtypes = [PT, PT, PT, PT, ctypes.POINTER(ConvP)]
        L.max_pool_forward.argtypes = [PT, PT, ctypes.POINTER(Params)]
        L.softmax_forward.argtypes = [PT, PT, ctypes.c_int]
        L.elementwise_chain_forward.argtypes = [PT, ctypes.POINTER(PT), ctypes.c_int, ctypes.POINTER(CStep),
                                                ctypes.c_int, PT]
        L.global_average_pool_forward.argtypes = [PT, PT]
        L.dynamic_quantize_linear_forward.argtypes = [PT, PT, PT, PT]
        L.dequantize_gemm_forward.argtypes = [PT, PT, PT, PT, ctypes.c_int, PT, PT, ctypes.c_float, ctypes.c_float,
                                              ctypes.c_int, ctypes.c_int]
        L.init_cos_lut()

    def dev(self, arr, dt):
        arr = np.ascontiguousarray(arr)
        shp = list(arr.shape) or [1]
        t = self.lib.create_tensor_device(ints(shp), len(shp), dt)
        if not t or self.lib.tensor_from_host(t, arr.ctypes.data) != 0:
            raise RuntimeError(self.err())
        return t

    def empty(self, shape, dt):
        t = self.lib.create_tensor_device(ints(list(shape)), len(shape), dt)
        if not t:
            raise RuntimeError(self.err())
        return t

    def err(self):
        e = self.lib.tensor_ops_hip_last_error()
        return e.decode() if e else ""

    def check(self, what):
        e = self.err()
        if e:
            raise RuntimeError(f"{what}: {e}")


# ------------------------------------------------------------------ inputs ---
def config2_input(rng):
    x = rng.normal(0, 1.5, (32, 512, 1024))
    x[rng.random(x.shape) < 0.001] *= 20
    return x.astype(np.float32)


def config2_variants(x):
    """(name, scale, zero point, code dtype, scale shape) per BASELINE configs[1]."""
    mn, mx = float(x.min()), float(x.max())
    s_u8 = np.float32((mx - mn) / 255)
    z_u8 = np.uint8(np.clip(np.round(-mn / float(s_u8)), 0, 255))
    amax = float(np.abs(x).max())
    s_ax = (np.abs(x).max(axis=(0, 2)) / 127).astype(np.float32)
    return [("u8_per_tensor", np.array([s_u8]), np.array([z_u8]), U8),
            ("i8_per_axis1", s_ax.reshape(1, 512, 1), np.zeros((1, 512, 1), np.int8), I8),
            ("e4m3", np.array([amax / 448], np.float32), np.zeros(1, np.uint8), E4M3),
            ("e5m2", np.array([amax / 57344], np.float32), np.zeros(1, np.uint8), E5M2)]


# ------------------------------------------------------------------ timing ---
class Timer:
    def __init__(self, torch):
        self.torch = torch

    def event(self):
        return self.torch.cuda.Event(enable_timing=True)


def run_headline(lib, torch, steps, warmup):
    rng = np.random.default_rng(1)
    x = config2_input(rng)
    variants = config2_variants(x)
    n = x.size
    R = 8
    X = [lib.dev(x, F32) for _ in range(R)]
    shp = list(x.shape)
    Y = [[lib.empty(shp, v[3]) for _ in range(R)] for v in variants]   # per-variant code sets
    XR = [lib.empty(shp, F32) for _ in range(R)]
    S = [lib.dev(v[1], F32) for v in variants]
    Z = [lib.dev(v[2], v[3]) for v in variants]
    L = lib.lib
    bytes_per_launch = 5 * n

    def step(k):
        # launch q reads input set q % R; the dequantize of variant v reads the
        # codes its quantize wrote one step earlier (4 launches, > 600 MB ago)
        for v in range(4):
            q = 4 * k + v
            L.quantize_linear_forward(X[q % R], S[v], Z[v], Y[v][k % R])
            L.dequantize_linear_forward(Y[v][(k - 1) % R], S[v], Z[v], XR[q % R])

    for k in range(warmup):
        step(k)
    lib.check("warmup")
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    t0.record()
    for k in range(steps):
        step(warmup + k)
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    lib.check("timed steps")
    ms = t0.elapsed_time(t1) / steps

    # Per-kernel average launch duration: `steps` back-to-back launches of one
    # kernel (rotating over the R sets) between one pair of HIP events on the
    # launch stream.
    kern = {}
    for v, var in enumerate(variants):
        def q_fn(i, v=v):
            L.quantize_linear_forward(X[i % R], S[v], Z[v], Y[v][i % R])

        def dq_fn(i, v=v):
            L.dequantize_linear_forward(Y[v][i % R], S[v], Z[v], XR[i % R])
        kern[f"quantize_f32_to_{var[0]}"] = bench_loop(torch, q_fn, steps, warm=4)
        kern[f"dequantize_{var[0]}_to_f32"] = bench_loop(torch, dq_fn, steps, warm=4)
    lib.check("per-kernel pass")
    dom = max(kern, key=kern.get)
    for t in X + [t for ys in Y for t in ys] + XR + S + Z:
        L.free_tensor(t)
    per_step_bytes = 8 * bytes_per_launch
    return {"ms_per_step": ms, "wall_s": wall, "bytes_per_step": per_step_bytes, "kernel_ms": kern,
            "dominant": dom, "bytes_per_launch": bytes_per_launch, "n": n}


def bench_loop(torch, fn, iters, warm=3, warm_ms=50.0):
    """Mean time of `iters` back-to-back calls.  The warm-up runs at least `warm`
    calls and `warm_ms` of wall time, so the GPU clocks have ramped up (a cold
    4096^3 Gemm runs ~20% slower for its first few milliseconds)."""
    t0, i = time.perf_counter(), 0
    while i < warm or (time.perf_counter() - t0) * 1e3 < warm_ms:
        fn(i)
        torch.cuda.synchronize()
        i += 1
    warm = i
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(iters):
        fn(warm + i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def run_suite(lib, torch):
    """Other configs: one line per operator, achieved vs roofline."""
    L = lib.lib
    out = []
    rng = np.random.default_rng(0)
    # Config 1: f32 elementwise on [8,64,56,56] (+ B [64,1,1]); 40 rotating sets (> 512 MB).
    A = rng.uniform(-4, 4, (8, 64, 56, 56)).astype(np.float32)
    B = rng.uniform(-4, 4, (64, 1, 1)).astype(np.float32)
    Bd = (np.sign(B) * np.maximum(np.abs(B), 0.1)).astype(np.float32)
    R = 40
    As = [lib.dev(A, F32) for _ in range(R)]
    Os = [lib.empty(list(A.shape), F32) for _ in range(R)]
    tb, tbd = lib.dev(B, F32), lib.dev(Bd, F32)
    nb = A.size * 8
    for name, fn in (("add", L.add_forward), ("mul", L.mul_forward), ("sub", L.sub_forward),
                     ("div", L.div_forward)):
        b = tbd if name == "div" else tb
        ms = bench_loop(torch, lambda i: fn(As[i % R], b, Os[i % R]), 200)
        out.append(op_line(f"{name}_f32_bcast", "config1 [8,64,56,56] (+) [64,1,1]", nb, ms, "hbm"))
    for name, fn in (("relu", L.relu_forward), ("abs", L.abs_forward), ("cos", L.cos_forward)):
        ms = bench_loop(torch, lambda i: fn(As[i % R], Os[i % R]), 200)
        out.append(op_line(f"{name}_f32", "config1 [8,64,56,56]", nb, ms, "hbm"))
    # The same chain fused into one kernel (bit-identical to the op-by-op chain):
    # 4 B in + 4 B out per element, plus the two [64,1,1] operands.
    steps = (CStep * 7)(CStep(0, 0, 0), CStep(2, 0, 0), CStep(1, 0, 0), CStep(3, 1, 0), CStep(4, 0, 0),
                        CStep(5, 0, 0), CStep(6, 0, 0))
    opnds = (PT * 2)(tb, tbd)
    ms = bench_loop(torch, lambda i: L.elementwise_chain_forward(As[i % R], opnds, 2, steps, 7, Os[i % R]), 200)
    out.append(op_line("chain7_f32_fused", "config1 Add>Mul>Sub>Div>Relu>Abs>Cos, one pass", nb, ms, "hbm"))
    I = rng.integers(-(2 ** 31), 2 ** 31 - 1, A.shape, dtype=np.int64).astype(np.int32)
    Is = [lib.dev(I, I32) for _ in range(20)]
    O64 = [lib.empty(list(A.shape), F64) for _ in range(20)]
    ms = bench_loop(torch, lambda i: L.add_forward(Is[i % 20], tb, O64[i % 20]), 100)
    out.append(op_line("add_i32_f32_to_f64", "config1 int32 [8,64,56,56] + f32 [64,1,1]", A.size * 12, ms, "hbm"))
    lib.check("config1")
    for t in As + Os + Is + O64 + [tb, tbd]:
        L.free_tensor(t)

    # Config 3: Gemm 4096^3 transB=1 with bias, f32 and f16.
    rng = np.random.default_rng(2)
    K = 4096
    a = rng.normal(0, 1 / 64, (4096, K)).astype(np.float32)
    b = rng.normal(0, 1 / 64, (4096, K)).astype(np.float32)
    c = rng.normal(0, 1 / 64, (4096,)).astype(np.float32)
    flops = 2 * 4096 ** 3
    tc = lib.dev(c, F32)
    for dt, peak in ((F32, MFMA_F32), (F16, MFMA_F16)):
        aa = a if dt == F32 else a.astype(np.float16)
        bb = b if dt == F32 else b.astype(np.float16)
        ta, tbb = lib.dev(aa, dt), lib.dev(bb, dt)
        ty = lib.empty([4096, 4096], dt)
        ms = bench_loop(torch, lambda i: L.gemm_forward(ta, tbb, tc, ty, 1.0, 1.0, 0, 1), 20, 1)
        out.append(op_line(f"gemm_{'f32' if dt == F32 else 'f16'}_4096", "config3 4096x4096x4096 transB=1 +bias",
                           flops, ms, "mfma", peak))
        for t in (ta, tbb, ty):
            L.free_tensor(t)
    lib.check("config3")
    # Config 3 weight-only-quant variant: B int8 [4096,4096] with per-row (axis 0)
    # scales, DequantizeLinear -> Gemm on A [256,4096]; fused (codes read in the
    # Gemm) and unfused (f32 weight written, then read).
    bw = rng.normal(0, 1 / 64, (4096, K))
    sw = (np.abs(bw).max(axis=1) / 127).astype(np.float32)
    bq = np.clip(np.rint(bw / sw[:, None]), -127, 127).astype(np.int8)
    a = rng.normal(0, 1 / 64, (256, K)).astype(np.float32)
    ta, tq, tbd = lib.dev(a, F32), lib.dev(bq, I8), lib.empty([4096, K], F32)
    ts1, tz1 = lib.dev(sw, F32), lib.dev(np.zeros(4096, np.int8), I8)
    ts2, tz2 = lib.dev(sw.reshape(-1, 1), F32), lib.dev(np.zeros((4096, 1), np.int8), I8)
    ty = lib.empty([256, 4096], F32)
    wflops = 2 * 256 * 4096 * K
    ms = bench_loop(torch, lambda i: L.dequantize_gemm_forward(ta, tq, ts1, tz1, 0, tc, ty, 1.0, 1.0, 0, 1), 20, 2)
    out.append(op_line("gemm_woq_int8_fused", "config3 WOQ A[256,4096] x int8 B[4096,4096]^T, axis-0 scales, +bias",
                       wflops, ms, "mfma", MFMA_F32))

    def unfused(i):
        L.dequantize_linear_forward(tq, ts2, tz2, tbd)
        L.gemm_forward(ta, tbd, tc, ty, 1.0, 1.0, 0, 1)
    ms = bench_loop(torch, unfused, 20, 2)
    out.append(op_line("gemm_woq_int8_unfused", "config3 WOQ DequantizeLinear -> Gemm (f32 weight in HBM)",
                       wflops, ms, "mfma", MFMA_F32))
    lib.check("config3 woq")
    for t in (ta, tq, tbd, ts1, tz1, ts2, tz2, ty):
        L.free_tensor(t)
    L.free_tensor(tc)

    # Config 4: conv layers + maxpool.
    rng = np.random.default_rng(3)
    for tag, xs, ws, pads, strides in (("stem7x7s2", (32, 3, 224, 224), (64, 3, 7, 7), [3, 3, 3, 3], [2, 2]),
                                       ("3x3", (32, 64, 56, 56), (64, 64, 3, 3), [1, 1, 1, 1], [1, 1]),
                                       ("1x1", (32, 64, 56, 56), (256, 64, 1, 1), [0, 0, 0, 0], [1, 1])):
        x = rng.normal(0, 1, xs).astype(np.float32)
        w = rng.normal(0, np.sqrt(2 / (ws[1] * ws[2] * ws[3])), ws).astype(np.float32)
        bias = rng.normal(0, 1 / 64, (ws[0],)).astype(np.float32)
        OH = (xs[2] + pads[0] + pads[2] - ws[2]) // strides[0] + 1
        OW = (xs[3] + pads[1] + pads[3] - ws[3]) // strides[1] + 1
        tx, tw, tbias = lib.dev(x, F32), lib.dev(w, F32), lib.dev(bias, F32)
        ty = lib.empty([xs[0], ws[0], OH, OW], F32)
        keep = [ints(pads), ints(strides), ints([1, 1])]
        p = ConvP(ctypes.cast(keep[0], ctypes.POINTER(ctypes.c_int)), ctypes.cast(keep[1], ctypes.POINTER(ctypes.c_int)),
                  ctypes.cast(keep[2], ctypes.POINTER(ctypes.c_int)), 1)
        fl = 2 * xs[0] * ws[0] * OH * OW * ws[1] * ws[2] * ws[3]
        ms = bench_loop(torch, lambda i: L.conv2d_forward(tx, tw, tbias, ty, ctypes.byref(p)), 5, 1)
        out.append(op_line(f"conv_{tag}", f"config4 x{list(xs)} w{list(ws)}", fl, ms, "mfma", MFMA_F32))
        for t in (tx, tw, tbias, ty):
            L.free_tensor(t)
    x = rng.normal(0, 1, (32, 64, 112, 112)).astype(np.float32)
    txs = [lib.dev(x, F32) for _ in range(4)]
    tys = [lib.empty([32, 64, 56, 56], F32) for _ in range(4)]
    keep = [ints([1, 1, 1, 1]), ints([2, 2]), ints([1, 1]), ints([3, 3])]
    pp = Params(*[ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep])
    ms = bench_loop(torch, lambda i: L.max_pool_forward(txs[i % 4], tys[i % 4], ctypes.byref(pp)), 40)
    out.append(op_line("maxpool_3x3s2", "config4 [32,64,112,112] -> [32,64,56,56]", x.size * 4 + x.size, ms, "hbm"))
    for t in txs + tys:
        L.free_tensor(t)
    lib.check("config4")

    # Config 5: softmax [64,32000] axis 1 (rotating 20 sets > 320 MB).
    rng = np.random.default_rng(4)
    s = rng.normal(0, 3, (64, 32000)).astype(np.float32)
    ts = [lib.dev(s, F32) for _ in range(20)]
    to = [lib.empty([64, 32000], F32) for _ in range(20)]
    ms = bench_loop(torch, lambda i: L.softmax_forward(ts[i % 20], to[i % 20], 1), 200)
    out.append(op_line("softmax_64x32000", "config5 [64,32000] axis=1", s.size * 8, ms, "hbm"))
    for t in ts + to:
        L.free_tensor(t)
    lib.check("config5")

    # Next rows: GlobalAveragePool at the config-5 classifier input and
    # DynamicQuantizeLinear over the config-2 activation tensor.
    rng = np.random.default_rng(5)
    g = rng.normal(0, 1, (64, 512, 7, 7)).astype(np.float32)
    tg = [lib.dev(g, F32) for _ in range(20)]
    to = [lib.empty([64, 512, 1, 1], F32) for _ in range(20)]
    ms = bench_loop(torch, lambda i: L.global_average_pool_forward(tg[i % 20], to[i % 20]), 200)
    out.append(op_line("global_avg_pool", "[64,512,7,7] -> [64,512,1,1]", g.size * 4 + 64 * 512 * 4, ms, "hbm"))
    for t in tg + to:
        L.free_tensor(t)
    x = config2_input(np.random.default_rng(1))
    tx = [lib.dev(x, F32) for _ in range(4)]
    ty = [lib.empty(list(x.shape), U8) for _ in range(4)]
    ts, tz = lib.empty([1], F32), lib.empty([1], U8)
    ms = bench_loop(torch, lambda i: L.dynamic_quantize_linear_forward(tx[i % 4], ty[i % 4], ts, tz), 50)
    # two reads of x (min / max, then quantize) and one write of the codes
    out.append(op_line("dynamic_quantize_linear", "x f32 [32,512,1024] -> u8", x.size * 9, ms, "hbm"))
    for t in tx + ty + [ts, tz]:
        L.free_tensor(t)
    lib.check("next rows")
    out.append(run_graph(torch))
    return out


def run_graph(torch, batch=64, iters=10):
    """Config 5: the QDQ ResNet-style ONNX graph (written by
    onnx_translator_amd.onnx.create_model, random-init weights, seed 4) through the
    device-resident Graph executor, batch 64 of [3,224,224] inputs ~N(0,1)."""
    from onnx_translator_amd.nn import Tensor
    from onnx_translator_amd.nn.ONNXImport import load_graph
    from onnx_translator_amd.onnx.create_model import resnet_qdq_model
    g = load_graph(resnet_qdq_model(batch=batch))
    x = np.random.default_rng(4).normal(0, 1, (batch, 3, 224, 224)).astype(np.float32)
    xd = Tensor(*x.shape, dtype="float32", data=x).to_device()
    t0, n = time.perf_counter(), 0
    while n < 2 or time.perf_counter() - t0 < 0.1:     # >= 100 ms: clocks ramped up
        g.forward(xd)
        torch.cuda.synchronize()
        n += 1
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    a.record()
    for _ in range(iters):
        y = g.forward(xd)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / iters
    wall = (time.perf_counter() - w0) / iters * 1e3
    # conv + gemm work of the graph: stem 2*64*64*112^2*147, blocks (3x3 + 1x1 projections), fc
    flops = 2 * batch * (64 * 112 * 112 * 147 + 64 * 56 * 56 * 576 + 128 * 28 * 28 * 576 + 128 * 28 * 28 * 64 +
                         256 * 14 * 14 * 1152 + 256 * 14 * 14 * 128 + 512 * 7 * 7 * 2304 + 512 * 7 * 7 * 256 +
                         1000 * 512)
    del y
    return {"op": "graph_resnet_qdq_b64", "shape": "config5 ONNX graph, batch 64 x [3,224,224], 37 nodes",
            "ms": round(ms, 4), "images/s": round(batch / (ms * 1e-3), 1), "host_ms": round(wall, 4),
            "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2), "fused_runs": len(g.fused_runs)}


def op_line(name, shape, work, ms, bound, peak=HBM_PEAK):
    rate = work / (ms * 1e-3)
    if bound == "hbm":
        return {"op": name, "shape": shape, "ms": round(ms, 5), "GB/s": round(rate / 1e9, 1),
                "frac_hbm": round(rate / peak, 4)}
    return {"op": name, "shape": shape, "ms": round(ms, 4), "TFLOP/s": round(rate / 1e12, 2),
            "frac_mfma": round(rate / peak, 4)}


# ---------------------------------------------------------------- CPU leg ---
def cpu_baseline(budget_s=10.0):
    """QuantizeLinear / DequantizeLinear of the same workload through the C ABI of
    the compiled reference (oracle/_ref) or the restatement, pre-broadcast
    scale / zero point as the reference's Python layer passes them."""
    from oracle import oracle as O
    ref = O.reference()
    lib, kind = (ref, "reference") if ref is not None else (O.oracle(), "port")
    rng = np.random.default_rng(1)
    x = config2_input(rng)
    variants = config2_variants(x)
    L = lib.lib
    tx = lib.tensor(x, O.F32)
    n = x.size
    total_bytes, elapsed, rounds = 0, 0.0, 0
    tensors = []
    for name, s, z, dt in variants:
        sf = lib.tensor(np.broadcast_to(s, x.shape), O.F32)
        zf = lib.tensor(np.broadcast_to(z, x.shape), dt)
        ty = lib.tensor(np.zeros(x.shape, O.STORAGE[dt]), dt)    # pre-touched
        tr = lib.tensor(np.zeros(x.shape, np.float32), O.F32)
        tensors.append((sf, zf, ty, tr))
    while elapsed < budget_s or rounds == 0:
        for sf, zf, ty, tr in tensors:
            t0 = time.perf_counter()
            L.quantize_linear_forward(tx, sf, zf, ty)
            L.dequantize_linear_forward(ty, sf, zf, tr)
            elapsed += time.perf_counter() - t0
            total_bytes += 2 * 5 * n
        rounds += 1
    for group in tensors:
        for t in group:
            L.free_tensor(t)
    L.free_tensor(tx)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    return {"value": round(total_bytes / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"{rounds} full round trips of the 4 Q/DQ variants on x f32 [32,512,1024] "
                      f"({elapsed:.1f} s of C calls, OpenMP threads={threads}, scale/zp pre-broadcast)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--graph-only", action="store_true",
                    help="only run the config-5 ONNX graph (batch 64, 10 timed forwards) and print its line "
                         "(for per-kernel profiles of the graph)")
    ap.add_argument("--calib", action="store_true",
                    help="only run a plain copy kernel (torch.neg, 512 MiB in + 512 MiB out, 5 launches) to "
                         "calibrate the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.calib:
        import torch
        src = torch.ones(1 << 27, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"calib": "torch.neg f32", "bytes_in": src.numel() * 4, "bytes_out": dst.numel() * 4,
                          "launches": 5}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(every hot op shards without exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.init()
    lib = Lib(os.environ.get("TENSOR_OPS_LIB", os.path.join(ROOT, "onnx_translator_amd", "libtensor_ops_hip.so")))
    # A created stream (default priority): launches on the legacy default stream
    # cost ~0.5 us more each on this runtime.  torch's events below are recorded
    # on this same stream, which is the one every kernel is launched on.
    side = torch.cuda.Stream()
    torch.cuda.set_stream(side)
    lib.lib.tensor_ops_hip_set_stream(ctypes.c_void_p(side.cuda_stream))
    if args.graph_only:
        print(json.dumps(run_graph(torch)), flush=True)
        return
    print("bench: headline Q/DQ round trips ...", file=sys.stderr, flush=True)
    h = run_headline(lib, torch, args.steps, args.warmup)
    value = h["bytes_per_step"] / (h["ms_per_step"] * 1e-3) / 1e9
    dom_ms = h["kernel_ms"][h["dominant"]]
    achieved = h["bytes_per_launch"] / (dom_ms * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get(h["dominant"])
    ops = []
    if not args.no_suite:
        print("bench: per-op suite ...", file=sys.stderr, flush=True)
        ops = run_suite(lib, torch)
    cpu = None
    if not args.no_cpu:
        print("bench: CPU baseline ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.cpu_budget)
    line = {
        "metric": "GB/s (% HBM peak) for elementwise+Q/DQ; TFLOP/s (% MFMA) Gemm/Conv",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(h["ms_per_step"], 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32->u8/i8/e4m3/e5m2->f32 (fp64 quotient)", "data": "synthetic",
        "config": {"workload": "configs[1]: QuantizeLinear->DequantizeLinear round trip, x f32 [32,512,1024] "
                               "N(0,1.5)+0.1% x20 outliers, seed 1; u8 per-tensor, i8 per-axis(1), e4m3, e5m2",
                   "elements": h["n"], "bytes_per_step": h["bytes_per_step"], "rotating_sets": 8},
        "frac_hbm": round(value * 1e9 / HBM_PEAK, 4),
        "roofline": {"bound": "hbm", "kernel": h["dominant"], "achieved": round(achieved, 1), "peak": 8000.0,
                     "unit": "GB/s", "frac": round(achieved / 8000.0, 4), "traffic": traffic,
                     "avg_launch_ms": round(dom_ms, 5), "algorithmic_bytes": h["bytes_per_launch"]},
        "kernels_ms": {k: round(v, 5) for k, v in h["kernel_ms"].items()},
        "cpu_baseline": cpu,
        "ops": ops,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
