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
        L.tensor_ops_hip_set_thread_stream.argtypes = [ctypes.c_void_p]
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


def capture(torch, fn):
    """fn's launches on the current (library) stream, captured into a graph."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=torch.cuda.current_stream()):
        fn()
    return g


def run_headline(lib, torch, steps, warmup, use_graph=False, nstreams=1):
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
    # The four variants are independent: variant v runs on stream v % nstreams
    # (default priority), so one variant's launch gap and tail overlap another's
    # kernel.  Every buffer is written by one stream only (Y[v][*] by variant v;
    # XR[q % R] with q = 4k + v is XR[v] or XR[v + 4]).
    main = torch.cuda.current_stream()
    streams = [torch.cuda.Stream() for _ in range(nstreams)] if nstreams > 1 else []

    def step(k):
        # launch q reads input set q % R; the dequantize of variant v reads the
        # codes its quantize wrote one step earlier (4 launches, > 600 MB ago)
        for v in range(4):
            q = 4 * k + v
            if streams:
                L.tensor_ops_hip_set_thread_stream(ctypes.c_void_p(streams[v % nstreams].cuda_stream))
            L.quantize_linear_forward(X[q % R], S[v], Z[v], Y[v][k % R])
            L.dequantize_linear_forward(Y[v][(k - 1) % R], S[v], Z[v], XR[q % R])
        if streams:
            L.tensor_ops_hip_set_thread_stream(None)

    def fork():
        e = torch.cuda.Event()
        e.record(main)
        for st in streams:
            st.wait_event(e)

    def join():
        for st in streams:
            e = torch.cuda.Event()
            e.record(st)
            main.wait_event(e)

    fork()
    for k in range(warmup):
        step(k)
    join()
    lib.check("warmup")
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if use_graph and not streams:
        # The K timed steps (8 launches each, the same rotation of buffers) are
        # captured once into a HIP graph on the library's stream; one untimed
        # replay, then one timed replay of exactly K steps.
        g = capture(torch, lambda: [step(warmup + k) for k in range(steps)])
        g.replay()
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        t0.record()
        g.replay()
        t1.record()
    else:
        w0 = time.perf_counter()
        t0.record(main)
        fork()
        for k in range(steps):
            step(warmup + k)
        join()
        t1.record(main)
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
        kern[f"quantize_f32_to_{var[0]}"] = bench_loop(torch, q_fn, steps, warm=4, graph=use_graph)
        kern[f"dequantize_{var[0]}_to_f32"] = bench_loop(torch, dq_fn, steps, warm=4, graph=use_graph)
    lib.check("per-kernel pass")
    dom = max(kern, key=kern.get)
    for t in X + [t for ys in Y for t in ys] + XR + S + Z:
        L.free_tensor(t)
    per_step_bytes = 8 * bytes_per_launch
    return {"ms_per_step": ms, "wall_s": wall, "bytes_per_step": per_step_bytes, "kernel_ms": kern,
            "dominant": dom, "bytes_per_launch": bytes_per_launch, "n": n}


def bench_loop(torch, fn, iters, warm=3, warm_ms=100.0, graph=False):
    """Mean time of `iters` back-to-back calls.  The warm-up runs at least `warm`
    calls and `warm_ms` of wall time, in batches of up to 8 calls with no host
    wait inside a batch, so the GPU stays busy while its clocks ramp up (a cold
    4096^3 Gemm runs ~20% slower for its first few milliseconds).  graph: the
    `iters` calls are captured into a HIP graph and timed as one replay (for
    calls that launch kernels only: no host staging, no workspace allocation)."""
    t0, i = time.perf_counter(), 0
    while i < warm or (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(min(8, warm - i) if i < warm else 8):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    warm = i
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if graph:
        g = capture(torch, lambda: [fn(warm + k) for k in range(iters)])
        g.replay()
        torch.cuda.synchronize()
        a.record()
        g.replay()
        b.record()
    else:
        a.record()
        for i in range(iters):
            fn(warm + i)
        b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


SUITE = ("add_f32_bcast", "mul_f32_bcast", "sub_f32_bcast", "div_f32_bcast", "relu_f32", "abs_f32", "cos_f32",
         "chain7_f32_fused", "add_i32_f32_to_f64", "gemm_f32_4096", "gemm_f16_4096", "gemm_f16_4096_vendor",
         "gemm_woq_int8_fused",
         "gemm_woq_int8_unfused", "conv_stem7x7s2", "conv_3x3", "conv_1x1", "maxpool_3x3s2", "softmax_64x32000",
         "global_avg_pool", "dynamic_quantize_linear", "graph_resnet_qdq_b64", "graph_resnet_qdq_b64_int8")


def run_suite(lib, torch, only=None, cpu=None):
    """Other configs: one line per operator, achieved vs roofline; with `cpu` (a
    CpuLeg) each line also carries the reference on this host's cores."""
    L = lib.lib
    out = []

    def want(*names):
        return only is None or any(n in only for n in names)

    def emit(line, cpu_fn=None):
        if cpu is not None and cpu_fn is not None:
            line.update(cpu.measure(cpu_fn, line))
        out.append(line)
        print(f"bench: {line['op']} done", file=sys.stderr, flush=True)

    # Config 1: f32 elementwise on [8,64,56,56] (+ B [64,1,1]); 40 rotating sets (> 512 MB).
    rng = np.random.default_rng(0)
    A = rng.uniform(-4, 4, (8, 64, 56, 56)).astype(np.float32)
    B = rng.uniform(-4, 4, (64, 1, 1)).astype(np.float32)
    Bd = (np.sign(B) * np.maximum(np.abs(B), 0.1)).astype(np.float32)
    nb = A.size * 8
    c1 = [n for n in SUITE[:9]]
    if want(*c1):
        R = 40
        As = [lib.dev(A, F32) for _ in range(R)]
        Os = [lib.empty(list(A.shape), F32) for _ in range(R)]
        tb, tbd = lib.dev(B, F32), lib.dev(Bd, F32)
        for name, fn in (("add", L.add_forward), ("mul", L.mul_forward), ("sub", L.sub_forward),
                         ("div", L.div_forward)):
            if not want(f"{name}_f32_bcast"):
                continue
            b = tbd if name == "div" else tb
            ms = bench_loop(torch, lambda i: fn(As[i % R], b, Os[i % R]), 200, graph=True)
            emit(op_line(f"{name}_f32_bcast", "config1 [8,64,56,56] (+) [64,1,1]", nb, ms, "hbm", rotated=R * nb),
                 CpuLeg.binary(name, A, Bd if name == "div" else B))
        for name, fn in (("relu", L.relu_forward), ("abs", L.abs_forward), ("cos", L.cos_forward)):
            if not want(f"{name}_f32"):
                continue
            ms = bench_loop(torch, lambda i: fn(As[i % R], Os[i % R]), 200, graph=True)
            emit(op_line(f"{name}_f32", "config1 [8,64,56,56]", nb, ms, "hbm", rotated=R * nb), CpuLeg.unary(name, A))
        if want("chain7_f32_fused"):
            # The same chain fused into one kernel (bit-identical to the op-by-op chain):
            # 4 B in + 4 B out per element, plus the two [64,1,1] operands.  The CPU
            # figure is the reference's op-by-op chain (7 calls) over the same bytes.
            steps = (CStep * 7)(CStep(0, 0, 0), CStep(2, 0, 0), CStep(1, 0, 0), CStep(3, 1, 0), CStep(4, 0, 0),
                                CStep(5, 0, 0), CStep(6, 0, 0))
            opnds = (PT * 2)(tb, tbd)
            ms = bench_loop(torch, lambda i: L.elementwise_chain_forward(As[i % R], opnds, 2, steps, 7, Os[i % R]),
                            200, graph=True)
            emit(op_line("chain7_f32_fused", "config1 Add>Mul>Sub>Div>Relu>Abs>Cos, one pass", nb, ms, "hbm",
                         rotated=R * nb),
                 CpuLeg.chain(A, B, Bd))
        for t in As + Os:
            L.free_tensor(t)
        if want("add_i32_f32_to_f64"):
            I = rng.integers(-(2 ** 31), 2 ** 31 - 1, A.shape, dtype=np.int64).astype(np.int32)
            RI = 30
            Is = [lib.dev(I, I32) for _ in range(RI)]
            O64 = [lib.empty(list(A.shape), F64) for _ in range(RI)]
            ms = bench_loop(torch, lambda i: L.add_forward(Is[i % RI], tb, O64[i % RI]), 100, graph=True)
            emit(op_line("add_i32_f32_to_f64", "config1 int32 [8,64,56,56] + f32 [64,1,1]", A.size * 12, ms, "hbm",
                         rotated=RI * A.size * 12), CpuLeg.binary("add", I, B, I32, F64))
            for t in Is + O64:
                L.free_tensor(t)
        lib.check("config1")
        for t in (tb, tbd):
            L.free_tensor(t)

    # Config 3: Gemm 4096^3 transB=1 with bias, f32 and f16.
    rng = np.random.default_rng(2)
    K = 4096
    flops = 2 * 4096 ** 3
    if want("gemm_f32_4096", "gemm_f16_4096", "gemm_f16_4096_vendor", "gemm_woq_int8_fused", "gemm_woq_int8_unfused"):
        a = rng.normal(0, 1 / 64, (4096, K)).astype(np.float32)
        b = rng.normal(0, 1 / 64, (4096, K)).astype(np.float32)
        c = rng.normal(0, 1 / 64, (4096,)).astype(np.float32)
        tc = lib.dev(c, F32)
        for dt, peak in ((F32, MFMA_F32), (F16, MFMA_F16)):
            name = f"gemm_{'f32' if dt == F32 else 'f16'}_4096"
            if not want(name):
                continue
            aa = a if dt == F32 else a.astype(np.float16)
            bb = b if dt == F32 else b.astype(np.float16)
            ta, tbb = lib.dev(aa, dt), lib.dev(bb, dt)
            ty = lib.empty([4096, 4096], dt)
            ms = bench_loop(torch, lambda i: L.gemm_forward(ta, tbb, tc, ty, 1.0, 1.0, 0, 1), 20, 1)
            emit(op_line(name, "config3 4096x4096x4096 transB=1 +bias", flops, ms, "mfma", peak),
                 CpuLeg.gemm(aa, bb, c, dt))
            for t in (ta, tbb, ty):
                L.free_tensor(t)
        if want("gemm_f16_4096_vendor"):
            # Context, not this library: the same f16 product through torch
            # (F.linear -> the ROCm BLAS library, hipBLASLt on gfx950) on the same
            # box, timed the same way; the bias is f16 there (torch requires it).
            ah = torch.from_numpy(a.astype(np.float16)).cuda()
            bh = torch.from_numpy(b.astype(np.float16)).cuda()
            ch = torch.from_numpy(c.astype(np.float16)).cuda()
            fl = torch.nn.functional.linear
            ms = bench_loop(torch, lambda i: fl(ah, bh, ch), 20, 1)
            line = op_line("gemm_f16_4096_vendor", "config3 4096^3 f16 through torch F.linear (vendor BLAS, "
                           "for comparison only)", flops, ms, "mfma", MFMA_F16)
            line["library"] = "torch " + torch.__version__ + " F.linear (ROCm BLAS)"
            emit(line)
            del ah, bh, ch
        lib.check("config3")
        # Config 3 weight-only-quant variant: B int8 [4096,4096] with per-row (axis 0)
        # scales, DequantizeLinear -> Gemm on A [256,4096]; fused (codes read in the
        # Gemm) and unfused (f32 weight written, then read).
        bw = rng.normal(0, 1 / 64, (4096, K))
        sw = (np.abs(bw).max(axis=1) / 127).astype(np.float32)
        bq = np.clip(np.rint(bw / sw[:, None]), -127, 127).astype(np.int8)
        a = rng.normal(0, 1 / 64, (256, K)).astype(np.float32)
        wflops = 2 * 256 * 4096 * K
        if want("gemm_woq_int8_fused", "gemm_woq_int8_unfused"):
            ta, tq, tbd = lib.dev(a, F32), lib.dev(bq, I8), lib.empty([4096, K], F32)
            ts1, tz1 = lib.dev(sw, F32), lib.dev(np.zeros(4096, np.int8), I8)
            ts2, tz2 = lib.dev(sw.reshape(-1, 1), F32), lib.dev(np.zeros((4096, 1), np.int8), I8)
            ty = lib.empty([256, 4096], F32)
            woq_cpu = CpuLeg.woq(a, bq, sw, c)
            if want("gemm_woq_int8_fused"):
                ms = bench_loop(torch, lambda i: L.dequantize_gemm_forward(ta, tq, ts1, tz1, 0, tc, ty, 1.0, 1.0, 0, 1),
                                20, 2)
                emit(op_line("gemm_woq_int8_fused",
                             "config3 WOQ A[256,4096] x int8 B[4096,4096]^T, axis-0 scales, +bias",
                             wflops, ms, "mfma", MFMA_F32), woq_cpu)

            def unfused(i):
                L.dequantize_linear_forward(tq, ts2, tz2, tbd)
                L.gemm_forward(ta, tbd, tc, ty, 1.0, 1.0, 0, 1)
            if want("gemm_woq_int8_unfused"):
                ms = bench_loop(torch, unfused, 20, 2)
                emit(op_line("gemm_woq_int8_unfused", "config3 WOQ DequantizeLinear -> Gemm (f32 weight in HBM)",
                             wflops, ms, "mfma", MFMA_F32), woq_cpu)
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
        if not want(f"conv_{tag}"):
            continue
        OH = (xs[2] + pads[0] + pads[2] - ws[2]) // strides[0] + 1
        OW = (xs[3] + pads[1] + pads[3] - ws[3]) // strides[1] + 1
        tx, tw, tbias = lib.dev(x, F32), lib.dev(w, F32), lib.dev(bias, F32)
        ty = lib.empty([xs[0], ws[0], OH, OW], F32)
        keep = [ints(pads), ints(strides), ints([1, 1])]
        p = ConvP(ctypes.cast(keep[0], ctypes.POINTER(ctypes.c_int)), ctypes.cast(keep[1], ctypes.POINTER(ctypes.c_int)),
                  ctypes.cast(keep[2], ctypes.POINTER(ctypes.c_int)), 1)
        fl = 2 * xs[0] * ws[0] * OH * OW * ws[1] * ws[2] * ws[3]
        ms = bench_loop(torch, lambda i: L.conv2d_forward(tx, tw, tbias, ty, ctypes.byref(p)), 20, 1)
        emit(op_line(f"conv_{tag}", f"config4 x{list(xs)} w{list(ws)}", fl, ms, "mfma", MFMA_F32),
             CpuLeg.conv(x, w, bias, pads, strides))
        for t in (tx, tw, tbias, ty):
            L.free_tensor(t)
    if want("maxpool_3x3s2"):
        x = rng.normal(0, 1, (32, 64, 112, 112)).astype(np.float32)
        RP = 10
        txs = [lib.dev(x, F32) for _ in range(RP)]
        tys = [lib.empty([32, 64, 56, 56], F32) for _ in range(RP)]
        keep = [ints([1, 1, 1, 1]), ints([2, 2]), ints([1, 1]), ints([3, 3])]
        pp = Params(*[ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep])
        ms = bench_loop(torch, lambda i: L.max_pool_forward(txs[i % RP], tys[i % RP], ctypes.byref(pp)), 40,
                        graph=True)
        emit(op_line("maxpool_3x3s2", "config4 [32,64,112,112] -> [32,64,56,56]", x.size * 4 + x.size, ms, "hbm",
                     rotated=RP * (x.size * 4 + x.size)), CpuLeg.maxpool(x))
        for t in txs + tys:
            L.free_tensor(t)
    lib.check("config4")

    # Config 5: softmax [64,32000] axis 1 (rotating 40 sets, 655 MB).
    if want("softmax_64x32000"):
        rng = np.random.default_rng(4)
        s = rng.normal(0, 3, (64, 32000)).astype(np.float32)
        RS = 40
        ts = [lib.dev(s, F32) for _ in range(RS)]
        to = [lib.empty([64, 32000], F32) for _ in range(RS)]
        ms = bench_loop(torch, lambda i: L.softmax_forward(ts[i % RS], to[i % RS], 1), 200)
        emit(op_line("softmax_64x32000", "config5 [64,32000] axis=1", s.size * 8, ms, "hbm", rotated=RS * s.size * 8),
             CpuLeg.softmax(s))
        for t in ts + to:
            L.free_tensor(t)
        lib.check("config5")

    # Next rows: GlobalAveragePool at the config-5 classifier input and
    # DynamicQuantizeLinear over the config-2 activation tensor.
    if want("global_avg_pool"):
        rng = np.random.default_rng(5)
        g = rng.normal(0, 1, (64, 512, 7, 7)).astype(np.float32)
        RG = 80
        tg = [lib.dev(g, F32) for _ in range(RG)]
        to = [lib.empty([64, 512, 1, 1], F32) for _ in range(RG)]
        ms = bench_loop(torch, lambda i: L.global_average_pool_forward(tg[i % RG], to[i % RG]), 200)
        gb = g.size * 4 + 64 * 512 * 4
        emit(op_line("global_avg_pool", "[64,512,7,7] -> [64,512,1,1]", gb, ms, "hbm", rotated=RG * gb),
             CpuLeg.gap(g))
        for t in tg + to:
            L.free_tensor(t)
    if want("dynamic_quantize_linear"):
        x = config2_input(np.random.default_rng(1))
        RD = 7
        tx = [lib.dev(x, F32) for _ in range(RD)]
        ty = [lib.empty(list(x.shape), U8) for _ in range(RD)]
        ts, tz = lib.empty([1], F32), lib.empty([1], U8)
        ms = bench_loop(torch, lambda i: L.dynamic_quantize_linear_forward(tx[i % RD], ty[i % RD], ts, tz), 50)
        # algorithmic bytes: x read once (4 B) and the codes written once (1 B)
        emit(op_line("dynamic_quantize_linear", "x f32 [32,512,1024] -> u8", x.size * 5, ms, "hbm",
                     rotated=RD * x.size * 5), CpuLeg.dql(x))
        for t in tx + ty + [ts, tz]:
            L.free_tensor(t)
    lib.check("next rows")
    if want("graph_resnet_qdq_b64"):
        emit(run_graph(torch), CpuLeg.graph())
    if want("graph_resnet_qdq_b64_int8"):
        emit(run_graph(torch, int8=True))
    return out


def run_graph(torch, batch=64, iters=10, int8=False):
    """Config 5: the QDQ ResNet-style ONNX graph (written by
    onnx_translator_amd.onnx.create_model, random-init weights, seed 4) through the
    device-resident Graph executor, batch 64 of [3,224,224] inputs ~N(0,1).
    int8: with the QDQ blocks on the int8 MFMA kernels (Graph.fuse(int8_conv=True),
    the convolution tolerance class instead of the default passes' bits)."""
    from onnx_translator_amd.nn import Tensor
    from onnx_translator_amd.nn.ONNXImport import load_graph
    from onnx_translator_amd.onnx.create_model import resnet_qdq_model
    g = load_graph(resnet_qdq_model(batch=batch), fuse=False)
    g.fuse(int8_conv=int8)
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
    return {"op": "graph_resnet_qdq_b64" + ("_int8" if int8 else ""),
            "shape": "config5 ONNX graph, batch 64 x [3,224,224], 37 nodes" +
                     (", QDQ blocks on int8 MFMA (tolerance class)" if int8 else ""),
            "ms": round(ms, 4), "images/s": round(batch / (ms * 1e-3), 1), "host_ms": round(wall, 4),
            "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2), "fused_runs": len(g.fused_runs)}


CACHE_BYTES = 256 << 20      # MI355X Infinity Cache


def op_line(name, shape, work, ms, bound, peak=HBM_PEAK, rotated=None):
    """rotated: bytes the timed calls cycle through (inputs and outputs); an HBM
    line states whether that exceeds 2x the Infinity Cache, so its fraction is
    of HBM traffic, or could have been served from the cache."""
    rate = work / (ms * 1e-3)
    if bound == "hbm":
        line = {"op": name, "shape": shape, "ms": round(ms, 5), "GB/s": round(rate / 1e9, 1),
                "frac_hbm": round(rate / peak, 4), "work": work}
        if rotated is not None:
            line["rotated_MB"] = round(rotated / 1e6, 1)
            line["regime"] = ("hbm (rotation > 2x the 256 MB Infinity Cache)" if rotated >= 2 * CACHE_BYTES
                              else "cache-resident possible (rotation below 2x the 256 MB Infinity Cache)")
        return line
    return {"op": name, "shape": shape, "ms": round(ms, 4), "TFLOP/s": round(rate / 1e12, 2),
            "frac_mfma": round(rate / peak, 4), "work": work}


# ---------------------------------------------------------------- CPU leg ---
def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))


class CpuLeg:
    """The reference tensor_ops.c (oracle/_ref, compiled from its source; the
    restatement where it was never built) on this host's cores, timed on a bounded
    sample of each suite line's workload, operands prepared as the reference's
    Python layer passes them (broadcast to full size).  Each sample function
    returns (fraction of the line's work it covers, seconds, description)."""

    def __init__(self, budget_s=1.0):
        from oracle import oracle as O
        self.O = O
        ref = O.reference()
        self.lib, self.kind = (ref, "reference") if ref is not None else (O.oracle(), "port")
        self.budget = budget_s
        self.cores = cpu_threads()
        self.model = cpu_model()

    def timed(self, fn, max_runs=5):
        """Median of repeated calls after one untimed call (first-touch faults)."""
        fn()
        ts, t_end = [], time.perf_counter() + self.budget
        while len(ts) < max_runs and (not ts or time.perf_counter() < t_end):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)), len(ts)

    def measure(self, sample_fn, line):
        frac, secs, desc = sample_fn(self)
        work = line.get("work")
        if "images/s" in line:
            value, unit = frac / secs, "images/s"
        elif "GB/s" in line:
            value, unit = work * frac / secs / 1e9, "GB/s"
        else:
            value, unit = work * frac / secs / 1e12, "TFLOP/s"
        return {"cpu": {"value": float(f"{value:.4g}"), "unit": unit, "cores": self.cores, "kind": self.kind,
                        "cpu_model": self.model, "sample": desc}}

    # -- tensors on the CPU library -------------------------------------------------
    def _t(self, arr, dt):
        return self.lib.tensor(arr, dt)

    def _free(self, *ts):
        for t in ts:
            if t:
                self.lib.lib.free_tensor(t)

    # -- samples (static constructors return closures over the inputs) ---------------
    @staticmethod
    def binary(name, a, b, dta=F32, dto=F32):
        def run(leg):
            bb = np.ascontiguousarray(np.broadcast_to(b, a.shape))
            ta, tb = leg._t(a, dta), leg._t(bb, F32)
            to = leg.lib.empty(a.shape, dto)
            fn = getattr(leg.lib.lib, f"{name}_forward")
            secs, n = leg.timed(lambda: fn(ta, tb, to))
            leg._free(ta, tb, to)
            return 1.0, secs, f"full size, B pre-broadcast, median of {n}"
        return run

    @staticmethod
    def unary(name, a):
        def run(leg):
            ta, to = leg._t(a, F32), leg.lib.empty(a.shape, F32)
            fn = getattr(leg.lib.lib, f"{name}_forward")
            secs, n = leg.timed(lambda: fn(ta, to))
            leg._free(ta, to)
            return 1.0, secs, f"full size, median of {n}"
        return run

    @staticmethod
    def chain(a, b, bd):
        def run(leg):
            L = leg.lib.lib
            tb = leg._t(np.ascontiguousarray(np.broadcast_to(b, a.shape)), F32)
            tbd = leg._t(np.ascontiguousarray(np.broadcast_to(bd, a.shape)), F32)
            t0, t1 = leg._t(a, F32), leg.lib.empty(a.shape, F32)

            def chain():
                L.add_forward(t0, tb, t1)
                L.mul_forward(t1, tb, t1)
                L.sub_forward(t1, tb, t1)
                L.div_forward(t1, tbd, t1)
                L.relu_forward(t1, t1)
                L.abs_forward(t1, t1)
                L.cos_forward(t1, t1)
            secs, n = leg.timed(chain)
            leg._free(tb, tbd, t0, t1)
            return 1.0, secs, f"the 7 reference calls op by op, full size, median of {n}"
        return run

    @staticmethod
    def gemm(a, b, c, dt, rows=64):
        def run(leg):
            ta, tb = leg._t(a[:rows], dt), leg._t(b, dt)
            tc = leg._t(c.reshape(1, -1), F32)
            ty = leg.lib.empty((rows, b.shape[0]), dt)
            secs, n = leg.timed(lambda: leg.lib.lib.gemm_forward(ta, tb, tc, ty, 1.0, 1.0, 0, 1), max_runs=3)
            leg._free(ta, tb, tc, ty)
            return rows / a.shape[0], secs, f"{rows} of {a.shape[0]} rows of A (same N, K), median of {n}"
        return run

    @staticmethod
    def woq(a, bq, sw, c, rows=16):
        def run(leg):
            L = leg.lib.lib
            tq = leg._t(bq, I8)
            ts = leg._t(np.ascontiguousarray(np.broadcast_to(sw.reshape(-1, 1), bq.shape)), F32)
            tz = leg._t(np.zeros(bq.shape, np.int8), I8)
            tw = leg.lib.empty(bq.shape, F32)
            t_dq, n1 = leg.timed(lambda: L.dequantize_linear_forward(tq, ts, tz, tw), max_runs=3)
            ta, tc, ty = leg._t(a[:rows], F32), leg._t(c.reshape(1, -1), F32), leg.lib.empty((rows, bq.shape[0]), F32)
            t_mm, n2 = leg.timed(lambda: L.gemm_forward(ta, tw, tc, ty, 1.0, 1.0, 0, 1), max_runs=3)
            leg._free(tq, ts, tz, tw, ta, tc, ty)
            full = t_dq + t_mm * a.shape[0] / rows
            return 1.0, full, (f"DequantizeLinear of the full weight ({t_dq * 1e3:.0f} ms) + Gemm on {rows} of "
                               f"{a.shape[0]} rows scaled to all rows")
        return run

    @staticmethod
    def conv(x, w, bias, pads, strides, images=1):
        def run(leg):
            OH = (x.shape[2] + pads[0] + pads[2] - w.shape[2]) // strides[0] + 1
            OW = (x.shape[3] + pads[1] + pads[3] - w.shape[3]) // strides[1] + 1
            tx, tw, tb = leg._t(x[:images], F32), leg._t(w, F32), leg._t(bias, F32)
            ty = leg.lib.empty((images, w.shape[0], OH, OW), F32)
            p = leg.O.CConvParams()
            keep = [leg.O._ints(pads), leg.O._ints(strides), leg.O._ints([1, 1])]
            p.pads, p.strides, p.dilations = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
            p.group = 1
            secs, n = leg.timed(lambda: leg.lib.lib.conv2d_forward(tx, tw, tb, ty, ctypes.byref(p)), max_runs=3)
            leg._free(tx, tw, tb, ty)
            return images / x.shape[0], secs, f"{images} of {x.shape[0]} images, median of {n}"
        return run

    @staticmethod
    def maxpool(x, images=4):
        def run(leg):
            tx, ty = leg._t(x[:images], F32), leg.lib.empty((images, x.shape[1], 56, 56), F32)
            p = leg.O.CPoolParams()
            keep = [leg.O._ints([1, 1, 1, 1]), leg.O._ints([2, 2]), leg.O._ints([1, 1]), leg.O._ints([3, 3])]
            p.pads, p.strides, p.dilations, p.kernel_shape = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int))
                                                              for k in keep]
            secs, n = leg.timed(lambda: leg.lib.lib.max_pool_forward(tx, ty, ctypes.byref(p)))
            leg._free(tx, ty)
            return images / x.shape[0], secs, f"{images} of {x.shape[0]} images, median of {n}"
        return run

    @staticmethod
    def softmax(s):
        def run(leg):
            ts, to = leg._t(s, F32), leg.lib.empty(s.shape, F32)
            secs, n = leg.timed(lambda: leg.lib.lib.softmax_forward(ts, to, 1))
            leg._free(ts, to)
            return 1.0, secs, f"full size, median of {n}"
        return run

    @staticmethod
    def gap(g):
        def run(leg):
            tg, to = leg._t(g, F32), leg.lib.empty(g.shape[:2] + (1, 1), F32)
            secs, n = leg.timed(lambda: leg.lib.lib.global_average_pool_forward(tg, to))
            leg._free(tg, to)
            return 1.0, secs, f"full size, median of {n}"
        return run

    @staticmethod
    def dql(x):
        def run(leg):
            tx, ty = leg._t(x, F32), leg.lib.empty(x.shape, U8)
            ts, tz = leg.lib.empty((1,), F32), leg.lib.empty((1,), U8)
            secs, n = leg.timed(lambda: leg.lib.lib.dynamic_quantize_linear_forward(tx, ty, ts, tz), max_runs=3)
            leg._free(tx, ty, ts, tz)
            return 1.0, secs, f"full size, median of {n}"
        return run

    @staticmethod
    def graph(images=1):
        def run(leg):
            from onnx_translator_amd.onnx.create_model import resnet_qdq_model
            from tests.graph_oracle import run_model
            m = resnet_qdq_model(batch=images)
            x = np.random.default_rng(4).normal(0, 1, (images, 3, 224, 224)).astype(np.float32)
            secs, n = leg.timed(lambda: run_model(leg.lib, m, {"input": (x, "float32")}), max_runs=2)
            return images, secs, (f"{images} image(s) node by node through the C ABI (the reference's per-op "
                                  f"path, host copies included), median of {n}")
        return run


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
    threads = cpu_threads()
    return {"value": round(total_bytes / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "cpu_model": cpu_model(),
            "sample": f"{rounds} full round trips of the 4 Q/DQ variants on x f32 [32,512,1024] "
                      f"({elapsed:.1f} s of C calls, OpenMP threads={threads}, scale/zp pre-broadcast)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--streams", type=int, default=1,
                    help="HIP streams the four headline variants are spread over (1: one stream, in order; "
                         "2 and 4 measured no faster on MI355X: the step is bandwidth-bound)")
    ap.add_argument("--graph", action="store_true",
                    help="time the headline steps as one HIP graph replay instead of eager back-to-back launches "
                         "(measured slower for these 84 MB launches on MI355X)")
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--only", default=None,
                    help="comma-separated suite lines to run instead of the full run (no headline, no CPU leg), "
                         f"e.g. for per-kernel profiles; names: {', '.join(SUITE)}")
    ap.add_argument("--cpu-line-budget", type=float, default=1.0,
                    help="seconds of reference calls per suite line in the CPU leg")
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
              "(every hot op shards along its outer dimension without exchange; run one process per GPU)",
              file=sys.stderr)
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
    if args.only:
        only = [n.strip() for n in args.only.split(",") if n.strip()]
        unknown = [n for n in only if n not in SUITE]
        if unknown:
            print(f"bench.py: unknown suite line(s) {unknown}; names: {', '.join(SUITE)}", file=sys.stderr)
            sys.exit(2)
        for line in run_suite(lib, torch, only=set(only)):
            print(json.dumps(line), flush=True)
        return
    print("bench: headline Q/DQ round trips ...", file=sys.stderr, flush=True)
    h = run_headline(lib, torch, args.steps, args.warmup, use_graph=args.graph, nstreams=args.streams)
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
        ops = run_suite(lib, torch, cpu=None if args.no_cpu else CpuLeg(args.cpu_line_budget))
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
                   "elements": h["n"], "bytes_per_step": h["bytes_per_step"], "rotating_sets": 8,
                   "timing": ("one HIP graph replay of the K steps" if args.graph and args.streams <= 1 else
                              f"eager launches, the 4 variants over {max(1, args.streams)} HIP stream(s)")},
        "frac_hbm": round(value * 1e9 / HBM_PEAK, 4),
        "roofline": {"bound": "hbm", "kernel": h["dominant"], "achieved": round(achieved, 1), "peak": 8000.0,
                     "unit": "GB/s", "frac": round(achieved / 8000.0, 4), "traffic": traffic,
                     "traffic_source": "profiles/traffic.json: calibrated rocprofv3 FETCH_SIZE / WRITE_SIZE runs of "
                                       "this kernel (profiles/qdq_config2_hbm_traffic.md), not this run",
                     "avg_launch_ms": round(dom_ms, 5), "algorithmic_bytes": h["bytes_per_launch"]},
        "kernels_ms": {k: round(v, 5) for k, v in h["kernel_ms"].items()},
        "cpu_baseline": cpu,
        "ops": ops,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
