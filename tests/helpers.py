"""Shared test helpers: golden cases, the C-ABI driver for the HIP library and
the comparison rules.

Comparison rules (the parity bar):
* bit-exact: integer / fp8 / f16 / bf16 codes and f32 / f64 bits must match,
  except that where the reference result is a NaN the result only has to be a
  NaN of the same format (the reference's own NaN sign/payload depends on
  which operand x86 SSE propagates, which its C code does not fix);
* tolerance (MFMA Gemm / Conv, tree-reduced Softmax): |g - r| <= rtol*|r| + atol
  with rtol 1e-5 for f32 / f64 outputs and atol = rtol * rms(r); for narrow
  float outputs one unit in the last place of the output format plus the same
  atol.
"""
from __future__ import annotations

import contextlib
import ctypes
import json
import os

import numpy as np

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
HIP_SO = os.path.join(ROOT, "onnx_translator_amd", "libtensor_ops_hip.so")

_cases = None


def load_cases():
    global _cases
    if _cases is None:
        with open(os.path.join(GOLDEN, "cases.json")) as f:
            cases = json.load(f)
        arrays = dict(np.load(os.path.join(GOLDEN, "cases.npz"), allow_pickle=False))
        _cases = (cases, arrays)
    return _cases


def case_by_name(name):
    cases, arrays = load_cases()
    for c in cases:
        if c["name"] == name:
            return c, arrays
    raise KeyError(name)


def run_case(lib, case, arrays):
    ins = [arrays[k] if k is not None else None for k in case["inputs"]]
    from tests.golden.make_golden import call
    return call(lib, case["op"], ins, case["dtypes"], case["out_dtype"], case["params"])


# ---------------------------------------------------------------- comparisons ---
def nan_mask(a, dt):
    dt = O.dtype_code(dt)
    a = np.asarray(a)
    if dt == O.F32 or dt == O.F64:
        return np.isnan(a)
    if dt == O.F16:
        b = a.view(np.uint16)
        return ((b & 0x7C00) == 0x7C00) & ((b & 0x3FF) != 0)
    if dt == O.BF16:
        b = a.view(np.uint16)
        return ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    if dt == O.E4M3:
        return (a.view(np.uint8) & 0x7F) == 0x7F
    if dt == O.E5M2:
        b = a.view(np.uint8)
        return ((b & 0x7C) == 0x7C) & ((b & 3) != 0)
    return np.zeros(a.shape, bool)


def bits(a):
    a = np.asarray(a)
    return a.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[a.itemsize])


def assert_bitexact(out, ref, dt, what=""):
    out, ref = np.asarray(out), np.asarray(ref)
    assert out.shape == ref.shape, f"{what}: shape {out.shape} vs {ref.shape}"
    rn, on = nan_mask(ref, dt), nan_mask(out, dt)
    bad = (~rn & (bits(out) != bits(ref))) | (rn & ~on)
    if bad.any():
        idx = np.argwhere(bad)[:8]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} differ; first at {idx.tolist()}: "
                             f"got {[out[tuple(i)] for i in idx]} want {[ref[tuple(i)] for i in idx]}")


def decode(a, dt):
    """Storage -> float64 values (uses the oracle's decoders via a Sub(x, 0) pass)."""
    dt = O.dtype_code(dt)
    a = np.asarray(a)
    if dt in (O.F32, O.F64) or dt >= O.I4:
        return a.astype(np.float64)
    if dt == O.F16:
        return a.view(np.float16).astype(np.float64)
    z = np.zeros(1, np.float32)
    return O.oracle().binary("sub", a, dt, z, O.F32, O.F64)


MANT_BITS = {O.F16: 10, O.BF16: 7, O.E4M3: 3, O.E5M2: 2}


def assert_close(out, ref, dt, rtol=1e-5, what=""):
    dt = O.dtype_code(dt)
    g, r = decode(out, dt), decode(ref, dt)
    assert g.shape == r.shape
    rn = np.isnan(r)
    assert not (np.isnan(g) & ~rn).any(), f"{what}: NaN where the reference is finite"
    finite = r[np.isfinite(r)]
    rms = float(np.sqrt(np.mean(finite ** 2))) if finite.size else 0.0
    if dt in MANT_BITS:
        tol = np.abs(r) * 2.0 ** -MANT_BITS[dt] + 1e-30
        # values below the format's normal range are spaced by its subnormal step
        tol = np.maximum(tol, {O.F16: 2 ** -24, O.BF16: 2 ** -133, O.E4M3: 2 ** -6, O.E5M2: 2 ** -14}[dt])
        # the same absolute floor as f32: results that cancel to near zero carry
        # the fp32 accumulation error of their terms, not of the result
        tol = tol + rtol * rms
    else:
        tol = rtol * np.abs(r) + rtol * rms
    fin = np.isfinite(r)
    with np.errstate(invalid="ignore"):        # inf - inf where both are infinite
        err = np.abs(g - r)
    bad = fin & ~(err <= tol)
    bad |= ~fin & ~rn & (g != r)
    if bad.any():
        idx = np.argwhere(bad)[:8]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside tolerance; first "
                             f"{[(tuple(i), g[tuple(i)], r[tuple(i)]) for i in idx]}")


TOL_OPS = {"gemm", "conv2d", "softmax"}


def out_dtypes(case):
    """Output dtype per output key (DynamicQuantizeLinear: y, y_scale, y_zero_point)."""
    if case["op"] == "dynamic_quantize_linear":
        return ["uint8", "float32", case["params"].get("zp_dtype", "uint8")]
    return [case["out_dtype"]]


def check_case(out, case, arrays, exact):
    if isinstance(case["out"], list):
        for i, (o, k, dt) in enumerate(zip(out, case["out"], out_dtypes(case))):
            assert_bitexact(o, arrays[k], dt, what=f"{case['name']} output {i}")
        return
    ref = arrays[case["out"]]
    if case["op"] in TOL_OPS and not exact:
        assert_close(out, ref, case["out_dtype"], what=case["name"])
    else:
        assert_bitexact(out, ref, case["out_dtype"], what=case["name"])


# ---------------------------------------------------------------- HIP driver ---
class HipLib(O.CpuLib):
    """libtensor_ops_hip.so driven through its C ABI (host tensors: reference semantics)."""

    def __init__(self, path=HIP_SO):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `python -m onnx_translator_amd.build` first")
        super().__init__(path)
        lib = self.lib
        lib.tensor_ops_hip_last_error.restype = ctypes.c_char_p
        lib.tensor_ops_hip_last_error.argtypes = []
        lib.tensor_ops_hip_clear_error.argtypes = []
        lib.tensor_ops_hip_device_count.restype = ctypes.c_int
        lib.tensor_ops_hip_set_exact.argtypes = [ctypes.c_int]
        lib.tensor_ops_hip_set_stream.argtypes = [ctypes.c_void_p]
        lib.tensor_ops_hip_sync.restype = ctypes.c_int
        lib.create_tensor_device.restype = O.PT
        lib.create_tensor_device.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        lib.tensor_wrap_device.restype = O.PT
        lib.tensor_wrap_device.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                           ctypes.c_int]
        lib.tensor_to_host.argtypes = [O.PT, ctypes.c_void_p]
        lib.tensor_to_host.restype = ctypes.c_int
        lib.tensor_from_host.argtypes = [O.PT, ctypes.c_void_p]
        lib.tensor_from_host.restype = ctypes.c_int
        lib.tensor_is_device.argtypes = [O.PT]
        lib.tensor_is_device.restype = ctypes.c_int
        for n in ("quantize_linear_axis_forward", "dequantize_linear_axis_forward"):
            getattr(lib, n).argtypes = [O.PT, O.PT, O.PT, O.PT, ctypes.c_int]
        lib.conv2d_fused_forward.argtypes = [O.PT, O.PT, O.PT, O.PT, ctypes.c_int, O.PT, ctypes.POINTER(O.CConvParams)]
        lib.dequantize_conv2d_fused_forward.argtypes = [O.PT, O.PT, O.PT, O.PT, O.PT, O.PT, ctypes.c_int, O.PT,
                                                        ctypes.POINTER(O.CConvParams)]
        lib.dequantize_gemm_forward.argtypes = [O.PT, O.PT, O.PT, O.PT, ctypes.c_int, O.PT, O.PT, ctypes.c_float,
                                                ctypes.c_float, ctypes.c_int, ctypes.c_int]
        lib.quantize_dequantize_linear_forward.argtypes = [O.PT] * 6 + [ctypes.c_int]
        lib.max_pool_qdq_forward.argtypes = [O.PT, O.PT, ctypes.POINTER(O.CPoolParams), O.PT, O.PT, O.PT, O.PT,
                                             ctypes.c_int, O.PT]
        lib.conv2d_fused_qdq_forward.argtypes = [O.PT, O.PT, O.PT, O.PT, ctypes.c_int, O.PT, O.PT, O.PT, O.PT,
                                                 ctypes.c_int, O.PT, ctypes.POINTER(O.CConvParams)]

    def device_count(self):
        return int(self.lib.tensor_ops_hip_device_count())

    @contextlib.contextmanager
    def poisoned(self, byte=0xFF):
        """Every device buffer the library hands out with undefined contents
        (device outputs from create_tensor_device_empty, staged host outputs) is
        filled with `byte` first (0xFF: NaN in every float format), so an
        element an operator fails to write shows up."""
        fn = self.lib.tensor_ops_hip_set_poison
        fn.argtypes, fn.restype = [ctypes.c_int], ctypes.c_int
        prev = fn(int(byte))
        try:
            yield
        finally:
            fn(prev)

    def last_error(self):
        e = self.lib.tensor_ops_hip_last_error()
        return e.decode() if e else ""

    def set_exact(self, on):
        self.lib.tensor_ops_hip_set_exact(1 if on else 0)

    def _run(self, fn, ins, out_shape, out_dt, *extra):
        self.lib.tensor_ops_hip_clear_error()
        out = super()._run(fn, ins, out_shape, out_dt, *extra)
        err = self.last_error()
        if err:
            raise RuntimeError(err)
        return out

    def binary_raw(self, name, a, dta, b, dtb, dto):
        """add/sub/mul/div_forward with the operands passed un-broadcast (the
        library broadcasts in-kernel); the output has the broadcast shape."""
        a, b = np.asarray(a), np.asarray(b)
        shape = np.broadcast_shapes(a.shape, b.shape)
        return self._run(getattr(self.lib, name + "_forward"), [(a, dta), (b, dtb)], shape, dto)

    def qdq_axis(self, name, x, dtx, s, z, dtz, dty, axis):
        """quantize / dequantize_linear_axis_forward with 1-D Scale / ZeroPoint."""
        x = np.asarray(x)
        return self._run(getattr(self.lib, name + "_linear_axis_forward"),
                         [(x, dtx), (np.atleast_1d(s), O.F32), (np.atleast_1d(z), dtz)], x.shape, dty,
                         ctypes.c_int(axis))

    def qdq1(self, name, x, dtx, s, z, dtz, dty):
        """quantize / dequantize_linear_forward with Scale and ZeroPoint passed as
        given (not broadcast to X's shape: one-element tensors stay per-tensor)."""
        return self._run(getattr(self.lib, name + "_linear_forward"),
                         [(np.asarray(x), dtx), (np.atleast_1d(s), O.F32), (np.atleast_1d(z), dtz)],
                         np.asarray(x).shape, dty)

    def qdq_fused(self, x, qs, qz, ds, dz, code_dt):
        """quantize_dequantize_linear_forward on host tensors (f32 x and scales,
        zero points of code_dt)."""
        x = np.asarray(x)
        return self._run(self.lib.quantize_dequantize_linear_forward,
                         [(x, O.F32), (np.atleast_1d(qs), O.F32), (np.atleast_1d(qz), code_dt),
                          (np.atleast_1d(ds), O.F32), (np.atleast_1d(dz), code_dt)], x.shape, O.F32,
                         ctypes.c_int(O.NAMES[code_dt] if isinstance(code_dt, str) else int(code_dt)))

    def dql(self, x, dtx, zdt="uint8"):
        self.lib.tensor_ops_hip_clear_error()
        out = super().dql(x, dtx, zdt)
        err = self.last_error()
        if err:
            raise RuntimeError(err)
        return out

    def dq_gemm(self, a, bq, dtb, s, z, axis, c, dty, alpha=1.0, beta=1.0, transA=0, transB=1):
        """dequantize_gemm_forward on host tensors: A f32, Bq codes of dtb, 1-D Scale (f32)
        and ZeroPoint (dtb, or None), bias c (f32 or None)."""
        M = a.shape[1] if transA else a.shape[0]
        N = bq.shape[0] if transB else bq.shape[1]
        ins = [self.tensor(a, "float32"), self.tensor(bq, dtb), self.tensor(np.atleast_1d(s), "float32"),
               self.tensor(np.atleast_1d(z), dtb) if z is not None else O.PT(),
               self.tensor(c, "float32") if c is not None else O.PT()]
        o = self.empty((M, N), dty)
        try:
            self.lib.tensor_ops_hip_clear_error()
            self.lib.dequantize_gemm_forward(ins[0], ins[1], ins[2], ins[3], int(axis), ins[4], o,
                                             ctypes.c_float(alpha), ctypes.c_float(beta), int(transA), int(transB))
            err = self.last_error()
            if err:
                raise RuntimeError(err)
            return self.read(o, dty)
        finally:
            for t in ins:
                if t:
                    self.lib.free_tensor(t)
            self.lib.free_tensor(o)

    def conv_fused(self, x, w, b, skip, relu, dty, pads, strides, dilations=(1, 1), group=1, skip_dt="float32"):
        """conv2d_fused_forward on host tensors (f32 x / w / b; skip of skip_dt or None)."""
        N, C, H, W = x.shape
        M, _, KH, KW = w.shape
        OH = (H + pads[0] + pads[2] - dilations[0] * (KH - 1) - 1) // strides[0] + 1
        OW = (W + pads[1] + pads[3] - dilations[1] * (KW - 1) - 1) // strides[1] + 1
        p = O.CConvParams()
        keep = [O._ints(pads), O._ints(strides), O._ints(dilations)]
        p.pads, p.strides, p.dilations = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        p.group = int(group)
        ins = [self.tensor(x, "float32"), self.tensor(w, "float32"),
               self.tensor(b, "float32") if b is not None else O.PT(),
               self.tensor(skip, skip_dt) if skip is not None else O.PT()]
        o = self.empty((N, M, OH, OW), dty)
        try:
            self.lib.tensor_ops_hip_clear_error()
            self.lib.conv2d_fused_forward(ins[0], ins[1], ins[2], ins[3], int(relu), o, ctypes.byref(p))
            err = self.last_error()
            if err:
                raise RuntimeError(err)
            return self.read(o, dty)
        finally:
            for t in ins:
                if t:
                    self.lib.free_tensor(t)
            self.lib.free_tensor(o)

    def maxpool_qdq(self, x, kernel_shape, pads, strides, qs, qz, ds, dz, code_dt):
        """max_pool_qdq_forward on host tensors: f32 x, f32 scales, zero points of
        code_dt; returns (Y, Yq)."""
        N, C, H, W = x.shape
        KH, KW = kernel_shape
        OH = (H + pads[0] + pads[2] - (KH - 1) - 1) // strides[0] + 1
        OW = (W + pads[1] + pads[3] - (KW - 1) - 1) // strides[1] + 1
        p = O.CPoolParams()
        keep = [O._ints(pads), O._ints(strides), O._ints((1, 1)), O._ints(kernel_shape)]
        p.pads, p.strides, p.dilations, p.kernel_shape = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        ins = [self.tensor(x, "float32"), self.tensor(np.atleast_1d(qs), "float32"),
               self.tensor(np.atleast_1d(qz), code_dt), self.tensor(np.atleast_1d(ds), "float32"),
               self.tensor(np.atleast_1d(dz), code_dt)]
        outs = [self.empty((N, C, OH, OW), "float32") for _ in range(2)]
        try:
            self.lib.tensor_ops_hip_clear_error()
            self.lib.max_pool_qdq_forward(ins[0], outs[0], ctypes.byref(p), *ins[1:], ctypes.c_int(O.NAMES[code_dt]),
                                          outs[1])
            err = self.last_error()
            if err:
                raise RuntimeError(err)
            return self.read(outs[0], "float32"), self.read(outs[1], "float32")
        finally:
            for t in ins + outs:
                self.lib.free_tensor(t)

    def conv_fused_qdq(self, x, w, b, skip, relu, qs, qz, ds, dz, code_dt, pads, strides, dilations=(1, 1),
                       group=1):
        """conv2d_fused_qdq_forward on host tensors: f32 x / w / b / skip (b, skip may be
        None), f32 scales and zero points of code_dt; f32 output."""
        N, C, H, W = x.shape
        M, _, KH, KW = w.shape
        OH = (H + pads[0] + pads[2] - dilations[0] * (KH - 1) - 1) // strides[0] + 1
        OW = (W + pads[1] + pads[3] - dilations[1] * (KW - 1) - 1) // strides[1] + 1
        p = O.CConvParams()
        keep = [O._ints(pads), O._ints(strides), O._ints(dilations)]
        p.pads, p.strides, p.dilations = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        p.group = int(group)
        ins = [self.tensor(x, "float32"), self.tensor(w, "float32"),
               self.tensor(b, "float32") if b is not None else O.PT(),
               self.tensor(skip, "float32") if skip is not None else O.PT(),
               self.tensor(np.atleast_1d(qs), "float32"), self.tensor(np.atleast_1d(qz), code_dt),
               self.tensor(np.atleast_1d(ds), "float32"), self.tensor(np.atleast_1d(dz), code_dt)]
        o = self.empty((N, M, OH, OW), "float32")
        try:
            self.lib.tensor_ops_hip_clear_error()
            self.lib.conv2d_fused_qdq_forward(*ins[:4], int(relu), *ins[4:], ctypes.c_int(O.NAMES[code_dt]), o,
                                              ctypes.byref(p))
            err = self.last_error()
            if err:
                raise RuntimeError(err)
            return self.read(o, "float32")
        finally:
            for t in ins:
                if t:
                    self.lib.free_tensor(t)
            self.lib.free_tensor(o)

    def dq_conv_fused(self, xq, xdt, s, z, w, b, skip, relu, pads, strides, dilations=(1, 1), group=1):
        """dequantize_conv2d_fused_forward on host tensors: codes xq of xdt, scale s (f32) and
        zero point z (xdt, or None), f32 w / b / skip."""
        N, C, H, W = xq.shape
        M, _, KH, KW = w.shape
        OH = (H + pads[0] + pads[2] - dilations[0] * (KH - 1) - 1) // strides[0] + 1
        OW = (W + pads[1] + pads[3] - dilations[1] * (KW - 1) - 1) // strides[1] + 1
        p = O.CConvParams()
        keep = [O._ints(pads), O._ints(strides), O._ints(dilations)]
        p.pads, p.strides, p.dilations = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        p.group = int(group)
        ins = [self.tensor(xq, xdt), self.tensor(np.atleast_1d(s), "float32"),
               self.tensor(np.atleast_1d(z), xdt) if z is not None else O.PT(), self.tensor(w, "float32"),
               self.tensor(b, "float32") if b is not None else O.PT(),
               self.tensor(skip, "float32") if skip is not None else O.PT()]
        o = self.empty((N, M, OH, OW), "float32")
        try:
            self.lib.tensor_ops_hip_clear_error()
            self.lib.dequantize_conv2d_fused_forward(ins[0], ins[1], ins[2], ins[3], ins[4], ins[5], int(relu), o,
                                                     ctypes.byref(p))
            err = self.last_error()
            if err:
                raise RuntimeError(err)
            return self.read(o, "float32")
        finally:
            for t in ins:
                if t:
                    self.lib.free_tensor(t)
            self.lib.free_tensor(o)

    # device tensors --------------------------------------------------------
    def dev_from(self, arr, dt):
        a = O.as_storage(arr, dt)
        shape = a.shape if a.ndim else (1,)
        t = self.lib.create_tensor_device((ctypes.c_int * len(shape))(*shape), len(shape), O.dtype_code(dt))
        assert t, self.last_error()
        assert self.lib.tensor_from_host(t, a.ctypes.data) == 0, self.last_error()
        return t

    def dev_empty(self, shape, dt):
        shape = tuple(shape) or (1,)
        t = self.lib.create_tensor_device((ctypes.c_int * len(shape))(*shape), len(shape), O.dtype_code(dt))
        assert t, self.last_error()
        return t

    def dev_read(self, t, dt):
        c = t.contents
        shape = [c.shape[i] for i in range(c.ndim)]
        out = np.empty(shape, dtype=O.STORAGE[O.dtype_code(dt)])
        assert self.lib.tensor_to_host(t, out.ctypes.data) == 0, self.last_error()
        return out
