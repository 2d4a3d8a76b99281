"""ctypes driver for the CPU checker libraries (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module.  It drives any library that exports the reference C ABI
(``tensor_ops/tensor_ops.h:28-179``):

* ``oracle/liboracle.so``       — the restatement in ``tensor_ops_oracle.c``;
* ``oracle/_ref/tensor_ops.so`` — the reference ``tensor_ops.c`` compiled from
  its own source by ``oracle/Makefile`` (present only where it was built), or
  the build that ``TENSOR_OPS_REF_SO`` names.

Arrays are passed in their storage form: float16 / bfloat16 as uint16 bits,
fp8 as uint8 codes, int4 as int8.  Callers pre-broadcast binary / Q / DQ
operands to the output shape, as the reference's Python layer does
(``nn/__init__.py:210-279``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "tensor_ops.so")

E4M3, E5M2, F16, BF16, F32, F64, I4, I8, U8, I16, I32, I64 = range(12)
NAMES = {
    "float8_e4m3": E4M3, "float8_e5m2": E5M2, "float16": F16, "bfloat16": BF16,
    "float32": F32, "float64": F64, "int4": I4, "int8": I8, "uint8": U8,
    "int16": I16, "int32": I32, "int64": I64,
}
STORAGE = {
    E4M3: np.uint8, E5M2: np.uint8, F16: np.uint16, BF16: np.uint16, F32: np.float32,
    F64: np.float64, I4: np.int8, I8: np.int8, U8: np.uint8, I16: np.int16,
    I32: np.int32, I64: np.int64,
}


def dtype_code(dt) -> int:
    return NAMES[dt] if isinstance(dt, str) else int(dt)


def as_storage(arr, dt) -> np.ndarray:
    """Contiguous array in the storage type of dtype code ``dt`` (bit views for f16)."""
    dt = dtype_code(dt)
    arr = np.asarray(arr)
    st = STORAGE[dt]
    if arr.dtype == np.float16 and st == np.uint16:
        arr = arr.view(np.uint16)
    return np.ascontiguousarray(arr.astype(st, copy=False))


class CTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("shape", ctypes.POINTER(ctypes.c_int)),
                ("ndim", ctypes.c_int), ("size", ctypes.c_size_t), ("dtype", ctypes.c_int)]


class CConvParams(ctypes.Structure):
    _fields_ = [("pads", ctypes.POINTER(ctypes.c_int)), ("strides", ctypes.POINTER(ctypes.c_int)),
                ("dilations", ctypes.POINTER(ctypes.c_int)), ("group", ctypes.c_int)]


class CPoolParams(ctypes.Structure):
    _fields_ = [("pads", ctypes.POINTER(ctypes.c_int)), ("strides", ctypes.POINTER(ctypes.c_int)),
                ("dilations", ctypes.POINTER(ctypes.c_int)),
                ("kernel_shape", ctypes.POINTER(ctypes.c_int))]


PT = ctypes.POINTER(CTensor)


def _ints(vals):
    return (ctypes.c_int * len(vals))(*[int(v) for v in vals])


class CpuLib:
    """One loaded checker library; every call is synchronous host code."""

    def __init__(self, path: str):
        self.path = path
        lib = ctypes.CDLL(path)
        lib.create_tensor.restype = PT
        lib.create_tensor.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        lib.free_tensor.argtypes = [PT]
        for n in ("relu_forward", "cos_forward", "abs_forward"):
            getattr(lib, n).argtypes = [PT, PT]
        for n in ("add_forward", "sub_forward", "mul_forward", "div_forward"):
            getattr(lib, n).argtypes = [PT, PT, PT]
        for n in ("quantize_linear_forward", "dequantize_linear_forward"):
            getattr(lib, n).argtypes = [PT, PT, PT, PT]
        lib.conv2d_forward.argtypes = [PT, PT, PT, PT, ctypes.POINTER(CConvParams)]
        lib.max_pool_forward.argtypes = [PT, PT, ctypes.POINTER(CPoolParams)]
        lib.gemm_forward.argtypes = [PT, PT, PT, PT, ctypes.c_float, ctypes.c_float,
                                     ctypes.c_int, ctypes.c_int]
        lib.softmax_forward.argtypes = [PT, PT, ctypes.c_int]
        for n in ("flatten_forward", "reshape_forward", "global_average_pool_forward"):
            getattr(lib, n).argtypes = [PT, PT]
        lib.dynamic_quantize_linear_forward.argtypes = [PT, PT, PT, PT]
        lib.init_cos_lut.argtypes = []
        lib.init_cos_lut()
        self.lib = lib
        self.has_probes = hasattr(lib, "oracle_encode_f32")
        if self.has_probes:
            lib.oracle_encode_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                              ctypes.c_int]
            lib.oracle_checksum.restype = ctypes.c_uint64
            lib.oracle_checksum.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                            ctypes.c_uint64]

    # -- tensors -----------------------------------------------------------
    def tensor(self, arr, dt):
        dt = dtype_code(dt)
        a = as_storage(arr, dt)
        shape = a.shape if a.ndim else (1,)
        t = self.lib.create_tensor(_ints(shape), len(shape), dt)
        if not t:
            raise MemoryError("create_tensor failed")
        ctypes.memmove(t.contents.data, a.ctypes.data, a.nbytes)
        return t

    def empty(self, shape, dt):
        shape = tuple(int(s) for s in shape) or (1,)
        t = self.lib.create_tensor(_ints(shape), len(shape), dtype_code(dt))
        if not t:
            raise MemoryError("create_tensor failed")
        return t

    def read(self, t, dt):
        dt = dtype_code(dt)
        c = t.contents
        shape = [c.shape[i] for i in range(c.ndim)]
        st = np.dtype(STORAGE[dt])
        buf = (ctypes.c_byte * (c.size * st.itemsize)).from_address(c.data)
        return np.frombuffer(buf, dtype=st).reshape(shape).copy()

    def _run(self, fn, ins, out_shape, out_dt, *extra):
        ts = [self.tensor(a, d) if a is not None else PT() for a, d in ins]
        o = self.empty(out_shape, out_dt)
        try:
            fn(*ts, o, *extra)
            return self.read(o, out_dt)
        finally:
            for t in ts:
                if t:
                    self.lib.free_tensor(t)
            self.lib.free_tensor(o)

    # -- operators ---------------------------------------------------------
    def unary(self, name, x, dtx, dto):
        x = np.asarray(x)
        return self._run(getattr(self.lib, name + "_forward"), [(x, dtx)], x.shape, dto)

    def binary(self, name, a, dta, b, dtb, dto):
        a, b = np.broadcast_arrays(np.asarray(a), np.asarray(b))
        return self._run(getattr(self.lib, name + "_forward"), [(a, dta), (b, dtb)], a.shape, dto)

    def qdq(self, name, x, dtx, s, dts, z, dtz, dty):
        x, s, z = np.broadcast_arrays(np.asarray(x), np.asarray(s), np.asarray(z))
        return self._run(getattr(self.lib, name + "_linear_forward"),
                         [(x, dtx), (s, dts), (z, dtz)], x.shape, dty)

    def conv(self, x, dtx, w, dtw, b, dtb, dty, pads, strides, dilations, group):
        N, C, H, W = x.shape
        M, _, KH, KW = w.shape
        OH = (H + pads[0] + pads[2] - dilations[0] * (KH - 1) - 1) // strides[0] + 1
        OW = (W + pads[1] + pads[3] - dilations[1] * (KW - 1) - 1) // strides[1] + 1
        p = CConvParams()
        keep = [_ints(pads), _ints(strides), _ints(dilations)]
        p.pads, p.strides, p.dilations = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        p.group = int(group)
        return self._run(self.lib.conv2d_forward, [(x, dtx), (w, dtw), (b, dtb)],
                         (N, M, OH, OW), dty, ctypes.byref(p))

    def maxpool(self, x, dtx, dty, kernel_shape, pads, strides, dilations=(1, 1)):
        N, C, H, W = x.shape
        KH, KW = kernel_shape
        OH = (H + pads[0] + pads[2] - dilations[0] * (KH - 1) - 1) // strides[0] + 1
        OW = (W + pads[1] + pads[3] - dilations[1] * (KW - 1) - 1) // strides[1] + 1
        p = CPoolParams()
        keep = [_ints(pads), _ints(strides), _ints(dilations), _ints(kernel_shape)]
        p.pads, p.strides, p.dilations, p.kernel_shape = [
            ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        return self._run(self.lib.max_pool_forward, [(x, dtx)], (N, C, OH, OW), dty,
                         ctypes.byref(p))

    def gemm(self, a, dta, b, dtb, c, dtc, dty, alpha=1.0, beta=1.0, transA=0, transB=0):
        M = a.shape[1] if transA else a.shape[0]
        N = b.shape[0] if transB else b.shape[1]
        if c is not None and c.ndim == 1:          # nn/Operators.py:638-645
            if c.shape[0] == N:
                c = c.reshape(1, -1)
            elif c.shape[0] == M:
                c = c.reshape(-1, 1)
        return self._run(self.lib.gemm_forward, [(a, dta), (b, dtb), (c, dtc)], (M, N), dty,
                         ctypes.c_float(alpha), ctypes.c_float(beta), int(transA), int(transB))

    def softmax(self, x, dtx, dty, axis):
        return self._run(self.lib.softmax_forward, [(x, dtx)], x.shape, dty, int(axis))

    def flatten(self, x, dtx, out_shape, dty=None, name="flatten"):
        """flatten_forward / reshape_forward: byte copy into a tensor of out_shape."""
        x = np.asarray(x)
        return self._run(getattr(self.lib, name + "_forward"), [(x, dtx)], out_shape,
                         dtx if dty is None else dty)

    def gap(self, x, dtx, dty):
        x = np.asarray(x)
        return self._run(self.lib.global_average_pool_forward, [(x, dtx)],
                         x.shape[:-2] + (1, 1), dty)

    def dql(self, x, dtx, zdt="uint8"):
        """dynamic_quantize_linear_forward -> (y uint8, scale float32 [1], zero point [1])."""
        x = np.asarray(x)
        tx = self.tensor(x, dtx)
        ty, ts, tz = self.empty(x.shape, U8), self.empty((1,), F32), self.empty((1,), zdt)
        try:
            self.lib.dynamic_quantize_linear_forward(tx, ty, ts, tz)
            return self.read(ty, U8), self.read(ts, F32), self.read(tz, zdt)
        finally:
            for t in (tx, ty, ts, tz):
                self.lib.free_tensor(t)

    # -- oracle-only probes -------------------------------------------------
    def encode_f32(self, x, dt):
        dt = dtype_code(dt)
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=STORAGE[dt])
        self.lib.oracle_encode_f32(x.ctypes.data, out.ctypes.data, x.size, dt)
        return out

    def checksum(self, codes, base=0):
        codes = np.ascontiguousarray(codes)
        return int(self.lib.oracle_checksum(codes.ctypes.data, codes.size, codes.itemsize,
                                            int(base)))


_lock = threading.Lock()
_cache: dict = {}


def build() -> None:
    """Compile liboracle.so (and oracle/_ref where the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _get(path):
    with _lock:
        if path not in _cache:
            _cache[path] = CpuLib(path)
        return _cache[path]


def oracle() -> CpuLib:
    if not os.path.exists(ORACLE_SO):
        build()
    return _get(ORACLE_SO)


def reference():
    """The compiled reference library, or None where it was never built.

    ``TENSOR_OPS_REF_SO`` names another build of the reference ``tensor_ops.c``
    (the reference's own Python layer loads a hard-coded ``./tensor_ops.so``,
    ``nn/__init__.py:150``); it must exist when set.  Unset: ``oracle/_ref``."""
    path = os.environ.get("TENSOR_OPS_REF_SO")
    if path:
        if not os.path.exists(path):
            raise FileNotFoundError(f"TENSOR_OPS_REF_SO={path} does not exist")
        return _get(os.path.abspath(path))
    return _get(REF_SO) if os.path.exists(REF_SO) else None
