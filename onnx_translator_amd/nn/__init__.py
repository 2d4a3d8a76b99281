"""Host-side operator layer over libtensor_ops_hip.so.

Mirrors the reference's FFI layer (``nn/__init__.py:1-344``): the same
``CTensor`` struct, dtype maps, ``Tensor`` / ``Tensor_`` classes and the
``Ops`` base with ``_execute_unary`` / ``_execute_binary`` /
``_execute_ternary`` / ``_numpy_to_ctensor`` / ``_ctensor_to_numpy``, so the
operator classes in :mod:`onnx_translator_amd.nn.Operators` keep the reference
constructor and ``forward`` API.

Differences, all additive:

* the library is ``libtensor_ops_hip.so`` (``TENSOR_OPS_LIB`` overrides the
  path) and every call is checked: a GPU-side failure, a missing GPU or a
  shape the library rejects raises ``RuntimeError`` instead of returning zeros;
* broadcasting happens in the kernels: operands are passed un-broadcast;
* ``Tensor.data`` may be a :class:`DeviceArray` (HBM-resident); an operator
  with any device operand keeps its output on the device, so graph
  intermediates never round-trip through the host.  ``Tensor.numpy()`` copies
  back.
"""
from __future__ import annotations

import ctypes
import os
import threading

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEFAULT_LIB = os.path.join(PKG_DIR, "libtensor_ops_hip.so")


class CTensor(ctypes.Structure):
    """C tensor struct (``tensor_ops.h:28-34``; reference mirror ``nn/__init__.py:9-17``)."""
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("shape", ctypes.POINTER(ctypes.c_int)),
        ("ndim", ctypes.c_int),
        ("size", ctypes.c_size_t),
        ("dtype", ctypes.c_int),
    ]


# nn/__init__.py:20-34
DTYPE_MAP = {
    "float8_e4m3": 0, "float8_e5m2": 1, "float16": 2, "bfloat16": 3, "float32": 4,
    "float64": 5, "int4": 6, "int8": 7, "uint8": 8, "int16": 9, "int32": 10, "int64": 11,
    "bool": 8,
}

# nn/__init__.py:37-51 (storage types; fp8 codes as uint8, bf16 bits as uint16)
DTYPE_TO_NUMPY = {
    "float8_e4m3": np.uint8, "float8_e5m2": np.uint8, "float16": np.float16,
    "bfloat16": np.uint16, "float32": np.float32, "float64": np.float64, "int4": np.int8,
    "int8": np.int8, "uint8": np.uint8, "int16": np.int16, "int32": np.int32,
    "int64": np.int64, "bool": np.bool_,
}

# nn/__init__.py:54-72
NUMPY_TO_DTYPE = {
    np.float16: "float16", np.uint16: "bfloat16", np.float32: "float32",
    np.float64: "float64", np.int8: "int8", np.uint8: "uint8", np.int16: "int16",
    np.int32: "int32", np.int64: "int64",
}
NUMPY_TO_DTYPE[np.dtype("intc").type] = "int32" if np.dtype("intc").itemsize == 4 else "int64"

# nn/__init__.py:75-92, plus the ONNX FP8 element types (17 float8e4m3fn, 19 float8e5m2)
onnx_dtype_mapping = {
    1: "float32", 2: "uint8", 3: "int8", 4: "uint16", 5: "int16", 6: "int32", 7: "int64",
    8: "string", 9: "bool", 10: "float16", 11: "float64", 12: "uint32", 13: "uint64",
    14: "complex64", 15: "complex128", 16: "bfloat16", 17: "float8_e4m3", 19: "float8_e5m2",
}

PT = ctypes.POINTER(CTensor)


def _shape_arr(shape):
    return (ctypes.c_int * max(len(shape), 1))(*[int(s) for s in shape])


class DeviceArray:
    """An HBM-resident tensor owned by libtensor_ops_hip (``create_tensor_device``)."""

    def __init__(self, lib, shape, dtype: str, ptr=None, zero: bool = True):
        self.lib = lib
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        if ptr is None:
            shp = self.shape or (1,)
            make = lib.create_tensor_device if zero else lib.create_tensor_device_empty
            ptr = make(_shape_arr(shp), len(shp), DTYPE_MAP[dtype])
            if not ptr:
                raise RuntimeError("create_tensor_device failed: " + Ops._last_error(lib))
        self.ptr = ptr

    @property
    def size(self):
        return int(np.prod(self.shape)) if self.shape else 1

    @property
    def ndim(self):
        return len(self.shape)

    @classmethod
    def from_numpy(cls, lib, arr: np.ndarray, dtype: str) -> "DeviceArray":
        arr = np.ascontiguousarray(np.asarray(arr).astype(DTYPE_TO_NUMPY[dtype], copy=False))
        d = cls(lib, arr.shape, dtype)
        if lib.tensor_from_host(d.ptr, arr.ctypes.data_as(ctypes.c_void_p)) != 0:
            raise RuntimeError("tensor_from_host failed: " + Ops._last_error(lib))
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=DTYPE_TO_NUMPY[self.dtype])
        if self.lib.tensor_to_host(self.ptr, out.ctypes.data_as(ctypes.c_void_p)) != 0:
            raise RuntimeError("tensor_to_host failed: " + Ops._last_error(self.lib))
        return out

    def __del__(self):
        ptr, self.ptr = getattr(self, "ptr", None), None
        if ptr:
            try:
                self.lib.free_tensor(ptr)
            except Exception:
                pass


class Tensor:
    """Tensor with host (numpy) or device (:class:`DeviceArray`) data (``nn/__init__.py:94-116``)."""

    def __init__(self, *size, dtype="float32", data=None):
        self.size = size[0] if (len(size) == 1 and isinstance(size[0], (list, tuple))) else size
        self.size = tuple(self.size)
        self.data_size = 1
        for s in self.size:
            self.data_size *= s
        self.dtype = dtype
        if data is not None:
            self.data = data
        else:
            self.data = np.zeros(self.size, dtype=DTYPE_TO_NUMPY[dtype])

    @property
    def on_device(self) -> bool:
        return isinstance(self.data, DeviceArray)

    def to_device(self) -> "Tensor":
        if self.on_device:
            return self
        lib = Ops._get_lib()
        return Tensor(*self.size, dtype=self.dtype,
                      data=DeviceArray.from_numpy(lib, self.data, self.dtype))

    def numpy(self) -> np.ndarray:
        return self.data.numpy() if self.on_device else np.asarray(self.data)


class Tensor_:
    """Shape / dtype placeholder for graph construction (``nn/__init__.py:118-133``)."""

    def __init__(self, *size, dtype="float32"):
        self.size = size[0] if (len(size) == 1 and isinstance(size[0], (list, tuple))) else size
        self.size = tuple(self.size)
        self.data_size = 1
        for s in self.size:
            self.data_size *= s
        self.dtype = dtype


def _sig(lib, name, restype, argtypes):
    f = getattr(lib, name)
    f.restype = restype
    f.argtypes = argtypes


class Ops:
    """Operator base class (``nn/__init__.py:135-344``)."""
    _lib = None
    _lib_initialized = False
    _lock = threading.Lock()

    @classmethod
    def _get_lib(cls):
        """Load libtensor_ops_hip.so once per process (``nn/__init__.py:141-173``)."""
        if cls._lib is None:
            with cls._lock:
                if cls._lib is None:
                    path = os.environ.get("TENSOR_OPS_LIB", DEFAULT_LIB)
                    if not os.path.exists(path):
                        raise RuntimeError(
                            f"{path} not found: build it with `python -m onnx_translator_amd.build`")
                    lib = ctypes.CDLL(path)
                    P = PT
                    _sig(lib, "create_tensor", P, [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int])
                    _sig(lib, "create_tensor_device", P,
                         [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int])
                    _sig(lib, "create_tensor_device_empty", P,
                         [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int])
                    _sig(lib, "tensor_wrap_device", P,
                         [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int])
                    _sig(lib, "free_tensor", None, [P])
                    for n in ("relu_forward", "cos_forward", "abs_forward"):
                        _sig(lib, n, None, [P, P])
                    for n in ("add_forward", "sub_forward", "mul_forward", "div_forward"):
                        _sig(lib, n, None, [P, P, P])
                    for n in ("quantize_linear_forward", "dequantize_linear_forward"):
                        _sig(lib, n, None, [P, P, P, P])
                    for n in ("quantize_linear_axis_forward", "dequantize_linear_axis_forward"):
                        _sig(lib, n, None, [P, P, P, P, ctypes.c_int])
                    for n in ("flatten_forward", "reshape_forward", "global_average_pool_forward"):
                        _sig(lib, n, None, [P, P])
                    _sig(lib, "dynamic_quantize_linear_forward", None, [P, P, P, P])
                    _sig(lib, "tensor_is_device", ctypes.c_int, [P])
                    _sig(lib, "tensor_to_host", ctypes.c_int, [P, ctypes.c_void_p])
                    _sig(lib, "tensor_from_host", ctypes.c_int, [P, ctypes.c_void_p])
                    _sig(lib, "tensor_ops_hip_sync", ctypes.c_int, [])
                    _sig(lib, "tensor_ops_hip_set_stream", None, [ctypes.c_void_p])
                    _sig(lib, "tensor_ops_hip_get_stream", ctypes.c_void_p, [])
                    _sig(lib, "tensor_ops_hip_device_count", ctypes.c_int, [])
                    _sig(lib, "tensor_ops_hip_last_error", ctypes.c_char_p, [])
                    _sig(lib, "tensor_ops_hip_clear_error", None, [])
                    _sig(lib, "tensor_ops_hip_version", ctypes.c_char_p, [])
                    _sig(lib, "tensor_ops_hip_set_exact", None, [ctypes.c_int])
                    _sig(lib, "init_cos_lut", None, [])
                    lib.init_cos_lut()
                    cls._lib = lib
                    cls._lib_initialized = True
        return cls._lib

    @staticmethod
    def _last_error(lib) -> str:
        e = lib.tensor_ops_hip_last_error()
        return e.decode() if e else ""

    def __init__(self, inputs, outputs):
        self.inputs = inputs
        self.outputs = outputs
        self.parameters = {}
        self.name = None
        self.lib = self._get_lib()

    # -- call checking ---------------------------------------------------------
    def _call(self, c_func_name, *args):
        self.lib.tensor_ops_hip_clear_error()
        getattr(self.lib, c_func_name)(*args)
        err = self._last_error(self.lib)
        if err:
            raise RuntimeError(f"{c_func_name}: {err}")

    # -- marshalling -------------------------------------------------------------
    def _in_ctensor(self, t: Tensor, keep: list):
        """C tensor for an input: the device tensor itself, or a host copy."""
        if isinstance(t.data, DeviceArray):
            return t.data.ptr
        arr = np.ascontiguousarray(np.asarray(t.data).astype(DTYPE_TO_NUMPY[t.dtype], copy=False))
        c = self._numpy_to_ctensor(arr, t.dtype)
        keep.append(c)
        return c

    def _out_ctensor(self, shape, dtype, device: bool):
        if device:
            # operators write their whole output: no zero fill needed
            d = DeviceArray(self.lib, shape, dtype, zero=False)
            return d, d.ptr
        shp = tuple(shape) or (1,)
        c = self.lib.create_tensor(_shape_arr(shp), len(shp), DTYPE_MAP[dtype])
        if not c:
            raise MemoryError("create_tensor failed")
        return None, c

    def _finish(self, shape, dtype, dev, c_out, keep):
        try:
            if dev is not None:
                return Tensor(*shape, dtype=dtype, data=dev)
            data = self._ctensor_to_numpy(c_out, dtype).reshape(shape)
            return Tensor(*shape, dtype=dtype, data=data)
        finally:
            if dev is None:
                self.lib.free_tensor(c_out)
            for c in keep:
                self.lib.free_tensor(c)

    def _run(self, c_func_name, ins, out_shape, out_dtype, *extra, arrange=None):
        """Call c_func_name(*inputs, output, *extra) (or the argument list
        ``arrange(inputs, output)`` builds) and wrap the output."""
        keep: list = []
        dev = any(isinstance(t.data, DeviceArray) for t in ins if t is not None)
        try:
            cins = [self._in_ctensor(t, keep) if t is not None else PT() for t in ins]
            dev_out, c_out = self._out_ctensor(out_shape, out_dtype, dev)
        except Exception:
            for c in keep:
                self.lib.free_tensor(c)
            raise
        try:
            if arrange is None:
                self._call(c_func_name, *cins, c_out, *extra)
            else:
                self._call(c_func_name, *arrange(cins, c_out))
        except Exception:
            if dev_out is None:
                self.lib.free_tensor(c_out)
            for c in keep:
                self.lib.free_tensor(c)
            raise
        return self._finish(out_shape, out_dtype, dev_out, c_out, keep)

    # -- reference execution templates (nn/__init__.py:189-279) --------------------
    def _execute_unary(self, input_tensor, c_func_name):
        out_dtype = self.dtype if self.dtype else input_tensor.dtype
        return self._run(c_func_name, [input_tensor], tuple(input_tensor.size), out_dtype)

    def _execute_binary(self, input_a, input_b, c_func_name):
        try:
            out_shape = np.broadcast_shapes(tuple(input_a.size), tuple(input_b.size))
        except ValueError:
            print(f"Broadcasting error: {input_a.size} vs {input_b.size}")
            raise
        if self.dtype:
            out_dtype = self.dtype
        else:
            res = np.result_type(np.dtype(DTYPE_TO_NUMPY[input_a.dtype]),
                                 np.dtype(DTYPE_TO_NUMPY[input_b.dtype]))
            out_dtype = NUMPY_TO_DTYPE.get(res.type, "float32")
        return self._run(c_func_name, [input_a, input_b], out_shape, out_dtype)

    def _execute_ternary(self, in_a, in_b, in_c, c_func_name):
        try:
            out_shape = np.broadcast_shapes(tuple(in_a.size), tuple(in_b.size), tuple(in_c.size))
        except ValueError:
            print(f"Broadcasting error in ternary op: {in_a.size}, {in_b.size}, {in_c.size}")
            raise
        out_dtype = self.dtype if self.dtype else "float32"
        return self._run(c_func_name, [in_a, in_b, in_c], out_shape, out_dtype)

    def forward(self, input):
        pass

    def forward_(self, input):
        pass

    def _numpy_to_ctensor(self, arr: np.ndarray, dtype: str):
        """Host C tensor holding a copy of ``arr`` (``nn/__init__.py:305-323``)."""
        shape = arr.shape if arr.ndim else (1,)
        c_tensor = self.lib.create_tensor(_shape_arr(shape), len(shape), DTYPE_MAP[dtype])
        if not c_tensor:
            raise MemoryError("create_tensor failed")
        ctypes.memmove(c_tensor.contents.data, arr.ctypes.data, arr.size * arr.itemsize)
        return c_tensor

    def _ctensor_to_numpy(self, c_tensor, dtype: str) -> np.ndarray:
        """Copy of a host C tensor's data (``nn/__init__.py:325-344``)."""
        c = c_tensor.contents
        shape = [c.shape[i] for i in range(c.ndim)]
        np_dtype = DTYPE_TO_NUMPY[dtype]
        nbytes = c.size * np.dtype(np_dtype).itemsize
        arr = np.frombuffer((ctypes.c_byte * nbytes).from_address(c.data), dtype=np_dtype)
        return arr.reshape(shape).copy()


def __getattr__(name):
    """``nn.Graph`` as in the reference (``nn/__init__.py:346``), imported lazily
    because the graph module builds on the operator classes."""
    if name == "Graph":
        from .graph import Graph
        return Graph
    raise AttributeError(name)
