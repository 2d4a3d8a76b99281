"""The C ABI of libtensor_ops_hip.so, checked without a GPU.

* every function declared in include/tensor_ops.h is exported;
* struct layouts match the reference (tensor_ops.h:28-54, LP64);
* tensor lifecycle works everywhere (host memory, zero-filled);
* with no GPU, operators leave the output untouched and report an error
  that the Python layer turns into an exception (never a silent CPU path).
"""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import HIP_SO, HipLib, ROOT

HEADER = os.path.join(ROOT, "include", "tensor_ops.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(\w+)\s*\([^;]*\)\s*;", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "while")))


@pytest.fixture(scope="module")
def lib():
    return HipLib()


def test_library_built():
    assert os.path.exists(HIP_SO), "run `python -m onnx_translator_amd.build`"


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 16 + 12, names
    missing = [n for n in names if not hasattr(lib.lib, n)]
    assert not missing, f"declared in include/tensor_ops.h but not exported: {missing}"


def test_reference_hot_path_symbols_present(lib):
    for n in ("create_tensor", "free_tensor", "init_cos_lut", "relu_forward", "cos_forward", "abs_forward",
              "add_forward", "sub_forward", "mul_forward", "div_forward", "quantize_linear_forward",
              "dequantize_linear_forward", "conv2d_forward", "max_pool_forward", "gemm_forward",
              "softmax_forward"):
        assert hasattr(lib.lib, n), n


def test_struct_layout():
    assert ctypes.sizeof(O.CTensor) == 40
    assert [O.CTensor.data.offset, O.CTensor.shape.offset, O.CTensor.ndim.offset, O.CTensor.size.offset,
            O.CTensor.dtype.offset] == [0, 8, 16, 24, 32]
    assert ctypes.sizeof(O.CConvParams) == 32 and O.CConvParams.group.offset == 24
    assert ctypes.sizeof(O.CPoolParams) == 32
    from onnx_translator_amd.nn import CTensor
    from onnx_translator_amd.nn.Operators import CConvParams, CPoolParams
    assert ctypes.sizeof(CTensor) == 40 and ctypes.sizeof(CConvParams) == 32 and ctypes.sizeof(CPoolParams) == 32


def test_dtype_codes_match_reference():
    from onnx_translator_amd.nn import DTYPE_MAP
    assert DTYPE_MAP == {"float8_e4m3": 0, "float8_e5m2": 1, "float16": 2, "bfloat16": 3, "float32": 4,
                         "float64": 5, "int4": 6, "int8": 7, "uint8": 8, "int16": 9, "int32": 10, "int64": 11,
                         "bool": 8}


def test_create_tensor_zeroed_and_sized(lib):
    for dt, nbytes in ((O.E4M3, 1), (O.F16, 2), (O.F32, 4), (O.F64, 8), (O.I4, 1), (O.I64, 8)):
        t = lib.empty((3, 5, 7), dt)
        c = t.contents
        assert c.ndim == 3 and c.size == 105 and c.dtype == dt
        assert [c.shape[i] for i in range(3)] == [3, 5, 7]
        assert not lib.read(t, dt).view(np.uint8).any()
        lib.lib.free_tensor(t)
    lib.lib.free_tensor(O.PT())          # NULL is ignored


def test_host_roundtrip_through_memmove(lib):
    a = np.arange(1000, dtype=np.float32)
    t = lib.tensor(a, O.F32)
    assert np.array_equal(lib.read(t, O.F32), a)
    assert lib.lib.tensor_is_device(t) == 0
    out = np.empty_like(a)
    assert lib.lib.tensor_to_host(t, out.ctypes.data) == 0 and np.array_equal(out, a)
    lib.lib.free_tensor(t)


def test_no_gpu_fails_loudly(lib):
    # Decided at run time, not at collection: loading the library while pytest
    # collects would bind the process to its HIP runtime before torch loads.
    if lib.device_count() > 0:
        pytest.skip("checks the no-GPU behaviour")
    with pytest.raises(RuntimeError, match="no HIP device"):
        lib.binary("add", np.ones(4, np.float32), O.F32, np.ones(4, np.float32), O.F32, O.F32)
    # output untouched (zeros), as the reference's silent no-op leaves it
    a = lib.tensor(np.ones(4, np.float32), O.F32)
    o = lib.empty((4,), O.F32)
    lib.lib.add_forward(a, a, o)
    assert "no HIP device" in lib.last_error()
    assert not lib.read(o, O.F32).any()
    lib.lib.free_tensor(a)
    lib.lib.free_tensor(o)
    from onnx_translator_amd.nn import Tensor
    from onnx_translator_amd.nn.Operators import ADD
    x = Tensor(2, 2, dtype="float32", data=np.ones((2, 2), np.float32))
    with pytest.raises(RuntimeError):
        ADD([], [], "float32").forward(x, x)


def test_free_tensor_ownership_per_header(lib):
    """Each header releases only what it owns: two wrappers over one buffer, and a
    wrapper over a library tensor's data, can be freed in either order."""
    L = lib.lib
    L.tensor_wrap_device.restype = O.PT
    L.tensor_wrap_device.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
    L.tensor_ops_hip_clear_error.argtypes = []
    buf = np.arange(16, dtype=np.float32)
    shp = (ctypes.c_int * 1)(16)
    w1 = L.tensor_wrap_device(buf.ctypes.data, shp, 1, O.F32)
    w2 = L.tensor_wrap_device(buf.ctypes.data, shp, 1, O.F32)
    L.free_tensor(w1)
    L.free_tensor(w2)                     # must not free() the caller's buffer
    assert np.array_equal(buf, np.arange(16, dtype=np.float32))
    for owner_first in (True, False):
        t = lib.tensor(np.ones(16, np.float32), O.F32)
        w = L.tensor_wrap_device(t.contents.data, shp, 1, O.F32)
        if owner_first:
            L.free_tensor(t)
            L.free_tensor(w)
        else:
            L.free_tensor(w)
            assert np.array_equal(lib.read(t, O.F32), np.ones(16, np.float32))
            L.free_tensor(t)
    # a header the library did not create is left alone, with an error
    foreign = O.CTensor(ctypes.c_void_p(buf.ctypes.data), ctypes.cast(shp, ctypes.POINTER(ctypes.c_int)), 1, 16, O.F32)
    L.tensor_ops_hip_clear_error()
    L.free_tensor(ctypes.byref(foreign))
    assert "not created by this library" in lib.last_error()
    L.tensor_ops_hip_clear_error()


def test_dequantize_conv_rejects_non_4d_input(lib):
    """A rank other than 4 is an error before any allocation (ranks above 8 once
    overran a fixed shape buffer on the unfused path)."""
    L = lib.lib
    xq = lib.tensor(np.zeros((1,) * 9, np.uint8), O.U8)
    s = lib.tensor(np.ones(1, np.float32), O.F32)
    w = lib.tensor(np.ones((1, 1, 1, 1), np.float32), O.F32)
    y = lib.empty((1, 1, 1, 1), O.F32)
    L.tensor_ops_hip_clear_error()
    L.dequantize_conv2d_fused_forward(xq, s, O.PT(), w, O.PT(), O.PT(), 0, y, ctypes.POINTER(O.CConvParams)())
    assert "must be 4-D" in lib.last_error()
    L.tensor_ops_hip_clear_error()
    for t in (xq, s, w, y):
        L.free_tensor(t)
