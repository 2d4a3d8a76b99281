"""Operator classes over libtensor_ops_hip.so: the 13 hot-path operators and
the ones a ResNet-style graph needs next to them (Flatten, Reshape,
GlobalAveragePool, DynamicQuantizeLinear).

Same class names, constructor signatures and ``forward`` / ``forward_``
results as the reference (``nn/Operators.py:9-704``):
``forward`` returns ``{"tensor": Tensor, "parameters": None, "graph": None}``
and stores it in ``self.parameters["values"]``.  Inputs may be host (numpy)
or device-resident tensors; see :mod:`onnx_translator_amd.nn`.

Additions: ``QuantizeLinear.forward_`` (absent in the reference),
``DequantizeLinear(axis=...)`` for per-axis scales (the reference ignores the
axis and lets numpy align a 1-D scale with the last dimension; ``axis=None``
keeps that behaviour), and ``MaxPool.forward_`` uses the dilation-aware
output formula of ``MaxPool.forward``.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import DTYPE_MAP, DTYPE_TO_NUMPY, DeviceArray, Ops, Tensor, Tensor_, PT

__all__ = ["CConvParams", "CPoolParams", "CReduceParams", "RELU", "COS", "ABS", "ADD", "SUB", "MUL", "DIV",
           "QuantizeLinear", "DequantizeLinear", "Conv", "MaxPool", "Gemm", "Softmax", "Flatten", "Reshape",
           "GlobalAveragePool", "DynamicQuantizeLinear", "ElementwiseChain", "CChainStep"]


class CConvParams(ctypes.Structure):
    """``ConvParams`` (tensor_ops.h:39-44; nn/Operators.py:9-15)."""
    _fields_ = [("pads", ctypes.POINTER(ctypes.c_int)), ("strides", ctypes.POINTER(ctypes.c_int)),
                ("dilations", ctypes.POINTER(ctypes.c_int)), ("group", ctypes.c_int)]


class CPoolParams(ctypes.Structure):
    """``PoolParams`` (tensor_ops.h:49-54; nn/Operators.py:17-23)."""
    _fields_ = [("pads", ctypes.POINTER(ctypes.c_int)), ("strides", ctypes.POINTER(ctypes.c_int)),
                ("dilations", ctypes.POINTER(ctypes.c_int)), ("kernel_shape", ctypes.POINTER(ctypes.c_int))]


class CReduceParams(ctypes.Structure):
    """``ReduceParams`` (tensor_ops.h:56-60; nn/Operators.py:25-30)."""
    _fields_ = [("axes", ctypes.POINTER(ctypes.c_int)), ("num_axes", ctypes.c_int), ("keepdims", ctypes.c_int)]


def _values(op, t):
    values = {"tensor": t, "parameters": None, "graph": None}
    op.parameters = {"values": values}
    return values


def _int_arr(vals):
    return (ctypes.c_int * len(vals))(*[int(v) for v in vals])


def _broadcast_dtype(a, b):
    """Output dtype of a binary op with no declared dtype (nn/Operators.py:216-230)."""
    import onnx_translator_amd.nn as nn
    res = np.result_type(np.dtype(DTYPE_TO_NUMPY[a.dtype]), np.dtype(DTYPE_TO_NUMPY[b.dtype]))
    if res.type in nn.NUMPY_TO_DTYPE:
        return nn.NUMPY_TO_DTYPE[res.type]
    if "float" in str(res):
        return "float64"
    if "int" in str(res):
        return "int64"
    return "float32"


class _Unary(Ops):
    c_name = ""

    def __init__(self, inputs, outputs, dtype, version="17"):
        super().__init__(inputs, outputs)
        self.dtype = dtype
        self.version = version

    def forward(self, input: Tensor):
        return _values(self, self._execute_unary(input, self.c_name))

    def forward_(self, input: Tensor_):
        return _values(self, Tensor_(*input.size, dtype=self.dtype))


class RELU(_Unary):
    """ReLU (nn/Operators.py:32-79 -> tensor_ops.c:708-728)."""
    c_name = "relu_forward"


class COS(_Unary):
    """Cos via the reference's table lookup (nn/Operators.py:81-128 -> tensor_ops.c:840-854)."""
    c_name = "cos_forward"


class ABS(_Unary):
    """Abs (nn/Operators.py:130-168 -> tensor_ops.c:736-757)."""
    c_name = "abs_forward"


class _Binary(Ops):
    c_name = ""
    label = ""

    def __init__(self, inputs, outputs, dtype, version="17"):
        super().__init__(inputs, outputs)
        self.dtype = dtype
        self.version = version

    def forward(self, *inputs):
        if len(inputs) != 2:
            raise ValueError(f"{self.label} operator expects 2 inputs, but got {len(inputs)}")
        return _values(self, self._execute_binary(inputs[0], inputs[1], self.c_name))

    def forward_(self, *inputs):
        if len(inputs) != 2:
            raise ValueError(f"{self.label} operator expects 2 inputs (Tensor_), but got {len(inputs)}")
        a, b = inputs
        try:
            shape = np.broadcast_shapes(tuple(a.size), tuple(b.size))
        except ValueError:
            print(f"Error during broadcasting shapes {a.size} and {b.size}")
            raise
        return _values(self, Tensor_(*shape, dtype=_broadcast_dtype(a, b)))


class ADD(_Binary):
    """A + B with broadcasting and type promotion (nn/Operators.py:170-240 -> tensor_ops.c:864-890)."""
    c_name, label = "add_forward", "ADD"


class SUB(_Binary):
    """A - B (nn/Operators.py:242-303 -> tensor_ops.c:900-925)."""
    c_name, label = "sub_forward", "SUB"


class MUL(_Binary):
    """A * B (nn/Operators.py:305-365 -> tensor_ops.c:935-960)."""
    c_name, label = "mul_forward", "MUL"


class DIV(_Binary):
    """A / B (nn/Operators.py:367-425 -> tensor_ops.c:970-997)."""
    c_name, label = "div_forward", "DIV"


def _is_1d(t):
    return len(tuple(t.size)) == 1


class QuantizeLinear(Ops):
    """y = saturate(rint(x / s) + zp) (nn/Operators.py:427-450 -> tensor_ops.c:999-1016)."""

    def __init__(self, inputs, outputs, axis=1, dtype=None, version="17"):
        super().__init__(inputs, outputs)
        self.dtype = dtype
        self.axis = axis
        self.version = version

    def forward(self, x, y_scale, y_zero_point):
        nd = len(tuple(x.size))
        if _is_1d(y_scale) and nd > 1:
            # nn/Operators.py:439-445 reshapes a 1-D scale onto `axis`; the library's
            # per-axis entry point does the same without touching the data.
            axis = self.axis if self.axis >= 0 else self.axis + nd
            out_dtype = self.dtype if self.dtype else "float32"
            t = self._run("quantize_linear_axis_forward", [x, y_scale, y_zero_point], tuple(x.size),
                          out_dtype, ctypes.c_int(axis))
            return _values(self, t)
        return _values(self, self._execute_ternary(x, y_scale, y_zero_point, "quantize_linear_forward"))

    def forward_(self, x, y_scale, y_zero_point):
        return _values(self, Tensor_(*x.size, dtype=self.dtype))


class DequantizeLinear(Ops):
    """y = (x - zp) * s (nn/Operators.py:452-473 -> tensor_ops.c:1018-1034)."""

    def __init__(self, inputs, outputs, dtype=None, version="17", axis=None):
        super().__init__(inputs, outputs)
        self.dtype = dtype
        self.version = version
        self.axis = axis

    def forward(self, x, x_scale, x_zero_point):
        nd = len(tuple(x.size))
        if self.axis is not None and _is_1d(x_scale) and nd > 1:
            axis = self.axis if self.axis >= 0 else self.axis + nd
            out_dtype = self.dtype if self.dtype else "float32"
            t = self._run("dequantize_linear_axis_forward", [x, x_scale, x_zero_point], tuple(x.size),
                          out_dtype, ctypes.c_int(axis))
            return _values(self, t)
        return _values(self, self._execute_ternary(x, x_scale, x_zero_point, "dequantize_linear_forward"))

    def forward_(self, x, x_scale, x_zero_point):
        if self.axis is not None and len(tuple(x_scale.size)) == 1 and len(tuple(x.size)) > 1:
            return _values(self, Tensor_(*x.size, dtype=self.dtype))      # per-axis scale: x's shape
        try:
            shape = np.broadcast_shapes(tuple(x.size), tuple(x_scale.size), tuple(x_zero_point.size))
        except ValueError:
            shape = tuple(x.size)
        return _values(self, Tensor_(*shape, dtype=self.dtype))


def _pool_out(h, w, pads, strides, dilations, kh, kw):
    """nn/Operators.py:499-501 and :569-570."""
    oh = (h + pads[0] + pads[2] - dilations[0] * (kh - 1) - 1) // strides[0] + 1
    ow = (w + pads[1] + pads[3] - dilations[1] * (kw - 1) - 1) // strides[1] + 1
    return oh, ow


class Conv(Ops):
    """2-D convolution, NCHW (nn/Operators.py:475-548 -> tensor_ops.c:1036-1114)."""

    def __init__(self, inputs, outputs, pads, strides, dilations, group, dtype, version="17"):
        super().__init__(inputs, outputs)
        self.pads, self.strides, self.dilations, self.group = pads, strides, dilations, group
        self.dtype = dtype
        self.version = version
        self.lib.conv2d_forward.argtypes = [PT, PT, PT, PT, ctypes.POINTER(CConvParams)]
        self.lib.conv2d_forward.restype = None

    def _params(self):
        keep = [_int_arr(self.pads), _int_arr(self.strides), _int_arr(self.dilations)]
        p = CConvParams()
        p.pads, p.strides, p.dilations = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        p.group = int(self.group)
        return p, keep

    def forward(self, x: Tensor, w: Tensor, b: Tensor = None):
        N, _, H, W = x.size
        M, _, KH, KW = w.size
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        p, keep = self._params()
        t = self._run("conv2d_forward", [x, w, b], (N, M, OH, OW), self.dtype, ctypes.byref(p))
        del keep
        return _values(self, t)

    def forward_(self, x: Tensor_, w: Tensor_, b: Tensor_ = None):
        N, _, H, W = x.size
        M, _, KH, KW = w.size
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        return _values(self, Tensor_(N, M, OH, OW, dtype=self.dtype))


class FusedConv(Conv):
    """Conv -> Relu -> Add(., skip) of a residual block in one call to
    ``conv2d_fused_forward``: y = [skip +] [Relu](Conv(x, w, b)), equal to the
    three operators (nn/Operators.py:475-548, :32-79, :170-219) bit for bit.
    ``inputs`` = [x, w, b or "", skip or ""]."""

    def __init__(self, inputs, outputs, pads, strides, dilations, group, dtype, relu, version="17"):
        super().__init__(inputs, outputs, pads, strides, dilations, group, dtype, version)
        self.relu = 1 if relu else 0
        self.lib.conv2d_fused_forward.argtypes = [PT, PT, PT, PT, ctypes.c_int, PT, ctypes.POINTER(CConvParams)]
        self.lib.conv2d_fused_forward.restype = None

    def forward(self, x: Tensor, w: Tensor, b: Tensor = None, skip: Tensor = None):
        N, _, H, W = x.size
        M, _, KH, KW = w.size
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        p, keep = self._params()
        relu = ctypes.c_int(self.relu)

        def arrange(ins, out):
            return (ins[0], ins[1], ins[2], ins[3], relu, out, ctypes.byref(p))
        t = self._run("conv2d_fused_forward", [x, w, b, skip], (N, M, OH, OW), self.dtype, arrange=arrange)
        del keep
        return _values(self, t)

    def forward_(self, x: Tensor_, w: Tensor_, b: Tensor_ = None, skip: Tensor_ = None):
        return super().forward_(x, w, b)


class FusedConvQDQ(FusedConv):
    """Conv -> Relu -> Add(., skip) -> QuantizeLinear -> DequantizeLinear in one
    call to ``conv2d_fused_qdq_forward``: y = DQ(Q([skip +] [Relu](Conv(x, w, b)))),
    the fake quantization applied in the convolution's epilogue, so neither the
    block output before quantization nor the codes are written.  Equal to the
    operator sequence (nn/Operators.py:475-548, :32-79, :170-219, :427-473) bit
    for bit.  ``inputs`` = [x, w, b or "", skip or "", q_scale, q_zero_point,
    d_scale, d_zero_point]; codes of dtype ``code_dtype``."""

    def __init__(self, inputs, outputs, pads, strides, dilations, group, dtype, relu, code_dtype, version="17"):
        super().__init__(inputs, outputs, pads, strides, dilations, group, dtype, relu, version)
        self.code_dtype = code_dtype
        self.lib.conv2d_fused_qdq_forward.argtypes = [PT, PT, PT, PT, ctypes.c_int, PT, PT, PT, PT, ctypes.c_int, PT,
                                                      ctypes.POINTER(CConvParams)]
        self.lib.conv2d_fused_qdq_forward.restype = None

    def forward(self, x: Tensor, w: Tensor, b: Tensor = None, skip: Tensor = None, q_scale: Tensor = None,
                q_zero_point: Tensor = None, d_scale: Tensor = None, d_zero_point: Tensor = None):
        N, _, H, W = x.size
        M, _, KH, KW = w.size
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        p, keep = self._params()
        relu, code = ctypes.c_int(self.relu), ctypes.c_int(DTYPE_MAP[self.code_dtype])

        def arrange(ins, out):
            return (ins[0], ins[1], ins[2], ins[3], relu, ins[4], ins[5], ins[6], ins[7], code, out, ctypes.byref(p))
        t = self._run("conv2d_fused_qdq_forward", [x, w, b, skip, q_scale, q_zero_point, d_scale, d_zero_point],
                      (N, M, OH, OW), self.dtype, arrange=arrange)
        del keep
        return _values(self, t)

    def forward_(self, x: Tensor_, w: Tensor_, b: Tensor_ = None, *rest):
        return super().forward_(x, w, b)


class DequantizeConv(FusedConv):
    """DequantizeLinear -> Conv [-> Relu] [-> Add(., skip)] of a QDQ block in one call
    to ``dequantize_conv2d_fused_forward``: the convolution reads the uint8 / int8
    activation codes and never materialises the float32 activation; equal to the
    operator sequence (nn/Operators.py:452-473, :475-548, :32-79, :170-219) bit for
    bit.  ``inputs`` = [x codes, x scale, x zero point or "", w, b or "", skip or ""];
    the scale and zero point hold one element."""

    def __init__(self, inputs, outputs, pads, strides, dilations, group, dtype, relu, version="17"):
        super().__init__(inputs, outputs, pads, strides, dilations, group, dtype, relu, version)
        self.lib.dequantize_conv2d_fused_forward.argtypes = [PT, PT, PT, PT, PT, PT, ctypes.c_int, PT,
                                                             ctypes.POINTER(CConvParams)]
        self.lib.dequantize_conv2d_fused_forward.restype = None

    def forward(self, xq: Tensor, x_scale: Tensor, x_zero_point: Tensor = None, w: Tensor = None, b: Tensor = None,
                skip: Tensor = None):
        N, _, H, W = xq.size
        M, _, KH, KW = w.size
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        p, keep = self._params()
        relu = ctypes.c_int(self.relu)

        def arrange(ins, out):
            return (ins[0], ins[1], ins[2], ins[3], ins[4], ins[5], relu, out, ctypes.byref(p))
        t = self._run("dequantize_conv2d_fused_forward", [xq, x_scale, x_zero_point, w, b, skip], (N, M, OH, OW),
                      self.dtype, arrange=arrange)
        del keep
        return _values(self, t)

    def forward_(self, xq: Tensor_, x_scale: Tensor_ = None, x_zero_point: Tensor_ = None, w: Tensor_ = None,
                 b: Tensor_ = None, skip: Tensor_ = None):
        return Conv.forward_(self, xq, w, b)


class QuantizeNHWC(Ops):
    """QuantizeLinear of a float32 NCHW tensor into the channels-last int8 codes
    that :class:`QConvBlock` reads (``quantize_linear_nhwc_forward``): the codes
    of QuantizeLinear (nn/Operators.py:427-450, tensor_ops.c:999-1016) bit for
    bit, stored [N, H, W, C] as code - 128 for uint8 (the code for int8).
    ``inputs`` = [x, scale, zero point or ""] with one-element parameters."""

    def __init__(self, inputs, outputs, code_dtype, version="17"):
        super().__init__(inputs, outputs)
        self.code_dtype = code_dtype
        self.version = version
        self.lib.quantize_linear_nhwc_forward.argtypes = [PT, PT, PT, ctypes.c_int, PT]
        self.lib.quantize_linear_nhwc_forward.restype = None

    def forward(self, x: Tensor, scale: Tensor, zero_point: Tensor = None):
        N, C, H, W = x.size
        code = ctypes.c_int(DTYPE_MAP[self.code_dtype])

        def arrange(ins, out):
            return (ins[0], ins[1], ins[2], code, out)
        t = self._run("quantize_linear_nhwc_forward", [x, scale, zero_point], (N, H, W, C), "int8", arrange=arrange)
        return _values(self, t)

    def forward_(self, x: Tensor_, *rest):
        N, C, H, W = x.size
        return _values(self, Tensor_(N, H, W, C, dtype="int8"))


class CQConvBlock(ctypes.Structure):
    """``QConvBlock`` (tensor_ops.h extension)."""
    _fields_ = [("x_scale", PT), ("x_zero", PT), ("x_codes", ctypes.c_int), ("w", PT), ("w_sum", PT),
                ("w_scale", PT), ("bias", PT), ("relu", ctypes.c_int), ("p", PT), ("p_sum", PT), ("p_scale", PT),
                ("skip", PT), ("q_scale", PT), ("q_zero", PT), ("y_codes", ctypes.c_int)]


class QConvBlock(Ops):
    """A QDQ residual block on int8 MFMA (``qconv_block_forward``): y =
    [Q](Relu?(Conv(DQ(x), DQ(w)) + b) [+ Conv1x1(DQ(x), DQ(p))] [+ skip]), the
    sequence QuantizeLinear -> DequantizeLinear -> Conv -> Relu -> Add (and the
    next block's QuantizeLinear) of nn/Operators.py:427-548, :32-79, :170-219
    with the convolution's integer sum taken exactly: the tolerance class of
    the MFMA convolution, not the sequence's bits.

    ``inputs`` = [x codes (channels-last, from QuantizeNHWC or another block),
    x scale, x zero point or "", packed weight codes [M, KH, KW, C], their
    per-tap sums [M, KH, KW], weight scales [M], bias or "", projection codes
    [M, 1, 1, C] or "", their sums, their scales, skip (f32 NCHW) or "",
    output scale or "", output zero point or ""]; with an output scale the
    block writes the next block's channels-last codes of ``y_codes``, else f32
    NCHW."""

    def __init__(self, inputs, outputs, pads, strides, dilations, relu, x_codes, y_codes=None, version="17"):
        super().__init__(inputs, outputs)
        self.pads, self.strides, self.dilations = pads, strides, dilations
        self.relu = 1 if relu else 0
        self.x_codes, self.y_codes = x_codes, y_codes
        self.version = version
        self.lib.qconv_block_forward.argtypes = [PT, ctypes.POINTER(CQConvBlock), PT, ctypes.POINTER(CConvParams)]
        self.lib.qconv_block_forward.restype = None

    def _shape(self, x, w):
        N, H, W, _ = x.size
        M, KH, KW, _ = w.size
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        return ((N, OH, OW, M), "int8") if self.y_codes else ((N, M, OH, OW), "float32")

    def forward(self, x, x_scale, x_zero, w, w_sum, w_scale, bias=None, p=None, p_sum=None, p_scale=None,
                skip=None, q_scale=None, q_zero=None):
        keep = [_int_arr(self.pads), _int_arr(self.strides), _int_arr(self.dilations)]
        prm = CConvParams()
        prm.pads, prm.strides, prm.dilations = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        prm.group = 1
        blk = CQConvBlock()

        def arrange(ins, out):
            (blk.x_scale, blk.x_zero, blk.w, blk.w_sum, blk.w_scale, blk.bias, blk.p, blk.p_sum, blk.p_scale,
             blk.skip, blk.q_scale, blk.q_zero) = ins[1:]
            blk.x_codes = DTYPE_MAP[self.x_codes]
            blk.relu = self.relu
            blk.y_codes = DTYPE_MAP[self.y_codes] if self.y_codes else 0
            return (ins[0], ctypes.byref(blk), out, ctypes.byref(prm))
        shape, dt = self._shape(x, w)
        t = self._run("qconv_block_forward", [x, x_scale, x_zero, w, w_sum, w_scale, bias, p, p_sum, p_scale, skip,
                                              q_scale, q_zero], shape, dt, arrange=arrange)
        del keep
        return _values(self, t)

    def forward_(self, x, x_scale=None, x_zero=None, w=None, *rest):
        shape, dt = self._shape(x, w)
        return _values(self, Tensor_(*shape, dtype=dt))


class MaxPool(Ops):
    """2-D max pooling (nn/Operators.py:550-611 -> tensor_ops.c:1116-1165)."""

    def __init__(self, inputs, outputs, kernel_shape, pads, strides, dtype, dilations=[1, 1], version="17"):
        super().__init__(inputs, outputs)
        self.kernel_shape, self.pads, self.strides, self.dilations = kernel_shape, pads, strides, dilations
        self.dtype = dtype
        self.version = version
        self.lib.max_pool_forward.argtypes = [PT, PT, ctypes.POINTER(CPoolParams)]
        self.lib.max_pool_forward.restype = None

    def forward(self, x: Tensor):
        N, C, H, W = x.size
        KH, KW = self.kernel_shape
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        keep = [_int_arr(self.pads), _int_arr(self.strides), _int_arr(self.dilations), _int_arr(self.kernel_shape)]
        p = CPoolParams()
        p.pads, p.strides, p.dilations, p.kernel_shape = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
        t = self._run("max_pool_forward", [x], (N, C, OH, OW), self.dtype, ctypes.byref(p))
        return _values(self, t)

    def forward_(self, x: Tensor_):
        N, C, H, W = x.size
        KH, KW = self.kernel_shape
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        return _values(self, Tensor_(N, C, OH, OW, dtype=self.dtype))


class MaxPoolQDQ(MaxPool):
    """MaxPool with a second output in one call to ``max_pool_qdq_forward``:
    outputs [y, yq] with y = MaxPool(x) and yq = DequantizeLinear(QuantizeLinear(y,
    q_scale, q_zero_point), d_scale, d_zero_point); equal to the MaxPool ->
    QuantizeLinear -> DequantizeLinear operators (nn/Operators.py:550-611,
    :427-473) bit for bit, y read once.  ``inputs`` = [x, q_scale, q_zero_point,
    d_scale, d_zero_point]; codes of dtype ``code_dtype``."""

    def __init__(self, inputs, outputs, kernel_shape, pads, strides, dtype, code_dtype, dilations=[1, 1],
                 version="17"):
        super().__init__(inputs, outputs, kernel_shape, pads, strides, dtype, dilations, version)
        self.code_dtype = code_dtype
        self.lib.max_pool_qdq_forward.argtypes = [PT, PT, ctypes.POINTER(CPoolParams), PT, PT, PT, PT, ctypes.c_int,
                                                  PT]
        self.lib.max_pool_qdq_forward.restype = None

    def forward(self, x: Tensor, q_scale: Tensor, q_zero_point: Tensor, d_scale: Tensor, d_zero_point: Tensor):
        N, C, H, W = x.size
        KH, KW = self.kernel_shape
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        arrs = [_int_arr(self.pads), _int_arr(self.strides), _int_arr(self.dilations), _int_arr(self.kernel_shape)]
        p = CPoolParams()
        p.pads, p.strides, p.dilations, p.kernel_shape = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in arrs]
        keep: list = []
        dev = any(isinstance(t.data, DeviceArray) for t in (x, q_scale, q_zero_point, d_scale, d_zero_point))
        outs = []
        try:
            cins = [self._in_ctensor(t, keep) for t in (x, q_scale, q_zero_point, d_scale, d_zero_point)]
            for _ in range(2):
                outs.append(((N, C, OH, OW), self.dtype) + self._out_ctensor((N, C, OH, OW), self.dtype, dev))
            self._call("max_pool_qdq_forward", cins[0], outs[0][3], ctypes.byref(p), *cins[1:],
                       ctypes.c_int(DTYPE_MAP[self.code_dtype]), outs[1][3])
        except Exception:
            for shape, dt, d, c in outs:
                if d is None:
                    self.lib.free_tensor(c)
            for c in keep:
                self.lib.free_tensor(c)
            raise
        tensors = [self._finish(shape, dt, d, c, []) for shape, dt, d, c in outs]
        for c in keep:
            self.lib.free_tensor(c)
        return _values(self, tensors)

    def forward_(self, x: Tensor_, *params):
        y = super().forward_(x)["tensor"]
        return _values(self, [y, Tensor_(*y.size, dtype=self.dtype)])


class MaxPoolQuantizeNHWC(MaxPool):
    """MaxPool whose output is also quantized into the channels-last int8 codes
    :class:`QConvBlock` reads, in one call to ``max_pool_quantize_nhwc_forward``:
    outputs [y, codes] with y = MaxPool(x) (nn/Operators.py:550-611) and codes =
    :class:`QuantizeNHWC` of y, both bit for bit, x read once.  ``inputs`` = [x,
    scale, zero point or ""] (one-element parameters of the codes' dtype)."""

    def __init__(self, inputs, outputs, kernel_shape, pads, strides, dtype, code_dtype, dilations=[1, 1],
                 version="17"):
        super().__init__(inputs, outputs, kernel_shape, pads, strides, dtype, dilations, version)
        self.code_dtype = code_dtype
        self.lib.max_pool_quantize_nhwc_forward.argtypes = [PT, PT, ctypes.POINTER(CPoolParams), PT, PT,
                                                            ctypes.c_int, PT]
        self.lib.max_pool_quantize_nhwc_forward.restype = None

    def forward(self, x: Tensor, scale: Tensor, zero_point: Tensor = None):
        N, C, H, W = x.size
        KH, KW = self.kernel_shape
        OH, OW = _pool_out(H, W, self.pads, self.strides, self.dilations, KH, KW)
        arrs = [_int_arr(self.pads), _int_arr(self.strides), _int_arr(self.dilations), _int_arr(self.kernel_shape)]
        p = CPoolParams()
        p.pads, p.strides, p.dilations, p.kernel_shape = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in arrs]
        keep: list = []
        dev = any(isinstance(t.data, DeviceArray) for t in (x, scale, zero_point) if t is not None)
        outs = []
        try:
            cins = [self._in_ctensor(t, keep) if t is not None else PT() for t in (x, scale, zero_point)]
            for shape, dt in (((N, C, OH, OW), self.dtype), ((N, OH, OW, C), "int8")):
                outs.append((shape, dt) + self._out_ctensor(shape, dt, dev))
            self._call("max_pool_quantize_nhwc_forward", cins[0], outs[0][3], ctypes.byref(p), cins[1], cins[2],
                       ctypes.c_int(DTYPE_MAP[self.code_dtype]), outs[1][3])
        except Exception:
            for shape, dt, d, c in outs:
                if d is None:
                    self.lib.free_tensor(c)
            for c in keep:
                self.lib.free_tensor(c)
            raise
        tensors = [self._finish(shape, dt, d, c, []) for shape, dt, d, c in outs]
        for c in keep:
            self.lib.free_tensor(c)
        return _values(self, tensors)

    def forward_(self, x: Tensor_, *params):
        y = super().forward_(x)["tensor"]
        N, C, OH, OW = y.size
        return _values(self, [y, Tensor_(N, OH, OW, C, dtype="int8")])


class Gemm(Ops):
    """Y = alpha * A' B' + beta * C (nn/Operators.py:613-669 -> tensor_ops.c:1167-1228)."""

    def __init__(self, inputs, outputs, alpha, beta, transA, transB, dtype, version="17"):
        super().__init__(inputs, outputs)
        self.alpha, self.beta, self.transA, self.transB = alpha, beta, transA, transB
        self.dtype = dtype
        self.lib.gemm_forward.argtypes = [PT, PT, PT, PT, ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int]
        self.lib.gemm_forward.restype = None

    def forward(self, A: Tensor, B: Tensor, C: Tensor = None):
        M = A.size[0] if self.transA == 0 else A.size[1]
        N = B.size[1] if self.transB == 0 else B.size[0]
        if C is not None and not isinstance(C.data, DeviceArray) and np.asarray(C.data).ndim == 1:
            # nn/Operators.py:638-645 (the library reads a 1-D C the same way)
            c = np.asarray(C.data)
            if c.shape[0] == N:
                c = c.reshape(1, -1)
            elif c.shape[0] == M:
                c = c.reshape(-1, 1)
            C = Tensor(*c.shape, dtype=C.dtype, data=np.ascontiguousarray(c))
        t = self._run("gemm_forward", [A, B, C], (M, N), self.dtype, ctypes.c_float(self.alpha),
                      ctypes.c_float(self.beta), ctypes.c_int(self.transA), ctypes.c_int(self.transB))
        return _values(self, t)

    def forward_(self, A: Tensor_, B: Tensor_, C: Tensor_ = None):
        M = A.size[0] if self.transA == 0 else A.size[1]
        N = B.size[1] if self.transB == 0 else B.size[0]
        return _values(self, Tensor_(M, N, dtype=self.dtype))


class GemmSoftmax(Gemm):
    """Gemm followed by Softmax over the last axis of its output in one call to
    ``gemm_softmax_forward``: outputs [y, p] with y = Gemm(A, B, C) and p =
    Softmax(y) (nn/Operators.py:613-669, :671-704), both bit for bit; on device
    tensors the Gemm's k-split reduction also takes the softmax."""

    def __init__(self, inputs, outputs, alpha, beta, transA, transB, dtype, version="17"):
        super().__init__(inputs, outputs, alpha, beta, transA, transB, dtype, version)
        self.lib.gemm_softmax_forward.argtypes = [PT] * 5 + [ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                                             ctypes.c_int]
        self.lib.gemm_softmax_forward.restype = None

    def forward(self, A: Tensor, B: Tensor, C: Tensor = None):
        M = A.size[0] if self.transA == 0 else A.size[1]
        N = B.size[1] if self.transB == 0 else B.size[0]
        if C is not None and not isinstance(C.data, DeviceArray) and np.asarray(C.data).ndim == 1:
            c = np.asarray(C.data)
            if c.shape[0] == N:
                c = c.reshape(1, -1)
            elif c.shape[0] == M:
                c = c.reshape(-1, 1)
            C = Tensor(*c.shape, dtype=C.dtype, data=np.ascontiguousarray(c))
        keep: list = []
        dev = any(isinstance(t.data, DeviceArray) for t in (A, B, C) if t is not None)
        outs = []
        try:
            cins = [self._in_ctensor(t, keep) if t is not None else PT() for t in (A, B, C)]
            for _ in range(2):
                outs.append(((M, N), self.dtype) + self._out_ctensor((M, N), self.dtype, dev))
            self._call("gemm_softmax_forward", cins[0], cins[1], cins[2], outs[0][3], outs[1][3],
                       ctypes.c_float(self.alpha), ctypes.c_float(self.beta), ctypes.c_int(self.transA),
                       ctypes.c_int(self.transB))
        except Exception:
            for shape, dt, d, c in outs:
                if d is None:
                    self.lib.free_tensor(c)
            for c in keep:
                self.lib.free_tensor(c)
            raise
        tensors = [self._finish(shape, dt, d, c, []) for shape, dt, d, c in outs]
        for c in keep:
            self.lib.free_tensor(c)
        return _values(self, tensors)

    def forward_(self, A: Tensor_, B: Tensor_, C: Tensor_ = None):
        y = super().forward_(A, B, C)["tensor"]
        return _values(self, [y, Tensor_(*y.size, dtype=self.dtype)])


class QuantizeDequantize(Ops):
    """DequantizeLinear(QuantizeLinear(x, q_scale, q_zero_point), d_scale,
    d_zero_point) in one call to ``quantize_dequantize_linear_forward``: the
    codes (dtype ``code_dtype``) stay in registers and are never written.
    Output equals the QuantizeLinear -> DequantizeLinear pair
    (nn/Operators.py:427-473) bit for bit.  ``inputs`` = [x, q_scale,
    q_zero_point, d_scale, d_zero_point]."""

    def __init__(self, inputs, outputs, code_dtype, dtype="float32", version="17"):
        super().__init__(inputs, outputs)
        self.code_dtype = code_dtype
        self.dtype = dtype
        self.version = version
        self.lib.quantize_dequantize_linear_forward.argtypes = [PT] * 6 + [ctypes.c_int]
        self.lib.quantize_dequantize_linear_forward.restype = None

    def forward(self, x: Tensor, q_scale: Tensor, q_zero_point: Tensor, d_scale: Tensor, d_zero_point: Tensor):
        code = ctypes.c_int(DTYPE_MAP[self.code_dtype])
        t = self._run("quantize_dequantize_linear_forward", [x, q_scale, q_zero_point, d_scale, d_zero_point],
                      tuple(x.size), self.dtype, code)
        return _values(self, t)

    def forward_(self, x: Tensor_, *params):
        return _values(self, Tensor_(*x.size, dtype=self.dtype))


class DequantizeGemm(Ops):
    """Gemm(A, DequantizeLinear(Bq, scale, zero_point), C) in one call to
    ``dequantize_gemm_forward``: the weight-only-quantized Gemm reads the int8 /
    uint8 codes and never writes the f32 weight.  Output equals the
    DequantizeLinear -> Gemm pair (nn/Operators.py:452-473 then :613-669) bit
    for bit.  ``inputs`` = [A, Bq, scale, zero_point or "", C (optional)];
    ``axis`` is the dequantisation axis of Bq (a 1-element scale is per-tensor)."""

    def __init__(self, inputs, outputs, alpha, beta, transA, transB, axis, dtype, version="17"):
        super().__init__(inputs, outputs)
        self.alpha, self.beta, self.transA, self.transB, self.axis = alpha, beta, transA, transB, axis
        self.dtype = dtype
        self.version = version
        self.lib.dequantize_gemm_forward.argtypes = [PT, PT, PT, PT, ctypes.c_int, PT, PT, ctypes.c_float,
                                                     ctypes.c_float, ctypes.c_int, ctypes.c_int]
        self.lib.dequantize_gemm_forward.restype = None

    def _mn(self, A, B):
        M = A.size[0] if self.transA == 0 else A.size[1]
        N = B.size[1] if self.transB == 0 else B.size[0]
        return M, N

    def forward(self, A: Tensor, Bq: Tensor, scale: Tensor, zero_point: Tensor = None, C: Tensor = None):
        M, N = self._mn(A, Bq)
        args = (ctypes.c_int(self.axis), ctypes.c_float(self.alpha), ctypes.c_float(self.beta),
                ctypes.c_int(self.transA), ctypes.c_int(self.transB))

        def arrange(ins, out):
            a, b, sc, zp, c = ins
            return (a, b, sc, zp, args[0], c, out) + args[1:]
        t = self._run("dequantize_gemm_forward", [A, Bq, scale, zero_point, C], (M, N), self.dtype,
                      arrange=arrange)
        return _values(self, t)

    def forward_(self, A: Tensor_, Bq: Tensor_, scale: Tensor_ = None, zero_point: Tensor_ = None,
                 C: Tensor_ = None):
        return _values(self, Tensor_(*self._mn(A, Bq), dtype=self.dtype))


class Softmax(Ops):
    """Softmax along one axis (nn/Operators.py:671-704 -> tensor_ops.c:1231-1270)."""

    def __init__(self, inputs, outputs, axis, dtype, version="17"):
        super().__init__(inputs, outputs)
        self.axis = axis
        self.dtype = dtype
        self.lib.softmax_forward.argtypes = [PT, PT, ctypes.c_int]
        self.lib.softmax_forward.restype = None

    def forward(self, input: Tensor):
        t = self._run("softmax_forward", [input], tuple(input.size), self.dtype, ctypes.c_int(self.axis))
        return _values(self, t)

    def forward_(self, input: Tensor_):
        return _values(self, Tensor_(*input.size, dtype=self.dtype))


class Flatten(Ops):
    """Collapse to 2-D around ``axis`` (nn/Operators.py:776-825 -> tensor_ops.c:1289-1294)."""

    def __init__(self, inputs, outputs, axis=1, dtype="float32", version="17"):
        super().__init__(inputs, outputs)
        self.axis = axis
        self.dtype = dtype
        self.version = version

    def _calc_shape(self, input_shape):
        axis = self.axis if self.axis >= 0 else len(input_shape) + self.axis
        d0 = int(np.prod(input_shape[:axis], dtype=np.int64)) if axis > 0 else 1
        d1 = int(np.prod(input_shape[axis:], dtype=np.int64))
        return (d0, d1)

    def forward(self, input: Tensor):
        return _values(self, self._run("flatten_forward", [input], self._calc_shape(input.size), self.dtype))

    def forward_(self, input: Tensor_):
        return _values(self, Tensor_(*self._calc_shape(input.size), dtype=self.dtype))


class Reshape(Ops):
    """Reshape to the shape held by the second input, -1 inferred
    (nn/Operators.py:827-871 -> tensor_ops.c:1297-1299)."""

    def __init__(self, inputs, outputs, dtype="float32", version="17"):
        super().__init__(inputs, outputs)
        self.dtype = dtype
        self.version = version

    @staticmethod
    def _target(data_size, shape):
        target = np.asarray(shape.numpy() if isinstance(shape, Tensor) else shape).astype(np.int64).reshape(-1).tolist()
        known = 1
        infer = -1
        for i, v in enumerate(target):
            if v == -1:
                infer = i
            else:
                known *= v
        if infer != -1:
            target[infer] = data_size // known
        return tuple(int(v) for v in target)

    def forward(self, data: Tensor, shape: Tensor):
        final = self._target(data.data_size, shape)
        return _values(self, self._run("reshape_forward", [data], final, self.dtype))

    def forward_(self, data: Tensor_, shape):
        return _values(self, Tensor_(*self._target(data.data_size, shape), dtype=self.dtype))


class GlobalAveragePool(Ops):
    """Mean over the two trailing (spatial) dims: NCHW -> NC11
    (nn/Operators.py:2997-3021 -> tensor_ops.c:2844-2868)."""

    def __init__(self, inputs, outputs, dtype="float32", version="17", flatten=False):
        super().__init__(inputs, outputs)
        self.dtype = dtype
        self.version = version
        # flatten: write the [N, C] result of a following Flatten(axis=1) directly (the
        # same values in the same order; global_average_pool_forward takes any output
        # of N*C elements)
        self.flatten = flatten

    def _out_shape(self, size):
        return (int(size[0]), int(np.prod(size[1:-2], dtype=np.int64))) if self.flatten else tuple(size[:-2]) + (1, 1)

    def forward(self, x: Tensor):
        return _values(self, self._run("global_average_pool_forward", [x], self._out_shape(x.size), self.dtype))

    def forward_(self, x: Tensor_):
        return _values(self, Tensor_(*self._out_shape(x.size), dtype=self.dtype))


class DynamicQuantizeLinear(Ops):
    """uint8 quantization with scale / zero point computed from the data
    (nn/Operators.py:3891-3927 -> tensor_ops.c:3760-3809).  ``forward`` returns
    ``{"tensor": [y, y_scale, y_zero_point], "parameters": None}``."""

    def __init__(self, inputs, outputs, dtype="uint8", version="17"):
        super().__init__(inputs, outputs)
        self.dtype = "uint8"
        self.version = version

    def forward(self, x: Tensor):
        keep: list = []
        dev = isinstance(x.data, DeviceArray)
        outs = []
        try:
            cx = self._in_ctensor(x, keep)
            for shape, dt in ((tuple(x.size), "uint8"), ((1,), "float32"), ((1,), "uint8")):
                outs.append((shape, dt) + self._out_ctensor(shape, dt, dev))
            self._call("dynamic_quantize_linear_forward", cx, *[o[3] for o in outs])
        except Exception:
            for shape, dt, d, c in outs:
                if d is None:
                    self.lib.free_tensor(c)
            for c in keep:
                self.lib.free_tensor(c)
            raise
        tensors = [self._finish(shape, dt, d, c, []) for shape, dt, d, c in outs]
        for c in keep:
            self.lib.free_tensor(c)
        values = {"tensor": tensors, "parameters": None}
        self.parameters = {"values": values}
        return values

    def forward_(self, x: Tensor_):
        return {"tensor": [Tensor_(*x.size, dtype="uint8"), Tensor_(1, dtype="float32"), Tensor_(1, dtype="uint8")],
                "parameters": None}


class CChainStep(ctypes.Structure):
    """``TensorOpsChainStep`` of include/tensor_ops.h."""
    _fields_ = [("op", ctypes.c_int), ("operand", ctypes.c_int), ("reversed", ctypes.c_int)]


CHAIN_OPS = {"Add": 0, "Sub": 1, "Mul": 2, "Div": 3, "Relu": 4, "Abs": 5, "Cos": 6}


class ElementwiseChain(Ops):
    """A run of elementwise operators on one float32 tensor in a single pass
    (extension; replaces consecutive ADD / SUB / MUL / DIV / RELU / ABS / COS
    calls).  ``steps`` is a list of ``(op, operand_index, reversed)`` with op in
    Add, Sub, Mul, Div, Relu, Abs, Cos; binary steps compute ``v op operand``
    (``operand op v`` when reversed).  Each step rounds to float32 as the
    standalone operator does, so the result equals the op-by-op chain bit for bit."""

    def __init__(self, inputs, outputs, steps, dtype="float32", version="17"):
        super().__init__(inputs, outputs)
        self.steps = [(op, None if arg is None else int(arg), bool(rev)) for op, arg, rev in steps]
        self.dtype = dtype
        self.version = version
        self.lib.elementwise_chain_forward.argtypes = [PT, ctypes.POINTER(PT), ctypes.c_int,
                                                       ctypes.POINTER(CChainStep), ctypes.c_int, PT]
        self.lib.elementwise_chain_forward.restype = None

    def forward(self, x: Tensor, *operands: Tensor):
        keep: list = []
        dev = isinstance(x.data, DeviceArray) or any(isinstance(o.data, DeviceArray) for o in operands)
        try:
            cx = self._in_ctensor(x, keep)
            cops = (PT * max(1, len(operands)))(*[self._in_ctensor(o, keep) for o in operands])
            csteps = (CChainStep * max(1, len(self.steps)))(
                *[CChainStep(CHAIN_OPS[op], -1 if arg is None else arg, int(rev)) for op, arg, rev in self.steps])
            dev_out, c_out = self._out_ctensor(tuple(x.size), self.dtype, dev)
        except Exception:
            for c in keep:
                self.lib.free_tensor(c)
            raise
        try:
            self._call("elementwise_chain_forward", cx, cops, len(operands), csteps, len(self.steps), c_out)
        except Exception:
            if dev_out is None:
                self.lib.free_tensor(c_out)
            for c in keep:
                self.lib.free_tensor(c)
            raise
        return _values(self, self._finish(tuple(x.size), self.dtype, dev_out, c_out, keep))

    def forward_(self, x: Tensor_, *operands):
        return _values(self, Tensor_(*x.size, dtype=self.dtype))
