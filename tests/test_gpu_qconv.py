"""QDQ convolution blocks on int8 MFMA (csrc/qconv.hip) against the operator
sequence they replace: QuantizeLinear -> DequantizeLinear of the activation,
DequantizeLinear of the int8 per-channel weights, Conv (+ bias) -> Relu -> Add
of a skip tensor or of a 1x1 projection Conv of the same activation, and the
next block's QuantizeLinear (reference: tensor_ops.c:999-1034 for Q / DQ,
:1036-1114 for Conv, nn/Operators.py for the graph's node order).

* The channels-last quantize is QuantizeLinear bit for bit (codes compared with
  the oracle's after the layout change).
* The block's f32 output is within the convolution tolerance (rtol 1e-5 plus
  1e-5 of the output rms) of the oracle's sequence on small shapes, and of the
  library's exact-mode (fp64) sequence on every element at the config-5 block
  shapes; its code output equals QuantizeLinear of its own f32 output bit for
  bit (the epilogue value is the same in both launches).
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


class QConvBlock(ctypes.Structure):
    _fields_ = [("x_scale", O.PT), ("x_zero", O.PT), ("x_codes", ctypes.c_int), ("w", O.PT), ("w_sum", O.PT),
                ("w_scale", O.PT), ("bias", O.PT), ("relu", ctypes.c_int), ("p", O.PT), ("p_sum", O.PT),
                ("p_scale", O.PT), ("skip", O.PT), ("q_scale", O.PT), ("q_zero", O.PT), ("y_codes", ctypes.c_int)]


def _bind(lib):
    lib.quantize_linear_nhwc_forward.argtypes = [O.PT, O.PT, O.PT, ctypes.c_int, O.PT]
    lib.qconv_pack_weights.argtypes = [O.PT, O.PT, O.PT]
    lib.qconv_block_forward.argtypes = [O.PT, ctypes.POINTER(QConvBlock), O.PT, ctypes.POINTER(O.CConvParams)]
    lib.create_tensor_device_empty.restype = O.PT
    lib.create_tensor_device_empty.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]


def _params(pads, strides):
    keep = [(ctypes.c_int * 4)(*pads), (ctypes.c_int * 2)(*strides), (ctypes.c_int * 2)(1, 1)]
    p = O.CConvParams()
    p.pads, p.strides, p.dilations = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
    p.group = 1
    return p, keep


def _stored(codes, dt):
    """Codes [N, C, H, W] -> the kernels' channels-last int8 (code - 128 for uint8)."""
    c = np.asarray(codes)
    s = (c.astype(np.int16) - 128).astype(np.int8) if dt == O.U8 else c.astype(np.int8)
    return np.ascontiguousarray(s.transpose(0, 2, 3, 1))


def _codes_from_stored(s, dt):
    """Channels-last stored bytes [N, H, W, C] -> codes [N, C, H, W]."""
    s = np.asarray(s).transpose(0, 3, 1, 2)
    return (s.astype(np.int16) + 128).astype(np.uint8) if dt == O.U8 else s.astype(np.int8)


def _weights(rng, m, c, kh, kw):
    w = rng.normal(0, np.sqrt(2.0 / (c * kh * kw)), (m, c, kh, kw))
    s = (np.abs(w).reshape(m, -1).max(axis=1) / 127).astype(np.float32)
    q = np.clip(np.rint(w / s[:, None, None, None]), -127, 127).astype(np.int8)
    return q, s


class _Dev:
    """Device tensors freed together."""

    def __init__(self, hip):
        self.hip, self.ts = hip, []

    def put(self, arr, dt):
        t = self.hip.dev_from(arr, dt)
        self.ts.append(t)
        return t

    def empty(self, shape, dt):
        t = self.hip.dev_empty(shape, dt)
        self.ts.append(t)
        return t

    def output(self, shape, dt):
        """Undefined contents (filled with the poison byte under hip.poisoned())."""
        shape = tuple(shape)
        t = self.hip.lib.create_tensor_device_empty((ctypes.c_int * len(shape))(*shape), len(shape), dt)
        assert t, self.hip.last_error()
        self.ts.append(t)
        return t

    def free(self):
        for t in self.ts:
            self.hip.lib.free_tensor(t)
        self.ts = []


def _pack(hip, dev, wq):
    m, c, kh, kw = wq.shape
    t = dev.put(wq, O.I8)
    wk, ws = dev.empty((m, kh, kw, c), O.I8), dev.empty((m, kh * kw), O.I32)
    hip.lib.tensor_ops_hip_clear_error()
    hip.lib.qconv_pack_weights(t, wk, ws)
    assert not hip.last_error(), hip.last_error()
    return wk, ws


def _run_block(hip, dev, xs, xdt, sx, zx, wq, sw, bias, relu, pq, sp, skip, pads, strides, qs=None, qz=None,
               ydt=O.U8):
    """qconv_block_forward on device copies; returns the f32 output or, with qs,
    the stored channels-last codes."""
    L = hip.lib
    N, H, W, C = xs.shape
    M, _, KH, KW = wq.shape
    OH = (H + pads[0] + pads[2] - KH) // strides[0] + 1
    OW = (W + pads[1] + pads[3] - KW) // strides[1] + 1
    b = QConvBlock()
    b.x_scale = dev.put(np.array([sx], np.float32), O.F32)
    b.x_zero = dev.put(np.array([zx]), xdt)
    b.x_codes = xdt
    b.w, b.w_sum = _pack(hip, dev, wq)
    b.w_scale = dev.put(sw, O.F32)
    b.bias = dev.put(bias, O.F32) if bias is not None else O.PT()
    b.relu = 1 if relu else 0
    if pq is not None:
        b.p, b.p_sum = _pack(hip, dev, pq)
        b.p_scale = dev.put(sp, O.F32)
    b.skip = dev.put(skip, O.F32) if skip is not None else O.PT()
    if qs is not None:
        b.q_scale = dev.put(np.array([qs], np.float32), O.F32)
        b.q_zero = dev.put(np.array([qz]), ydt)
        b.y_codes = ydt
    x = dev.put(xs, O.I8)
    p, keep = _params(pads, strides)
    with hip.poisoned():
        y = dev.output((N, OH, OW, M), O.I8) if qs is not None else dev.output((N, M, OH, OW), O.F32)
        L.tensor_ops_hip_clear_error()
        L.qconv_block_forward(x, ctypes.byref(b), y, ctypes.byref(p))
    assert not hip.last_error(), hip.last_error()
    del keep
    return hip.dev_read(y, O.I8 if qs is not None else O.F32)


def _oracle_block(ol, xq, xdt, sx, zx, wq, sw, bias, relu, pq, sp, skip, pads, strides):
    """The operator sequence through the compiled restatement of the reference."""
    xd = ol.qdq("dequantize", xq, xdt, np.float32(sx), O.F32, np.array(zx), xdt, O.F32)
    wd = ol.qdq("dequantize", wq, O.I8, sw[:, None, None, None], O.F32, np.zeros(1, np.int8), O.I8, O.F32)
    y = ol.conv(xd, O.F32, wd, O.F32, bias, O.F32 if bias is not None else O.F32, O.F32, pads, strides, (1, 1), 1)
    if relu:
        y = ol.unary("relu", y, O.F32, O.F32)
    if pq is not None:
        pd = ol.qdq("dequantize", pq, O.I8, sp[:, None, None, None], O.F32, np.zeros(1, np.int8), O.I8, O.F32)
        pr = ol.conv(xd, O.F32, pd, O.F32, None, O.F32, O.F32, (0, 0, 0, 0), strides, (1, 1), 1)
        y = ol.binary("add", y, O.F32, pr, O.F32, O.F32)
    if skip is not None:
        y = ol.binary("add", y, O.F32, skip, O.F32, O.F32)
    return y


def test_quantize_nhwc_matches_quantize_linear(hip, oracle_lib):
    _bind(hip.lib)
    rng = np.random.default_rng(11)
    dev = _Dev(hip)
    try:
        for shape, dt, s, z in (((2, 64, 9, 13), O.U8, 8 / 255, 0), ((1, 96, 8, 8), O.U8, 0.05, 37),
                                ((3, 32, 5, 7), O.I8, 0.04, -3), ((1, 64, 64, 3), O.U8, 0.02, 128),
                                ((2, 32, 10, 10), O.U8, 0.03, 5), ((2, 128, 10, 10), O.I8, 0.05, -7)):
            x = rng.normal(0.5, 2.0, shape).astype(np.float32)
            x.flat[::97] = np.float32(s) * (np.rint(x.flat[::97] / s) + 0.5)      # ties
            ref = oracle_lib.qdq("quantize", x, O.F32, np.float32(s), O.F32, np.array(z), dt, dt)
            tx, ts, tz = dev.put(x, O.F32), dev.put(np.array([s], np.float32), O.F32), dev.put(np.array([z]), dt)
            n, c, h, w = shape
            with hip.poisoned():
                ty = dev.output((n, h, w, c), O.I8)
                hip.lib.tensor_ops_hip_clear_error()
                hip.lib.quantize_linear_nhwc_forward(tx, ts, tz, dt, ty)
            assert not hip.last_error(), hip.last_error()
            got = _codes_from_stored(hip.dev_read(ty, O.I8), dt)
            assert_bitexact(got, ref, dt, what=f"quantize_linear_nhwc {shape} {dt}")
            dev.free()
    finally:
        dev.free()


def _pool_params(pads, strides):
    keep = [(ctypes.c_int * 4)(*pads), (ctypes.c_int * 2)(*strides), (ctypes.c_int * 2)(1, 1),
            (ctypes.c_int * 2)(3, 3)]
    p = O.CPoolParams()
    p.pads, p.strides, p.dilations, p.kernel_shape = [ctypes.cast(k, ctypes.POINTER(ctypes.c_int)) for k in keep]
    return p, keep


# (shape, pads, code dtype, scale, zero point): the config-5 pool (strips of 4 output
# rows, 16 channels per block), a partial last strip with an int8 zero point, an odd
# input height with W % 4 == 2, 128 and 32 channels, and a shape the fused kernel does
# not take (W != 2 OW): max_pool_forward then quantize_linear_nhwc_forward.
MAXPOOL_Q = [((2, 64, 112, 112), (1, 1, 1, 1), O.U8, 8 / 255, 0),
             ((3, 64, 20, 22), (1, 1, 1, 1), O.I8, 0.05, -3),
             ((2, 128, 15, 18), (1, 1, 1, 1), O.U8, 0.03, 17),
             ((1, 32, 16, 16), (1, 1, 1, 1), O.U8, 0.02, 0),
             ((2, 64, 16, 17), (1, 1, 0, 0), O.I8, 0.04, 5)]


@pytest.mark.parametrize("case", MAXPOOL_Q, ids=[f"{c[0]}-{c[2]}" for c in MAXPOOL_Q])
def test_maxpool_quantize_nhwc(hip, oracle_lib, case):
    """max_pool_quantize_nhwc_forward = max_pool_forward -> quantize_linear_nhwc_forward
    bit for bit (both outputs against the oracle's MaxPool and QuantizeLinear), with
    NaN, +-inf and rounding ties among the inputs."""
    shape, pads, dt, s, z = case
    L = hip.lib
    _bind(L)
    L.max_pool_quantize_nhwc_forward.argtypes = [O.PT, O.PT, ctypes.POINTER(O.CPoolParams), O.PT, O.PT,
                                                 ctypes.c_int, O.PT]
    rng = np.random.default_rng(shape[1] + shape[2])
    x = rng.normal(0.5, 2.0, shape).astype(np.float32)
    x.flat[::89] = np.float32(s) * (np.rint(x.flat[::89] / s) + 0.5)     # ties after pooling, some of them
    x.flat[5::1013] = np.nan
    x.flat[7::2039] = np.inf
    x.flat[11::3001] = -np.inf
    x[0, 0, :3, :3] = np.nan                                             # a window of NaN only: -inf out
    ref_y = oracle_lib.maxpool(x, O.F32, O.F32, (3, 3), pads, (2, 2))
    ref_c = oracle_lib.qdq("quantize", ref_y, O.F32, np.float32(s), O.F32, np.array(z), dt, dt)
    n, c, oh, ow = ref_y.shape
    dev = _Dev(hip)
    try:
        tx, ts, tz = dev.put(x, O.F32), dev.put(np.array([s], np.float32), O.F32), dev.put(np.array([z]), dt)
        p, keep = _pool_params(pads, (2, 2))
        with hip.poisoned():
            ty, tc = dev.output((n, c, oh, ow), O.F32), dev.output((n, oh, ow, c), O.I8)
            L.tensor_ops_hip_clear_error()
            L.max_pool_quantize_nhwc_forward(tx, ty, ctypes.byref(p), ts, tz, dt, tc)
        assert not hip.last_error(), hip.last_error()
        assert_bitexact(hip.dev_read(ty, O.F32), ref_y, O.F32, what=f"pooled {shape}")
        assert_bitexact(_codes_from_stored(hip.dev_read(tc, O.I8), dt), ref_c, dt, what=f"codes {shape}")
        del keep
    finally:
        dev.free()


def test_pack_weights(hip):
    _bind(hip.lib)
    rng = np.random.default_rng(12)
    dev = _Dev(hip)
    try:
        for shape in ((64, 64, 3, 3), (128, 96, 1, 1), (64, 32, 3, 2)):
            wq = rng.integers(-127, 128, shape).astype(np.int8)
            wk, ws = _pack(hip, dev, wq)
            np.testing.assert_array_equal(hip.dev_read(wk, O.I8), wq.transpose(0, 2, 3, 1))
            taps = wq.transpose(0, 2, 3, 1).reshape(shape[0], shape[2] * shape[3], shape[1])
            np.testing.assert_array_equal(hip.dev_read(ws, O.I32), taps.sum(2, dtype=np.int64))
            dev.free()
    finally:
        dev.free()


# name, N, C, H, W, M, stride, projection, skip, x code dtype, x zero point[, kernel size (3)].
# Grids this small run two k groups per block; the 1x1 cases put the second group's
# stages wholly in the projection, or leave it none.
SMALL = [
    ("s1_skip_u8", 2, 64, 12, 12, 64, 1, False, True, O.U8, 0),
    ("s1_skip_u8_zp", 2, 64, 11, 9, 64, 1, False, True, O.U8, 41),
    ("s2_proj_u8", 2, 64, 13, 13, 128, 2, True, False, O.U8, 0),
    ("s2_proj_i8_zp", 1, 96, 10, 7, 64, 2, True, False, O.I8, -5),
    ("s1_plain_c32", 3, 32, 6, 6, 64, 1, False, False, O.U8, 200),
    ("k1_s2_proj_u8", 2, 64, 9, 9, 64, 2, True, False, O.U8, 0, 1),
    ("k1_skip_c128_i8", 1, 128, 8, 8, 128, 1, False, True, O.I8, 7, 1),
    ("k1_one_stage_c64", 2, 64, 6, 6, 64, 1, False, True, O.U8, 3, 1),
]


@pytest.mark.parametrize("case", SMALL, ids=[c[0] for c in SMALL])
def test_qconv_block_against_sequence(hip, oracle_lib, case):
    _bind(hip.lib)
    name, N, C, H, W, M, stride, proj, has_skip, xdt, zx = case[:11]
    ks = case[11] if len(case) > 11 else 3
    rng = np.random.default_rng(sum(map(ord, name)))
    lo, hi = (0, 256) if xdt == O.U8 else (-128, 128)
    xq = rng.integers(lo, hi, (N, C, H, W)).astype(np.uint8 if xdt == O.U8 else np.int8)
    sx = np.float32(8.0 / 255)
    wq, sw = _weights(rng, M, C, ks, ks)
    pq, sp = _weights(rng, M, C, 1, 1) if proj else (None, None)
    bias = rng.normal(0, 1 / 64, M).astype(np.float32)
    pd = ks // 2
    OH, OW = (H + 2 * pd - ks) // stride + 1, (W + 2 * pd - ks) // stride + 1
    skip = rng.normal(0, 1, (N, M, OH, OW)).astype(np.float32) if has_skip else None
    pads, strides = (pd, pd, pd, pd), (stride, stride)
    ref = _oracle_block(oracle_lib, xq, xdt, sx, zx, wq, sw, bias, True, pq, sp, skip, pads, strides)
    dev = _Dev(hip)
    try:
        xs = _stored(xq, xdt)
        print(f"qconv {name}: f32 output", flush=True)
        y = _run_block(hip, dev, xs, xdt, sx, zx, wq, sw, bias, True, pq, sp, skip, pads, strides)
        assert_close(y, ref, O.F32, what=f"qconv {name}")
        for ydt, qs, qz in ((O.U8, 0.03, 0), (O.I8, 0.02, 3)):
            print(f"qconv {name}: codes {ydt}", flush=True)
            yc = _run_block(hip, dev, xs, xdt, sx, zx, wq, sw, bias, True, pq, sp, skip, pads, strides, qs, qz, ydt)
            want = oracle_lib.qdq("quantize", y, O.F32, np.float32(qs), O.F32, np.array(qz), ydt, ydt)
            assert_bitexact(_codes_from_stored(yc, ydt), want, ydt, what=f"qconv {name} codes")
    finally:
        dev.free()


def test_qconv_refuses_exact_mode(hip):
    _bind(hip.lib)
    rng = np.random.default_rng(13)
    xq = rng.integers(0, 256, (1, 32, 4, 4)).astype(np.uint8)
    wq, sw = _weights(rng, 64, 32, 3, 3)
    dev = _Dev(hip)
    hip.set_exact(True)
    try:
        with pytest.raises(AssertionError, match="no exact mode"):
            _run_block(hip, dev, _stored(xq, O.U8), O.U8, 0.1, 0, wq, sw, None, True, None, None, None,
                       (1, 1, 1, 1), (1, 1))
    finally:
        hip.set_exact(False)
        dev.free()


# config-5 blocks at batch 64: (C, H, M, stride, projection); block 1 adds the
# pooled f32 activation, blocks 2-4 a 1x1 projection of the block input
CONFIG5 = [("block1", 64, 56, 64, 1, False), ("block2", 64, 56, 128, 2, True), ("block3", 128, 28, 256, 2, True),
           ("block4", 256, 14, 512, 2, True)]


def _dq(q, s, z=0):
    """DequantizeLinear as the reference computes it: (q - z) * s in double, rounded once to f32."""
    return ((np.asarray(q, np.float64) - z) * np.asarray(s, np.float64)).astype(np.float32)


@pytest.mark.parametrize("case", CONFIG5, ids=[c[0] for c in CONFIG5])
def test_qconv_block_config5_size(hip, case):
    """Every element of the config-5 block output against the library's exact-mode
    (fp64, the reference's summation) convolution sequence on the same codes."""
    _bind(hip.lib)
    name, C, H, M, stride, proj = case
    N = 64
    rng = np.random.default_rng(500 + C + M)
    sx = np.float32(8.0 / 255)
    xq = np.clip(np.rint(np.abs(rng.normal(0, 1.2, (N, C, H, H))) / sx), 0, 255).astype(np.uint8)
    wq, sw = _weights(rng, M, C, 3, 3)
    pq, sp = _weights(rng, M, C, 1, 1) if proj else (None, None)
    bias = rng.normal(0, 1 / 64, M).astype(np.float32)
    OH = (H - 1) // stride + 1
    skip = None if proj else rng.normal(0, 1, (N, M, OH, OH)).astype(np.float32)
    pads, strides = (1, 1, 1, 1), (stride, stride)
    xd = _dq(xq, sx)
    hip.set_exact(True)
    try:
        print(f"qconv {name}: exact-mode sequence", flush=True)
        ref = hip.conv(xd, O.F32, _dq(wq, sw[:, None, None, None]), O.F32, bias, O.F32, O.F32, pads, strides,
                       (1, 1), 1)
        ref = np.where(ref > 0, ref, np.float32(0))
        if proj:
            pr = hip.conv(xd, O.F32, _dq(pq, sp[:, None, None, None]), O.F32, None, O.F32, O.F32, (0, 0, 0, 0),
                          strides, (1, 1), 1)
            ref = (ref + pr).astype(np.float32)
        else:
            ref = (ref + skip).astype(np.float32)
    finally:
        hip.set_exact(False)
    dev = _Dev(hip)
    try:
        print(f"qconv {name}: int8 block", flush=True)
        y = _run_block(hip, dev, _stored(xq, O.U8), O.U8, sx, 0, wq, sw, bias, True, pq, sp, skip, pads, strides)
        assert_close(y, ref, O.F32, what=f"qconv {name}: every element against the exact sequence")
    finally:
        dev.free()


def test_qconv_blocks_under_graph_capture(hip):
    """The channels-last quantize and two chained blocks (skip + codes out, then
    projection + f32 out) captured into a HIP graph on the library's stream and
    replayed three times with the outputs overwritten before each replay and
    eager library work between replays: every replay equals the eager results
    bit for bit (the calls allocate nothing and record no memset)."""
    import torch
    _bind(hip.lib)
    torch.cuda.init()
    side = torch.cuda.Stream()
    L = hip.lib
    L.tensor_ops_hip_set_stream(ctypes.c_void_p(side.cuda_stream))
    keep = []
    dev = _Dev(hip)

    def wrap(t, dt):
        shape = list(t.shape)
        p = L.tensor_wrap_device(ctypes.c_void_p(t.data_ptr()), (ctypes.c_int * len(shape))(*shape), len(shape), dt)
        assert p
        keep.append(p)
        return p

    try:
        with torch.cuda.stream(side):
            rng = np.random.default_rng(17)
            N, C, H, M2 = 4, 64, 20, 128
            x = torch.from_numpy(np.abs(rng.normal(0, 1.2, (N, C, H, H))).astype(np.float32)).cuda()
            sx = np.float32(8.0 / 255)
            w1, s1 = _weights(rng, C, C, 3, 3)
            w2, s2 = _weights(rng, M2, C, 3, 3)
            p2, sp2 = _weights(rng, M2, C, 1, 1)
            b1 = rng.normal(0, 1 / 64, C).astype(np.float32)
            b2 = rng.normal(0, 1 / 64, M2).astype(np.float32)
            xs_t = torch.empty((N, H, H, C), dtype=torch.int8, device="cuda")
            c1_t = torch.empty((N, H, H, C), dtype=torch.int8, device="cuda")
            OH = (H - 1) // 2 + 1
            y_t = torch.empty((N, M2, OH, OH), dtype=torch.float32, device="cuda")
            tx, txs, tc1, ty = wrap(x, O.F32), wrap(xs_t, O.I8), wrap(c1_t, O.I8), wrap(y_t, O.F32)
            tsx, tzx = dev.put(np.array([sx], np.float32), O.F32), dev.put(np.array([0]), O.U8)
            tsy, tzy = dev.put(np.array([np.float32(0.04)], np.float32), O.F32), dev.put(np.array([0]), O.U8)
            blk1, blk2 = QConvBlock(), QConvBlock()
            blk1.x_scale, blk1.x_zero, blk1.x_codes = tsx, tzx, O.U8
            blk1.w, blk1.w_sum = _pack(hip, dev, w1)
            blk1.w_scale, blk1.bias, blk1.relu = dev.put(s1, O.F32), dev.put(b1, O.F32), 1
            blk1.skip = tx
            blk1.q_scale, blk1.q_zero, blk1.y_codes = tsy, tzy, O.U8
            blk2.x_scale, blk2.x_zero, blk2.x_codes = tsy, tzy, O.U8
            blk2.w, blk2.w_sum = _pack(hip, dev, w2)
            blk2.w_scale, blk2.bias, blk2.relu = dev.put(s2, O.F32), dev.put(b2, O.F32), 1
            blk2.p, blk2.p_sum = _pack(hip, dev, p2)
            blk2.p_scale = dev.put(sp2, O.F32)
            p1, k1 = _params((1, 1, 1, 1), (1, 1))
            pp2, k2 = _params((1, 1, 1, 1), (2, 2))
            torch.cuda.synchronize()

            def step():
                L.quantize_linear_nhwc_forward(tx, tsx, tzx, O.U8, txs)
                L.qconv_block_forward(txs, ctypes.byref(blk1), tc1, ctypes.byref(p1))
                L.qconv_block_forward(tc1, ctypes.byref(blk2), ty, ctypes.byref(pp2))

            L.tensor_ops_hip_clear_error()
            step()
            torch.cuda.synchronize()
            assert not hip.last_error(), hip.last_error()
            outs = {"xs": xs_t, "c1": c1_t, "y": y_t}
            eager = {k: v.cpu().numpy().copy() for k, v in outs.items()}
            assert np.isfinite(eager["y"]).all()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                step()
            assert not hip.last_error(), hip.last_error()
            for r in range(3):
                for v in outs.values():
                    v.view(torch.uint8).fill_(0xA5)
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
                for k, v in outs.items():
                    assert np.array_equal(v.cpu().numpy().view(np.uint8), eager[k].view(np.uint8)), f"replay {r} {k}"
                L.quantize_linear_nhwc_forward(tx, tsy, tzy, O.U8, txs)      # eager work between replays
                torch.cuda.synchronize()
            del k1, k2
    finally:
        for p in keep:
            L.free_tensor(p)
        dev.free()
        L.tensor_ops_hip_set_stream(None)
