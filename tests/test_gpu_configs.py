"""GPU parity at the BASELINE configuration sizes.

Elementwise, Q/DQ, MaxPool: bit-exact against the oracle at full size.
Gemm / Conv: MFMA results within tolerance of a float64 reference on sampled
rows / images (the oracle itself on the images it finishes in seconds), and
bit-exact in exact mode on the same samples.  Softmax: tolerance plus
rows summing to one.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


def config1_inputs():
    rng = np.random.default_rng(0)
    A = rng.uniform(-4, 4, (8, 64, 56, 56)).astype(np.float32)
    B = rng.uniform(-4, 4, (64, 1, 1)).astype(np.float32)
    Bd = (np.sign(B) * np.maximum(np.abs(B), 0.1)).astype(np.float32)
    return A, B, Bd


def test_config1_chain_full_size(hip, oracle_lib):
    A, B, Bd = config1_inputs()
    o, h = oracle_lib, hip
    t_o, t_h = A, A
    for op, b in (("add", B), ("mul", B), ("sub", B), ("div", Bd)):
        t_o = o.binary(op, t_o, O.F32, b, O.F32, O.F32)
        t_h = h.binary(op, t_h, O.F32, b, O.F32, O.F32)
        assert_bitexact(t_h, t_o, O.F32, what=op)
        t_h = t_o
    for op in ("relu", "abs", "cos"):
        t_o2 = o.unary(op, t_o, O.F32, O.F32)
        assert_bitexact(h.unary(op, t_o, O.F32, O.F32), t_o2, O.F32, what=op)
        t_o = t_o2


@pytest.mark.parametrize("wide", [True, False])
def test_config1_int32_promotion(hip, oracle_lib, wide):
    rng = np.random.default_rng(0)
    _, B, _ = config1_inputs()
    lo, hi = (-(2 ** 31), 2 ** 31 - 1) if wide else (-(2 ** 20), 2 ** 20)
    I = rng.integers(lo, hi, (8, 64, 56, 56), dtype=np.int64).astype(np.int32)
    for dt in (O.F64, O.F32):
        assert_bitexact(hip.binary("add", I, O.I32, B, O.F32, dt), oracle_lib.binary("add", I, O.I32, B, O.F32, dt),
                        dt, what=f"int32+f32 -> {dt}")


# The calls bench.py times pass the [64,1,1] operand un-broadcast, so the library
# broadcasts it in-kernel (k_bin_f32_v4 / k_bin_typed over a collapsed stride
# descriptor); the oracle gets it pre-broadcast, as the reference's Python layer
# passes it (nn/__init__.py:210-279, tensor_ops.c:864-997).
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_config1_binary_unbroadcast_full_size(hip, oracle_lib, op):
    A, B, Bd = config1_inputs()
    b = Bd if op == "div" else B
    got = hip.binary_raw(op, A, O.F32, b, O.F32, O.F32)
    assert_bitexact(got, oracle_lib.binary(op, A, O.F32, b, O.F32, O.F32), O.F32, what=f"{op} [64,1,1] in-kernel")


@pytest.mark.parametrize("wide", [True, False], ids=["full_range", "pm2e20"])
@pytest.mark.parametrize("dt", [O.F64, O.F32], ids=["to_f64", "to_f32"])
def test_config1_int32_promotion_unbroadcast(hip, oracle_lib, wide, dt):
    rng = np.random.default_rng(0)
    _, B, _ = config1_inputs()
    lo, hi = (-(2 ** 31), 2 ** 31 - 1) if wide else (-(2 ** 20), 2 ** 20)
    I = rng.integers(lo, hi, (8, 64, 56, 56), dtype=np.int64).astype(np.int32)
    got = hip.binary_raw("add", I, O.I32, B, O.F32, dt)
    assert_bitexact(got, oracle_lib.binary("add", I, O.I32, B, O.F32, dt), dt, what="int32 + f32[64,1,1]")


# int32 x f32 -> f64 / f32 runs four elements per thread when the last
# dimension is a multiple of 4 (k_bin_i32f32_v4), one otherwise (k_bin_typed):
# the int32 operand broadcast, the f32 operand broadcast along the last
# dimension, and a ragged last dimension, over the four operators.
I32_LAYOUTS = {"i32_bcast_channel": ((64, 1, 1), (4, 64, 56, 56)), "f32_last_dim": ((4, 64, 56, 56), (56,)),
               "ragged_last_dim": ((4, 64, 56, 55), (4, 64, 56, 55))}


@pytest.mark.parametrize("layout", list(I32_LAYOUTS))
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("dt", [O.F64, O.F32], ids=["to_f64", "to_f32"])
def test_int32_f32_promotion_layouts(hip, oracle_lib, layout, op, dt):
    rng = np.random.default_rng(5)
    sa, sb = I32_LAYOUTS[layout]
    I = rng.integers(-(2 ** 31), 2 ** 31 - 1, sa, dtype=np.int64).astype(np.int32)
    F = rng.uniform(-4, 4, sb).astype(np.float32)
    if op == "div":
        F = np.where(np.abs(F) < 0.1, np.float32(0.5), F).astype(np.float32)
    got = hip.binary_raw(op, I, O.I32, F, O.F32, dt)
    shape = np.broadcast_shapes(I.shape, F.shape)
    want = oracle_lib.binary(op, np.broadcast_to(I, shape).copy(), O.I32, np.broadcast_to(F, shape).copy(), O.F32, dt)
    assert_bitexact(got, want, dt, what=f"int32 {sa} {op} f32 {sb} -> {dt}")


def config2_input():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1.5, (32, 512, 1024))
    x[rng.random(x.shape) < 0.001] *= 20
    return x.astype(np.float32)


def config2_variants(x):
    mn, mx = float(x.min()), float(x.max())
    s_u8 = np.float32((mx - mn) / 255)
    z_u8 = np.uint8(np.clip(np.round(-mn / float(s_u8)), 0, 255))
    amax = float(np.abs(x).max())
    return [
        ("u8", np.array([s_u8]), np.array([z_u8]), O.U8, None),
        ("i8axis", (np.abs(x).max(axis=(0, 2)) / 127).astype(np.float32), np.zeros(512, np.int8), O.I8, 1),
        ("e4m3", np.array([amax / 448], np.float32), np.zeros(1, np.uint8), O.E4M3, None),
        ("e5m2", np.array([amax / 57344], np.float32), np.zeros(1, np.uint8), O.E5M2, None),
        ("e4m3_stress", np.array([amax / 448 / 16], np.float32), np.zeros(1, np.uint8), O.E4M3, None),
        ("e5m2_stress", np.array([amax / 57344 / 16], np.float32), np.zeros(1, np.uint8), O.E5M2, None),
    ]


@pytest.fixture(scope="module")
def x2():
    return config2_input()


@pytest.mark.parametrize("idx", range(6), ids=["u8", "i8axis", "e4m3", "e5m2", "e4m3_stress", "e5m2_stress"])
def test_config2_qdq_full_size(hip, oracle_lib, x2, idx):
    tag, s, z, ydt, axis = config2_variants(x2)[idx]
    sv, zv = (s.reshape(1, -1, 1), z.reshape(1, -1, 1)) if axis is not None else (s, z)
    y_ref = oracle_lib.qdq("quantize", x2, O.F32, sv, O.F32, zv, ydt, ydt)
    y = hip.qdq("quantize", x2, O.F32, sv, O.F32, zv, ydt, ydt)
    assert_bitexact(y, y_ref, ydt, what=f"Q {tag}")
    xr_ref = oracle_lib.qdq("dequantize", y_ref, ydt, sv, O.F32, zv, ydt, O.F32)
    xr = hip.qdq("dequantize", y_ref, ydt, sv, O.F32, zv, ydt, O.F32)
    assert_bitexact(xr, xr_ref, O.F32, what=f"DQ {tag}")
    if ydt in (O.U8, O.I8):
        # round-trip property: unsaturated codes reproduce x within half a step
        lo, hi = (0, 255) if ydt == O.U8 else (-128, 127)
        ok = (y > lo) & (y < hi)
        step = np.broadcast_to(sv, x2.shape)[ok].astype(np.float64)
        assert np.all(np.abs(xr[ok].astype(np.float64) - x2[ok]) <= step * 0.5 * (1 + 1e-6))


@pytest.mark.parametrize("idx", range(6), ids=["u8", "i8axis", "e4m3", "e5m2", "e4m3_stress", "e5m2_stress"])
def test_config2_qdq_unbroadcast_full_size(hip, oracle_lib, x2, idx):
    """The calls bench.py times: one-element scale / zero point (per-tensor kernels)
    or a [1,512,1] scale and zero point (per-axis kernels), passed as they are;
    the oracle gets them broadcast to x's shape (tensor_ops.c:999-1034)."""
    tag, s, z, ydt, axis = config2_variants(x2)[idx]
    sv, zv = (s.reshape(1, -1, 1), z.reshape(1, -1, 1)) if axis is not None else (s, z)
    y_ref = oracle_lib.qdq("quantize", x2, O.F32, sv, O.F32, zv, ydt, ydt)
    y = hip.qdq1("quantize", x2, O.F32, sv, zv, ydt, ydt)
    assert_bitexact(y, y_ref, ydt, what=f"Q {tag} un-broadcast")
    xr = hip.qdq1("dequantize", y_ref, ydt, sv, zv, ydt, O.F32)
    assert_bitexact(xr, oracle_lib.qdq("dequantize", y_ref, ydt, sv, O.F32, zv, ydt, O.F32), O.F32,
                    what=f"DQ {tag} un-broadcast")
    if axis is not None:
        # the axis entry points with 1-D parameters reach the same kernels
        assert_bitexact(hip.qdq_axis("quantize", x2, O.F32, s, z, ydt, ydt, axis), y_ref, ydt, what="Q axis 1-D")
        assert_bitexact(hip.qdq_axis("dequantize", y_ref, ydt, s, z, ydt, O.F32, axis), xr, O.F32,
                        what="DQ axis 1-D")


def test_config2_per_axis_entry_point(hip, oracle_lib, x2):
    import ctypes
    tag, s, z, ydt, axis = config2_variants(x2)[1]
    y = hip._run(hip.lib.quantize_linear_axis_forward, [(x2, O.F32), (s, O.F32), (z, O.I8)], x2.shape, O.I8,
                 ctypes.c_int(1))
    ref = oracle_lib.qdq("quantize", x2, O.F32, s.reshape(1, -1, 1), O.F32, z.reshape(1, -1, 1), O.I8, O.I8)
    assert_bitexact(y, ref, O.I8, what="axis entry point")


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_config3_gemm_4096(hip, oracle_lib, dt):
    """Config-3 Gemm at full size.  Every element of the MFMA result (output
    poisoned with NaN first, so an unwritten tile fails) is compared with the
    exact-mode result of the same call (fp64 accumulation in the reference's
    order); the exact mode is anchored bit for bit to the oracle on 16 rows,
    and the MFMA result to a float64 product on 48 rows."""
    rng = np.random.default_rng(2)
    K = 4096
    a = rng.normal(0, 1 / np.sqrt(K), (4096, K)).astype(np.float32)
    b = rng.normal(0, 1 / np.sqrt(K), (4096, K)).astype(np.float32)
    c = rng.normal(0, 1 / 64, (4096,)).astype(np.float32)
    if dt == "float16":
        a, b = a.astype(np.float16), b.astype(np.float16)
    with hip.poisoned():
        y = hip.gemm(a, dt, b, dt, c, "float32", dt, 1.0, 1.0, 0, 1)
        hip.set_exact(True)
        try:
            ye = hip.gemm(a, dt, b, dt, c, "float32", dt, 1.0, 1.0, 0, 1)
        finally:
            hip.set_exact(False)
    assert_close(y, ye, dt, what=f"gemm {dt} 4096: every element, MFMA vs exact mode")
    rows = rng.choice(4096, 48, replace=False)
    ref = a[rows].astype(np.float64) @ b.astype(np.float64).T + c.astype(np.float64)
    if dt == "float16":
        ref_codes = O.oracle().encode_f32(ref.astype(np.float32), O.F16)
        assert_close(y[rows], ref_codes, O.F16, what="gemm f16 4096")
    else:
        assert_close(y[rows], ref.astype(np.float32), O.F32, what="gemm f32 4096")
    few = rows[:16]
    want = oracle_lib.gemm(a[few], dt, b, dt, c, "float32", dt, 1.0, 1.0, 0, 1)
    assert_bitexact(ye[few], want, dt, what=f"gemm {dt} 4096 exact mode vs oracle")


def test_config3_woq(hip, oracle_lib):
    rng = np.random.default_rng(2)
    bw = rng.normal(0, 1 / 64, (4096, 4096))
    sw = (np.abs(bw).max(axis=1) / 127).astype(np.float32)
    bq = np.clip(np.rint(bw / sw[:, None]), -127, 127).astype(np.int8)
    z = np.zeros(4096, np.int8)
    deq = hip.qdq("dequantize", bq, O.I8, sw.reshape(-1, 1), O.F32, z.reshape(-1, 1), O.I8, O.F32)
    ref = oracle_lib.qdq("dequantize", bq, O.I8, sw.reshape(-1, 1), O.F32, z.reshape(-1, 1), O.I8, O.F32)
    assert_bitexact(deq, ref, O.F32, what="WOQ DQ")
    a = rng.normal(0, 1 / 64, (256, 4096)).astype(np.float32)
    cb = rng.normal(0, 1 / 64, (4096,)).astype(np.float32)
    y = hip.gemm(a, O.F32, deq, O.F32, cb, O.F32, O.F32, 1.0, 1.0, 0, 1)
    r = a.astype(np.float64) @ deq.astype(np.float64).T + cb
    assert_close(y, r.astype(np.float32), O.F32, what="WOQ gemm")


CONVS = [("stem", (32, 3, 224, 224), (64, 3, 7, 7), [3, 3, 3, 3], [2, 2]),
         ("3x3", (32, 64, 56, 56), (64, 64, 3, 3), [1, 1, 1, 1], [1, 1]),
         ("1x1", (32, 64, 56, 56), (256, 64, 1, 1), [0, 0, 0, 0], [1, 1])]


@pytest.mark.parametrize("layer", CONVS, ids=[c[0] for c in CONVS])
def test_config4_conv_full_size(hip, oracle_lib, layer):
    """Config-4 convolution at full size.  Every element of the MFMA result
    (output poisoned with NaN first) is compared with the exact-mode result of
    the same call over the whole batch; the exact mode is anchored bit for bit
    to the oracle on the first and last images, as is the MFMA mode within
    tolerance."""
    tag, xs, ws, pads, strides = layer
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, xs).astype(np.float32)
    w = rng.normal(0, np.sqrt(2 / (ws[1] * ws[2] * ws[3])), ws).astype(np.float32)
    b = rng.normal(0, 1 / 64, (ws[0],)).astype(np.float32)
    with hip.poisoned():
        y = hip.conv(x, O.F32, w, O.F32, b, O.F32, O.F32, pads, strides, [1, 1], 1)
        hip.set_exact(True)
        try:
            ye = hip.conv(x, O.F32, w, O.F32, b, O.F32, O.F32, pads, strides, [1, 1], 1)
        finally:
            hip.set_exact(False)
    assert_close(y, ye, O.F32, what=f"conv {tag}: every element, MFMA vs exact mode")
    imgs = [0, xs[0] - 1]
    ref = oracle_lib.conv(x[imgs], O.F32, w, O.F32, b, O.F32, O.F32, pads, strides, [1, 1], 1)
    assert_close(y[imgs], ref, O.F32, what=f"conv {tag}")
    assert_bitexact(ye[imgs], ref, O.F32, what=f"conv {tag} exact")


def test_config4_maxpool_full_size(hip, oracle_lib):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (32, 64, 112, 112)).astype(np.float32)
    y = hip.maxpool(x, O.F32, O.F32, [3, 3], [1, 1, 1, 1], [2, 2])
    assert_bitexact(y, oracle_lib.maxpool(x, O.F32, O.F32, [3, 3], [1, 1, 1, 1], [2, 2]), O.F32, what="maxpool")


# 3x3 / stride 2 / pad 1 runs the strip kernel (odd input and output heights,
# W % 4 == 0 and == 2 included).
POOLS = [("3x3s2p1", (2, 3, 30, 28), [3, 3], [1, 1, 1, 1], [2, 2], [1, 1]),
         ("3x3s2p1_odd_h", (2, 3, 29, 28), [3, 3], [1, 1, 1, 1], [2, 2], [1, 1]),
         ("3x3s2p1_w26_strip", (2, 3, 30, 26), [3, 3], [1, 1, 1, 1], [2, 2], [1, 1]),
         ("2x2s2", (2, 4, 16, 12), [2, 2], [0, 0, 0, 0], [2, 2], [1, 1]),
         ("3x3s1p1_dil2", (1, 5, 20, 24), [3, 3], [1, 1, 1, 1], [1, 1], [2, 2]),
         ("7x7_asym", (1, 3, 36, 40), [7, 5], [3, 2, 1, 0], [2, 3], [1, 1]),
         ("allpad_window", (1, 2, 8, 8), [2, 2], [3, 3, 3, 3], [4, 4], [1, 1]),
         # the strip kernel's resident blocks walking 1500 planes (one or two each)
         ("3x3s2p1_1500_planes", (3, 500, 14, 12), [3, 3], [1, 1, 1, 1], [2, 2], [1, 1])]


@pytest.mark.parametrize("case", POOLS, ids=[c[0] for c in POOLS])
def test_maxpool_plane_kernel(hip, oracle_lib, case):
    """f32 planes that fit in LDS (one block per plane), with NaN, +-0 and -inf planted."""
    tag, xs, k, pads, strides, dil = case
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, xs).astype(np.float32)
    flat = x.reshape(-1)
    flat[rng.choice(flat.size, 20, replace=False)] = np.nan
    flat[rng.choice(flat.size, 20, replace=False)] = -0.0
    flat[rng.choice(flat.size, 20, replace=False)] = 0.0
    flat[rng.choice(flat.size, 5, replace=False)] = -np.inf
    y = hip.maxpool(x, O.F32, O.F32, k, pads, strides, dil)
    assert_bitexact(y, oracle_lib.maxpool(x, O.F32, O.F32, k, pads, strides, dil), O.F32, what=f"maxpool {tag}")


def test_config5_softmax(hip, oracle_lib):
    rng = np.random.default_rng(4)
    x = rng.normal(0, 3, (64, 32000)).astype(np.float32)
    y = hip.softmax(x, O.F32, O.F32, 1)
    ref = oracle_lib.softmax(x, O.F32, O.F32, 1)
    assert_close(y, ref, O.F32, what="softmax")
    # exp runs as fp64 range reduction + fp32 core: within a few f32 ulp of the
    # reference's double exp (outputs are positive, so ulp = bit distance)
    ulp = np.abs(y.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert int(ulp.max()) <= 8, int(ulp.max())
    np.testing.assert_allclose(y.astype(np.float64).sum(axis=1), 1.0, rtol=1e-5)
    x2 = rng.normal(0, 3, (64, 1000)).astype(np.float32)
    assert_close(hip.softmax(x2, O.F32, O.F32, -1), oracle_lib.softmax(x2, O.F32, O.F32, -1), O.F32)


# Few long rows run the one-launch split kernel (each row over G blocks that
# exchange partial (max, sum) pairs); chunks over 4096 elements run the
# two-launch form.  spin = 0 makes every block recompute every other block's
# pair from X instead of waiting for it: the result must not change by a bit.
SOFTMAX_SPLIT = [((64, 32000), "float32", O.F32, O.F32), ((8, 20000), "float32", O.F32, O.F32),
                 ((3, 31999), "float32", O.F32, O.F32), ((5, 6000), "float64", O.F64, O.F64),
                 ((4, 9000), "float16", O.F16, O.F32), ((2, 70001), "float32", O.F32, O.F32),
                 ((2, 300000), "float32", O.F32, O.F32)]


@pytest.mark.parametrize("shape,npdt,dtx,dty", SOFTMAX_SPLIT,
                         ids=[f"{s[0]}x{s[1]}-{n}" for s, n, _, _ in SOFTMAX_SPLIT])
def test_softmax_split_rows(hip, oracle_lib, shape, npdt, dtx, dty):
    rng = np.random.default_rng(shape[1])
    x = rng.normal(0, 3, shape).astype(npdt)
    x.reshape(-1)[rng.choice(x.size, 7, replace=False)] = 40.0    # a few clear maxima per tensor
    y = hip.softmax(x, dtx, dty, 1)
    assert_close(y, oracle_lib.softmax(x, dtx, dty, 1), dty, what=f"softmax {shape}")
    old = hip.lib.tensor_ops_hip_set_softmax_spin(0)
    try:
        y0 = hip.softmax(x, dtx, dty, 1)
    finally:
        hip.lib.tensor_ops_hip_set_softmax_spin(old)
    assert np.array_equal(y0.view(np.uint8), y.view(np.uint8)), f"recomputed partials changed softmax {shape}"


@pytest.mark.parametrize("ydt,zdt", [(O.U8, O.U8), (O.I8, O.I8), (O.E4M3, O.E4M3), (O.E5M2, O.E5M2),
                                     (O.I8, O.F32), (O.U8, O.F32), (O.E4M3, O.F32), (O.E5M2, O.F32)])
def test_quantize_fast_path_boundaries(hip, oracle_lib, ydt, zdt):
    """Inputs placed on and next to rounding ties of x / s, huge quotients and
    special scales: the fp32 fast path must hand every doubtful lane to fp64."""
    rng = np.random.default_rng(int(ydt) * 13 + int(zdt))
    n = 1 << 16
    s = np.float32(rng.uniform(0.003, 3.0))
    k = rng.integers(-200, 200, n).astype(np.float64)
    rel = rng.choice([0.0, 1e-7, -1e-7, 3e-7, -3e-7, 1e-6, -1e-6, 6e-8, -6e-8], n)
    x = ((k + 0.5) * float(s) * (1.0 + rel)).astype(np.float32)
    ulp = np.spacing(x).astype(np.float32)
    x = np.where(rng.random(n) < 0.3, x + ulp * rng.integers(-2, 3, n).astype(np.float32), x).astype(np.float32)
    x[:64] = np.array([2 ** 22, 2 ** 22 + 1, 2 ** 23 + 0.5, -2 ** 24, 1e30, -1e30, np.inf, -np.inf, np.nan, 0.0, -0.0,
                       1e-40, -1e-45, 0.5, -0.5, 1.5] * 4, np.float32) * np.float32(s)
    # quotients between 2^17 and 2^28 (fp32 spacing of x / s above 1), and around the fp8 saturation points
    big = np.float64(s) * np.concatenate([rng.uniform(2 ** 17, 2 ** 28, 96) * rng.choice([-1, 1], 96),
                                          np.array([447.5, 448.5, 463.5, 464.5, 57343.5, 61439.5, 61440.5, 65535.5])])
    x[64:168] = big.astype(np.float32)
    # zero points: integral, fractional (0x01 codes, -2.5, 0.001: fp8 flush-to-zero band of r + zp),
    # beyond the fast path's |zp| < 2^22 and huge
    zvals = {O.U8: [0, 3, 128, 255], O.I8: [0, -5, 127, -128], O.E4M3: [0x00, 0x38, 0xB8, 0x01, 0x80],
             O.E5M2: [0x00, 0x3C, 0xBC, 0x01, 0x80],
             O.F32: [0.0, 3.0, -2.5, 1e30, 0.001, 2.0 ** 22, 2.0 ** 22 + 2, -(2.0 ** 22 - 1)]}[zdt]
    for zv in zvals:
        z = np.array([zv], O.STORAGE[zdt])
        # special scales, including ones whose reciprocal is subnormal (|s| > 2^126) or overflows
        for sv in (s, np.float32(-s), np.float32(0.0), np.float32(-0.0), np.float32(1e-42), np.float32(np.inf),
                   np.float32(np.nan), np.float32(1e38), np.float32(-3e38), np.float32(1.2e-38)):
            sa = np.array([sv], np.float32)
            got = hip.qdq("quantize", x, O.F32, sa, O.F32, z, zdt, ydt)
            ref = oracle_lib.qdq("quantize", x, O.F32, sa, O.F32, z, zdt, ydt)
            assert_bitexact(got, ref, ydt, what=f"Q y={ydt} z={zv} s={sv}")
    # per-axis scales with mixed magnitudes
    x3 = x[: 64 * 1024].reshape(4, 64, 256)
    sax = rng.uniform(0.001, 5.0, 64).astype(np.float32)
    sax[:6] = [0.0, -1.5, np.inf, np.nan, 1e38, 1e-42]
    sax = sax.reshape(1, 64, 1)
    zax = np.array(zvals * 16, O.STORAGE[zdt])[:64].reshape(1, 64, 1)
    assert_bitexact(hip.qdq("quantize", x3, O.F32, sax, O.F32, zax, zdt, ydt),
                    oracle_lib.qdq("quantize", x3, O.F32, sax, O.F32, zax, zdt, ydt), ydt, what="Q per-axis")
    # inner dimension not a multiple of 256 (parameters per 4-element group rather than per wave)
    x4 = x[: 64 * 1000].reshape(50, 64, 20)
    assert_bitexact(hip.qdq("quantize", x4, O.F32, sax, O.F32, zax, zdt, ydt),
                    oracle_lib.qdq("quantize", x4, O.F32, sax, O.F32, zax, zdt, ydt), ydt, what="Q per-axis inner 20")
    # full-size scale and zero point (the reference's Python pre-broadcasts them): per-element parameters
    sfull = np.broadcast_to(sax, x3.shape).copy()
    sfull[:, :, ::7] = s
    zfull = np.broadcast_to(zax, x3.shape).copy()
    assert_bitexact(hip.qdq("quantize", x3, O.F32, sfull, O.F32, zfull, zdt, ydt),
                    oracle_lib.qdq("quantize", x3, O.F32, sfull, O.F32, zfull, zdt, ydt), ydt, what="Q full-size")


@pytest.mark.parametrize("xdt", [O.U8, O.I8, O.E4M3, O.E5M2])
def test_dequantize_all_codes(hip, oracle_lib, xdt):
    """Every code of every 1-byte format through the dequantize kernels (per-tensor,
    per-axis and full-size parameters): pins the hardware fp8 decode and the fp64
    (x - zp) * s against the reference, bit for bit."""
    rng = np.random.default_rng(int(xdt))
    codes = np.tile(np.arange(256, dtype=np.uint8), 64).reshape(4, 16, 256)
    zdts = [xdt, O.F32]
    for zdt in zdts:
        zv = {O.U8: [0, 7, 255], O.I8: [0, -9, 127], O.E4M3: [0x00, 0x39, 0xC4, 0x7F], O.E5M2: [0x00, 0x3D, 0xBA, 0x7D],
              O.F32: [0.0, 0.3, -1e30, 5.0]}[zdt]
        for z0 in zv:
            for s0 in (np.float32(0.0123), np.float32(-3.5), np.float32(1e38), np.float32(0.0), np.float32(np.inf),
                       np.float32(np.nan), np.float32(1e-45)):
                sa, za = np.array([s0], np.float32), np.array([z0], O.STORAGE[zdt])
                assert_bitexact(hip.qdq("dequantize", codes, xdt, sa, O.F32, za, zdt, O.F32),
                                oracle_lib.qdq("dequantize", codes, xdt, sa, O.F32, za, zdt, O.F32), O.F32,
                                what=f"DQ x={xdt} z={z0} s={s0}")
        sax = rng.uniform(-2, 2, 16).astype(np.float32)
        sax[:3] = [0.0, np.inf, 1e30]
        zax = np.array((zv * 16)[:16], O.STORAGE[zdt])
        c2 = codes.reshape(64, 16, 16)
        assert_bitexact(hip.qdq("dequantize", c2, xdt, sax.reshape(1, 16, 1), O.F32, zax.reshape(1, 16, 1), zdt, O.F32),
                        oracle_lib.qdq("dequantize", c2, xdt, sax.reshape(1, 16, 1), O.F32, zax.reshape(1, 16, 1), zdt,
                                       O.F32), O.F32, what="DQ per-axis inner 16")
        assert_bitexact(hip.qdq("dequantize", codes, xdt, sax.reshape(1, 16, 1), O.F32, zax.reshape(1, 16, 1), zdt,
                                O.F32),
                        oracle_lib.qdq("dequantize", codes, xdt, sax.reshape(1, 16, 1), O.F32, zax.reshape(1, 16, 1),
                                       zdt, O.F32), O.F32, what="DQ per-axis")
        sfull = np.broadcast_to(sax.reshape(1, 16, 1), codes.shape).copy()
        sfull[..., ::5] = np.float32(0.75)
        zfull = np.broadcast_to(zax.reshape(1, 16, 1), codes.shape).copy()
        assert_bitexact(hip.qdq("dequantize", codes, xdt, sfull, O.F32, zfull, zdt, O.F32),
                        oracle_lib.qdq("dequantize", codes, xdt, sfull, O.F32, zfull, zdt, O.F32), O.F32,
                        what="DQ full-size")


@pytest.mark.parametrize("words", [1, 255, 1023, 1025, 3 * 1024 + 517, 40 * 1024 + 1])
def test_dequantize_ragged_lengths(hip, oracle_lib, words):
    """Lengths (in 4-code words) that end inside a thread's group of code words and
    inside a block's pass: with outputs pre-filled with NaN, every word must be
    written (the fp8 cases with a zero point other than 0 take the fp64 branch)."""
    rng = np.random.default_rng(words)
    for xdt, zdt, z0 in ((O.U8, O.U8, 3), (O.E4M3, O.E4M3, 0), (O.E5M2, O.E5M2, 0x3D)):
        codes = rng.integers(0, 256, 4 * words, dtype=np.uint8)
        codes[(codes & 0x7F) >= (0x7C if xdt == O.E5M2 else 0x7F)] = 0x11     # finite codes only: NaN would mask a miss
        sa, za = np.array([0.0371], np.float32), np.array([z0], O.STORAGE[zdt])
        with hip.poisoned():
            got = hip.qdq("dequantize", codes, xdt, sa, O.F32, za, zdt, O.F32)
        assert_bitexact(got, oracle_lib.qdq("dequantize", codes, xdt, sa, O.F32, za, zdt, O.F32), O.F32,
                        what=f"DQ {xdt} {words} words")


# ---------------------------------------------------------------- next rows ---
def test_dql_reciprocal_path_ties(hip, oracle_lib):
    """The quantize pass multiplies by 1/scale and falls back to the division
    near half-integers: with scale = 3 (1/3 inexact), inputs 3k + 1.5 are exact
    ties of x / scale and their float neighbours sit next to them."""
    k = np.arange(-2, 253, dtype=np.float64)
    t = (3 * k + 1.5).astype(np.float32)
    x = np.concatenate([np.array([-6.0, 759.0], np.float32), t, np.nextafter(t, np.float32(np.inf)),
                        np.nextafter(t, np.float32(-np.inf)), (3 * k).astype(np.float32)])
    x = np.tile(x, 64)
    y, s, z = hip.dql(x, O.F32)
    ry, rs, rz = oracle_lib.dql(x, O.F32)
    assert float(rs[0]) == 3.0 and int(rz[0]) == 2
    assert_bitexact(s, rs, O.F32, what="dql scale")
    assert_bitexact(z, rz, O.U8, what="dql zero point")
    assert_bitexact(y, ry, O.U8, what="dql codes at ties")


def test_dynamic_quantize_linear_full_size(hip, oracle_lib, x2):
    """DynamicQuantizeLinear on the config-2 activation tensor (16.8 M values), bit-exact."""
    y, s, z = hip.dql(x2, O.F32)
    ry, rs, rz = oracle_lib.dql(x2, O.F32)
    assert_bitexact(s, rs, O.F32, what="dql scale")
    assert_bitexact(z, rz, O.U8, what="dql zero point")
    assert_bitexact(y, ry, O.U8, what="dql codes")


def _dql_case(name):
    rng = np.random.default_rng(len(name))
    if name == "normal_1M":
        return rng.normal(0, 3, 1 << 20).astype(np.float32)
    if name == "nan_inf":
        x = rng.normal(0, 2, 1 << 16).astype(np.float32)
        x[rng.choice(x.size, 9, replace=False)] = np.nan
        x[rng.choice(x.size, 3, replace=False)] = np.inf
        x[rng.choice(x.size, 3, replace=False)] = -np.inf
        return x
    if name == "all_nan":
        return np.full(4096, np.nan, np.float32)
    if name == "zeros":
        return np.zeros(1 << 14, np.float32)
    if name == "negative":
        return -np.abs(rng.normal(0, 5, 1 << 15)).astype(np.float32)
    if name == "positive":
        return np.abs(rng.normal(0, 5, 1 << 15)).astype(np.float32) + 1
    if name == "tiny":     # scale below 2^-120: every code through the double path
        return (rng.normal(0, 1, 1 << 14) * 1e-38).astype(np.float32)
    if name == "huge":     # scale above 2^120
        return (rng.uniform(-1, 1, 1 << 14) * 3e38).astype(np.float32)
    if name == "odd_size":  # n % 4 != 0: the three-launch path
        return rng.normal(0, 1, 100_003).astype(np.float32)
    if name == "ragged_62_blocks":  # 250,001 float4s: 62 blocks, the last one partial
        return rng.normal(1, 2, 4 * 250_001).astype(np.float32)
    if name == "full_minus_one_float4":  # 256 blocks of 16 float4s per thread, the last block one short
        return rng.normal(0, 1, 32 * 512 * 1024 - 4).astype(np.float32)
    raise ValueError(name)


DQL_CASES = ["normal_1M", "nan_inf", "all_nan", "zeros", "negative", "positive", "tiny", "huge", "odd_size",
             "ragged_62_blocks", "full_minus_one_float4"]


@pytest.mark.parametrize("name", DQL_CASES)
def test_dql_one_launch_cases(hip, oracle_lib, name):
    """DynamicQuantizeLinear's one-launch kernel (x read once, blocks exchange
    their min / max) against the oracle, bit for bit, on special values and
    scales outside the f32 reciprocal's range; spin = 0 makes every block
    recompute the other blocks' min / max from x instead of waiting."""
    x = _dql_case(name)
    ry, rs, rz = oracle_lib.dql(x, O.F32)
    old = hip.lib.tensor_ops_hip_set_softmax_spin(-1)
    try:
        for spin in (-1, 0):
            hip.lib.tensor_ops_hip_set_softmax_spin(spin)
            y, s, z = hip.dql(x, O.F32)
            assert_bitexact(s, rs, O.F32, what=f"dql scale {name} spin {spin}")
            assert_bitexact(z, rz, O.U8, what=f"dql zero point {name} spin {spin}")
            assert_bitexact(y, ry, O.U8, what=f"dql codes {name} spin {spin}")
    finally:
        hip.lib.tensor_ops_hip_set_softmax_spin(old)


@pytest.mark.parametrize("shape", [(64, 512, 7, 7), (8, 64, 56, 56), (3, 5, 1, 1), (1, 300, 3, 3), (2, 70, 10, 11)])
def test_global_average_pool_sizes(hip, oracle_lib, shape):
    rng = np.random.default_rng(sum(shape))
    x = rng.normal(0, 1, shape).astype(np.float32)
    for ydt in (O.F32, O.F64, O.F16):
        assert_bitexact(hip.gap(x, O.F32, ydt), oracle_lib.gap(x, O.F32, ydt), ydt, what=f"gap {shape} -> {ydt}")


def test_next_row_ops_device_resident(hip):
    """Flatten / Reshape / GlobalAveragePool / DynamicQuantizeLinear through the
    Python layer on device tensors give the host path's bits."""
    from onnx_translator_amd.nn import Tensor
    from onnx_translator_amd.nn.Operators import DynamicQuantizeLinear, Flatten, GlobalAveragePool, Reshape
    rng = np.random.default_rng(8)
    x = rng.normal(0, 1, (4, 32, 7, 7)).astype(np.float32)
    host = Tensor(*x.shape, dtype="float32", data=x)
    dev = host.to_device() if hasattr(host, "to_device") else None
    assert dev is not None
    for op, args in ((GlobalAveragePool(["x"], ["y"], dtype="float32"), ()),
                     (Flatten(["x"], ["y"], axis=1, dtype="float32"), ()),
                     (Reshape(["x", "s"], ["y"], dtype="float32"), (np.array([4, -1], np.int64),))):
        h = op.forward(host, *args)["tensor"]
        d = op.forward(dev, *args)["tensor"]
        assert d.on_device and d.size == h.size
        assert_bitexact(d.numpy(), h.numpy(), O.F32, what=type(op).__name__)
    q = DynamicQuantizeLinear(["x"], ["y", "s", "z"])
    hs = [t.numpy() for t in q.forward(host)["tensor"]]
    ds = [t.numpy() for t in q.forward(dev)["tensor"]]
    for a, b, dt in zip(ds, hs, (O.U8, O.F32, O.U8)):
        assert_bitexact(a, b, dt, what="dql device")


# ------------------------------------------------------------ fused chain ---
CONFIG1_CHAIN = [("Add", 0, False), ("Mul", 0, False), ("Sub", 0, False), ("Div", 1, False), ("Relu", None, False),
                 ("Abs", None, False), ("Cos", None, False)]


def oracle_chain(o, x, operands, steps):
    """The chain op by op through the oracle (each op pinned to the reference's golden vectors)."""
    v = x
    for op, arg, rev in steps:
        if op in ("Relu", "Abs", "Cos"):
            v = o.unary(op.lower(), v, O.F32, O.F32)
        else:
            b = operands[arg]
            a0, a1 = (b, v) if rev else (v, b)
            v = o.binary(op.lower(), a0, O.F32, a1, O.F32, O.F32)
    return v


def test_config1_chain_fused_full_size(hip, oracle_lib):
    """The config-1 chain in one kernel equals the op-by-op reference chain bit for bit."""
    from onnx_translator_amd.nn import Tensor
    from onnx_translator_amd.nn.Operators import ElementwiseChain
    rng = np.random.default_rng(0)
    A = rng.uniform(-4, 4, (8, 64, 56, 56)).astype(np.float32)
    B = rng.uniform(-4, 4, (64, 1, 1)).astype(np.float32)
    Bd = (np.sign(B) * np.maximum(np.abs(B), 0.1)).astype(np.float32)
    ref = oracle_chain(oracle_lib, A, [B, Bd], CONFIG1_CHAIN)
    op = ElementwiseChain(["A", "B", "Bd"], ["Y"], CONFIG1_CHAIN)
    got = op.forward(Tensor(*A.shape, dtype="float32", data=A), Tensor(*B.shape, dtype="float32", data=B),
                     Tensor(*Bd.shape, dtype="float32", data=Bd))["tensor"]
    assert_bitexact(got.numpy(), ref, O.F32, what="config1 chain (host)")
    dev = op.forward(Tensor(*A.shape, dtype="float32", data=A).to_device(),
                     Tensor(*B.shape, dtype="float32", data=B).to_device(),
                     Tensor(*Bd.shape, dtype="float32", data=Bd).to_device())["tensor"]
    assert dev.on_device
    assert_bitexact(dev.numpy(), ref, O.F32, what="config1 chain (device)")


@pytest.mark.parametrize("seed", range(6))
def test_random_chains(hip, oracle_lib, seed):
    """Random op sequences, reversed operands, operand shapes that broadcast along
    inner / outer / all dims, the vector path (inner % 4 == 0) and the scalar one."""
    from onnx_translator_amd.nn import Tensor
    from onnx_translator_amd.nn.Operators import ElementwiseChain
    rng = np.random.default_rng(100 + seed)
    shape = [(3, 5, 8), (2, 7, 9), (4, 16), (6, 1, 12)][seed % 4]
    x = rng.uniform(-3, 3, shape).astype(np.float32)
    x.reshape(-1)[:3] = [np.nan, -0.0, np.inf]
    cands = [shape[-1:], (1,) + tuple(shape[1:]), (1,), tuple(shape), (shape[0],) + (1,) * (len(shape) - 1)]
    operands = [rng.uniform(0.5, 2, cands[int(rng.integers(len(cands)))]).astype(np.float32) for _ in range(3)]
    ops = ["Add", "Sub", "Mul", "Div", "Relu", "Abs", "Cos"]
    steps = []
    for _ in range(int(rng.integers(3, 12))):
        op = ops[int(rng.integers(len(ops)))]
        steps.append((op, int(rng.integers(3)), bool(rng.integers(2))) if op in ops[:4] else (op, None, False))
    with np.errstate(all="ignore"):
        ref = oracle_chain(oracle_lib, x, operands, steps)
    got = ElementwiseChain(["x"], ["y"], steps).forward(
        Tensor(*x.shape, dtype="float32", data=x), *[Tensor(*o.shape, dtype="float32", data=o) for o in operands])
    assert_bitexact(got["tensor"].numpy(), ref, O.F32, what=f"chain {steps}")


def test_cos_near_multiples_of_two_pi(hip, oracle_lib):
    """The exact fmod(|x|, 2pi) shortcut: inputs on and next to k * 2pi (where the
    quotient estimate is off by one), random magnitudes below 2^30 and just above it."""
    rng = np.random.default_rng(31)
    k = np.unique(np.concatenate([np.arange(1, 2000), rng.integers(1, 2 ** 27, 4000)])).astype(np.float64)
    base = (k * (2 * np.pi)).astype(np.float32)
    near = np.concatenate([base, np.nextafter(base, 0), np.nextafter(base, np.inf)])
    wide = np.concatenate([rng.uniform(0, 2.0 ** 30, 20000), rng.uniform(2.0 ** 30, 2.0 ** 34, 2000),
                           -rng.uniform(0, 1e4, 2000)]).astype(np.float32)
    x = np.concatenate([near, -near, wide]).astype(np.float32)
    assert_bitexact(hip.unary("cos", x, O.F32, O.F32), oracle_lib.unary("cos", x, O.F32, O.F32), O.F32,
                    what="cos near 2pi multiples")
    xd = np.concatenate([k * 2 * np.pi, np.nextafter(k * 2 * np.pi, 0), rng.uniform(0, 2.0 ** 31, 5000)])
    assert_bitexact(hip.unary("cos", xd, O.F64, O.F64), oracle_lib.unary("cos", xd, O.F64, O.F64), O.F64,
                    what="cos f64 near 2pi multiples")


@pytest.mark.parametrize("shape,axis", [((3, 40, 1024), 1), ((2, 7, 2048), 1), ((130, 1024), 0), ((1, 3, 4096), 1),
                                        ((5, 6, 768), 1), ((4, 9, 256), 1), ((3, 5, 12), 1), ((6, 3, 4, 1024), 2)],
                         ids=["inner1024", "inner2048", "axis0", "inner4096", "inner768", "inner256", "inner12",
                              "rank4"])
@pytest.mark.parametrize("ydt", [O.I8, O.U8], ids=["i8", "u8"])
def test_per_axis_qdq_layouts(hip, oracle_lib, shape, axis, ydt):
    """Per-axis QuantizeLinear / DequantizeLinear over channel runs that take the
    per-wave parameter kernels (runs a multiple of 1024 elements for quantize,
    256 for dequantize) and the per-unit ones (shorter runs), with per-channel
    zero points, rounding ties and saturation, against the oracle
    (tensor_ops.c:999-1034)."""
    rng = np.random.default_rng(hash((shape, axis, ydt)) % 2 ** 32)
    C = shape[axis]
    s = rng.uniform(0.01, 0.2, C).astype(np.float32)
    lo, hi = (-6, 6) if ydt == O.I8 else (0, 12)
    z = rng.integers(lo, hi, C).astype(np.int8 if ydt == O.I8 else np.uint8)
    x = rng.normal(0, 8, shape).astype(np.float32)
    on = [1] * len(shape)
    on[axis] = C
    sb, zb = np.broadcast_to(s.reshape(on), shape), np.broadcast_to(z.reshape(on), shape)
    x.reshape(-1)[::7] = ((np.rint(x.reshape(-1)[::7] / sb.reshape(-1)[::7]) + 0.5) * sb.reshape(-1)[::7])
    want = oracle_lib.qdq("quantize", x, O.F32, s.reshape(on), O.F32, z.reshape(on), ydt, ydt)
    assert_bitexact(hip.qdq1("quantize", x, O.F32, s.reshape(on), z.reshape(on), ydt, ydt), want, ydt,
                    what=f"Q {shape} axis {axis}")
    assert_bitexact(hip.qdq_axis("quantize", x, O.F32, s, z, ydt, ydt, axis), want, ydt, what="Q axis entry")
    back = oracle_lib.qdq("dequantize", want, ydt, s.reshape(on), O.F32, z.reshape(on), ydt, O.F32)
    assert_bitexact(hip.qdq1("dequantize", want, ydt, s.reshape(on), z.reshape(on), ydt, O.F32), back, O.F32,
                    what=f"DQ {shape} axis {axis}")
    assert_bitexact(hip.qdq_axis("dequantize", want, ydt, s, z, ydt, O.F32, axis), back, O.F32, what="DQ axis entry")
