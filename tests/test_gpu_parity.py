"""GPU parity: every golden case through libtensor_ops_hip.so's C ABI.

* host tensors (reference semantics: synchronous, staged through HBM);
* Gemm / Conv in both precision modes: MFMA (tolerance class) and exact
  (fp64, reference summation order: bit-exact);
* device-resident tensors through the Python operator layer, which must give
  the same bits as the host path;
* error paths forced from the host (bad shapes) return an error, never fault.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import HipLib, assert_bitexact, check_case, load_cases, run_case

pytestmark = pytest.mark.gpu

CASES, ARRAYS = load_cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden_default_mode(hip, case):
    hip.set_exact(False)
    out = run_case(hip, case, ARRAYS)
    check_case(out, case, ARRAYS, exact=False)


EXACT_CASES = [c for c in CASES if c["op"] in ("gemm", "conv2d")]


@pytest.mark.parametrize("case", EXACT_CASES, ids=[c["name"] for c in EXACT_CASES])
def test_golden_exact_mode(hip, case):
    hip.set_exact(True)
    try:
        out = run_case(hip, case, ARRAYS)
    finally:
        hip.set_exact(False)
    assert_bitexact(out, ARRAYS[case["out"]], case["out_dtype"], what=case["name"])


def test_mfma_f32_layout_single_tile(hip):
    """A 32x2 @ 2x32 product (one MFMA) checks the operand / result lane layout."""
    rng = np.random.default_rng(0)
    a = rng.integers(-8, 8, (32, 2)).astype(np.float32)
    b = rng.integers(-8, 8, (2, 32)).astype(np.float32)
    out = hip.gemm(a, O.F32, b, O.F32, None, O.F32, O.F32, 1.0, 0.0, 0, 0)
    assert np.array_equal(out, a @ b)
    a16 = rng.integers(-8, 8, (32, 16)).astype(np.float16)
    b16 = rng.integers(-8, 8, (32, 16)).astype(np.float16)
    out = hip.gemm(a16, O.F16, b16, O.F16, None, O.F32, O.F32, 1.0, 0.0, 0, 1)
    assert np.array_equal(out, a16.astype(np.float32) @ b16.astype(np.float32).T)


@pytest.mark.parametrize("shape", [(1, 1, 1), (127, 129, 67), (200, 64, 300), (64, 250, 17)])
@pytest.mark.parametrize("trans", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_ragged_shapes(hip, oracle_lib, shape, trans):
    M, N, K = shape
    ta, tb = trans
    rng = np.random.default_rng(M * 7 + N)
    a = rng.normal(0, 1, (K, M) if ta else (M, K)).astype(np.float32)
    b = rng.normal(0, 1, (N, K) if tb else (K, N)).astype(np.float32)
    c = rng.normal(0, 1, (N,)).astype(np.float32)
    for dt in ("float32", "float16"):
        aa = a if dt == "float32" else a.astype(np.float16).view(np.uint16)
        bb = b if dt == "float32" else b.astype(np.float16).view(np.uint16)
        ref = oracle_lib.gemm(aa, dt, bb, dt, c, "float32", "float32", 1.25, 0.5, ta, tb)
        got = hip.gemm(aa, dt, bb, dt, c, "float32", "float32", 1.25, 0.5, ta, tb)
        from tests.helpers import assert_close
        assert_close(got, ref, O.F32, what=f"gemm {dt} {shape} {trans}")


# f32 x f32 with transB = 1 and K % 4 == 0 runs the tiled NT kernel: 128x256
# tiles when the grid has >= 192 of them, else 128x64 tiles with the k range
# split over up to 16 slices (partial sums reduced in a second pass).  The
# cases cover one slice, several slices with a ragged last one, K % 16 != 0,
# ragged M / N and every bias mode of the inline and out-of-line epilogues.
F32_NT = [(300, 200, 136, "col"), (64, 256, 2048, "none"), (70, 130, 1100, "scalar"), (96, 72, 5200, "row"),
          (3000, 3100, 68, "col"), (1000, 1000, 4, "2d"), (1, 1000, 512, "col")]


@pytest.mark.parametrize("M,N,K,bias", F32_NT, ids=[f"{m}x{n}x{k}-{b}" for m, n, k, b in F32_NT])
@pytest.mark.parametrize("ydt", ["float32", "float16"])
def test_gemm_f32_tiled_kernel(hip, M, N, K, bias, ydt):
    from tests.helpers import assert_close
    rng = np.random.default_rng(M + 5 * N + 11 * K)
    a = rng.normal(0, 1, (M, K)).astype(np.float32)
    b = rng.normal(0, 1, (N, K)).astype(np.float32)
    c = {"none": None, "scalar": rng.normal(0, 1, (1,)), "row": rng.normal(0, 1, (M,)),
         "col": rng.normal(0, 1, (N,)), "2d": rng.normal(0, 1, (M, N))}[bias]
    if c is not None:
        c = c.astype(np.float32)
    alpha, beta = 0.75, 1.5
    y = hip.gemm(a, O.F32, b, O.F32, c, O.F32, ydt, alpha, beta, 0, 1)
    rows = np.arange(M) if M * N <= 1 << 20 else np.unique(np.r_[rng.choice(M, 40, replace=False), 0, M - 1])
    ref = alpha * (a[rows].astype(np.float64) @ b.astype(np.float64).T)
    if c is not None:
        cc = {"row": lambda: c[rows].reshape(-1, 1), "2d": lambda: c[rows]}.get(bias, lambda: c.reshape(1, -1))()
        ref = ref + beta * cc.astype(np.float64)
    if ydt == "float16":
        assert_close(y[rows], O.oracle().encode_f32(ref.astype(np.float32), O.F16), O.F16,
                     what=f"f32 nt {M}x{N}x{K} {bias}")
    else:
        assert_close(y[rows], ref.astype(np.float32), O.F32, what=f"f32 nt {M}x{N}x{K} {bias}")


# dequantize_gemm_forward: the fused weight-only-quantized Gemm returns the
# bits of dequantize_linear_axis_forward followed by gemm_forward (same
# schedule, and the dequantised operand is the same fp32 value), and matches
# the oracle's DequantizeLinear -> Gemm within the Gemm tolerance.  Cases: int8
# per-row scales (split-K and single slice), uint8 with per-row zero points,
# per-tensor parameters, no zero point, K % 16 != 0, ragged M / N, and cases
# the fused kernel does not take (transB = 0, axis 1 scales, K % 4 != 0),
# which run the unfused pair.
DQ_GEMM = [("i8_row", 64, 256, 2048, "int8", "row", 1, 0), ("i8_row_big", 300, 2100, 96, "int8", "row", 1, 0),
           ("u8_zp", 70, 130, 1100, "uint8", "row", 1, 0), ("u8_tensor", 33, 65, 260, "uint8", "tensor", 1, 0),
           ("i8_nozp", 128, 64, 512, "int8", "nozp", 1, 0), ("i8_nn", 40, 50, 60, "int8", "row", 0, 1),
           ("i8_axis1", 40, 50, 64, "int8", "col", 1, 1), ("i8_k_odd", 17, 19, 23, "int8", "row", 1, 0)]


@pytest.mark.parametrize("case", DQ_GEMM, ids=[c[0] for c in DQ_GEMM])
@pytest.mark.parametrize("ydt", ["float32", "float16"])
def test_dequantize_gemm(hip, oracle_lib, case, ydt):
    import ctypes
    from tests.helpers import assert_close
    tag, M, N, K, bdt, params, tb, axis = case
    rng = np.random.default_rng(M * 3 + N + K)
    shape = (N, K) if tb else (K, N)
    lo, hi = (-128, 128) if bdt == "int8" else (0, 256)
    bq = rng.integers(lo, hi, shape).astype(np.int8 if bdt == "int8" else np.uint8)
    nax = shape[axis]
    s = (rng.uniform(0.5, 2.0, nax) / 127).astype(np.float32)
    z = rng.integers(-3, 4, nax) if bdt == "int8" else rng.integers(100, 156, nax)
    z = z.astype(bq.dtype)
    if params == "tensor":
        s, z = s[:1], z[:1]
    elif params == "nozp":
        z = None
    a = rng.normal(0, 1, (M, K)).astype(np.float32)
    c = rng.normal(0, 1, (N,)).astype(np.float32)
    got = hip.dq_gemm(a, bq, bdt, s, z, axis, c, ydt, 0.75, 1.25, 0, tb)
    # unfused pair through the same library
    zz = z if z is not None else np.zeros(1, bq.dtype)
    bd = hip._run(hip.lib.dequantize_linear_axis_forward, [(bq, bdt), (s, O.F32), (zz, bdt)], bq.shape, O.F32,
                  ctypes.c_int(axis))
    two = hip.gemm(a, O.F32, bd, O.F32, c, O.F32, ydt, 0.75, 1.25, 0, tb)
    assert np.array_equal(got.view(np.uint8), two.view(np.uint8)), f"{tag}: fused differs from the unfused pair"
    # oracle: DequantizeLinear with the parameters on their axis, then Gemm
    on_axis = [1, 1]
    on_axis[axis] = -1
    zo = zz if zz.size > 1 else np.broadcast_to(zz, s.shape)
    ref_b = oracle_lib.qdq("dequantize", bq, bdt, s.reshape(on_axis) if s.size > 1 else s, O.F32,
                           zo.reshape(on_axis) if zo.size > 1 else zo, bdt, O.F32)
    assert np.array_equal(bd, ref_b), f"{tag}: dequantised weight differs from the oracle"
    ref = oracle_lib.gemm(a, O.F32, ref_b, O.F32, c, O.F32, ydt, 0.75, 1.25, 0, tb)
    assert_close(got, ref, ydt, what=f"dequantize_gemm {tag}")


# quantize_dequantize_linear_forward = quantize_linear_forward ->
# dequantize_linear_forward bit for bit: the one-pass kernel (one-element
# scales, zero points of the code dtype, f32, n % 4 == 0) for every 1-byte code
# format, with special values (NaN, +-inf, +-0, ties of the rounding, values
# that saturate) and different quantize / dequantize parameters; the fallback
# through a temporary (n % 4 != 0, a per-channel scale).  The oracle's pair
# gives the same bits.
QDQ_FUSED = [("u8", "uint8", 128, 0.037, 128, 0.037, (64, 64, 4)),
             ("i8_zp", "int8", -3, 0.02, 5, 0.031, (3, 1000, 4)),
             ("e4m3", "float8_e4m3", 0, 0.011, 0, 0.011, (4096,)),
             ("e5m2", "float8_e5m2", 0, 0.5, 0, 0.25, (2, 2048)),
             ("u8_tail_fallback", "uint8", 7, 0.05, 7, 0.05, (3, 5, 7)),
             ("i8_per_channel_fallback", "int8", 0, None, 0, 0.02, (2, 6, 8, 8))]


@pytest.mark.parametrize("case", QDQ_FUSED, ids=[c[0] for c in QDQ_FUSED])
def test_quantize_dequantize_fused(hip, oracle_lib, case):
    tag, cdt, qz, qs, dz, ds, shape = case
    rng = np.random.default_rng(len(tag) * 7 + len(shape))
    x = rng.normal(0, 3, shape).astype(np.float32)
    flat = x.reshape(-1)
    specials = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1e30, -1e30]
    flat[:len(specials)] = specials
    sq = np.float32(qs if qs is not None else 0.03)
    flat[len(specials):len(specials) + 64] = (np.arange(-32, 32) + 0.5) * sq      # ties of rint
    npz = np.int8 if cdt == "int8" else np.uint8
    zq, zd = np.array([qz], npz), np.array([dz], npz)
    if qs is None:   # per-channel quantize scale [1, C, 1, 1]: the library runs the pair
        qsv = (0.01 + 0.02 * rng.random(shape[1])).astype(np.float32).reshape(1, -1, 1, 1)
    else:
        qsv = np.array([qs], np.float32)
    dsv = np.array([ds], np.float32)
    got = hip.qdq_fused(x, qsv, zq, dsv, zd, cdt)
    codes = hip.qdq1("quantize", x, O.F32, qsv, zq, cdt, cdt)
    pair = hip.qdq1("dequantize", codes, cdt, dsv, zd, cdt, O.F32)
    assert np.array_equal(got.view(np.uint32), pair.view(np.uint32)), f"{tag}: fused differs from the pair"
    ref_codes = oracle_lib.qdq("quantize", x, O.F32, qsv, O.F32, zq, cdt, cdt)
    ref = oracle_lib.qdq("dequantize", ref_codes, cdt, dsv, O.F32, zd, cdt, O.F32)
    assert_bitexact(got, ref, O.F32, what=f"qdq fused {tag}")


# f16 x f16 with transB = 1 and K % 8 == 0 runs the tiled kernel (buffer loads,
# K tail masked in registers): 128x128 tiles for small grids, 256x256 tiles when
# the grid has >= 192 of them.  Ragged M / N and K % 64 != 0 exercise the edges;
# the bias modes cover the inline epilogue (none / scalar / per row / per
# column) and the out-of-line one (2-D bias).  Grids of >= 192 256x256 tiles
# with K % 64 == 0 and an inline epilogue run the direct-to-LDS kernel (the
# last four cases: ragged M / N load as zeros past the operands' ends).
F16_NT = [(300, 200, 136, "col"), (130, 1000, 8, "none"), (257, 129, 64, "scalar"), (96, 72, 520, "row"),
          (3600, 3500, 72, "col"), (3584, 3584, 200, "2d"),
          (3600, 3500, 128, "col"), (3584, 3712, 64, "row"), (3300, 3850, 192, "scalar"), (4000, 3000, 256, "none")]
# alpha = 1 takes the direct-to-LDS kernel's lean epilogue on whole blocks (the
# ragged edge blocks keep the general one): no bias, scalar and per-column bias.
F16_NT_A1 = [(3584, 3584, 128, "none"), (3600, 3500, 64, "scalar"), (3584, 3712, 192, "col")]


@pytest.mark.parametrize("M,N,K,bias,alpha", [c + (0.75,) for c in F16_NT] + [c + (1.0,) for c in F16_NT_A1],
                         ids=[f"{m}x{n}x{k}-{b}" for m, n, k, b in F16_NT] + [f"{m}x{n}x{k}-{b}-a1" for m, n, k, b in F16_NT_A1])
@pytest.mark.parametrize("ydt", ["float16", "float32"])
def test_gemm_f16_tiled_kernel(hip, M, N, K, bias, alpha, ydt):
    from tests.helpers import assert_close
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    a = rng.normal(0, 1, (M, K)).astype(np.float16)
    b = rng.normal(0, 1, (N, K)).astype(np.float16)
    c = {"none": None, "scalar": rng.normal(0, 1, (1,)), "row": rng.normal(0, 1, (M,)),
         "col": rng.normal(0, 1, (N,)), "2d": rng.normal(0, 1, (M, N))}[bias]
    if c is not None:
        c = c.astype(np.float32)
    beta = 1.5
    y = hip.gemm(a, O.F16, b, O.F16, c, O.F32, ydt, alpha, beta, 0, 1)
    rows = np.arange(M) if M * N <= 1 << 20 else np.unique(np.r_[rng.choice(M, 40, replace=False), 0, M - 1])
    ref = alpha * (a[rows].astype(np.float64) @ b.astype(np.float64).T)
    if c is not None:
        cc = {"row": lambda: c[rows].reshape(-1, 1), "2d": lambda: c[rows]}.get(bias, lambda: c.reshape(1, -1))()
        ref = ref + beta * cc.astype(np.float64)
    if ydt == "float16":
        assert_close(y[rows], O.oracle().encode_f32(ref.astype(np.float32), O.F16), O.F16,
                     what=f"f16 nt {M}x{N}x{K} {bias}")
    else:
        assert_close(y[rows], ref.astype(np.float32), O.F32, rtol=2e-5, what=f"f16 nt {M}x{N}x{K} {bias}")


# f32 x f32 Conv runs the tiled implicit GEMM: MODE 0 (gathered im2col),
# MODE 1 (1x1 / stride 1 / no padding with HW % 4 == 0) and MODE 2 (channel
# counts a multiple of 16, tap-blocked k order), 64-channel and
# 128-channel block tiles, groups, dilation, asymmetric padding, ragged channel
# and pixel counts, no bias, and a narrow output through the generic epilogue.
CONV_TILED = [
    ("gather_dil_pads", (2, 5, 13, 11), (7, 5, 3, 2), [1, 0, 2, 1], [2, 1], [1, 2], 1, True, "float32"),
    ("depthwise", (1, 8, 9, 9), (8, 1, 3, 3), [1, 1, 1, 1], [1, 1], [1, 1], 8, True, "float32"),
    ("grouped", (2, 12, 10, 9), (18, 4, 3, 3), [0, 1, 1, 0], [1, 2], [1, 1], 3, True, "float32"),
    ("direct_m160", (2, 64, 12, 12), (160, 64, 1, 1), [0, 0, 0, 0], [1, 1], [1, 1], 1, True, "float32"),
    ("direct_m32_nobias", (3, 16, 10, 10), (32, 16, 1, 1), [0, 0, 0, 0], [1, 1], [1, 1], 1, False, "float32"),
    ("1x1_hw49", (2, 16, 7, 7), (32, 16, 1, 1), [0, 0, 0, 0], [1, 1], [1, 1], 1, True, "float32"),
    ("1x1_stride2", (2, 32, 14, 14), (64, 32, 1, 1), [0, 0, 0, 0], [2, 2], [1, 1], 1, True, "float32"),
    ("3x3_m200_k1170", (1, 130, 20, 20), (200, 130, 3, 3), [1, 1, 1, 1], [1, 1], [1, 1], 1, True, "float32"),
    ("stem_like", (2, 3, 37, 41), (64, 3, 7, 7), [3, 3, 3, 3], [2, 2], [1, 1], 1, True, "float32"),
    ("f16_out", (2, 5, 13, 11), (7, 5, 3, 2), [1, 0, 2, 1], [2, 1], [1, 2], 1, True, "float16"),
    ("direct_f16_out", (2, 64, 12, 12), (160, 64, 1, 1), [0, 0, 0, 0], [1, 1], [1, 1], 1, False, "float16"),
    # few pixels, long k: the k range is split over slices reduced in a second pass
    ("split_3x3_s2", (2, 256, 14, 14), (512, 256, 3, 3), [1, 1, 1, 1], [2, 2], [1, 1], 1, True, "float32"),
    ("split_direct", (1, 512, 8, 8), (256, 512, 1, 1), [0, 0, 0, 0], [1, 1], [1, 1], 1, True, "float32"),
    ("split_grouped_nobias", (2, 256, 9, 9), (256, 128, 3, 3), [1, 1, 1, 1], [1, 1], [1, 1], 2, False, "float32"),
    ("split_ragged_k", (3, 37, 11, 11), (70, 37, 3, 3), [1, 1, 1, 1], [1, 1], [1, 1], 1, True, "float32"),
    # MODE 2 (channels a multiple of 16; (channel block, kh, kw, channel) k order):
    # 128-row tiles with ragged rows and a split k range, groups with dilation
    # and asymmetric padding, a strided 1x1 with ragged rows, a narrow output
    ("tap_m144_split", (2, 32, 16, 16), (144, 32, 3, 3), [1, 1, 1, 1], [1, 1], [1, 1], 1, True, "float32"),
    ("tap_groups_dil", (2, 32, 20, 19), (40, 16, 3, 3), [2, 1, 1, 2], [1, 1], [2, 1], 2, True, "float32"),
    ("tap_1x1_s2_m96", (3, 48, 15, 15), (96, 48, 1, 1), [0, 0, 0, 0], [2, 2], [1, 1], 1, False, "float32"),
    ("tap_m128_s2", (4, 64, 30, 30), (128, 64, 3, 3), [1, 1, 1, 1], [2, 2], [1, 1], 1, True, "float32"),
    ("tap_m160_k144", (2, 16, 24, 24), (160, 16, 3, 3), [1, 1, 1, 1], [1, 1], [1, 1], 1, True, "float32"),
    ("tap_f16_out", (2, 32, 16, 16), (40, 32, 3, 3), [1, 1, 1, 1], [1, 1], [1, 1], 1, True, "float16"),
    # 128x128 MODE 2 tiles: small images with >= 128 output channels (split k),
    # and a strided 1x1 with 256 output channels over >= 192 tiles
    ("tap_small_img_m192_split", (2, 64, 14, 14), (192, 64, 3, 3), [1, 1, 1, 1], [2, 2], [1, 1], 1, True, "float32"),
    ("tap_1x1_m256_wide", (12, 16, 64, 64), (256, 16, 1, 1), [0, 0, 0, 0], [2, 2], [1, 1], 1, True, "float32"),
    ("tap_groups_m128_split", (1, 64, 10, 10), (256, 32, 3, 3), [1, 1, 1, 1], [1, 1], [1, 1], 2, True, "float32"),
    # the 3-channel 7x7 / stride-2 stem plan (whole k range in LDS): a second, partial
    # channel tile; asymmetric padding without bias
    ("stem_plan_m80", (2, 3, 20, 180), (80, 3, 7, 7), [3, 3, 3, 3], [2, 2], [1, 1], 1, True, "float32"),
    # one partial channel tile (the weights-resident-in-LDS form with channels past M)
    ("stem_plan_m40", (2, 3, 20, 180), (40, 3, 7, 7), [3, 3, 3, 3], [2, 2], [1, 1], 1, True, "float32"),
    # a single tile (one busy block in the persistent grid)
    ("stem_plan_one_tile", (1, 3, 3, 224), (64, 3, 7, 7), [3, 3, 3, 3], [2, 2], [1, 1], 1, True, "float32"),
    ("stem_plan_asym_nobias", (1, 3, 17, 224), (64, 3, 7, 7), [2, 3, 4, 1], [2, 2], [1, 1], 1, False, "float32"),
    # direct 1x1 layers of the config-4 shape class (64 input channels, 256 and 512
    # output channels)
    ("direct_m256", (2, 64, 16, 16), (256, 64, 1, 1), [0, 0, 0, 0], [1, 1], [1, 1], 1, True, "float32"),
    ("direct_m512_nobias", (3, 64, 14, 16), (512, 64, 1, 1), [0, 0, 0, 0], [1, 1], [1, 1], 1, False, "float32"),
]


@pytest.mark.parametrize("case", CONV_TILED, ids=[c[0] for c in CONV_TILED])
def test_conv_tiled_kernel(hip, oracle_lib, case):
    from tests.helpers import assert_close
    tag, xs, ws, pads, strides, dil, group, has_b, ydt = case
    rng = np.random.default_rng(len(tag) * 131 + xs[1])
    x = rng.normal(0, 1, xs).astype(np.float32)
    w = rng.normal(0, np.sqrt(2 / (ws[1] * ws[2] * ws[3])), ws).astype(np.float32)
    b = rng.normal(0, 1, (ws[0],)).astype(np.float32) if has_b else None
    got = hip.conv(x, O.F32, w, O.F32, b, O.F32, ydt, pads, strides, dil, group)
    ref = oracle_lib.conv(x, O.F32, w, O.F32, b, O.F32, ydt, pads, strides, dil, group)
    assert_close(got, ref, ydt, what=f"conv {tag}")


# conv2d_fused_forward = conv2d_forward -> relu_forward -> add_forward(., Skip)
# bit for bit, through the kernel epilogue (gather, direct 1x1 and split-k
# paths, with / without bias, Relu only, Skip only) and through the fallbacks
# (f16 output, broadcast Skip, exact mode); and close to the oracle's sequence.
CONV_FUSED = [
    ("gather_relu_skip", (2, 16, 13, 11), (24, 16, 3, 3), [1, 1, 1, 1], [1, 1], 1, True, True, "full", "float32"),
    ("direct_relu_skip", (2, 64, 12, 12), (96, 64, 1, 1), [0, 0, 0, 0], [1, 1], 1, True, True, "full", "float32"),
    ("split_relu_skip", (2, 256, 14, 14), (512, 256, 3, 3), [1, 1, 1, 1], [2, 2], 1, True, True, "full", "float32"),
    ("stem_relu_only", (2, 3, 37, 41), (64, 3, 7, 7), [3, 3, 3, 3], [2, 2], 1, True, True, None, "float32"),
    ("skip_only_nobias", (2, 12, 10, 9), (18, 4, 3, 3), [0, 1, 1, 0], [1, 2], 3, False, False, "full", "float32"),
    ("tail_rows_m200", (1, 30, 9, 9), (200, 30, 3, 3), [1, 1, 1, 1], [1, 1], 1, True, True, "full", "float32"),
    ("f16_out_fallback", (2, 5, 13, 11), (7, 5, 3, 2), [1, 0, 2, 1], [2, 1], 1, True, True, "full", "float16"),
    ("bcast_skip_fallback", (2, 16, 13, 11), (24, 16, 3, 3), [1, 1, 1, 1], [1, 1], 1, True, True, "chan", "float32"),
    ("tap_split_relu_skip", (2, 32, 16, 16), (144, 32, 3, 3), [1, 1, 1, 1], [1, 1], 1, True, True, "full", "float32"),
    ("tap_m128_relu_skip", (4, 64, 30, 30), (128, 64, 3, 3), [1, 1, 1, 1], [2, 2], 1, True, True, "full", "float32"),
    ("tap_small_img_relu_skip", (2, 64, 14, 14), (192, 64, 3, 3), [1, 1, 1, 1], [2, 2], 1, True, True, "full", "float32"),
    ("stem_plan_relu_skip", (2, 3, 20, 180), (64, 3, 7, 7), [3, 3, 3, 3], [2, 2], 1, True, True, "full", "float32"),
    ("stem_plan_m40_skip", (2, 3, 20, 180), (40, 3, 7, 7), [3, 3, 3, 3], [2, 2], 1, True, False, "full", "float32"),
    ("stem_plan_one_tile_relu", (1, 3, 3, 224), (64, 3, 7, 7), [3, 3, 3, 3], [2, 2], 1, True, True, None, "float32"),
    ("stem_plan_m80_relu_skip", (2, 3, 20, 180), (80, 3, 7, 7), [3, 3, 3, 3], [2, 2], 1, True, True, "full", "float32"),
    ("direct_m256_relu_skip", (2, 64, 16, 16), (256, 64, 1, 1), [0, 0, 0, 0], [1, 1], 1, True, True, "full", "float32"),
    ("direct_m512_skip_nobias", (1, 64, 8, 32), (512, 64, 1, 1), [0, 0, 0, 0], [1, 1], 1, False, False, "full", "float32"),
]


@pytest.mark.parametrize("case", CONV_FUSED, ids=[c[0] for c in CONV_FUSED])
@pytest.mark.parametrize("exact", [False, True], ids=["mfma", "exact"])
def test_conv_fused_epilogue(hip, oracle_lib, case, exact):
    from tests.helpers import assert_close
    tag, xs, ws, pads, strides, group, has_b, relu, skip_kind, ydt = case
    rng = np.random.default_rng(len(tag) * 17 + xs[1])
    x = rng.normal(0, 1, xs).astype(np.float32)
    w = rng.normal(0, np.sqrt(2 / (ws[1] * ws[2] * ws[3])), ws).astype(np.float32)
    b = rng.normal(0, 1, (ws[0],)).astype(np.float32) if has_b else None
    y0 = oracle_lib.conv(x, O.F32, w, O.F32, b, O.F32, O.F32, pads, strides, [1, 1], group)
    skip = None
    if skip_kind == "full":
        skip = rng.normal(0, 1, y0.shape).astype(np.float32)
    elif skip_kind == "chan":
        skip = rng.normal(0, 1, (y0.shape[1], 1, 1)).astype(np.float32)
    if ydt == "float16" and skip is not None:
        skip = skip.astype(np.float16).view(np.uint16)
    sdt = ydt
    hip.set_exact(exact)
    try:
        got = hip.conv_fused(x, w, b, skip, relu, ydt, pads, strides, [1, 1], group, skip_dt=sdt)
        seq = hip.conv(x, O.F32, w, O.F32, b, O.F32, ydt, pads, strides, [1, 1], group)
        if relu:
            seq = hip.unary("relu", seq, ydt, ydt)
        if skip is not None:
            seq = hip.binary("add", seq, ydt, skip, sdt, ydt)
    finally:
        hip.set_exact(False)
    assert np.array_equal(got.view(np.uint8), seq.view(np.uint8)), f"{tag}: fused differs from the sequence"
    ref = oracle_lib.conv(x, O.F32, w, O.F32, b, O.F32, ydt, pads, strides, [1, 1], group)
    if relu:
        ref = oracle_lib.unary("relu", ref, ydt, ydt)
    if skip is not None:
        ref = oracle_lib.binary("add", ref, ydt, skip, sdt, ydt)
    assert_close(got, ref, ydt, what=f"conv fused {tag}")


# conv2d_fused_qdq_forward = conv2d_fused_forward -> quantize_dequantize_linear_forward
# bit for bit on every conv plan: tap-blocked tiles (64x128, 128x128, 128x256), the
# split-k reductions (16-byte and scalar), the gather and direct 1x1 plans, the
# generic epilogue of partial channel tiles, the stem plan (fake quantization in a
# second pass), and the sequence fallbacks (fp8 codes, exact mode).  Output channel 0
# has zero weights and bias, so with Relu its value is the skip tensor's, which holds
# rint ties and non-finite values there (the fp64 fallback of the quantize step).
CONV_QDQ = [
    ("tap_u8_relu_skip", (2, 64, 28, 28), (64, 64, 3, 3), [1, 1, 1, 1], [1, 1], "uint8", 0, 8 / 255, 0, 8 / 255),
    ("tap_i8_m128_s2", (2, 64, 30, 30), (128, 64, 3, 3), [1, 1, 1, 1], [2, 2], "int8", -3, 0.05, 2, 0.04),
    ("tap_m256_small_img", (2, 128, 14, 14), (256, 128, 3, 3), [1, 1, 1, 1], [2, 2], "uint8", 3, 0.03, 3, 0.03),
    ("split4_u8", (2, 256, 14, 14), (512, 256, 3, 3), [1, 1, 1, 1], [2, 2], "uint8", 0, 8 / 255, 0, 8 / 255),
    ("split_scalar_i8", (1, 256, 9, 9), (129, 256, 3, 3), [1, 1, 1, 1], [2, 2], "int8", 0, 0.05, 0, 0.05),
    ("gather_u8", (2, 12, 13, 11), (24, 12, 3, 3), [1, 1, 1, 1], [1, 1], "uint8", 9, 0.02, 9, 0.02),
    ("direct_1x1_u8", (2, 40, 12, 12), (96, 40, 1, 1), [0, 0, 0, 0], [1, 1], "uint8", 0, 0.04, 0, 0.04),
    ("direct_m256_i8", (2, 64, 16, 16), (256, 64, 1, 1), [0, 0, 0, 0], [1, 1], "int8", 2, 0.04, 2, 0.04),
    ("tail_rows_m200_i8", (1, 30, 9, 9), (200, 30, 3, 3), [1, 1, 1, 1], [1, 1], "int8", 1, 0.03, 1, 0.03),
    ("stem_u8", (2, 3, 20, 180), (64, 3, 7, 7), [3, 3, 3, 3], [2, 2], "uint8", 0, 8 / 255, 0, 8 / 255),
    ("e4m3_fallback", (2, 64, 12, 12), (64, 64, 3, 3), [1, 1, 1, 1], [1, 1], "float8_e4m3", 0, 0.01, 0, 0.01),
]


@pytest.mark.parametrize("case", CONV_QDQ, ids=[c[0] for c in CONV_QDQ])
@pytest.mark.parametrize("exact", [False, True], ids=["mfma", "exact"])
def test_conv_fused_qdq(hip, oracle_lib, case, exact):
    tag, xs, ws, pads, strides, cdt, qz, qs, dz, ds = case
    rng = np.random.default_rng(len(tag) * 13 + ws[0])
    x = rng.normal(0, 1, xs).astype(np.float32)
    w = rng.normal(0, np.sqrt(2 / (ws[1] * ws[2] * ws[3])), ws).astype(np.float32)
    b = rng.normal(0, 0.1, (ws[0],)).astype(np.float32)
    w[0], b[0] = 0.0, 0.0
    OH = (xs[2] + pads[0] + pads[2] - ws[2]) // strides[0] + 1
    OW = (xs[3] + pads[1] + pads[3] - ws[3]) // strides[1] + 1
    skip = rng.normal(0, 1, (xs[0], ws[0], OH, OW)).astype(np.float32)
    c0 = skip[0, 0].reshape(-1)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e30, -1e30], np.float32)
    c0[:7] = specials
    ties = ((np.arange(-16, 16) + 0.5) * np.float32(qs)).astype(np.float32)
    c0[7:7 + min(32, c0.size - 7)] = ties[:c0.size - 7]
    npz = {"int8": np.int8, "uint8": np.uint8}.get(cdt, np.uint8)
    qsv, dsv = np.array([qs], np.float32), np.array([ds], np.float32)
    zq, zd = np.array([qz], npz), np.array([dz], npz)
    hip.set_exact(exact)
    try:
        got = hip.conv_fused_qdq(x, w, b, skip, True, qsv, zq, dsv, zd, cdt, pads, strides)
        y = hip.conv_fused(x, w, b, skip, True, "float32", pads, strides)
        seq = hip.qdq_fused(y, qsv, zq, dsv, zd, cdt)
    finally:
        hip.set_exact(False)
    assert np.array_equal(got.view(np.uint32), seq.view(np.uint32)), f"{tag}: fused differs from the sequence"
    # against the oracle: Conv -> Relu -> Add -> QuantizeLinear -> DequantizeLinear
    yr = oracle_lib.conv(x, O.F32, w, O.F32, b, O.F32, O.F32, pads, strides, [1, 1], 1)
    yr = oracle_lib.binary("add", oracle_lib.unary("relu", yr, O.F32, O.F32), O.F32, skip, O.F32, O.F32)
    codes = oracle_lib.qdq("quantize", yr, O.F32, qsv, O.F32, zq, cdt, cdt)
    ref = oracle_lib.qdq("dequantize", codes, cdt, dsv, O.F32, zd, cdt, O.F32)
    if exact:
        assert_bitexact(got, ref, O.F32, what=f"conv qdq {tag}")
    else:
        # fp32 MFMA accumulation moves a few values across a rounding boundary of
        # the quantizer: those differ by one code step, everything else is exact
        assert_bitexact(got[0, 0], ref[0, 0], O.F32, what=f"conv qdq {tag} channel 0")
        fin = np.isfinite(ref)
        assert np.array_equal(np.isfinite(got), fin)
        diff = np.abs(got[fin].astype(np.float64) - ref[fin])
        if not cdt.startswith("float8"):   # integer codes: one step of the dequantize scale
            assert diff.max() <= np.float64(np.float32(ds)) * 1.0001
        assert (diff > 0).mean() < 0.01, f"{tag}: {(diff > 0).mean():.4f} of the values differ"


# Config-5 sizes (batch 64): block 1's 3x3 conv (full grid of 64x128 tap-blocked tiles)
# and block 3's strided 3x3 conv (5 k-slices and the 16-byte reduction) with the Relu,
# residual and fake quantization of the graph; fused == sequence bit for bit.
CONV_QDQ_FULL = [("block1", (64, 64, 56, 56), (64, 64, 3, 3), [1, 1]),
                 ("block3", (64, 128, 28, 28), (256, 128, 3, 3), [2, 2])]


@pytest.mark.parametrize("case", CONV_QDQ_FULL, ids=[c[0] for c in CONV_QDQ_FULL])
def test_conv_fused_qdq_config5_size(hip, case):
    tag, xs, ws, strides = case
    rng = np.random.default_rng(xs[1] + ws[0])
    x = np.maximum(rng.normal(0, 1, xs), 0).astype(np.float32)
    w = rng.normal(0, np.sqrt(2 / (ws[1] * 9)), ws).astype(np.float32)
    b = rng.normal(0, 1 / 64, (ws[0],)).astype(np.float32)
    OH = (xs[2] + 2 - 3) // strides[0] + 1
    skip = rng.normal(0, 1, (xs[0], ws[0], OH, OH)).astype(np.float32)
    qs, zp = np.array([8 / 255], np.float32), np.array([0], np.uint8)
    got = hip.conv_fused_qdq(x, w, b, skip, True, qs, zp, qs, zp, "uint8", [1, 1, 1, 1], strides)
    y = hip.conv_fused(x, w, b, skip, True, "float32", [1, 1, 1, 1], strides)
    seq = hip.qdq_fused(y, qs, zp, qs, zp, "uint8")
    assert np.array_equal(got.view(np.uint32), seq.view(np.uint32)), f"{tag}: fused differs from the sequence"
    # the fake-quantized values are multiples of the scale in [0, 255 * scale]
    codes = got / np.float32(8 / 255)
    assert np.all(np.abs(codes - np.rint(codes)) < 1e-3) and got.min() >= 0 and got.max() <= 8.0 + 1e-6
    assert (got > 0).mean() > 0.3


# max_pool_qdq_forward: Y = max_pool_forward(X) and Yq = quantize_dequantize_linear_forward(Y)
# bit for bit (the strip kernel for 3x3 / stride 2, the sequence otherwise), and equal to
# the oracle's MaxPool -> QuantizeLinear -> DequantizeLinear (all three are exact).
POOL_QDQ = [
    ("strip_u8_stem_shape", (2, 64, 112, 112), (3, 3), [1, 1, 1, 1], [2, 2], "uint8", 0, 8 / 255, 0, 8 / 255),
    ("strip_i8_odd", (3, 5, 21, 22), (3, 3), [1, 1, 1, 1], [2, 2], "int8", -7, 0.02, 4, 0.03),
    ("rows_fallback_u8", (2, 4, 17, 19), (2, 2), [0, 0, 0, 0], [2, 2], "uint8", 5, 0.05, 5, 0.05),
    ("e5m2_fallback", (2, 4, 16, 16), (3, 3), [1, 1, 1, 1], [2, 2], "float8_e5m2", 0, 0.25, 0, 0.25),
]


@pytest.mark.parametrize("case", POOL_QDQ, ids=[c[0] for c in POOL_QDQ])
def test_maxpool_qdq(hip, oracle_lib, case):
    tag, xs, ks, pads, strides, cdt, qz, qs, dz, ds = case
    rng = np.random.default_rng(len(tag) + xs[1])
    x = rng.normal(0, 2, xs).astype(np.float32)
    flat = x[0, 0].reshape(-1)
    flat[:7] = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1e30, -1e30]
    # rint ties where they survive the max: whole plane 1 of image 0 at tie values
    x[0, 1] = ((rng.integers(-40, 40, xs[2:]) + 0.5) * np.float32(qs)).astype(np.float32)
    npz = {"int8": np.int8, "uint8": np.uint8}.get(cdt, np.uint8)
    qsv, dsv = np.array([qs], np.float32), np.array([ds], np.float32)
    zq, zd = np.array([qz], npz), np.array([dz], npz)
    y, yq = hip.maxpool_qdq(x, ks, pads, strides, qsv, zq, dsv, zd, cdt)
    y1 = hip.maxpool(x, O.F32, O.F32, ks, pads, strides)
    assert np.array_equal(y.view(np.uint32), y1.view(np.uint32)), f"{tag}: Y differs from max_pool_forward"
    seq = hip.qdq_fused(y1, qsv, zq, dsv, zd, cdt)
    assert np.array_equal(yq.view(np.uint32), seq.view(np.uint32)), f"{tag}: Yq differs from the sequence"
    ry = oracle_lib.maxpool(x, O.F32, O.F32, ks, pads, strides)
    codes = oracle_lib.qdq("quantize", ry, O.F32, qsv, O.F32, zq, cdt, cdt)
    ref = oracle_lib.qdq("dequantize", codes, cdt, dsv, O.F32, zd, cdt, O.F32)
    assert_bitexact(y, ry, O.F32, what=f"maxpool qdq {tag} Y")
    assert_bitexact(yq, ref, O.F32, what=f"maxpool qdq {tag} Yq")


# dequantize_conv2d_fused_forward = dequantize_linear_forward -> conv2d_fused_forward
# bit for bit: uint8 / int8 codes read by the gather (zero points that make the
# padding taps differ from (0 - zp) * s), the direct 1x1 path, the split-k path,
# stride / groups, no zero point; and the fallbacks (exact mode, a per-channel
# scale).  Against the oracle: DequantizeLinear then Conv / Relu / Add.
DQ_CONV = [
    ("u8_pad_relu_skip", (2, 16, 13, 11), "uint8", 37, (24, 16, 3, 3), [1, 1, 1, 1], [1, 1], 1, True, True, True),
    ("i8_pad", (2, 8, 9, 10), "int8", -5, (12, 8, 3, 3), [1, 0, 2, 1], [2, 1], 1, True, False, False),
    ("u8_direct_1x1", (2, 64, 12, 12), "uint8", 128, (96, 64, 1, 1), [0, 0, 0, 0], [1, 1], 1, True, True, True),
    ("u8_split", (2, 256, 14, 14), "uint8", 3, (512, 256, 3, 3), [1, 1, 1, 1], [2, 2], 1, True, True, True),
    ("u8_groups_nozp", (2, 12, 10, 9), "uint8", None, (18, 4, 3, 3), [0, 1, 1, 0], [1, 2], 3, False, True, False),
    ("u8_stride2_proj", (2, 32, 14, 14), "uint8", 0, (64, 32, 1, 1), [0, 0, 0, 0], [2, 2], 1, False, False, False),
    ("u8_tap_split", (2, 32, 16, 16), "uint8", 7, (144, 32, 3, 3), [1, 1, 1, 1], [1, 1], 1, True, True, True),
    ("i8_tap_m128_s2", (4, 64, 30, 30), "int8", -3, (128, 64, 3, 3), [1, 1, 1, 1], [2, 2], 1, True, True, False),
    ("u8_tap_small_img", (2, 64, 14, 14), "uint8", 9, (192, 64, 3, 3), [1, 1, 1, 1], [2, 2], 1, True, True, True),
    ("u8_stem_shape", (2, 3, 20, 180), "uint8", 5, (64, 3, 7, 7), [3, 3, 3, 3], [2, 2], 1, True, True, False),
]


@pytest.mark.parametrize("case", DQ_CONV, ids=[c[0] for c in DQ_CONV])
@pytest.mark.parametrize("mode", ["mfma", "exact", "per_channel_fallback"])
def test_dequantize_conv_fused(hip, oracle_lib, case, mode):
    import ctypes
    from tests.helpers import assert_close
    tag, xs, xdt, zp, ws, pads, strides, group, has_b, relu, has_skip = case
    rng = np.random.default_rng(len(tag) * 29 + xs[1])
    lo, hi = (0, 256) if xdt == "uint8" else (-128, 128)
    xq = rng.integers(lo, hi, xs).astype(np.uint8 if xdt == "uint8" else np.int8)
    sc = np.array([0.037], np.float32)
    z = None if zp is None else np.array([zp], xq.dtype)
    w = rng.normal(0, np.sqrt(2 / (ws[1] * ws[2] * ws[3])), ws).astype(np.float32)
    b = rng.normal(0, 1, (ws[0],)).astype(np.float32) if has_b else None
    # dequantised input, as DequantizeLinear writes it (the oracle)
    zz = z if z is not None else np.zeros(1, xq.dtype)
    if mode == "per_channel_fallback":
        sc = (0.02 + 0.01 * rng.random(xs[1])).astype(np.float32)
        zz = np.full(xs[1], zp if zp is not None else 0, xq.dtype)
        z = zz
        xd = oracle_lib.qdq("dequantize", xq, xdt, sc.reshape(1, -1, 1, 1), O.F32, zz.reshape(1, -1, 1, 1), xdt, O.F32)
    else:
        xd = oracle_lib.qdq("dequantize", xq, xdt, sc, O.F32, zz, xdt, O.F32)
    y0 = oracle_lib.conv(xd, O.F32, w, O.F32, b, O.F32, O.F32, pads, strides, [1, 1], group)
    skip = rng.normal(0, 1, y0.shape).astype(np.float32) if has_skip else None
    hip.set_exact(mode == "exact")
    try:
        if mode == "per_channel_fallback":
            with pytest.raises(RuntimeError):
                # a 1-D per-channel scale does not broadcast against [N, C, H, W] in
                # DequantizeLinear (numpy alignment): the sequence reports the error
                hip.dq_conv_fused(xq, xdt, sc, z, w, b, skip, relu, pads, strides, [1, 1], group)
            return
        got = hip.dq_conv_fused(xq, xdt, sc, z, w, b, skip, relu, pads, strides, [1, 1], group)
        xdh = hip.qdq("dequantize", xq, xdt, sc, O.F32, zz, xdt, O.F32)
        seq = hip.conv_fused(xdh, w, b, skip, relu, O.F32, pads, strides, [1, 1], group)
    finally:
        hip.set_exact(False)
    assert np.array_equal(xdh, xd), f"{tag}: DequantizeLinear differs from the oracle"
    assert np.array_equal(got.view(np.uint32), seq.view(np.uint32)), f"{tag}: fused differs from the sequence"
    ref = y0
    if relu:
        ref = oracle_lib.unary("relu", ref, O.F32, O.F32)
    if skip is not None:
        ref = oracle_lib.binary("add", ref, O.F32, skip, O.F32, O.F32)
    assert_close(got, ref, O.F32, what=f"dq conv {tag}")


# Grids of >= 256 tiles take the store-first MODE 2 pipeline without a k
# split: 64x256 tiles for 64 output channels, 128x256 for >= 128; f32 input and
# uint8 / int8 codes dequantised in the gather.
D3_PLANS = [("f32_m256_128x256", (8, 16, 64, 64), (256, 16, 3, 3), None),
            ("u8_m64_64x256", (16, 16, 64, 64), (64, 16, 3, 3), "uint8"),
            ("i8_m256_128x256", (8, 16, 64, 64), (256, 16, 3, 3), "int8")]


@pytest.mark.parametrize("case", D3_PLANS, ids=[c[0] for c in D3_PLANS])
def test_conv_store_first_plans(hip, oracle_lib, case):
    from tests.helpers import assert_close
    tag, xs, ws, xdt = case
    rng = np.random.default_rng(len(tag) + xs[0])
    w = rng.normal(0, np.sqrt(2 / (ws[1] * 9)), ws).astype(np.float32)
    b = rng.normal(0, 1, (ws[0],)).astype(np.float32)
    pads, strides = [1, 1, 1, 1], [1, 1]
    if xdt is None:
        x = rng.normal(0, 1, xs).astype(np.float32)
        got = hip.conv(x, O.F32, w, O.F32, b, O.F32, "float32", pads, strides, [1, 1], 1)
    else:
        lo, hi = (0, 256) if xdt == "uint8" else (-128, 128)
        xq = rng.integers(lo, hi, xs).astype(np.uint8 if xdt == "uint8" else np.int8)
        sc, z = np.array([0.029], np.float32), np.array([3 if xdt == "uint8" else -2], xq.dtype)
        x = oracle_lib.qdq("dequantize", xq, xdt, sc, O.F32, z, xdt, O.F32)
        got = hip.dq_conv_fused(xq, xdt, sc, z, w, b, None, False, pads, strides, [1, 1], 1)
        seq = hip.conv_fused(hip.qdq("dequantize", xq, xdt, sc, O.F32, z, xdt, O.F32), w, b, None, False, O.F32,
                             pads, strides, [1, 1], 1)
        assert np.array_equal(got.view(np.uint32), seq.view(np.uint32)), f"{tag}: fused differs from the sequence"
    ref = oracle_lib.conv(x, O.F32, w, O.F32, b, O.F32, O.F32, pads, strides, [1, 1], 1)
    assert_close(got, ref, O.F32, what=f"conv {tag}")


def test_device_path_matches_host_path(hip):
    """Config-1 chain with device-resident tensors (no host round trips between ops)."""
    from onnx_translator_amd.nn import Tensor
    from onnx_translator_amd.nn.Operators import ABS, ADD, COS, DIV, MUL, RELU, SUB
    rng = np.random.default_rng(0)
    A = rng.uniform(-4, 4, (2, 64, 14, 14)).astype(np.float32)
    B = rng.uniform(-4, 4, (64, 1, 1)).astype(np.float32)
    Bd = (np.sign(B) * np.maximum(np.abs(B), 0.1)).astype(np.float32)
    ta, tb, tbd = [Tensor(*x.shape, dtype="float32", data=x) for x in (A, B, Bd)]

    def chain(a, b, bd):
        t = ADD([], [], "float32").forward(a, b)["tensor"]
        t = MUL([], [], "float32").forward(t, b)["tensor"]
        t = SUB([], [], "float32").forward(t, b)["tensor"]
        t = DIV([], [], "float32").forward(t, bd)["tensor"]
        t = RELU([], [], "float32").forward(t)["tensor"]
        t = ABS([], [], "float32").forward(t)["tensor"]
        return COS([], [], "float32").forward(t)["tensor"]

    host = chain(ta, tb, tbd)
    dev = chain(ta.to_device(), tb.to_device(), tbd.to_device())
    assert dev.on_device and not host.on_device
    assert_bitexact(dev.numpy(), host.numpy(), O.F32, what="device chain")
    # and against the oracle, op by op on the host
    o = O.oracle()
    t = o.binary("add", A, O.F32, B, O.F32, O.F32)
    t = o.binary("mul", t, O.F32, B, O.F32, O.F32)
    t = o.binary("sub", t, O.F32, B, O.F32, O.F32)
    t = o.binary("div", t, O.F32, Bd, O.F32, O.F32)
    t = o.unary("cos", o.unary("abs", o.unary("relu", t, O.F32, O.F32), O.F32, O.F32), O.F32, O.F32)
    assert_bitexact(host.numpy(), t, O.F32, what="host chain vs oracle")


def test_operator_layer_qdq_axis_and_gemm(hip):
    from onnx_translator_amd.nn import Tensor
    from onnx_translator_amd.nn.Operators import DequantizeLinear, Gemm, QuantizeLinear, Softmax
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1.5, (4, 16, 64)).astype(np.float32)
    s = (np.abs(x).max(axis=(0, 2)) / 127).astype(np.float32)
    z = np.zeros(16, np.int8)
    X = Tensor(*x.shape, dtype="float32", data=x)
    S = Tensor(16, dtype="float32", data=s)
    Z = Tensor(16, dtype="int8", data=z)
    for dev in (False, True):
        xs, ss, zs = (X.to_device(), S.to_device(), Z.to_device()) if dev else (X, S, Z)
        y = QuantizeLinear([], [], axis=1, dtype="int8").forward(xs, ss, zs)["tensor"]
        xr = DequantizeLinear([], [], dtype="float32", axis=1).forward(y, ss, zs)["tensor"]
        ref_y = O.oracle().qdq("quantize", x, O.F32, s.reshape(1, 16, 1), O.F32, z.reshape(1, 16, 1), O.I8, O.I8)
        assert_bitexact(y.numpy(), ref_y, O.I8, what="q axis")
        ref_x = O.oracle().qdq("dequantize", ref_y, O.I8, s.reshape(1, 16, 1), O.F32, z.reshape(1, 16, 1), O.I8,
                               O.F32)
        assert_bitexact(xr.numpy(), ref_x, O.F32, what="dq axis")
    a = rng.normal(0, 1, (33, 70)).astype(np.float32)
    b = rng.normal(0, 1, (17, 70)).astype(np.float32)
    c = rng.normal(0, 1, (17,)).astype(np.float32)
    g = Gemm([], [], 1.0, 1.0, 0, 1, "float32").forward(
        Tensor(*a.shape, data=a), Tensor(*b.shape, data=b), Tensor(17, data=c))["tensor"]
    np.testing.assert_allclose(g.numpy(), a.astype(np.float64) @ b.T.astype(np.float64) + c, rtol=1e-5,
                               atol=1e-5)
    sm = Softmax([], [], axis=1, dtype="float32").forward(Tensor(*a.shape, data=a))["tensor"].numpy()
    np.testing.assert_allclose(sm.sum(axis=1), 1.0, rtol=1e-5)


def test_errors_are_reported_not_faulted(hip):
    with pytest.raises(RuntimeError, match="broadcast"):
        hip._run(hip.lib.add_forward, [(np.ones((3, 4), np.float32), O.F32), (np.ones((5,), np.float32), O.F32)],
                 (3, 4), O.F32)
    with pytest.raises(RuntimeError, match="inner dimensions"):
        hip._run(hip.lib.gemm_forward, [(np.ones((4, 5), np.float32), O.F32), (np.ones((6, 7), np.float32), O.F32),
                                        (None, O.F32)], (4, 7), O.F32, ctypes.c_float(1), ctypes.c_float(0), 0, 0)
    with pytest.raises(RuntimeError, match="sizes differ"):
        hip._run(hip.lib.relu_forward, [(np.ones(5, np.float32), O.F32)], (6,), O.F32)
    # the library still works afterwards
    out = hip.unary("relu", np.array([-1.0, 2.0], np.float32), O.F32, O.F32)
    assert out.tolist() == [0.0, 2.0]


def test_zero_size_tensors(hip):
    out = hip.binary("add", np.zeros((0, 3), np.float32), O.F32, np.zeros((0, 3), np.float32), O.F32, O.F32)
    assert out.shape == (0, 3)


@pytest.mark.gpu
@pytest.mark.parametrize("against", ["reference", "oracle"])
@pytest.mark.parametrize("exact", [False, True], ids=["mfma", "exact"])
def test_verifier_plans(hip, oracle_lib, exact, against):
    """The verifier harness (tests/verify.py) over all 45 reference plans with
    fresh seeded inputs: every iteration inside its parity class, against the
    reference's own tensor_ops.c (oracle/_ref, compiled from its source) and
    against the restatement."""
    from tests.verify import verify
    truth = oracle_lib
    if against == "reference":
        truth = O.reference()
        if truth is None:
            pytest.skip("oracle/_ref/tensor_ops.so not built (the reference source was absent at build time)")
    failures, stats = verify(hip, truth, iterations=3, seed=7, exact=exact, log=lambda *a: None)
    assert not failures, failures[:3]
    assert sum(len(s["abs"]) for s in stats.values()) == 45 * 3
