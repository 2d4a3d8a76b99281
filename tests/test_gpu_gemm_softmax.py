"""gemm_softmax_forward against gemm_forward followed by softmax_forward over the
last axis (reference: tensor_ops.c:1167-1228 then :1231-1270), bit for bit on both
outputs: the k-split path whose reduction takes the softmax (the config-5 head,
[64,512] x [1000,512]^T with a per-column bias), shapes that run the two calls
(no split, rows longer than one block), scalar and absent biases, alpha / beta
other than 1, and rows with infinite and NaN logits."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu

# name, M, K, N, bias ("col", "one", None), alpha, beta, poison (inf / nan rows in A)
CASES = [
    ("head_config5", 64, 512, 1000, "col", 1.0, 1.0, False),
    ("head_alpha_beta", 64, 512, 1000, "col", 0.75, -1.5, False),
    ("split_no_bias", 32, 1024, 256, None, 1.0, 1.0, False),
    ("split_scalar_bias_nonfinite", 64, 512, 1000, "one", 1.0, 1.0, True),
    ("no_split_small", 8, 64, 100, "col", 1.0, 1.0, False),
    ("rows_past_block", 16, 512, 1500, "col", 1.0, 1.0, False),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_gemm_softmax_matches_the_two_calls(hip, oracle_lib, case):
    name, M, K, N, bias, alpha, beta, poison = case
    L = hip.lib
    L.gemm_forward.argtypes = [O.PT] * 4 + [ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int]
    L.gemm_softmax_forward.argtypes = [O.PT] * 5 + [ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int]
    L.softmax_forward.argtypes = [O.PT, O.PT, ctypes.c_int]
    rng = np.random.default_rng(M + K + N)
    a = rng.normal(0, 1, (M, K)).astype(np.float32)
    if poison:
        a[3, 7] = np.inf
        a[5, :] = -np.inf
        a[9, 11] = np.nan
    b = rng.normal(0, 1 / np.sqrt(K), (N, K)).astype(np.float32)
    c = None if bias is None else rng.normal(0, 0.1, (N,) if bias == "col" else (1,)).astype(np.float32)
    from tests.test_gpu_qconv import _Dev, _bind
    _bind(L)
    dev = _Dev(hip)
    try:
        ta, tb = dev.put(a, O.F32), dev.put(b, O.F32)
        tc = dev.put(c, O.F32) if c is not None else O.PT()
        y1, p1 = dev.empty((M, N), O.F32), dev.empty((M, N), O.F32)
        L.tensor_ops_hip_clear_error()
        L.gemm_forward(ta, tb, tc, y1, alpha, beta, 0, 1)
        L.softmax_forward(y1, p1, 1)
        assert not hip.last_error(), hip.last_error()
        with hip.poisoned():
            y2, p2 = dev.output((M, N), O.F32), dev.output((M, N), O.F32)
            L.gemm_softmax_forward(ta, tb, tc, y2, p2, alpha, beta, 0, 1)
        assert not hip.last_error(), hip.last_error()
        ry, rp = hip.dev_read(y1, O.F32), hip.dev_read(p1, O.F32)
        assert_bitexact(hip.dev_read(y2, O.F32), ry, O.F32, what=f"{name} logits")
        assert_bitexact(hip.dev_read(p2, O.F32), rp, O.F32, what=f"{name} softmax")
        if not poison:
            # and the pair itself within the MFMA tolerance of the compiled reference
            ref_y = oracle_lib.gemm(a, O.F32, b, O.F32, c, O.F32, O.F32, alpha, beta, 0, 1)
            assert_close(ry, ref_y, O.F32, what=f"{name} gemm vs oracle")
    finally:
        dev.free()
