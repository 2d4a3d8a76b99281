"""dynamic_quantize_linear_forward_noalloc: the no-allocation variant of
dynamic_quantize_linear_forward (its min / max partials live in a file-scope
device array instead of the HBM pool).  Called through the C ABI on device
tensors, it must return the existing entry point's outputs bit for bit, on two
calls in a row (the second with a smaller input, so it reuses the scratch the
first one left behind); host tensors are refused with an error.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_bitexact

pytestmark = pytest.mark.gpu


def _dql(hip, fn, x):
    L = hip.lib
    tx = hip.dev_from(x, O.F32)
    ty = hip.dev_empty(x.shape, O.U8)
    ts, tz = hip.dev_empty((1,), O.F32), hip.dev_empty((1,), O.U8)
    try:
        L.tensor_ops_hip_clear_error()
        fn(tx, ty, ts, tz)
        err = hip.last_error()
        assert not err, err
        return hip.dev_read(ty, O.U8), hip.dev_read(ts, O.F32), hip.dev_read(tz, O.U8)
    finally:
        for t in (tx, ty, ts, tz):
            L.free_tensor(t)


def test_noalloc_matches_dynamic_quantize_linear(hip, oracle_lib):
    L = hip.lib
    L.dynamic_quantize_linear_forward_noalloc.argtypes = [O.PT, O.PT, O.PT, O.PT]
    rng = np.random.default_rng(9)
    big = rng.normal(0, 1.5, (32, 512, 1024)).astype(np.float32)
    small = rng.uniform(-3, 7, (3, 1001)).astype(np.float32)     # ragged, all outputs differ from the first call
    for x in (big, small):
        print(f"noalloc dql: shape {x.shape}", flush=True)
        want = _dql(hip, L.dynamic_quantize_linear_forward, x)
        got = _dql(hip, L.dynamic_quantize_linear_forward_noalloc, x)
        for g, w, dt, what in zip(got, want, (O.U8, O.F32, O.U8), ("y", "y_scale", "y_zero_point")):
            assert_bitexact(g, w, dt, what=f"{what} {x.shape}")
    # the small case against the oracle as well
    ref = oracle_lib.dql(small, O.F32)
    for g, w, dt in zip(got, ref, (O.U8, O.F32, O.U8)):
        assert_bitexact(g, w, dt, what="noalloc vs oracle")


def test_noalloc_refuses_host_tensors(hip):
    L = hip.lib
    L.dynamic_quantize_linear_forward_noalloc.argtypes = [O.PT, O.PT, O.PT, O.PT]
    x = np.ones((4, 8), np.float32)
    tx, ty = hip.tensor(x, O.F32), hip.empty(x.shape, O.U8)
    ts, tz = hip.empty((1,), O.F32), hip.empty((1,), O.U8)
    try:
        L.tensor_ops_hip_clear_error()
        L.dynamic_quantize_linear_forward_noalloc(tx, ty, ts, tz)
        assert "device-resident" in hip.last_error()
        L.tensor_ops_hip_clear_error()
    finally:
        for t in (tx, ty, ts, tz):
            L.free_tensor(t)
