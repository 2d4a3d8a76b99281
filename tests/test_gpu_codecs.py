"""Exhaustive codec sweeps on the GPU.

All 2^32 float32 bit patterns go through sub_forward(x, 0) on device-resident
tensors with f16 / bf16 / e4m3 / e5m2 / int64 outputs (the reference's
observable encoder path, tensor_ops.c:571-588 and 520-546).  Each 2^24 chunk's
position-weighted checksum must equal the digest of the reference's own
outputs (tests/golden/codecs.npz, made by the compiled tensor_ops.c).
torch is used only as device-memory plumbing (arange, checksum reduction).
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

CHUNK = 1 << 24
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "codecs.npz")


@pytest.fixture(scope="module")
def env(hip):
    import torch
    torch.cuda.init()
    s = torch.cuda.current_stream()
    hip.lib.tensor_ops_hip_set_stream(ctypes.c_void_p(s.cuda_stream))
    yield torch
    torch.cuda.synchronize()
    hip.lib.tensor_ops_hip_set_stream(None)


def wrap(hip, t, shape, dt):
    arr = (ctypes.c_int * len(shape))(*shape)
    p = hip.lib.tensor_wrap_device(ctypes.c_void_p(t.data_ptr()), arr, len(shape), dt)
    assert p
    return p


@pytest.mark.parametrize("name,dt,nbytes", [("f16", O.F16, 2), ("bf16", O.BF16, 2), ("e4m3", O.E4M3, 1),
                                            ("e5m2", O.E5M2, 1), ("i64", O.I64, 8)])
def test_encoder_sweep_2pow32(hip, env, name, dt, nbytes):
    torch = env
    want = np.load(GOLD, allow_pickle=False)[f"enc_{name}_digest"]
    dev = "cuda"
    idx = torch.arange(CHUNK, dtype=torch.int64, device=dev)
    x = torch.empty(CHUNK, dtype=torch.int32, device=dev)
    zero = torch.zeros(1, dtype=torch.float32, device=dev)
    out = torch.empty(CHUNK * nbytes, dtype=torch.uint8, device=dev)
    tx, tz, to = wrap(hip, x, [CHUNK], O.F32), wrap(hip, zero, [1], O.F32), wrap(hip, out, [CHUNK], dt)
    sums = []
    try:
        for c in range(256):
            x.copy_(((idx + c * CHUNK) & 0xFFFFFFFF).to(torch.int64).sub_(
                ((idx + c * CHUNK) >= 2 ** 31).to(torch.int64) * 2 ** 32).to(torch.int32))
            hip.lib.tensor_ops_hip_clear_error()
            hip.lib.sub_forward(tx, tz, to)
            assert not hip.last_error(), hip.last_error()
            if nbytes == 1:
                codes = out.to(torch.int64)
            elif nbytes == 2:
                codes = out.view(torch.int16).to(torch.int64) & 0xFFFF
            else:
                codes = out.view(torch.int64)
            w = idx + (c * CHUNK + 1)
            sums.append(int(((codes + 1) * w).sum().item()) & 0xFFFFFFFFFFFFFFFF)
    finally:
        for p in (tx, tz, to):
            hip.lib.free_tensor(p)
    bad = [c for c in range(256) if sums[c] != int(want[c])]
    assert not bad, f"{name}: chunks {bad[:10]} differ from the reference digests"


def test_cos_f32_fast_path_every_input(hip, env, oracle_lib):
    """The f32 Cos kernels (standalone and in the fused chain: table in LDS, the
    index quotient by reciprocal multiply plus one fma correction instead of a
    division) against the division path that f64 outputs take (the reference's
    arithmetic, tensor_ops.c:815-833), over all 2^32 float32 patterns; eight
    chunks also against the oracle directly."""
    torch = env
    dev = "cuda"
    idx = torch.arange(CHUNK, dtype=torch.int64, device=dev)
    x = torch.empty(CHUNK, dtype=torch.int32, device=dev)
    y32 = torch.empty(CHUNK, dtype=torch.float32, device=dev)
    ych = torch.empty(CHUNK, dtype=torch.float32, device=dev)
    y64 = torch.empty(CHUNK, dtype=torch.float64, device=dev)
    tx, t32, tch, t64 = (wrap(hip, x, [CHUNK], O.F32), wrap(hip, y32, [CHUNK], O.F32),
                         wrap(hip, ych, [CHUNK], O.F32), wrap(hip, y64, [CHUNK], O.F64))

    class Step(ctypes.Structure):
        _fields_ = [("op", ctypes.c_int), ("operand", ctypes.c_int), ("reversed", ctypes.c_int)]
    step = (Step * 1)(Step(6, 0, 0))
    hip.lib.elementwise_chain_forward.argtypes = [O.PT, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                                  O.PT]
    check_oracle = {0, 37, 64, 100, 127, 128, 190, 250}
    bad = []
    try:
        for c in range(256):
            x.copy_(((idx + c * CHUNK) & 0xFFFFFFFF).sub_(((idx + c * CHUNK) >= 2 ** 31).to(torch.int64) * 2 ** 32)
                    .to(torch.int32))
            hip.lib.tensor_ops_hip_clear_error()
            hip.lib.cos_forward(tx, t32)
            hip.lib.cos_forward(tx, t64)
            hip.lib.elementwise_chain_forward(tx, None, 0, step, 1, tch)
            assert not hip.last_error(), hip.last_error()
            ref = y64.to(torch.float32)
            both_nan = torch.isnan(ref) & torch.isnan(y32) & torch.isnan(ych)
            diff = ((y32.view(torch.int32) != ref.view(torch.int32)) |
                    (ych.view(torch.int32) != ref.view(torch.int32))) & ~both_nan
            n = int(diff.sum().item())
            if n:
                first = int(torch.nonzero(diff)[0].item())
                bad.append((c, n, hex((c * CHUNK + first) & 0xFFFFFFFF)))
            if c in check_oracle:
                xs = x.cpu().numpy().view(np.float32)
                want = oracle_lib.unary("cos", xs, O.F32, O.F32)
                got = y32.cpu().numpy()
                mism = (got.view(np.uint32) != want.view(np.uint32)) & ~(np.isnan(got) & np.isnan(want))
                if mism.any():
                    bad.append((c, int(mism.sum()), "vs oracle"))
    finally:
        for p in (tx, t32, tch, t64):
            hip.lib.free_tensor(p)
    assert not bad, f"cos f32 fast path differs: {bad[:10]}"


DIVISORS = [1.0, -1.0, 3.0, 0.1, 1.0 / 3.0, 7.0, -2.5, np.pi, 1.0000001, 0.99999994, 1.17549435e-38, 1e-40, 1.4e-45,
            -3e-42, 3.4028235e38, -1e30, 1e-30, 0.0, -0.0, np.inf, -np.inf, np.nan, 12345.678, -0.007]


def test_chain_division_by_item_operand_every_dividend(hip, env):
    """The fused chain divides by a one-per-item operand as RN32(v * RN64(1 / b));
    for every f32 dividend (all 2^32 patterns) and each divisor above it must
    equal div_forward's correctly rounded f32 division (tensor_ops.c:949-997)
    bit for bit (any NaN where that gives a NaN)."""
    torch = env
    dev = "cuda"
    idx = torch.arange(CHUNK, dtype=torch.int64, device=dev)
    x = torch.empty(CHUNK, dtype=torch.int32, device=dev)
    bt = torch.empty(1, dtype=torch.float32, device=dev)
    yd = torch.empty(CHUNK, dtype=torch.float32, device=dev)
    yc = torch.empty(CHUNK, dtype=torch.float32, device=dev)
    tx, tb, tyd, tyc = (wrap(hip, x, [CHUNK], O.F32), wrap(hip, bt, [1], O.F32), wrap(hip, yd, [CHUNK], O.F32),
                        wrap(hip, yc, [CHUNK], O.F32))

    class Step(ctypes.Structure):
        _fields_ = [("op", ctypes.c_int), ("operand", ctypes.c_int), ("reversed", ctypes.c_int)]
    step = (Step * 1)(Step(3, 0, 0))
    opnds = (O.PT * 1)(tb)
    hip.lib.elementwise_chain_forward.argtypes = [O.PT, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                                  O.PT]
    bad = []
    try:
        for bv in DIVISORS:
            bt.fill_(float(np.float32(bv)))
            for c in range(256):
                x.copy_(((idx + c * CHUNK) & 0xFFFFFFFF).sub_(((idx + c * CHUNK) >= 2 ** 31).to(torch.int64) * 2 ** 32)
                        .to(torch.int32))
                hip.lib.tensor_ops_hip_clear_error()
                hip.lib.div_forward(tx, tb, tyd)
                hip.lib.elementwise_chain_forward(tx, ctypes.cast(opnds, ctypes.c_void_p), 1, step, 1, tyc)
                assert not hip.last_error(), hip.last_error()
                diff = (yd.view(torch.int32) != yc.view(torch.int32)) & ~(torch.isnan(yd) & torch.isnan(yc))
                n = int(diff.sum().item())
                if n:
                    first = int(torch.nonzero(diff)[0].item())
                    bad.append((bv, c, n, hex((c * CHUNK + first) & 0xFFFFFFFF)))
                    break
    finally:
        for p in (tx, tb, tyd, tyc):
            hip.lib.free_tensor(p)
    assert not bad, f"chain division differs from div_forward: {bad[:10]}"
