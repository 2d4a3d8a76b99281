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
