"""Concurrent calls into libtensor_ops_hip.so from several Python threads.

ctypes releases the GIL around every foreign call, so threads really do enter
the library at the same time, as callers of the reference can
(tensor_ops.c:21-25,763-807: the reference is re-entrant, its one-time cosine
table set-up is mutex-guarded).  Each thread runs host-tensor calls (staged,
synchronous), device-tensor calls (asynchronous on the library stream, or on
a stream of the thread's own for half of them) and its own precision mode,
and every result must equal the oracle's to its parity class; the precision
mode one thread sets must not reach another.
"""
import ctypes
import threading

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu

THREADS = 8
ROUNDS = 6


def _inputs(seed):
    rng = np.random.default_rng(seed)
    a = rng.uniform(-4, 4, (4, 64, 28, 28)).astype(np.float32)
    b = rng.uniform(-4, 4, (64, 1, 1)).astype(np.float32)
    x = rng.normal(0, 1.5, (8, 64, 256)).astype(np.float32)
    s = np.array([np.abs(x).max() / 127], np.float32)
    ga = rng.normal(0, 1, (192, 160)).astype(np.float32)
    gb = rng.normal(0, 1, (136, 160)).astype(np.float32)
    gc = rng.normal(0, 1, (136,)).astype(np.float32)
    return a, b, x, s, ga, gb, gc


def test_concurrent_calls_match_the_oracle(hip, oracle_lib):
    L = hip.lib
    L.tensor_ops_hip_get_exact.restype = ctypes.c_int
    L.tensor_ops_hip_get_exact.argtypes = []
    cases = []
    for t in range(THREADS):
        a, b, x, s, ga, gb, gc = _inputs(100 + t)
        z = np.zeros(1, np.int8)
        cases.append(dict(
            a=a, b=b, x=x, s=s, z=z, ga=ga, gb=gb, gc=gc,
            add=oracle_lib.binary("add", a, O.F32, b, O.F32, O.F32),
            cos=oracle_lib.unary("cos", a, O.F32, O.F32),
            q=oracle_lib.qdq("quantize", x, O.F32, s, O.F32, z, O.I8, O.I8),
            gemm=oracle_lib.gemm(ga, O.F32, gb, O.F32, gc, O.F32, O.F32, 1.0, 1.0, 0, 1)))
    errors = []
    start = threading.Barrier(THREADS)

    import torch
    torch.cuda.init()
    L.tensor_ops_hip_set_thread_stream.argtypes = [ctypes.c_void_p]
    # threads 2, 3, 6, 7 launch on a stream of their own (tensor_ops_hip_set_thread_stream)
    own = {t: torch.cuda.Stream() for t in range(THREADS) if t % 4 >= 2}

    def work(t):
        c = cases[t]
        exact = t % 2 == 1
        try:
            hip.set_exact(exact)
            if t in own:
                L.tensor_ops_hip_set_thread_stream(ctypes.c_void_p(own[t].cuda_stream))
            start.wait(timeout=120)
            for r in range(ROUNDS):
                # host tensors: staged through HBM, synchronous
                assert_bitexact(hip.binary_raw("add", c["a"], O.F32, c["b"], O.F32, O.F32), c["add"], O.F32,
                                what=f"thread {t} add")
                assert_bitexact(hip.qdq1("quantize", c["x"], O.F32, c["s"], c["z"], O.I8, O.I8), c["q"], O.I8,
                                what=f"thread {t} quantize")
                g = hip.gemm(c["ga"], O.F32, c["gb"], O.F32, c["gc"], O.F32, O.F32, 1.0, 1.0, 0, 1)
                if exact:
                    assert_bitexact(g, c["gemm"], O.F32, what=f"thread {t} gemm exact")
                else:
                    assert_close(g, c["gemm"], O.F32, what=f"thread {t} gemm")
                assert L.tensor_ops_hip_get_exact() == int(exact), f"thread {t}: precision mode changed"
                # device tensors: asynchronous on the library stream, read back at the end
                ta = hip.dev_from(c["a"], O.F32)
                tb = hip.dev_from(c["b"], O.F32)
                to = hip.dev_empty(c["a"].shape, O.F32)
                tc = hip.dev_empty(c["a"].shape, O.F32)
                L.add_forward(ta, tb, to)
                L.cos_forward(ta, tc)
                got_add, got_cos = hip.dev_read(to, O.F32), hip.dev_read(tc, O.F32)
                err = hip.last_error()
                for p in (ta, tb, to, tc):
                    L.free_tensor(p)
                assert not err, err
                assert_bitexact(got_add, c["add"], O.F32, what=f"thread {t} device add round {r}")
                assert_bitexact(got_cos, c["cos"], O.F32, what=f"thread {t} device cos round {r}")
        except BaseException as e:          # reported by the main thread
            errors.append(f"thread {t}: {e!r}"[:600])
        finally:
            hip.set_exact(False)
            L.tensor_ops_hip_set_thread_stream(None)

    print(f"threads: {THREADS} x {ROUNDS} rounds of add / quantize / gemm / device add+cos", flush=True)
    threads = [threading.Thread(target=work, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=300)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors[:3]
    # the main thread's mode was never touched by the workers
    assert L.tensor_ops_hip_get_exact() == 0
