"""Library calls captured into a HIP graph (as bench.py times the headline).

Two more tests capture Softmax over few long rows and f32 -> uint8
DynamicQuantizeLinear, whose eager forms are one launch whose blocks exchange
per-call tagged partials: under capture they must take their multi-launch
forms, so replays on changed inputs stay correct.

The calls of one headline step (per-tensor u8 and per-axis i8 QuantizeLinear,
their DequantizeLinear, the fused config-1 chain) are captured on the
library's stream; the graph is replayed several times with the program's own
eager work and synchronisations between replays, the outputs overwritten
before each replay, and every replay must reproduce the eager results bit for
bit.  None of these calls records a memset or allocates inside the capture.
torch provides device memory and the graph object only.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


class Step(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int), ("operand", ctypes.c_int), ("reversed", ctypes.c_int)]


def test_graph_replays_match_eager(hip):
    import torch
    torch.cuda.init()
    side = torch.cuda.Stream()
    L = hip.lib
    L.tensor_ops_hip_set_stream(ctypes.c_void_p(side.cuda_stream))
    keep = []

    def wrap(t, shape, dt):
        arr = (ctypes.c_int * len(shape))(*shape)
        p = L.tensor_wrap_device(ctypes.c_void_p(t.data_ptr()), arr, len(shape), dt)
        assert p
        keep.append(p)
        return p

    try:
        with torch.cuda.stream(side):
            rng = np.random.default_rng(11)
            xs = rng.normal(0, 1.5, (8, 512, 1024)).astype(np.float32)
            shp = list(xs.shape)
            x = torch.from_numpy(xs).cuda()
            s_u8 = torch.tensor([np.abs(xs).max() / 127], dtype=torch.float32, device="cuda")
            z_u8 = torch.tensor([128], dtype=torch.uint8, device="cuda")
            s_ax = torch.from_numpy((np.abs(xs).max(axis=(0, 2)) / 127).astype(np.float32).reshape(1, 512, 1)).cuda()
            z_ax = torch.zeros((1, 512, 1), dtype=torch.int8, device="cuda")
            a = torch.from_numpy(rng.uniform(-4, 4, (8, 64, 56, 56)).astype(np.float32)).cuda()
            bb = torch.from_numpy(rng.uniform(0.5, 4, (64, 1, 1)).astype(np.float32)).cuda()
            outs = {"q_u8": torch.empty(shp, dtype=torch.uint8, device="cuda"),
                    "q_i8": torch.empty(shp, dtype=torch.int8, device="cuda"),
                    "dq_u8": torch.empty(shp, dtype=torch.float32, device="cuda"),
                    "dq_i8": torch.empty(shp, dtype=torch.float32, device="cuda"),
                    "chain": torch.empty_like(a)}
            tx, ta, tb = wrap(x, shp, O.F32), wrap(a, list(a.shape), O.F32), wrap(bb, [64, 1, 1], O.F32)
            ts_u8, tz_u8 = wrap(s_u8, [1], O.F32), wrap(z_u8, [1], O.U8)
            ts_ax, tz_ax = wrap(s_ax, [1, 512, 1], O.F32), wrap(z_ax, [1, 512, 1], O.I8)
            t = {"q_u8": wrap(outs["q_u8"], shp, O.U8), "q_i8": wrap(outs["q_i8"], shp, O.I8),
                 "dq_u8": wrap(outs["dq_u8"], shp, O.F32), "dq_i8": wrap(outs["dq_i8"], shp, O.F32),
                 "chain": wrap(outs["chain"], list(a.shape), O.F32)}
            steps = (Step * 7)(Step(0, 0, 0), Step(2, 0, 0), Step(1, 0, 0), Step(3, 0, 0), Step(4, 0, 0),
                               Step(5, 0, 0), Step(6, 0, 0))
            opnds = (O.PT * 1)(tb)
            L.elementwise_chain_forward.argtypes = [O.PT, ctypes.POINTER(O.PT), ctypes.c_int, ctypes.POINTER(Step),
                                                    ctypes.c_int, O.PT]

            def step():
                L.quantize_linear_forward(tx, ts_u8, tz_u8, t["q_u8"])
                L.quantize_linear_forward(tx, ts_ax, tz_ax, t["q_i8"])
                L.dequantize_linear_forward(t["q_u8"], ts_u8, tz_u8, t["dq_u8"])
                L.dequantize_linear_forward(t["q_i8"], ts_ax, tz_ax, t["dq_i8"])
                L.elementwise_chain_forward(ta, opnds, 1, steps, 7, t["chain"])

            hip.lib.tensor_ops_hip_clear_error()
            step()
            torch.cuda.synchronize()
            assert not hip.last_error(), hip.last_error()
            eager = {k: v.cpu().numpy() for k, v in outs.items()}
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
                    dt = {"q_u8": O.U8, "q_i8": O.I8, "chain": O.F32}.get(k, O.F32)
                    assert_bitexact(v.cpu().numpy(), eager[k], dt, what=f"replay {r} {k}")
                # eager library work between replays
                L.add_forward(ta, tb, t["chain"])
                torch.cuda.synchronize()
        # the captured Q / DQ results are the oracle's too
        o = O.oracle()
        want = o.qdq("quantize", xs, O.F32, s_u8.cpu().numpy(), O.F32, z_u8.cpu().numpy(), O.U8, O.U8)
        assert_bitexact(eager["q_u8"], want, O.U8, what="eager q_u8 vs oracle")
    finally:
        for p in keep:
            L.free_tensor(p)
        L.tensor_ops_hip_set_stream(None)


def test_softmax_split_rows_under_capture(hip):
    """Softmax [64, 32000] captured after an eager call on the same stream;
    the input is rewritten before every replay and each replay must equal an
    eager call on that input bit for bit (a replayed one-launch kernel would
    find the previous replay's partials under its capture-time tag)."""
    import torch
    torch.cuda.init()
    side = torch.cuda.Stream()
    L = hip.lib
    L.tensor_ops_hip_set_stream(ctypes.c_void_p(side.cuda_stream))
    keep = []

    def wrap(t, shape, dt):
        arr = (ctypes.c_int * len(shape))(*shape)
        p = L.tensor_wrap_device(ctypes.c_void_p(t.data_ptr()), arr, len(shape), dt)
        assert p
        keep.append(p)
        return p

    try:
        with torch.cuda.stream(side):
            rng = np.random.default_rng(21)
            inputs = [rng.normal(0, 3, (64, 32000)).astype(np.float32) for _ in range(4)]
            x = torch.from_numpy(inputs[0]).cuda()
            y = torch.empty_like(x)
            ye = torch.empty_like(x)
            tx, ty, tye = wrap(x, [64, 32000], O.F32), wrap(y, [64, 32000], O.F32), wrap(ye, [64, 32000], O.F32)
            hip.lib.tensor_ops_hip_clear_error()
            L.softmax_forward(tx, ty, 1)
            torch.cuda.synchronize()
            assert not hip.last_error(), hip.last_error()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                L.softmax_forward(tx, ty, 1)
            assert not hip.last_error(), hip.last_error()
            for r in range(1, 4):
                x.copy_(torch.from_numpy(inputs[r]))
                y.fill_(0)
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
                L.softmax_forward(tx, tye, 1)
                torch.cuda.synchronize()
                assert not hip.last_error(), hip.last_error()
                assert_bitexact(y.cpu().numpy(), ye.cpu().numpy(), O.F32, what=f"softmax replay {r}")
    finally:
        for p in keep:
            L.free_tensor(p)
        L.tensor_ops_hip_set_stream(None)


def test_dynamic_quantize_linear_under_capture(hip):
    """f32 -> uint8 DynamicQuantizeLinear captured after an eager call (eager:
    one launch whose blocks exchange call-tagged (min, max) pairs; captured: the
    three-launch form).  The input is rewritten before every replay and each
    replay must equal an eager call on that input bit for bit."""
    import torch
    torch.cuda.init()
    side = torch.cuda.Stream()
    L = hip.lib
    L.tensor_ops_hip_set_stream(ctypes.c_void_p(side.cuda_stream))
    keep = []

    def wrap(t, shape, dt):
        arr = (ctypes.c_int * len(shape))(*shape)
        p = L.tensor_wrap_device(ctypes.c_void_p(t.data_ptr()), arr, len(shape), dt)
        assert p
        keep.append(p)
        return p

    try:
        with torch.cuda.stream(side):
            rng = np.random.default_rng(31)
            shp = [8, 512, 1024]
            inputs = [rng.normal(0, s, shp).astype(np.float32) for s in (1.0, 3.0, 0.5, 2.0)]
            x = torch.from_numpy(inputs[0]).cuda()
            y, ye = (torch.empty(shp, dtype=torch.uint8, device="cuda") for _ in range(2))
            sc, sce = (torch.empty([1], dtype=torch.float32, device="cuda") for _ in range(2))
            zp, zpe = (torch.empty([1], dtype=torch.uint8, device="cuda") for _ in range(2))
            tx, ty, tye = wrap(x, shp, O.F32), wrap(y, shp, O.U8), wrap(ye, shp, O.U8)
            ts, tse, tz, tze = wrap(sc, [1], O.F32), wrap(sce, [1], O.F32), wrap(zp, [1], O.U8), wrap(zpe, [1], O.U8)
            hip.lib.tensor_ops_hip_clear_error()
            L.dynamic_quantize_linear_forward(tx, ty, ts, tz)
            torch.cuda.synchronize()
            assert not hip.last_error(), hip.last_error()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                L.dynamic_quantize_linear_forward(tx, ty, ts, tz)
            assert not hip.last_error(), hip.last_error()
            for r in range(1, 4):
                x.copy_(torch.from_numpy(inputs[r]))
                y.fill_(0xA5)
                sc.fill_(-1.0)
                zp.fill_(7)
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
                L.dynamic_quantize_linear_forward(tx, tye, tse, tze)
                torch.cuda.synchronize()
                assert not hip.last_error(), hip.last_error()
                assert_bitexact(sc.cpu().numpy(), sce.cpu().numpy(), O.F32, what=f"dql scale replay {r}")
                assert_bitexact(zp.cpu().numpy(), zpe.cpu().numpy(), O.U8, what=f"dql zero point replay {r}")
                assert_bitexact(y.cpu().numpy(), ye.cpu().numpy(), O.U8, what=f"dql codes replay {r}")
        ry, rs, rz = O.oracle().dql(inputs[3], O.F32)
        assert_bitexact(ye.cpu().numpy(), ry, O.U8, what="eager dql vs oracle")
        assert_bitexact(sce.cpu().numpy(), rs, O.F32, what="eager dql scale vs oracle")
    finally:
        for p in keep:
            L.free_tensor(p)
        L.tensor_ops_hip_set_stream(None)


def _wrapper(L, keep):
    def wrap(t, shape, dt):
        arr = (ctypes.c_int * len(shape))(*shape)
        p = L.tensor_wrap_device(ctypes.c_void_p(t.data_ptr()), arr, len(shape), dt)
        assert p
        keep.append(p)
        return p
    return wrap


def test_allocation_and_host_work_refused_under_capture(hip):
    """Under capture, calls that would allocate or synchronise (device tensor
    creation, host operands, tensor_to_host) return an error instead, the
    device-only call captured beside them replays correctly, and the library
    works as before once the capture has ended."""
    import torch
    torch.cuda.init()
    side = torch.cuda.Stream()
    L = hip.lib
    L.tensor_ops_hip_set_stream(ctypes.c_void_p(side.cuda_stream))
    L.create_tensor_device_empty.restype = O.PT
    L.create_tensor_device_empty.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
    keep = []
    wrap = _wrapper(L, keep)
    rng = np.random.default_rng(51)
    xs = rng.normal(0, 1, (4, 1000)).astype(np.float32)
    relu = np.where(xs > 0, xs, np.float32(0)).astype(np.float32)     # tensor_ops.c:708-728
    hx, hy = hip.tensor(xs, O.F32), hip.empty(xs.shape, O.F32)
    dt = hip.dev_from(xs, O.F32)
    host = np.empty(xs.shape, np.float32)
    try:
        with torch.cuda.stream(side):
            x = torch.from_numpy(xs).cuda()
            y = torch.empty_like(x)
            tx, ty = wrap(x, [4, 1000], O.F32), wrap(y, [4, 1000], O.F32)
            torch.cuda.synchronize()
            shape = (ctypes.c_int * 2)(4, 1000)
            errors = {}
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                L.relu_forward(tx, ty)                          # device only: captured
                L.tensor_ops_hip_clear_error()
                errors["create_tensor_device"] = (L.create_tensor_device(shape, 2, O.F32), hip.last_error())
                L.tensor_ops_hip_clear_error()
                errors["create_tensor_device_empty"] = (L.create_tensor_device_empty(shape, 2, O.F32),
                                                        hip.last_error())
                L.tensor_ops_hip_clear_error()
                L.relu_forward(hx, hy)
                errors["host operands"] = (None, hip.last_error())
                L.tensor_ops_hip_clear_error()
                errors["tensor_to_host"] = (L.tensor_to_host(dt, host.ctypes.data), hip.last_error())
                L.tensor_ops_hip_clear_error()
            for what, (ret, err) in errors.items():
                print(f"capture refusal: {what}: {err}", flush=True)
                assert not ret or ret == -1, f"{what} returned {ret} under capture"
                assert "captur" in err, f"{what}: no capture error ({err!r})"
            y.fill_(-1)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert_bitexact(y.cpu().numpy(), relu, O.F32, what="captured relu")
        # after the capture: the refused calls work again
        L.tensor_ops_hip_clear_error()
        t = L.create_tensor_device(shape, 2, O.F32)
        assert t, hip.last_error()
        L.free_tensor(t)
        L.relu_forward(hx, hy)
        assert not hip.last_error(), hip.last_error()
        assert_bitexact(hip.read(hy, O.F32), relu, O.F32, what="host relu after capture")
        assert L.tensor_to_host(dt, host.ctypes.data) == 0
        assert_bitexact(host, xs, O.F32, what="tensor_to_host after capture")
    finally:
        for p in keep + [hx, hy, dt]:
            L.free_tensor(p)
        L.tensor_ops_hip_set_stream(None)


def test_capture_first_on_fresh_stream(hip, oracle_lib):
    """Calls captured on a stream the library has never used, with no eager call
    before them: Softmax over few long rows and DynamicQuantizeLinear (partials
    in the fixed capture workspaces), the no-allocation DynamicQuantizeLinear
    and a Gemm whose eager plan splits k (captured unsplit).  Nothing may
    allocate inside the capture; the graph is replayed on changed inputs and
    every replay is compared with eager calls on the same inputs (bit for bit;
    the Gemm against the oracle within tolerance, its eager plan differing)."""
    import torch
    torch.cuda.init()
    side = torch.cuda.Stream()
    L = hip.lib
    L.dynamic_quantize_linear_forward_noalloc.argtypes = [O.PT, O.PT, O.PT, O.PT]
    L.tensor_ops_hip_set_stream(ctypes.c_void_p(side.cuda_stream))
    keep = []
    wrap = _wrapper(L, keep)
    rng = np.random.default_rng(53)
    try:
        with torch.cuda.stream(side):
            sm_x = torch.empty((64, 32000), dtype=torch.float32, device="cuda")
            dq_x = torch.empty((8, 512, 1024), dtype=torch.float32, device="cuda")
            ga = torch.empty((64, 512), dtype=torch.float32, device="cuda")
            gb = torch.from_numpy(rng.normal(0, 0.05, (1000, 512)).astype(np.float32)).cuda()
            gc = torch.from_numpy(rng.normal(0, 1, (1, 1000)).astype(np.float32)).cuda()
            outs = {"softmax": torch.empty_like(sm_x), "gemm": torch.empty((64, 1000), dtype=torch.float32, device="cuda")}
            for k in ("dql", "dql_noalloc"):
                outs[k] = torch.empty((8, 512, 1024), dtype=torch.uint8, device="cuda")
                outs[k + "_scale"] = torch.empty([1], dtype=torch.float32, device="cuda")
                outs[k + "_zp"] = torch.empty([1], dtype=torch.uint8, device="cuda")
            t = {"sm_x": wrap(sm_x, [64, 32000], O.F32), "dq_x": wrap(dq_x, [8, 512, 1024], O.F32),
                 "ga": wrap(ga, [64, 512], O.F32), "gb": wrap(gb, [1000, 512], O.F32), "gc": wrap(gc, [1, 1000], O.F32)}
            dts = {"softmax": O.F32, "gemm": O.F32, "dql": O.U8, "dql_noalloc": O.U8}
            for k, v in outs.items():
                dt = dts.get(k, O.F32 if k.endswith("scale") else O.U8)
                t[k] = wrap(v, list(v.shape), dt)

            def calls(o):
                L.softmax_forward(t["sm_x"], o["softmax"], 1)
                L.dynamic_quantize_linear_forward(t["dq_x"], o["dql"], o["dql_scale"], o["dql_zp"])
                L.dynamic_quantize_linear_forward_noalloc(t["dq_x"], o["dql_noalloc"], o["dql_noalloc_scale"],
                                                          o["dql_noalloc_zp"])
                L.gemm_forward(t["ga"], t["gb"], t["gc"], o["gemm"], 1.0, 1.0, 0, 1)

            hip.lib.tensor_ops_hip_clear_error()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                calls({k: t[k] for k in outs})
            assert not hip.last_error(), hip.last_error()
        # eager results on the library's own stream, into separate outputs
        L.tensor_ops_hip_set_stream(None)
        eo = {k: torch.empty_like(v) for k, v in outs.items()}
        et = {k: wrap(v, list(v.shape), dts.get(k, O.F32 if k.endswith("scale") else O.U8)) for k, v in eo.items()}
        for r in range(3):
            sm_np = rng.normal(0, 3 + r, (64, 32000)).astype(np.float32)
            dq_np = rng.normal(0, 0.5 + r, (8, 512, 1024)).astype(np.float32)
            ga_np = rng.normal(0, 1, (64, 512)).astype(np.float32)
            sm_x.copy_(torch.from_numpy(sm_np))
            dq_x.copy_(torch.from_numpy(dq_np))
            ga.copy_(torch.from_numpy(ga_np))
            for v in outs.values():
                v.view(torch.uint8).fill_(0xA5)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            L.tensor_ops_hip_clear_error()
            calls({k: et[k] for k in outs})
            torch.cuda.synchronize()
            assert not hip.last_error(), hip.last_error()
            print(f"capture-first replay {r}", flush=True)
            for k, v in outs.items():
                if k == "gemm":
                    continue
                dt = dts.get(k, O.F32 if k.endswith("scale") else O.U8)
                assert_bitexact(v.cpu().numpy(), eo[k].cpu().numpy(), dt, what=f"replay {r} {k}")
            want = oracle_lib.gemm(ga_np, O.F32, gb.cpu().numpy(), O.F32, gc.cpu().numpy(), O.F32, O.F32,
                                   1.0, 1.0, 0, 1)
            assert_close(outs["gemm"].cpu().numpy(), want, O.F32, what=f"replay {r} gemm (unsplit) vs oracle")
            assert_close(eo["gemm"].cpu().numpy(), want, O.F32, what=f"eager {r} gemm (split) vs oracle")
        ry, rs, rz = oracle_lib.dql(dq_np, O.F32)
        assert_bitexact(outs["dql"].cpu().numpy(), ry, O.U8, what="captured dql vs oracle")
        assert_bitexact(outs["dql_noalloc_scale"].cpu().numpy(), rs, O.F32, what="captured noalloc scale vs oracle")
    finally:
        for p in keep:
            L.free_tensor(p)
        L.tensor_ops_hip_set_stream(None)
