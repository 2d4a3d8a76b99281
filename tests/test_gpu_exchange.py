"""One-launch exchanges: Softmax over few long rows ([64, 32000]) and f32 ->
uint8 DynamicQuantizeLinear run one launch whose blocks publish partial results
as 64-bit words (call tag << 32 | payload) and poll for each other's.  A word
must count as published only if the current call wrote it.

* Device-memory pool buffers of the exchange sizes, filled with words carrying
  the next calls' tags, are freed back to the pool just before those calls:
  the exchange buffers are kept apart from the pool, so the results still
  equal the oracle (a slot taken from the pool would fold these words).
* The 32-bit tag wraps: a call made after the count is moved into the next
  epoch, with the same tag as the previous call on the same buffer, must not
  see that call's words (the buffer is zero-filled at the epoch change).

Each test runs on a fresh stream of its own (tensor_ops_hip_set_thread_stream),
so the library's free lists for that stream hold only what the test put there.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu

SM_SHAPE = (64, 32000)          # 8 blocks per row: 64 * 8 * 4 words of 8 bytes = 16 KB of slots
DQL_SHAPE = (8, 512, 1024)      # 256 blocks: 2 * 256 words = 4 KB of slots


@pytest.fixture
def fresh_stream(hip):
    import torch
    torch.cuda.init()
    st = torch.cuda.Stream()
    L = hip.lib
    L.tensor_ops_hip_set_thread_stream.argtypes = [ctypes.c_void_p]
    L.tensor_ops_hip_advance_exchange_count.argtypes = [ctypes.c_ulonglong]
    L.tensor_ops_hip_advance_exchange_count.restype = ctypes.c_ulonglong
    L.tensor_ops_hip_set_thread_stream(ctypes.c_void_p(st.cuda_stream))
    try:
        yield st
    finally:
        L.tensor_ops_hip_set_thread_stream(None)
        torch.cuda.synchronize()


def _softmax(hip, x):
    L = hip.lib
    tx, ty = hip.dev_from(x, O.F32), hip.dev_empty(x.shape, O.F32)
    try:
        L.tensor_ops_hip_clear_error()
        L.softmax_forward(tx, ty, 1)
        assert not hip.last_error(), hip.last_error()
        return hip.dev_read(ty, O.F32)
    finally:
        L.free_tensor(tx)
        L.free_tensor(ty)


def _dql(hip, x):
    L = hip.lib
    tx = hip.dev_from(x, O.F32)
    ty, ts, tz = hip.dev_empty(x.shape, O.U8), hip.dev_empty((1,), O.F32), hip.dev_empty((1,), O.U8)
    try:
        L.tensor_ops_hip_clear_error()
        L.dynamic_quantize_linear_forward(tx, ty, ts, tz)
        assert not hip.last_error(), hip.last_error()
        return hip.dev_read(ty, O.U8), hip.dev_read(ts, O.F32), hip.dev_read(tz, O.U8)
    finally:
        for t in (tx, ty, ts, tz):
            L.free_tensor(t)


def _check_softmax(oracle_lib, x, got, what):
    assert_close(got, oracle_lib.softmax(x, O.F32, O.F32, 1), O.F32, what=what)


def _check_dql(oracle_lib, x, got, what):
    for g, w, dt, name in zip(got, oracle_lib.dql(x, O.F32), (O.U8, O.F32, O.U8), ("y", "scale", "zero point")):
        assert_bitexact(g, w, dt, what=f"{what} {name}")


def _plant(hip, words, nwords, reps):
    """`reps` pool buffers of nwords 8-byte words each, filled with `words`
    (cycled), then freed back to the pool of the current stream."""
    L = hip.lib
    fill = np.resize(np.asarray(words, np.uint64), nwords)
    ts = []
    for _ in range(reps):
        t = hip.dev_empty((nwords,), O.I64)
        assert L.tensor_from_host(t, fill.ctypes.data) == 0, hip.last_error()
        ts.append(t)
    for t in ts:
        L.free_tensor(t)


def test_pool_buffers_with_tagged_words_are_not_exchange_slots(hip, oracle_lib, fresh_stream):
    L = hip.lib
    rng = np.random.default_rng(41)
    xs = rng.normal(0, 3, SM_SHAPE).astype(np.float32)
    xd = rng.normal(0, 1.5, DQL_SHAPE).astype(np.float32)
    base = int(L.tensor_ops_hip_advance_exchange_count(0))
    # words that look published for each of the next 8 calls: tag << 32 | junk
    tags = [((base + k) & 0xFFFFFFFF) or 1 for k in range(1, 9)]
    junk = [(t << 32) | j for t in tags for j in (0x3FF00000, 0x00000000, 0x40490FDB, 0xFF800000)]
    print(f"exchange: planting words for tags {tags[0]}..{tags[-1]}", flush=True)
    for nwords in (4 * 64 * 8, 2 * 256):      # the slot sizes of the two calls
        _plant(hip, junk, nwords, reps=3)
    _check_softmax(oracle_lib, xs, _softmax(hip, xs), "softmax after planted pool words")
    _check_dql(oracle_lib, xd, _dql(hip, xd), "dql after planted pool words")


def test_tag_wrap_zero_fills_exchange_buffers(hip, oracle_lib, fresh_stream):
    L = hip.lib
    rng = np.random.default_rng(43)
    for name, run, check, shapes in (
            ("softmax", _softmax, _check_softmax, [rng.normal(0, s, SM_SHAPE) for s in (3.0, 0.5)]),
            ("dql", _dql, _check_dql, [rng.normal(0, s, DQL_SHAPE) for s in (1.5, 40.0)])):
        a, b = (v.astype(np.float32) for v in shapes)
        run(hip, a)                          # the buffer now holds words tagged with this call's tag
        c = int(L.tensor_ops_hip_advance_exchange_count(0))
        tag = c & 0xFFFFFFFF
        assert tag != 0
        # the next call gets the same tag in the next epoch
        target = (((c >> 32) + 1) << 32) | (tag - 1)
        assert int(L.tensor_ops_hip_advance_exchange_count(target)) == target
        print(f"exchange: {name} tag {tag:#x} reused in epoch {(target >> 32)}", flush=True)
        check(oracle_lib, b, run(hip, b), f"{name} after the tag wrapped")
        assert int(L.tensor_ops_hip_advance_exchange_count(0)) == target + 1
