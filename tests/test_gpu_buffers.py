"""The device-buffer entry points the Node executor's acquireOutput /
releaseOutput, upload and readback go through (evalCore.ts:14-17,38-43;
test/gpu.ts:73-83), called through the C-ABI on the GPU: bytes written come
back unchanged, a buffer feeds a kernel (moe_topk on an uploaded logits
buffer matches the oracle's topk), a zero-byte buffer and NULL pointers are
refused without disturbing other buffers, and freeing NULL is a no-op."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import ref
from runntime_amd import _lib

pytestmark = pytest.mark.gpu


def _ctx():
    return _lib.context(0, torch.cuda.current_stream().cuda_stream)


def _alloc(lib, ctx, n):
    p = ctypes.c_void_p()
    _lib.check(lib.moe_buffer_alloc(ctx, n, ctypes.byref(p)))
    assert p.value
    return p


def test_buffer_round_trip_and_refusals():
    lib, ctx = _lib.load(), _ctx()
    print("moe_buffer alloc/write/read/free round trip", flush=True)
    rng = np.random.default_rng(4)
    for n in (1, 3, 4096, (1 << 20) + 5):
        data = rng.integers(0, 256, n, dtype=np.uint8)
        p = _alloc(lib, ctx, n)
        _lib.check(lib.moe_buffer_write(ctx, p, data.ctypes.data, n))
        back = np.zeros(n, np.uint8)
        _lib.check(lib.moe_buffer_read(ctx, back.ctypes.data, p, n))
        assert np.array_equal(back, data), n
        _lib.check(lib.moe_buffer_free(ctx, p))
    # refusals
    q = ctypes.c_void_p()
    assert lib.moe_buffer_alloc(ctx, 0, ctypes.byref(q)) != 0
    keep = _alloc(lib, ctx, 64)
    host = np.zeros(4, np.uint8)
    assert lib.moe_buffer_write(ctx, None, host.ctypes.data, 4) != 0
    assert lib.moe_buffer_write(ctx, keep, None, 4) != 0
    assert lib.moe_buffer_write(ctx, keep, host.ctypes.data, 0) != 0
    assert lib.moe_buffer_read(ctx, None, keep, 4) != 0
    _lib.check(lib.moe_buffer_free(ctx, None))
    ones = np.full(64, 7, np.uint8)
    _lib.check(lib.moe_buffer_write(ctx, keep, ones.ctypes.data, 64))
    back = np.zeros(64, np.uint8)
    _lib.check(lib.moe_buffer_read(ctx, back.ctypes.data, keep, 64))
    assert np.array_equal(back, ones)
    _lib.check(lib.moe_buffer_free(ctx, keep))


def test_buffers_feed_topk():
    """An uploaded logits buffer through moe_topk into an allocated route
    buffer, read back: ids bit-exact and gates as the oracle's topk."""
    lib, ctx = _lib.load(), _ctx()
    T, E, k = 37, 24, 4
    print(f"moe_topk on moe_buffer memory T={T} E={E} k={k}", flush=True)
    logits = np.random.default_rng(9).standard_normal((T, E)).astype(np.float32)
    lp = _alloc(lib, ctx, logits.nbytes)
    rp = _alloc(lib, ctx, T * 2 * k * 4)
    _lib.check(lib.moe_buffer_write(ctx, lp, logits.ctypes.data, logits.nbytes))
    _lib.check(lib.moe_topk(ctx, lp, _lib.MOE_F32, T, E, k, rp))
    got = np.zeros((T, 2 * k), np.float32)
    _lib.check(lib.moe_buffer_read(ctx, got.ctypes.data, rp, got.nbytes))
    want = ref.topk(logits, k)
    assert np.array_equal(got[:, :k], want[:, :k])
    np.testing.assert_allclose(got[:, k:], want[:, k:], rtol=1e-6, atol=1e-7)
    for p in (lp, rp):
        _lib.check(lib.moe_buffer_free(ctx, p))
