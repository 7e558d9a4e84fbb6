"""Device allocator of the C ABI (ernie_hip_malloc / ernie_hip_free): a freed block is kept
and handed to the next allocation of the same rounded size, and carries the new owner's
data; other sizes get other blocks."""
import ctypes

import numpy as np
import pytest

import ernie_amd as E


@pytest.mark.gpu
def test_freed_block_is_reused_and_carries_new_data():
    ctx = E.Context(0, use_torch_stream=False)
    try:
        a = ctypes.c_void_p()
        ctx.call("malloc", 1000, ctypes.byref(a))
        src = np.arange(256, dtype=np.float32)
        ctx.call("memcpy_h2d", a, src.ctypes.data_as(ctypes.c_void_p), src.nbytes)
        ctx.call("free", a)
        b = ctypes.c_void_p()
        ctx.call("malloc", 1024, ctypes.byref(b))  # 1000 and 1024 bytes both round to 1024
        assert b.value == a.value
        c = ctypes.c_void_p()
        ctx.call("malloc", 4096, ctypes.byref(c))
        assert c.value not in (None, b.value)
        new = (np.arange(256, dtype=np.float32) * -3.0 + 7.0)
        ctx.call("memcpy_h2d", b, new.ctypes.data_as(ctypes.c_void_p), new.nbytes)
        back = np.zeros(256, np.float32)
        ctx.call("memcpy_d2h", back.ctypes.data_as(ctypes.c_void_p), b, back.nbytes)
        np.testing.assert_array_equal(back, new)
        ctx.call("free", b)
        ctx.call("free", c)
        ctx.call("free", None)  # freeing null is a no-op
    finally:
        del ctx
