"""The allocation-free argmax entry point (ds_hip_argmax_bf16_noalloc: candidate keys in the library's
static device array) against the allocating one (ds_hip_argmax_bf16), through the C-ABI, on two
calls in a row -- the second smaller, so stale keys of the first would show -- and its size limit."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_ROWS = 64 * 4096


def argmax_both(dev, W, x, in_dim, out_dim):
    L = dev.load()
    wd = dev.DeviceBuffer.from_array(W)
    xd = dev.DeviceBuffer.from_array(x)
    a = dev.DeviceBuffer(4)
    b = dev.DeviceBuffer(4)
    a.write(np.array([-5], np.int32))
    b.write(np.array([-6], np.int32))
    dev.check(L.ds_hip_argmax_bf16(a.ptr, xd.ptr, wd.ptr, in_dim, out_dim), "argmax")
    dev.check(L.ds_hip_argmax_bf16_noalloc(b.ptr, xd.ptr, wd.ptr, in_dim, out_dim), "argmax without allocation")
    dev.check(L.ds_hip_sync(), "sync")
    return int(a.to_array(np.int32)[0]), int(b.to_array(np.int32)[0])


def test_noalloc_argmax_equals_allocating_entry_point(dev, B):
    L = dev.load()
    for threads in (16, 1):
        L.ds_set_threads(threads)
        # 1: the full LM head shape; 2: a smaller matrix whose best row sits in a block that the first
        # call's keys would win if they were left behind
        H1, V1 = 1280, 129280
        W1 = B.normal_bf16(V1 * H1, 901, 0.02)
        x1 = B.normal_f32(H1, 902)
        a1, b1 = argmax_both(dev, W1, x1, H1, V1)
        want1 = B.oracle().or_argmax_bf16(x1, W1, H1, V1, threads, None)
        print(f"threads {threads}: full head {a1} / {b1} (oracle {want1})")
        assert a1 == b1 == want1
        H2, V2 = 256, 3000
        W2 = B.normal_bf16(V2 * H2, 903, 0.02).reshape(V2, H2)
        W2[2999] = W2[17]  # a duplicated row that the input favours: the lower index must win
        x2 = (W2[17].astype(np.uint32) << 16).view(np.float32) * np.float32(50.0) + B.normal_f32(H2, 904)
        a2, b2 = argmax_both(dev, W2.ravel(), x2, H2, V2)
        want2 = B.oracle().or_argmax_bf16(x2, W2.ravel(), H2, V2, threads, None)
        print(f"threads {threads}: small {a2} / {b2} (oracle {want2})")
        assert a2 == b2 == want2
    L.ds_set_threads(1)


def test_noalloc_argmax_refuses_beyond_its_scratch(dev):
    L = dev.load()
    w = dev.DeviceBuffer(1024)
    x = dev.DeviceBuffer(1024)
    o = dev.DeviceBuffer(4)
    assert L.ds_hip_argmax_bf16_noalloc(o.ptr, x.ptr, w.ptr, 64, MAX_ROWS + 1) == -1
    assert b"exceeds the maximum" in L.ds_hip_last_error()
    assert L.ds_hip_argmax_bf16_noalloc(None, x.ptr, w.ptr, 64, 10) == -1
