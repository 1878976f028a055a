"""GPU: the attention half of a decoder layer (ds_hip_attn_*; decoder_layer_forward,
ds_moe_decoder.c:339-431) against the oracle's or_decoder_attn (pinned bit for bit against the
reference in test_oracle_attn.py): the K and V cache rows bit-identical (RMSNorm, the threaded QKV
split, per-head norms and RoPE are exact), h and n within f32 rounding of the attention's output sum
(the device sums the online softmax's V rows in parallel with the same branches and exp arguments)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_oracle_attn import attn_weights, or_attn, rnd  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-5


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def make(dev, w, H, nh, hd, max_seq):
    L = dev.load()
    p = lambda k: w[k].ctypes.data if k in w else None  # noqa: E731
    A = L.ds_hip_attn_create(H, nh, hd, max_seq, 1e-6, 10000.0, p("wq"), p("wk"), p("wv"), p("wo"),
                             p("input_norm"), p("post_norm"), p("q_norm"), p("k_norm"))
    assert A, L.ds_hip_last_error()
    return A


def caches(dev, A, n_pos, qd):
    L = dev.load()
    kp, vp, st = C.c_void_p(), C.c_void_p(), C.c_int()
    dev.check(L.ds_hip_attn_kv(A, C.byref(kp), C.byref(vp), C.byref(st)), "kv")
    out = []
    for ptr in (kp, vp):
        buf = np.empty(n_pos * st.value, np.float32)
        dev.check(L.ds_hip_memcpy_d2h(buf.ctypes.data, ptr.value, buf.nbytes), "d2h")
        out.append(buf.reshape(n_pos, st.value)[:, :qd])
    return out


def run(dev, B, H, nh, hd, positions, pre, win, T, qk_norm, prefill_kv=0, seed=40):
    L = dev.load()
    O = B.oracle()
    qd, max_seq = nh * hd, max(positions) + 1
    w = attn_weights(H, nh, hd, seed, qk_norm)
    stride = (qd + 15) // 16 * 16
    Kc, Vc = np.zeros(max_seq * stride, np.float32), np.zeros(max_seq * stride, np.float32)
    A = make(dev, w, H, nh, hd, max_seq)
    L.ds_set_threads(T)
    try:
        dev.check(L.ds_hip_attn_set_window(A, pre, win), "window")
        if prefill_kv:
            kp, vp = rnd(prefill_kv * qd, seed + 50, 0.3), rnd(prefill_kv * qd, seed + 51)
            Kc.reshape(max_seq, stride)[:prefill_kv, :qd] = kp.reshape(prefill_kv, qd)
            Vc.reshape(max_seq, stride)[:prefill_kv, :qd] = vp.reshape(prefill_kv, qd)
            dev.check(L.ds_hip_attn_load_kv(A, kp.ctypes.data, vp.ctypes.data, prefill_kv, qd), "load kv")
        oa = or_attn(w, H, nh, hd, stride)
        worst = 0.0
        for pos in positions:
            x = rnd(H, 300 + pos)
            xd = dev.DeviceBuffer.from_array(x)
            hd_, nd_ = dev.DeviceBuffer(H * 4), dev.DeviceBuffer(H * 4)
            dev.check(L.ds_hip_attn_forward(A, hd_.ptr, nd_.ptr, xd.ptr, pos), "forward")
            h1, n1 = np.empty(H, np.float32), np.empty(H, np.float32)
            O.or_decoder_attn(h1, n1, x, C.byref(oa), Kc, Vc, pos, pre, win, T)
            kg, vg = caches(dev, A, pos + 1, qd)
            assert np.array_equal(bits(kg[pos]), bits(Kc.reshape(max_seq, stride)[pos, :qd])), pos
            assert np.array_equal(bits(vg[pos]), bits(Vc.reshape(max_seq, stride)[pos, :qd])), pos
            e = max(rel(hd_.to_array(np.float32), h1), rel(nd_.to_array(np.float32), n1))
            worst = max(worst, e)
            assert e < TOL, (pos, e)
        return worst
    finally:
        L.ds_set_threads(1)
        L.ds_hip_attn_destroy(A)


@pytest.mark.parametrize("qk_norm", [False, True])
@pytest.mark.parametrize("T", [1, 5])
def test_attention_block_vs_oracle(dev, B, qk_norm, T):
    worst = run(dev, B, 512, 4, 128, list(range(40)), 10, 16, T, qk_norm)
    print(f"attention block T={T} qk_norm={qk_norm}: worst rel err {worst:.2e}")


def test_attention_block_deepseek_size_rswa(dev, B):
    """1280 hidden, 10 heads x 128; a 200-position cache uploaded, then tokens 200-219 with R-SWA
    (reference 200 tokens, window 8) and without."""
    for pre, win in ((200, 8), (0, 0)):
        worst = run(dev, B, 1280, 10, 128, list(range(200, 220)), pre, win, 1, False, prefill_kv=200, seed=60)
        print(f"attention block 1280/10x128 R-SWA ({pre},{win}): worst rel err {worst:.2e}")


def test_attention_rejects_bad_shapes(dev):
    L = dev.load()
    z = np.zeros(1, np.uint16)
    assert not L.ds_hip_attn_create(500, 4, 128, 64, 1e-6, 1e4, z.ctypes.data, z.ctypes.data, z.ctypes.data,
                                    z.ctypes.data, z.ctypes.data, z.ctypes.data, None, None)
    assert not L.ds_hip_attn_create(512, 4, 128, 100000, 1e-6, 1e4, z.ctypes.data, z.ctypes.data, z.ctypes.data,
                                    z.ctypes.data, z.ctypes.data, z.ctypes.data, None, None)
