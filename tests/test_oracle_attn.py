"""Pins the oracle's decoder attention block (oracle.c: or_rms_norm ... or_decoder_attn;
ds_moe_decoder.c:339-431, ds_kernels.c) bit for bit against the reference's own compiled
functions (oracle/_ref, built from the reference sources by oracle/build_ref.sh): RMSNorm with and
without a tail, the fused residual RMSNorm, the RoPE cache and rotation, the per-head norm, the
threaded QKV split, causal and R-SWA attention, and the whole block composed from the reference's
calls in decoder_layer_forward's order."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import bindings as B  # noqa: E402

flags = open("/proc/cpuinfo").read()
pytestmark = [pytest.mark.skipif(not os.path.exists(B.ref_path("v4")),
                                 reason="oracle/_ref not built (reference sources absent)"),
              pytest.mark.skipif(" avx512f " not in flags, reason="the pinned reference build needs AVX-512")]


class _LazyRef:
    """The reference build, loaded at the first use by a test of this file (not at collection)."""

    def __getattr__(self, name):
        return getattr(B.ref("v4"), name)


R = _LazyRef()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def rnd(n, seed, scale=1.0):
    return B.normal_f32(n, seed) * np.float32(scale)


@pytest.mark.parametrize("n", [1280, 1288, 128, 40])
def test_rms_norms(n):
    O = B.oracle()
    x, w, r = rnd(n, 1), rnd(n, 2, 0.1) + 1, rnd(n, 3, 0.5)
    a, b = np.empty(n, np.float32), np.empty(n, np.float32)
    O.or_rms_norm(a, x, w, n, 1e-6)
    R.ds_rms_norm(b, x, w, 1, n, 1e-6)
    assert np.array_equal(bits(a), bits(b))
    o1, n1, o2, n2 = (np.empty(n, np.float32) for _ in range(4))
    O.or_residual_rms_norm(o1, n1, x, r, w, n, 1e-6)
    R.ds_residual_rms_norm(o2, n2, x, r, w, n, 1e-6)
    assert np.array_equal(bits(o1), bits(o2)) and np.array_equal(bits(n1), bits(n2))


@pytest.mark.parametrize("head_dim", [128, 64])
def test_rope_and_head_norm(head_dim):
    O = B.oracle()
    nh = 10
    for pos in (0, 1, 37, 999, 8191):
        c1, s1 = np.empty(head_dim, np.float32), np.empty(head_dim, np.float32)
        O.or_rope_row(c1, s1, pos, head_dim, 10000.0)
        c2, s2 = np.empty(head_dim, np.float32), np.empty(head_dim, np.float32)
        R.ds_compute_rope_neox(c2, s2, np.array([pos], np.int32), 1, head_dim, 10000.0)
        assert np.array_equal(bits(c1), bits(c2)) and np.array_equal(bits(s1), bits(s2))
        x = rnd(nh * head_dim, 10 + pos)
        a, b = x.copy(), x.copy()
        O.or_apply_rope(a, c1, s1, nh, head_dim)
        R.ds_apply_rope_neox(b, c2, s2, 1, nh, head_dim)
        assert np.array_equal(bits(a), bits(b)), pos
    w = rnd(head_dim, 5, 0.1) + 1
    x = rnd(nh * head_dim, 6)
    a, b = x.copy(), x.copy()
    O.or_rms_norm_per_head(a, w, nh, head_dim, 1e-6)
    R.ds_rms_norm_per_head(b, w, 1, nh, head_dim, 1e-6)
    assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("T", [1, 3, 7, 16])
def test_qkv_split_over_threads(T):
    O = B.oracle()
    H, qd = 512, 384
    Wq, Wk, Wv = (B.normal_bf16(qd * H, s, 0.02) for s in (20, 21, 22))
    x = rnd(H, 23)
    outs = [np.empty(qd, np.float32) for _ in range(6)]
    O.or_qkv(outs[0], outs[1], outs[2], x, Wq, Wk, Wv, H, qd, qd, T)
    R.ds_set_threads(T)
    try:
        R.ds_linear_nobias_bf16_qkv(outs[3], outs[4], outs[5], x, Wq, Wk, Wv, H, qd, qd)
    finally:
        R.ds_set_threads(1)
    for i in range(3):
        assert np.array_equal(bits(outs[i]), bits(outs[3 + i])), i


@pytest.mark.parametrize("T", [1, 4])
def test_attention_causal_and_rswa(T):
    O = B.oracle()
    nh, hd, stride, kv = 4, 128, 528, 300
    q = rnd(nh * hd, 30, 0.3)
    K = rnd(kv * stride, 31, 0.3)
    V = rnd(kv * stride, 32)
    scale = np.float32(1.0 / np.sqrt(hd))
    R.ds_set_threads(T)
    try:
        for pos, pre, win in ((0, 0, 0), (150, 0, 0), (299, 0, 0), (299, 100, 64), (299, 100, 250), (120, 130, 64)):
            rng = np.zeros(4, np.int32)
            nr = O.or_attn_ranges(rng, pos, pre, win)
            a, b = np.empty(nh * hd, np.float32), np.empty(nh * hd, np.float32)
            O.or_attention_decode(a, q, K, V, nh, hd, scale, stride, rng, nr)
            if nr == 1:
                R.ds_causal_attention_aligned(b, q, K, V, 1, pos + 1, nh, nh, hd, scale, pos, stride)
            else:
                R.ds_rswa_attention_aligned(b, q, K, V, 1, nh, nh, hd, scale, stride, pre, int(rng[2]), pos + 1)
            assert np.array_equal(bits(a), bits(b)), (pos, pre, win)
        assert O.or_attn_ranges(rng, 299, 100, 64) == 2 and list(rng) == [0, 100, 236, 300]
    finally:
        R.ds_set_threads(1)


def attn_weights(H, nh, hd, seed, qk_norm=False):
    qd = nh * hd
    w = {"wq": B.normal_bf16(qd * H, seed, 0.02), "wk": B.normal_bf16(qd * H, seed + 1, 0.02),
         "wv": B.normal_bf16(qd * H, seed + 2, 0.02), "wo": B.normal_bf16(H * qd, seed + 3, 0.02),
         "input_norm": rnd(H, seed + 4, 0.1) + 1, "post_norm": rnd(H, seed + 5, 0.1) + 1}
    if qk_norm:
        w["q_norm"] = rnd(hd, seed + 6, 0.1) + 1
        w["k_norm"] = rnd(hd, seed + 7, 0.1) + 1
    return w


def or_attn(w, H, nh, hd, stride):
    a = B.OrAttn()
    a.hidden, a.n_heads, a.head_dim, a.kv_stride, a.eps, a.theta = H, nh, hd, stride, 1e-6, 10000.0
    for k in ("wq", "wk", "wv", "wo", "input_norm", "post_norm", "q_norm", "k_norm"):
        setattr(a, k, w[k].ctypes.data if k in w else None)
    return a


def ref_block(w, x, Kc, Vc, pos, pre, win, H, nh, hd, stride, T):
    """decoder_layer_forward's attention half from the reference's calls, in its order."""
    qd = nh * hd
    R.ds_set_threads(T)
    try:
        xn = np.empty(H, np.float32)
        R.ds_rms_norm(xn, x, w["input_norm"], 1, H, 1e-6)
        q, k, v = (np.empty(qd, np.float32) for _ in range(3))
        R.ds_linear_nobias_bf16_qkv(q, k, v, xn, w["wq"], w["wk"], w["wv"], H, qd, qd)
        if "q_norm" in w:
            R.ds_rms_norm_per_head(q, w["q_norm"], 1, nh, hd, 1e-6)
            R.ds_rms_norm_per_head(k, w["k_norm"], 1, nh, hd, 1e-6)
        c, s = np.empty(hd, np.float32), np.empty(hd, np.float32)
        R.ds_compute_rope_neox(c, s, np.array([pos], np.int32), 1, hd, 10000.0)
        R.ds_apply_rope_neox(q, c, s, 1, nh, hd)
        R.ds_apply_rope_neox(k, c, s, 1, nh, hd)
        Kc[pos * stride:pos * stride + qd] = k
        Vc[pos * stride:pos * stride + qd] = v
        att = np.empty(qd, np.float32)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))  # 1.0f / sqrtf((float)head_dim), in f32
        kv = pos + 1
        ws = max(pre, kv - win) if win > 0 and pos >= pre else 0
        if win > 0 and pos >= pre and ws > pre:
            R.ds_rswa_attention_aligned(att, q, Kc, Vc, 1, nh, nh, hd, scale, stride, pre, ws, kv)
        else:
            R.ds_causal_attention_aligned(att, q, Kc, Vc, 1, kv, nh, nh, hd, scale, pos, stride)
        proj = np.empty(H, np.float32)
        R.ds_linear_nobias_bf16(proj, att, w["wo"], 1, qd, H)
        h, n = np.empty(H, np.float32), np.empty(H, np.float32)
        R.ds_residual_rms_norm(h, n, x, proj, w["post_norm"], H, 1e-6)
        return h, n
    finally:
        R.ds_set_threads(1)


@pytest.mark.parametrize("qk_norm", [False, True])
@pytest.mark.parametrize("T", [1, 5])
def test_decoder_attention_block(qk_norm, T):
    O = B.oracle()
    H, nh, hd, stride, steps = 512, 4, 128, 528, 40
    w = attn_weights(H, nh, hd, 40, qk_norm)
    A = or_attn(w, H, nh, hd, stride)
    Ko, Vo = np.zeros(steps * stride, np.float32), np.zeros(steps * stride, np.float32)
    Kr, Vr = Ko.copy(), Vo.copy()
    for pos in range(steps):
        x = rnd(H, 100 + pos)
        pre, win = (10, 16) if pos >= 10 else (0, 0)
        h1, n1 = np.empty(H, np.float32), np.empty(H, np.float32)
        O.or_decoder_attn(h1, n1, x, C.byref(A), Ko, Vo, pos, pre, win, T)
        h2, n2 = ref_block(w, x, Kr, Vr, pos, pre, win, H, nh, hd, stride, T)
        assert np.array_equal(bits(h1), bits(h2)) and np.array_equal(bits(n1), bits(n2)), pos
