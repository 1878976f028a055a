"""Properties the mathematics fixes, checked on the oracle independently of the reference build:
quantizer invariants, f64 brute force for the matvecs and the argmax, closed forms of the fast exp,
top-k and combine identities, and a one-token prefill equal to the decode layer."""
import ctypes as C

import numpy as np
import pytest


def f32(a):
    return np.asarray(a, np.float32)


@pytest.mark.parametrize("seed", [1, 2])
def test_quantizer_invariants(B, seed):
    W = B.normal_bf16(64 * 300, 70 + seed, 0.05).reshape(64, 300)
    blk = B.or_quantize_bf16(W)
    w = B.bf16_to_f32(W).reshape(64, 300)
    u = blk.q.astype(np.int32) + 128
    assert u.min() >= 0 and u.max() <= 255
    # offset is the row minimum, scale the range / 255, the minimum maps to code 0, the max to 255
    assert np.array_equal(blk.offset, w.min(axis=1))
    assert np.array_equal(blk.scale, f32((w.max(axis=1) - w.min(axis=1)) / np.float32(255.0)))
    assert (u[np.arange(64), w.argmin(axis=1)] == 0).all()
    assert (u[np.arange(64), w.argmax(axis=1)] == 255).all()
    # dequantization error is at most half a step (plus rounding of the f32 arithmetic)
    deq = blk.scale[:, None].astype(np.float64) * u + blk.offset[:, None]
    err = np.abs(deq - w)
    assert (err <= blk.scale[:, None] * 0.5 * (1 + 1e-5) + 1e-7).all()


def test_quantizer_half_way_rounds_away_from_zero(B):
    # min 0, max 255 -> scale 1, inv 1: (w - 0) * 1 = k + 0.5 exactly -> roundf gives k + 1
    row = np.array([0.0, 255.0] + [k + 0.5 for k in range(100)], np.float32)
    W = B.f32_to_bf16_rne(row)[None, :]
    blk = B.or_quantize_bf16(W)
    u = blk.q[0].astype(np.int32) + 128
    assert blk.scale[0] == 1.0
    assert list(u[2:]) == [k + 1 for k in range(100)]


def test_quantizer_constant_row_and_zero_ties(B):
    W = B.f32_to_bf16_rne(np.array([[0.5] * 40, [0.0, -0.0] * 20, [-0.0, 0.0] * 20], np.float32))
    blk = B.or_quantize_bf16(W)
    assert blk.scale[0] == np.float32(1e-10)
    assert (blk.q[0] == -128).all()
    # the first zero seen is the minimum (strict '<'): +0 in row 1, -0 in row 2
    assert blk.offset[1].view(np.uint32) == 0x00000000
    assert blk.offset[2].view(np.uint32) == 0x80000000


@pytest.mark.parametrize("shape", [(1792, 1280), (1280, 896), (17, 33)])
def test_int8_matvec_vs_f64_brute_force(B, shape):
    O = B.oracle()
    o, i = shape
    W = B.normal_bf16(o * i, 90 + o, 0.02).reshape(o, i)
    blk = B.or_quantize_bf16(W)
    x = B.normal_f32(i, 91 + i)
    y = np.empty(o, np.float32)
    O.or_int8_matvec_rows(y, x, blk.q, blk.scale, blk.offset, i, 0, o)
    yd = np.empty(o, np.float64)
    O.or_int8_matvec_f64(yd, x, blk.q, blk.scale, blk.offset, i, o)
    assert np.abs(y - yd).max() / np.abs(yd).max() < 1e-5
    # the identity scale*Σ(q+128)x + off*Σx equals the dequantized dot product
    deq = np.empty((o, i), np.float32)
    O.or_dequantize_f32(deq, blk.q, blk.scale, blk.offset, o, i)
    assert np.abs(deq.astype(np.float64) @ x - yd).max() / np.abs(yd).max() < 1e-5


def test_fast_expf_closed_form(B):
    O = B.oracle()
    assert O.or_fast_expf(-88.5) == 0.0
    assert O.or_fast_expf(88.5) == np.float32(1e38)
    # Schraudolph: bits = 12102203*x + 1064866816 (the constant rounds to a multiple of 64)
    for x in [0.0, 1.0, -1.0, 2.5, -10.0, 40.0]:
        v = np.float32(np.float64(12102203.0) * np.float64(x) + np.float64(1064866816.0))
        expect = np.array([int(v)], np.uint32).view(np.float32)[0]
        assert O.or_fast_expf(x) == expect
    xs = np.linspace(-20, 20, 1001)
    rel = np.abs(np.array([O.or_fast_expf(v) for v in xs]) / np.exp(xs) - 1)
    assert rel.max() < 0.065  # the approximation's known error envelope (a few percent)


def test_argmax_vs_f64_brute_force_and_edges(B):
    O = B.oracle()
    V, H = 500, 96
    W = B.normal_bf16(V * H, 95, 0.02)
    x = B.normal_f32(H, 96)
    logits = B.bf16_to_f32(W).reshape(V, H).astype(np.float64) @ x.astype(np.float64)
    for T in (1, 3, 8):
        assert O.or_argmax_bf16(x, W, H, V, T, None) == int(np.argmax(logits))
    # duplicated best row (later index) and an all-NaN row: lowest index wins, NaN never chosen.
    # One thread: both rows then use the same accumulation order, so their logits are equal bits
    # (with 4 threads row 499 is a chunk-tail row in the single-accumulator order and rounds
    # differently, which the reference does too).
    best = int(np.argmax(logits))
    W2 = W.reshape(V, H).copy()
    W2[V - 1] = W2[best]
    W2[0] = 0x7FC0
    assert O.or_argmax_bf16(x, np.ascontiguousarray(W2.reshape(-1)), H, V, 1, None) == best
    # every logit <= -1e30: index 0
    W3 = np.full(V * H, B.f32_to_bf16_rne(np.array([-3e38], np.float32))[0], np.uint16)
    x3 = np.ones(H, np.float32)
    assert O.or_argmax_bf16(x3, W3, H, V, 1, None) == 0


def test_topk_renorm_identity(B):
    O = B.oracle()
    s = B.normal_f32(64, 97, 1.0)
    idx = np.empty(6, np.int32)
    w = np.empty(6, np.float32)
    O.or_moe_top_k(idx, w, s, 64, 6)
    assert list(idx) == list(np.argsort(-s, kind="stable")[:6])
    assert abs(float(w.sum()) - 1.0) < 1e-6
    e = np.exp(np.float64(s[idx]) - s[idx].max())
    assert np.allclose(w, e / e.sum(), rtol=1e-6)


def test_decode_routing_identity(B):
    O = B.oracle()
    s = B.normal_f32(64, 98, 0.7)
    sc = s.copy()
    idx = np.empty(6, np.int32)
    w = np.empty(6, np.float32)
    O.or_softmax_topk_decode(idx, w, sc, 64, 6)
    assert list(idx) == list(np.argsort(-s, kind="stable")[:6])
    p = np.exp(np.float64(s) - s.max())
    p /= p.sum()
    assert np.allclose(w, p[idx], rtol=0.07)  # fast exp: a few percent
    assert abs(float(sc.sum()) - 1.0) < 1e-5   # probabilities over all experts sum to 1


def test_combine_closed_form(B):
    eo = B.normal_f32(6 * 100, 99)
    w = B.normal_f32(6, 100)
    out = np.empty(100, np.float32)
    B.oracle().or_expert_combine(out, eo, w, 6, 100)
    ref = (w.astype(np.float64)[:, None] * eo.reshape(6, 100)).sum(axis=0)
    assert np.abs(out - ref).max() < 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_one_token_equals_decode_layer(B, mode):
    """The f64 prefill block on one token equals the decode layer (same routing) within f32 noise."""
    O = B.oracle()
    L = B.make_moe_layer(21, hidden=256, inter=128, n_experts=16)
    orl = L.or_layer()
    x = B.normal_f32(256, 102)
    o = np.empty(256, np.float32)
    idx = np.empty(6, np.int32)
    w = np.empty(6, np.float32)
    O.or_moe_layer_decode(o, x, C.byref(orl), mode, 0, 1, idx, w)
    pidx = np.empty(6, np.int32)
    pw = np.empty(6, np.float32)
    if mode == 1:
        O.or_prefill_route(pidx, pw, x, 1, C.byref(orl), mode)
        assert np.array_equal(pidx, idx)
    op = np.empty(256, np.float64)
    O.or_prefill_moe_f64(op, x, 1, C.byref(orl), idx, w)
    assert np.abs(op - o).max() / np.abs(op).max() < 1e-5
