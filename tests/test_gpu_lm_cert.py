"""The decode stack's bounded LM head (ds_hip_stack_set_lm_certified: an int8 copy of the head with
per-row bounds on the exact logit, then the reference's order on each block's rows whose bound
reaches the block's best lower bound) against the one-pass head and the oracle's argmax of the same hidden state
(or_argmax_bf16, the reference's ds_argmax_matvec_bf16): tokens bit for bit. Heads: random, and
planted with exact ties (the lowest index wins), one-ulp near ties (the exact order decides), rows
that all bound together (every row a candidate), a NaN in the best row (never chosen), an all-zero
head, and a head rewritten after the stack was created (the copy rebuilt)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from test_gpu_moe import upload_layer  # noqa: E402

pytestmark = pytest.mark.gpu
BF16_NAN = 0x7FC0


def layers(dev, B, seed, H, n_layers=2):
    lays = [B.make_moe_layer(seed + i, hidden=H, inter=128, n_experts=16) for i in range(n_layers)]
    return lays, [upload_layer(dev, lay) for lay in lays]


def run_stack(dev, hs, lm_w, vocab, xs, cert, kernels, rewrite=None):
    """Tokens and hidden states of len(xs) steps; rewrite (optional): a head written over the first
    one after the stack was created, before the copy is rebuilt."""
    L = dev.load()
    H = xs.shape[1]
    lm = dev.DeviceBuffer.from_array(lm_w)
    xd = dev.DeviceBuffer.from_array(xs)
    n = xs.shape[0]
    td = dev.DeviceBuffer(4 * n)
    arr = (C.c_void_p * len(hs))(*hs)
    T0 = L.ds_get_threads()
    L.ds_set_threads(1)  # the reference's thread count: one chunk, whole groups of 4 rows
    S = L.ds_hip_stack_create(arr, len(hs), lm.ptr, vocab, dev.ROUTE_CFG)
    L.ds_set_threads(T0)
    assert S, L.ds_hip_last_error()
    try:
        dev.check(L.ds_hip_stack_set_layer_kernels(S, 1 if kernels == 1 else 0), "kernels")
        if rewrite is not None:
            lm.write(rewrite)
        dev.check(L.ds_hip_stack_set_lm_certified(S, cert), "certified")
        assert L.ds_hip_stack_lm_certified(S) == cert
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, n, td.ptr, n), "bind")
        hid = []
        for _ in range(n):
            dev.check(L.ds_hip_stack_run(S, 1), "run")
            hx = np.empty(H, np.float32)
            dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
            hid.append(hx)
        return td.to_array(np.int32), np.stack(hid)
    finally:
        L.ds_hip_stack_destroy(S)


def check(B, lm_w, vocab, H, toks, hid, label):
    for s in range(len(toks)):
        want = B.oracle().or_argmax_bf16(hid[s], lm_w, H, vocab, 1, None)
        print(f"{label} step {s}: token {toks[s]} oracle {want}")
        assert toks[s] == want


@pytest.mark.parametrize("kernels", [1, 2])
@pytest.mark.parametrize("H,vocab", [(256, 3000), (512, 20480), (768, 5000), (1280, 8192), (2048, 4096)])
def test_bounded_head_random(dev, B, H, vocab, kernels):
    L = dev.load()
    lays, hs = layers(dev, B, 700 + H, H)
    try:
        lm_w = B.normal_bf16(vocab * H, 710 + H, 0.02)
        xs = np.stack([B.normal_f32(H, 7200 + s) for s in range(6)])
        t1, h1 = run_stack(dev, hs, lm_w, vocab, xs, 1, kernels)
        check(B, lm_w, vocab, H, t1, h1, f"bounded H {H} vocab {vocab} kernels {kernels}")
        t0, h0 = run_stack(dev, hs, lm_w, vocab, xs, 0, kernels)
        check(B, lm_w, vocab, H, t0, h0, f"one-pass H {H} vocab {vocab} kernels {kernels}")
        if kernels == 2:  # deterministic layers: the same hidden states, so the same tokens
            assert np.array_equal(h0, h1) and np.array_equal(t0, t1)
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)


def planted_head(B, kind, h0, vocab, H, seed):
    """A head whose argmax for the hidden state h0 is decided by the planted rows."""
    W = B.normal_bf16(vocab * H, seed, 0.02).reshape(vocab, H)
    big = B.f32_to_bf16_rne(np.sign(h0) * 0.05)
    a, b = vocab // 3, vocab - 5
    if kind == "ties":
        W[a] = big
        W[b] = big
    elif kind == "near":
        W[a] = big
        W[b] = big
        # one bf16 ulp more magnitude in the column of h0's largest entry: w and h share signs
        # there, so row b's logit is slightly larger than row a's
        j = int(np.argmax(np.abs(h0)))
        W[b, j] = W[b, j] + 1
    elif kind == "flat":
        W[:] = W[7]
    elif kind == "nan":
        W[a] = big
        W[a, H // 2] = BF16_NAN
        W[b] = B.f32_to_bf16_rne(np.sign(h0) * 0.04)
    elif kind == "zero":
        W[:] = 0
    return np.ascontiguousarray(W)


@pytest.mark.parametrize("kind", ["ties", "near", "flat", "nan", "zero"])
def test_bounded_head_planted(dev, B, kind):
    L = dev.load()
    H, vocab = 256, 6000
    lays, hs = layers(dev, B, 760, H)
    try:
        xs = np.stack([B.normal_f32(H, 7600 + s) for s in range(2)])
        base = B.normal_bf16(vocab * H, 761, 0.02)
        _, h_ref = run_stack(dev, hs, base, vocab, xs, 0, 2)
        lm_w = planted_head(B, kind, h_ref[0], vocab, H, 761)
        t1, h1 = run_stack(dev, hs, lm_w, vocab, xs, 1, 2)
        t0, h0 = run_stack(dev, hs, lm_w, vocab, xs, 0, 2)
        assert np.array_equal(h0, h1) and np.array_equal(h1[0], h_ref[0])
        check(B, lm_w, vocab, H, t1, h1, f"planted {kind}")
        assert np.array_equal(t0, t1)
        if kind == "ties":
            assert t1[0] == vocab // 3
        if kind in ("flat", "zero"):
            assert t1[0] == 0
        if kind in ("nan", "near"):
            assert t1[0] == vocab - 5
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)


def test_bounded_head_rebuilt_after_rewrite(dev, B):
    """The copy is built from the head's contents: rewriting the head and calling
    ds_hip_stack_set_lm_certified(S, 1) again gives the new head's tokens."""
    L = dev.load()
    H, vocab = 256, 4000
    lays, hs = layers(dev, B, 780, H)
    try:
        xs = np.stack([B.normal_f32(H, 7800 + s) for s in range(3)])
        first = B.normal_bf16(vocab * H, 781, 0.02)
        second = B.normal_bf16(vocab * H, 782, 0.02)
        t1, h1 = run_stack(dev, hs, first, vocab, xs, 1, 2, rewrite=second)
        check(B, second, vocab, H, t1, h1, "rewritten head")
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)
