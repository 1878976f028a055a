"""The decode stack's input and output on the GPU: the capacity the bound buffers give (calls that
would run past it are refused before anything is launched), and the autoregressive embedding feed
(ds_ocr.c:2271-2278: each step's input is the widened bf16 embedding of the previous step's token,
written on the device), against the oracle composed the same way."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from test_gpu_moe import oracle_decode, rel_err, upload_layer  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-3


def small_stack(dev, B, seed, n_layers=2, H=256, vocab=3000):
    lays = [B.make_moe_layer(seed + i, hidden=H, inter=128, n_experts=16) for i in range(n_layers)]
    hs = [upload_layer(dev, lay) for lay in lays]
    lm_w = B.normal_bf16(vocab * H, seed + 50, 0.02)
    return lays, hs, lm_w


def widen(row_bf16):
    return (row_bf16.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("kernels", [1, 2])
def test_capacity_refuses_overrun_before_launch(dev, B, kernels):
    L = dev.load()
    H, vocab = 256, 3000
    lays, hs, lm_w = small_stack(dev, B, 500)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(H, 5000 + s) for s in range(3)])
    xd = dev.DeviceBuffer.from_array(xs)
    td = dev.DeviceBuffer(4 * 4)
    td.write(np.full(4, -7, np.int32))
    arr = (C.c_void_p * len(hs))(*hs)
    S = L.ds_hip_stack_create(arr, len(hs), lm.ptr, vocab, dev.ROUTE_CFG)
    assert S, L.ds_hip_last_error()
    try:
        dev.check(L.ds_hip_stack_set_layer_kernels(S, 1 if kernels == 1 else 0), "kernels")
        assert L.ds_hip_stack_bind(S, xd.ptr, H, 0, td.ptr, 4) == -1  # no rows
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, 3, td.ptr, 4), "bind")
        assert L.ds_hip_stack_capacity(S) == 3 and L.ds_hip_stack_steps_left(S) == 3
        dev.check(L.ds_hip_stack_run(S, 2), "run")
        assert L.ds_hip_stack_run(S, 2) == -1  # 2 + 2 > 3 rows of input
        assert b"capacity" in L.ds_hip_last_error()
        ms = C.c_float(0)
        assert L.ds_hip_time_stack(S, 2, C.byref(ms)) == -1
        assert L.ds_hip_stack_run_eager(S, 2) == -1
        assert L.ds_hip_profile_stack(S, 2, np.zeros(64, np.float32)) == -1
        assert L.ds_hip_time_stack_each(S, 2, np.zeros(2, np.float32)) == -1
        assert L.ds_hip_stack_steps_left(S) == 1
        dev.check(L.ds_hip_sync(), "sync")
        t = td.to_array(np.int32)
        assert (t[:2] >= 0).all() and t[2] == -7 and t[3] == -7  # the refused calls launched nothing
        dev.check(L.ds_hip_stack_run(S, 1), "run")
        assert L.ds_hip_stack_run(S, 1) == -1
        dev.check(L.ds_hip_stack_reset(S), "reset")
        dev.check(L.ds_hip_stack_run(S, 3), "run after reset")
        dev.check(L.ds_hip_sync(), "sync")
        assert td.to_array(np.int32)[3] == -7
        # stride 0: the token slots are the limit
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, 0, 1, td.ptr, 4), "bind")
        assert L.ds_hip_stack_capacity(S) == 4
        dev.check(L.ds_hip_stack_run(S, 4), "run")
        assert L.ds_hip_stack_run(S, 1) == -1
        dev.check(L.ds_hip_sync(), "sync")
    finally:
        L.ds_hip_stack_destroy(S)
        for h in hs:
            L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("mode,kernels", [(1, 1), (1, 2), (0, 1)])
def test_embedding_feed_autoregressive(dev, B, mode, kernels):
    """Six fed-back steps: step 0 reads the bound row, every later step the embedding of the token the
    step before chose; tokens and hidden states against the oracle fed the GPU's own tokens (so a
    near tie cannot make the two runs diverge), and the tokens must equal the oracle's argmax of
    the GPU's hidden state bit for bit. Graph and eager runs agree on the tokens."""
    L = dev.load()
    H, vocab, n = 256, 3000, 6
    lays, hs, lm_w = small_stack(dev, B, 520)
    emb = B.normal_bf16(vocab * H, 530, 0.5).reshape(vocab, H)
    lm = dev.DeviceBuffer.from_array(lm_w)
    ed = dev.DeviceBuffer.from_array(emb)
    x0 = B.normal_f32(H, 5300)
    xd = dev.DeviceBuffer.from_array(x0)
    td = dev.DeviceBuffer(4 * n)
    arr = (C.c_void_p * len(hs))(*hs)
    S = L.ds_hip_stack_create(arr, len(hs), lm.ptr, vocab, mode)
    assert S, L.ds_hip_last_error()
    try:
        dev.check(L.ds_hip_stack_set_layer_kernels(S, 1 if kernels == 1 else 0), "kernels")
        dev.check(L.ds_hip_stack_set_embedding(S, ed.ptr, vocab), "embedding")
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, 1, td.ptr, n), "bind")
        assert L.ds_hip_stack_capacity(S) == n  # one input row serves: later inputs come from the table
        hid = []
        for _ in range(n):
            dev.check(L.ds_hip_stack_run(S, 1), "run")
            hx = np.empty(H, np.float32)
            dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
            hid.append(hx)
        toks = td.to_array(np.int32)
        x = x0.copy()
        for s in range(n):
            _, rh = oracle_decode(B, lays, lm_w, vocab, x[None, :], mode)
            err = rel_err(hid[s], rh[0])
            want = B.oracle().or_argmax_bf16(hid[s], lm_w, H, vocab, 1, None)
            print(f"embedding feed mode {mode} kernels {kernels} step {s}: token {toks[s]} (oracle on GPU state "
                  f"{want}), hidden err {err:.2e}")
            assert err < TOL and toks[s] == want
            x = widen(emb[toks[s]])
        dev.check(L.ds_hip_stack_reset(S), "reset")
        dev.check(L.ds_hip_stack_run_eager(S, n), "eager")
        assert np.array_equal(td.to_array(np.int32), toks)
    finally:
        L.ds_hip_stack_destroy(S)
        for h in hs:
            L.ds_hip_layer_destroy(h)


def test_embedding_feed_with_sampling(dev, B):
    """With the repetition penalty and n-gram ban after the argmax, the fed-back row is the embedding
    of the token the rules chose (written after them)."""
    L = dev.load()
    H, vocab, n = 256, 3000, 8
    lays, hs, lm_w = small_stack(dev, B, 540)
    emb = B.normal_bf16(vocab * H, 550, 0.5).reshape(vocab, H)
    lm = dev.DeviceBuffer.from_array(lm_w)
    ed = dev.DeviceBuffer.from_array(emb)
    x0 = B.normal_f32(H, 5500)
    xd = dev.DeviceBuffer.from_array(x0)
    td = dev.DeviceBuffer(4 * n)
    arr = (C.c_void_p * len(hs))(*hs)
    S = L.ds_hip_stack_create(arr, len(hs), lm.ptr, vocab, dev.ROUTE_CFG)
    assert S, L.ds_hip_last_error()
    try:
        dev.check(L.ds_hip_stack_set_sampling(S, 1.3, 2, n), "sampling")
        dev.check(L.ds_hip_stack_set_embedding(S, ed.ptr, vocab), "embedding")
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, 0, 1, td.ptr, n), "bind")
        hid = []
        for _ in range(n):
            dev.check(L.ds_hip_stack_run(S, 1), "run")
            hx = np.empty(H, np.float32)
            dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
            hid.append(hx)
        toks = td.to_array(np.int32)
        x = x0.copy()
        for s in range(n):
            _, rh = oracle_decode(B, lays, lm_w, vocab, x[None, :], dev.ROUTE_CFG)
            assert rel_err(hid[s], rh[0]) < TOL
            x = widen(emb[toks[s]])  # the next input is the embedding of the token the rules chose
    finally:
        L.ds_hip_stack_destroy(S)
        for h in hs:
            L.ds_hip_layer_destroy(h)


def test_rewritten_input_rows_are_seen(dev, B):
    """One-kernel layers in CFG routing: the step's final kernel also computes the next step's first
    router partials, and every run call recomputes the current step's. Rows of the bound input the
    caller rewrites between run calls must be what the later steps read: two steps, rows 2 and 3
    rewritten, two more steps; those steps against a stack bound to the rewritten rows from the
    start and against the oracle."""
    L = dev.load()
    H, vocab, n = 256, 3000, 4
    lays, hs, lm_w = small_stack(dev, B, 560)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(H, 5600 + s) for s in range(n)])
    xs_new = xs.copy()
    xs_new[2:] = np.stack([B.normal_f32(H, 5700 + s) for s in range(2)])
    arr = (C.c_void_p * len(hs))(*hs)

    def run(x_bind, rewrite):
        xd = dev.DeviceBuffer.from_array(x_bind)
        td = dev.DeviceBuffer(4 * n)
        S = L.ds_hip_stack_create(arr, len(hs), lm.ptr, vocab, dev.ROUTE_CFG)
        assert S, L.ds_hip_last_error()
        try:
            dev.check(L.ds_hip_stack_set_layer_kernels(S, 1), "kernels")
            dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, n, td.ptr, n), "bind")
            names = [L.ds_hip_stack_kernel_name(S, i).decode() for i in range(L.ds_hip_stack_kernel_count(S))]
            assert names[-1] == "lm_head.final+scores" and "scores" not in names, names
            hid = []
            for s in range(n):
                if s == 2 and rewrite:
                    dev.check(L.ds_hip_sync(), "sync")
                    xd.write(xs_new)
                dev.check(L.ds_hip_stack_run(S, 1), "run")
                hx = np.empty(H, np.float32)
                dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
                hid.append(hx)
            return td.to_array(np.int32), np.stack(hid)
        finally:
            L.ds_hip_stack_destroy(S)

    try:
        toks, hid = run(xs, True)
        toks_ref, hid_ref = run(xs_new, False)
        _, rh = oracle_decode(B, lays, lm_w, vocab, xs_new, dev.ROUTE_CFG)
        for s in range(n):
            err, err_ref = rel_err(hid[s], rh[s]), rel_err(hid[s], hid_ref[s])
            print(f"rewritten input, step {s}: vs oracle {err:.2e}, vs a stack bound to the new rows {err_ref:.2e}")
            assert err < TOL and err_ref < 1e-5
            assert toks[s] == B.oracle().or_argmax_bf16(hid[s], lm_w, H, vocab, 1, None)
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)


def test_step_ending_at_the_lm_head_across_runs(dev, B):
    """Three one-kernel layers, CFG routing, bound input: the step ends with the LM head. The last
    layer's extra blocks compute the next step's router partials, the next step's first layer turns
    the previous step's keys into its token, and one kernel after each run finishes the last token.
    Eight steps run in chunks (1, 0 and 3 graph steps, 2 eager steps, then 2 graph steps after rows 6
    and 7 are rewritten) must give every token and the chunk-end hidden states of a stack bound to
    the final rows and run one step per call, and the oracle's hidden states."""
    L = dev.load()
    H, vocab, n = 256, 3000, 8
    lays, hs, lm_w = small_stack(dev, B, 580, n_layers=3)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(H, 5800 + s) for s in range(n)])
    xs_new = xs.copy()
    xs_new[6:] = np.stack([B.normal_f32(H, 5900 + s) for s in range(2)])
    arr = (C.c_void_p * len(hs))(*hs)

    def make(xd, td):
        S = L.ds_hip_stack_create(arr, len(hs), lm.ptr, vocab, dev.ROUTE_CFG)
        assert S, L.ds_hip_last_error()
        dev.check(L.ds_hip_stack_set_layer_kernels(S, 1), "kernels")
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, n, td.ptr, n), "bind")
        names = [L.ds_hip_stack_kernel_name(S, i).decode() for i in range(L.ds_hip_stack_kernel_count(S))]
        assert names == ["layer"] * 3 + ["lm_head.argmax"], names
        return S

    def hidden(S):
        hx = np.empty(H, np.float32)
        dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
        return hx

    try:
        # reference: bound to the final rows, one step per run call
        xd_r, td_r = dev.DeviceBuffer.from_array(xs_new), dev.DeviceBuffer(4 * n)
        S = make(xd_r, td_r)
        try:
            hid_ref = []
            for s in range(n):
                dev.check(L.ds_hip_stack_run(S, 1), "run")
                hid_ref.append(hidden(S))
            toks_ref = td_r.to_array(np.int32)
        finally:
            L.ds_hip_stack_destroy(S)
        # chunked: the steps that end each chunk are 0, 3, 5 and 7
        xd, td = dev.DeviceBuffer.from_array(xs), dev.DeviceBuffer(4 * n)
        S = make(xd, td)
        ends = {}
        try:
            dev.check(L.ds_hip_stack_run(S, 1), "run 1")
            ends[0] = hidden(S)
            dev.check(L.ds_hip_stack_run(S, 0), "run 0")
            dev.check(L.ds_hip_stack_run(S, 3), "run 3")
            ends[3] = hidden(S)
            dev.check(L.ds_hip_stack_run_eager(S, 2), "eager 2")
            ends[5] = hidden(S)
            dev.check(L.ds_hip_sync(), "sync")
            xd.write(xs_new)
            dev.check(L.ds_hip_stack_run(S, 2), "run 2")
            ends[7] = hidden(S)
            toks = td.to_array(np.int32)
        finally:
            L.ds_hip_stack_destroy(S)
        _, rh = oracle_decode(B, lays, lm_w, vocab, xs_new, dev.ROUTE_CFG)
        for s in range(n):
            err = rel_err(hid_ref[s], rh[s])
            assert err < TOL, (s, err)
            assert toks_ref[s] == B.oracle().or_argmax_bf16(hid_ref[s], lm_w, H, vocab, 1, None), s
        for s, hx in ends.items():
            err, err_ref = rel_err(hx, rh[s]), rel_err(hx, hid_ref[s])
            print(f"chunked run, step {s}: vs oracle {err:.2e}, vs one step per call {err_ref:.2e}")
            assert err < TOL and err_ref < 1e-5
            assert toks[s] == B.oracle().or_argmax_bf16(hx, lm_w, H, vocab, 1, None), s
        assert np.array_equal(toks, toks_ref), (toks, toks_ref)
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("mode,kernels,feed", [(1, 1, False), (1, 2, False), (0, 1, False), (1, 1, True)])
def test_steps_per_graph_launch(dev, B, mode, kernels, feed):
    """Runs of several steps launch a graph of k steps at a time, then 1-step graphs: 11 steps with
    k = 1 and with k = 4 (two 4-step launches and three single ones, and again through the timed
    run) give the same tokens, and the same last hidden state (bit for bit with the two-kernel
    layers; within the one-kernel layers' float-atomic order otherwise). Three layers, so the bound
    input's steps end at the LM head (the last layer's extra blocks and the token of the next step's
    first layer), and the embedding feed (each step's input from the token before)."""
    L = dev.load()
    H, vocab, n = 256, 3000, 11
    lays, hs, lm_w = small_stack(dev, B, 540, n_layers=3)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(H, 5400 + s) for s in range(n)])
    xd = dev.DeviceBuffer.from_array(xs)
    emb = B.normal_bf16(vocab * H, 541, 0.5).reshape(vocab, H)
    ed = dev.DeviceBuffer.from_array(emb)
    td = dev.DeviceBuffer(4 * n)
    arr = (C.c_void_p * len(hs))(*hs)
    S = L.ds_hip_stack_create(arr, len(hs), lm.ptr, vocab, mode)
    assert S, L.ds_hip_last_error()
    try:
        assert L.ds_hip_stack_set_graph_steps(S, 0) == -1 and L.ds_hip_stack_set_graph_steps(S, 17) == -1
        dev.check(L.ds_hip_stack_set_layer_kernels(S, 1 if kernels == 1 else 0), "kernels")
        if feed:
            dev.check(L.ds_hip_stack_set_embedding(S, ed.ptr, vocab), "embedding")
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, 1 if feed else n, td.ptr, n), "bind")
        runs = []
        for k, timed in [(1, False), (4, False), (4, True), (1, True)]:
            dev.check(L.ds_hip_stack_set_graph_steps(S, k), "graph steps")
            dev.check(L.ds_hip_stack_reset(S), "reset")
            td.write(np.full(n, -1, np.int32))
            if timed:
                ms = C.c_float(0)
                dev.check(L.ds_hip_time_stack(S, n, C.byref(ms)), "timed run")
            else:
                dev.check(L.ds_hip_stack_run(S, n), "run")
            hx = np.empty(H, np.float32)
            dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
            runs.append((k, timed, td.to_array(np.int32), hx))
            assert L.ds_hip_stack_steps_left(S) == 0
        k0, _, t0, h0 = runs[0]
        assert (t0 >= 0).all() and (t0 < vocab).all()
        for k, timed, t, hx in runs[1:]:
            err = rel_err(hx, h0)
            print(f"mode {mode} kernels {kernels} feed {feed}: k={k} timed={timed} tokens equal "
                  f"{int((t == t0).sum())}/{n}, hidden err {err:.2e}")
            assert np.array_equal(t, t0)
            if kernels == 2:
                assert np.array_equal(hx.view(np.uint32), h0.view(np.uint32))
            else:
                assert err < 1e-5
    finally:
        L.ds_hip_stack_destroy(S)
        for h in hs:
            L.ds_hip_layer_destroy(h)
