"""GPU: the greedy token choice with the reference's repetition penalty and n-gram ban
(ds_moe_decoder.c:1036-1095, :1105-1237) — ds_hip_lm_head_sample and a stack with
ds_hip_stack_set_sampling against the oracle's or_lm_sample_greedy (pinned in
test_oracle_sample.py): tokens bit-identical, for both the fast and the full-logits paths."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_gpu_moe import run_stack, upload_layer  # noqa: E402
from test_oracle_sample import H, V, near_tie, setup  # noqa: E402

pytestmark = pytest.mark.gpu


def oracle_choice(B, W, x, hist, rp, ngram, T):
    h = np.ascontiguousarray(hist, np.int32) if len(hist) else None
    used = C.c_int(-1)
    t = B.oracle().or_lm_sample_greedy(np.ascontiguousarray(x, np.float32), W, H, V, h, len(hist), rp, ngram, T,
                                       C.byref(used))
    return t, used.value


def device_choice(dev, Wd, x, hist, rp, ngram):
    L = dev.load()
    xd = dev.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    hd = dev.DeviceBuffer.from_array(np.ascontiguousarray(hist, np.int32)) if len(hist) else None
    td = dev.DeviceBuffer(4)
    dev.check(L.ds_hip_lm_head_sample(xd.ptr, Wd.ptr, H, V, hd.ptr if hd else None, len(hist), rp, ngram, td.ptr),
              "sample")
    return int(td.to_array(np.int32)[0])


def cases(B):
    O = B.oracle()
    rng = np.random.default_rng(5)
    out = []
    for seed in range(6):
        W, x = setup(4800 + 10 * seed)
        best0 = O.or_argmax_bf16(x, W, H, V, 1, None)
        lg = np.empty(V, np.float32)
        O.or_argmax_logits_avx512(lg, x, W, H, V, 1)
        top = np.argsort(-lg)[:30]
        hist = list(rng.choice(top, 25)) + [best0, -4, V + 9]
        rng.shuffle(hist)
        out.append((W, x, hist, 1.3, 0))  # penalty only
        a, b = rng.integers(0, V, 2)
        out.append((W, x, hist + [a, b, best0] + hist[:3] + [a, b], 1.2, 3))  # banned: full path
        out.append((W, x, [3, best0, 11], 1.0, 1))  # every history token banned
        out.append((W, x, [], 1.5, 2))  # empty history
    for seed in (4700, 4710):
        W, x = near_tie(seed)
        out.append((W, x, [7, 1, 0, 9], 1.2, 0))  # the penalty switches to row 1
    return out


@pytest.mark.parametrize("T", [1, 8])
def test_lm_head_sample_vs_oracle(dev, B, T):
    L = dev.load()
    L.ds_set_threads(T)
    try:
        kinds = set()
        for W, x, hist, rp, ngram in cases(B):
            Wd = dev.DeviceBuffer.from_array(W)
            want, used = oracle_choice(B, W, x, hist, rp, ngram, T)
            got = device_choice(dev, Wd, x, hist, rp, ngram)
            assert got == want, (len(hist), rp, ngram, used)
            kinds.add(used)
        assert kinds == {0, 1}  # both paths ran
    finally:
        L.ds_set_threads(1)


@pytest.mark.parametrize("cap", [64, 3])
def test_stack_sampling_vs_oracle(dev, B, cap):
    """The same input every step: the argmax repeats, the n-gram rule then bans it (full path) on
    alternate steps; with cap 3 only the first three tokens count as history."""
    L = dev.load()
    lays = [B.make_moe_layer(80 + i, hidden=H, inter=128, n_experts=16) for i in range(2)]
    hs = [upload_layer(dev, lay) for lay in lays]
    W = B.normal_bf16(V * H, 81, 0.02)
    lm = dev.DeviceBuffer.from_array(W)
    x = B.normal_f32(H, 82)
    n_steps = 10
    arr = (C.c_void_p * len(hs))(*hs)
    S = L.ds_hip_stack_create(arr, len(hs), lm.ptr, V, dev.ROUTE_CFG)
    assert S, L.ds_hip_last_error()
    try:
        dev.check(L.ds_hip_stack_set_sampling(S, 1.3, 2, cap), "sampling")
        names = [L.ds_hip_stack_kernel_name(S, i).decode() for i in range(L.ds_hip_stack_kernel_count(S))]
        assert names[-1] == "sample"
        xd = dev.DeviceBuffer.from_array(x)
        td = dev.DeviceBuffer(4 * n_steps)
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, 0, 1, td.ptr, n_steps), "bind")
        assert L.ds_hip_stack_set_sampling(S, 1.0, 0, 0) == -1  # only before binding
        hidden = []
        for _ in range(n_steps):
            dev.check(L.ds_hip_stack_run(S, 1), "run")
            hx = np.empty(H, np.float32)
            dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
            hidden.append(hx)
        toks = td.to_array(np.int32)
        full = 0
        for s in range(n_steps):
            want, used = oracle_choice(B, W, hidden[s], toks[:min(s, cap)], 1.3, 2, 1)
            assert toks[s] == want, s
            full += used
        assert full >= 2 if cap > 3 else full >= 1
        assert len(set(toks.tolist())) >= 2
    finally:
        L.ds_hip_stack_destroy(S)
        for h in hs:
            L.ds_hip_layer_destroy(h)
