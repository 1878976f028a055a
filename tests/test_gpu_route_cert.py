"""Certified CFG expert selection on the GPU (dsh_cert.h; ds_hip_route_stats, ds_hip_set_route_log):
every decode routing, in the two-kernel layers (ds_hip_layer_forward and two-kernel stacks) and in
the one-kernel layers of the stacks (speculative selection, verified per XCD), must pick exactly the
experts, in rank order, that the reference's ds_moe_router + ds_moe_top_k pick on the same input
(the oracle's or_linear_f32 and or_moe_top_k, pinned to ds_kernels.c:639-652 and :193-243).

Each routing is logged with the input it was made on, so the check runs on the GPU's own layer
inputs at every layer and step. The routers are planted with near ties that no summation order
other than ds_linear's can rank: pairs of rows equal but for one coordinate moved by one ulp, and a
pair of identical rows (the lower index wins). Those ties send most routings to the recomputation in
ds_linear's order, and in the one-kernel layers make the speculative selection wrong often enough that
the extra blocks add the difference (corrections are counted). Weights: within 2 ulp (the device's correctly rounded expf
against the oracle's) where the output carries the weights of a recomputation in ds_linear's
order, else within 2e-5 relative (scores within the bound of ds_linear's)."""
import ctypes as C

import numpy as np
import pytest
from test_gpu_moe import make_device_layer, run_stack, upload_layer

pytestmark = pytest.mark.gpu


def planted_router(seed, E, H, pairs):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    for i in range(pairs):
        a, b = 2 * i, 2 * i + 1
        W[b] = W[a]
        k = (7 * i) % H
        W[b, k] = np.nextafter(W[a, k], np.float32(np.inf))
    W[E - 1] = W[E - 2]  # an exact tie: the lower index is ranked first
    return np.ascontiguousarray(W)


def bf16_of(B, W):
    return np.ascontiguousarray(B.f32_to_bf16_rne(W.reshape(-1)).reshape(W.shape))


class RouteLog:
    def __init__(self, dev, cap, H):
        self.dev, self.cap, self.H = dev, cap, H
        self.buf = dev.DeviceBuffer(4 * (64 + cap * (32 + H)))
        self.buf.write(np.zeros(64 + cap * (32 + H), np.int32))
        dev.check(dev.load().ds_hip_set_route_log(self.buf.ptr, cap), "route log")

    def close(self):
        self.dev.load().ds_hip_set_route_log(None, 0)

    def entries(self):
        a = self.buf.to_array(np.int32)
        n = int(a[0])
        assert n <= self.cap, (n, self.cap)
        e = a[64:64 + n * (32 + self.H)].reshape(n, 32 + self.H)
        return e[:, :8], e[:, 8:16].view(np.float32), e[:, 16], e[:, 17], e[:, 32:].view(np.float32)


def check_log(B, log, routers, K, label, expect=None, one_kernel=False):
    """Every logged routing against the oracle. Weights: exact (2 ulp) where the output carries the
    weights of a recomputation in ds_linear's order (two-kernel layers; one-kernel layers where the
    selection was corrected), else within 2e-5 (the one-kernel layers keep the weights of their
    speculative selection when its experts are the certified ones)."""
    idx, w, flags, tags, xs = log.entries()
    if expect is not None:
        assert len(idx) == expect, (len(idx), expect)
    n_re = 0
    for j in range(len(idx)):
        W = routers[int(tags[j])]
        E, H = W.shape
        s = np.empty(E, np.float32)
        B.oracle().or_linear_f32(s, np.ascontiguousarray(xs[j]), W, H, E)
        ri, rw = np.empty(K, np.int32), np.empty(K, np.float32)
        B.oracle().or_moe_top_k(ri, rw, s, E, K)
        assert np.array_equal(idx[j, :K], ri), (label, j, int(tags[j]), idx[j, :K], ri, int(flags[j]))
        n_re += int(flags[j] & 1)
        if flags[j] & 1 and (not one_kernel or flags[j] & 2):
            d = np.abs(w[j, :K].view(np.int32).astype(np.int64) - rw.view(np.int32).astype(np.int64))
            assert d.max() <= 2, (label, j, w[j, :K], rw)
        else:
            assert np.allclose(w[j, :K], rw, rtol=2e-5, atol=1e-7), (label, j, w[j, :K], rw)
    print(f"{label}: {len(idx)} routings equal to ds_moe_top_k on ds_linear's scores; {n_re} recomputed")
    return len(idx), n_re


def stats(L, reset=0):
    c = (C.c_ulonglong * 3)()
    assert L.ds_hip_route_stats(c, reset) == 0
    return list(c)


@pytest.mark.parametrize("shape", [(256, 128, 16, 6, 2), (1280, 896, 64, 6, 2)])
def test_layer_forward_certified(dev, B, shape):
    """ds_hip_layer_forward (two-kernel layer, CFG): 24 inputs through a layer with planted ties."""
    H, I, E, K, NS = shape
    L = dev.load()
    if H == 1280:
        h, rf, rb = make_device_layer(dev, 301)
    else:
        h = upload_layer(dev, B.make_moe_layer(301, hidden=H, inter=I, n_experts=E, top_k=K, n_shared=NS))
    W = planted_router(302, E, H, pairs=E // 4)
    Wb = bf16_of(B, W)
    dev.check(L.ds_hip_layer_set_router(h, W.ctypes.data, Wb.ctypes.data), "router")
    log = RouteLog(dev, 64, H)
    stats(L, 1)
    try:
        xd = dev.DeviceBuffer(4 * H)
        od = dev.DeviceBuffer(4 * H)
        idd, wd = dev.DeviceBuffer(4 * K), dev.DeviceBuffer(4 * K)
        for s in range(24):
            xd.write(B.normal_f32(H, 3030 + s))
            dev.check(L.ds_hip_layer_forward(h, od.ptr, xd.ptr, dev.ROUTE_CFG, 0, idd.ptr, wd.ptr), "forward")
        n, n_re = check_log(B, log, {0: W}, K, f"layer_forward {shape}", expect=24)
        c = stats(L)
        print(f"counters {c}")
        assert c[0] == 24 and c[1] == n_re and n_re >= 1
    finally:
        log.close()
        L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("kernels,ties", [(1, True), (2, True), (1, False)])
def test_config5_stack_routing_certified(dev, B, kernels, ties):
    """A config-5-shape stack (11 layers of the config-2 shape, the 129280 x 1280 head), 20 steps:
    all 220 routings equal the reference's on the GPU's own layer inputs, in the one-kernel layers
    (certified by their extra blocks) and in the two-kernel layers. With every router planted with
    near ties most routings are recomputed and some one-kernel outputs corrected; with plain random
    routers nearly every routing is certified from the intervals alone (in the one-kernel layers:
    the routed blocks' own selection certified as it stands)."""
    L = dev.load()
    n_layers, vocab, H, K, E, steps = 11, 129280, 1280, 6, 64, 20
    made = [make_device_layer(dev, 310 + l) for l in range(n_layers)]
    hs = [m[0] for m in made]
    routers = {}
    for l, h in enumerate(hs):
        if ties:
            W = planted_router(320 + l, E, H, pairs=16)
        else:
            W = (np.random.default_rng(320 + l).standard_normal((E, H)) * 0.02).astype(np.float32)
        Wb = bf16_of(B, W)  # held while the library reads it (a temporary's buffer is freed at once)
        dev.check(L.ds_hip_layer_set_router(h, W.ctypes.data, Wb.ctypes.data), "router")
        routers[l] = W
    lm = dev.DeviceBuffer(vocab * H * 2)
    dev.check(L.ds_hip_fill_normal_bf16(lm.ptr, vocab * H, 4343, 0.02), "fill")
    xs = np.stack([B.normal_f32(H, 3300 + s) for s in range(steps)])
    log = RouteLog(dev, n_layers * steps + 8, H)
    stats(L, 1)
    arr = (C.c_void_p * n_layers)(*hs)
    S = L.ds_hip_stack_create(arr, n_layers, lm.ptr, vocab, dev.ROUTE_CFG)
    assert S, L.ds_hip_last_error()
    try:
        xd = dev.DeviceBuffer.from_array(xs)
        td = dev.DeviceBuffer(4 * steps)
        dev.check(L.ds_hip_stack_set_layer_kernels(S, kernels == 1), "kernels")
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, steps, td.ptr, steps), "bind")
        assert L.ds_hip_stack_layer_kernels(S) == kernels
        print(f"config-5 stack, {kernels}-kernel layers: {steps} steps", flush=True)
        dev.check(L.ds_hip_stack_run(S, steps), "run")
        dev.check(L.ds_hip_sync(), "sync")
        n, n_re = check_log(B, log, routers, K, f"config-5 stack, {kernels}-kernel layers, ties {ties}",
                            expect=n_layers * steps, one_kernel=kernels == 1)
        c = stats(L)
        print(f"counters {c}")
        assert c[0] == n_layers * steps and c[1] == n_re
        if ties:
            assert n_re >= 1
            if kernels == 1:
                assert c[2] >= 1  # some layers' outputs were corrected to the certified selection
        else:
            assert n_re <= n // 10 and c[2] <= n // 10, c
    finally:
        L.ds_hip_stack_destroy(S)
        log.close()
        for h in hs:
            L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("path", ["layer_forward", "stack1", "stack2"])
def test_nonfinite_inputs_route_like_reference(dev, B, path):
    """Inputs with a +inf, a NaN or a -inf coordinate (CFG routing, whose reference selection is
    defined for them: ds_moe_top_k never selects a NaN or floor score and fills empty slots with
    expert 0, weight 0). Such scores or bounds are never certified, so every expert's score is
    recomputed in ds_linear's order: an expert's score is ±inf by the sign of its router weight at the
    +inf coordinate, the +inf scores tie (the lowest indices win) and their softmax weights are NaN as
    in the reference; a NaN input selects nothing. One +inf coordinate is picked where fewer than K
    experts, expert 0 among them, have a positive router weight: the empty slots then repeat expert 0,
    which the one-kernel layers' verifier must not take for a selected expert. Every logged routing
    (two-kernel layer, one- and two-kernel stacks, whose later layers see the non-finite outputs) must
    give the oracle's indices, NaN weights where the oracle's are NaN, the rest within 2e-5."""
    L = dev.load()
    H, I, E, K, NS, nl = 256, 128, 16, 6, 2, 3
    lays = [B.make_moe_layer(330 + l, hidden=H, inter=I, n_experts=E, top_k=K, n_shared=NS) for l in range(nl)]
    hs = [upload_layer(dev, lay) for lay in lays]
    routers = {l: np.ascontiguousarray(lays[l].router_f32.reshape(E, H)) for l in range(nl)}
    pos = (routers[0] > 0).sum(axis=0)
    few = [c for c in range(H) if routers[0][0, c] > 0 and 2 <= pos[c] <= K - 2]
    many = [c for c in range(H) if pos[c] >= K + 2]
    assert few and many
    xs = np.stack([B.normal_f32(H, 3400 + s) for s in range(6)])
    xs[1, few[0]] = np.inf
    xs[2, 9] = np.nan
    xs[4, 3] = -np.inf
    xs[5, many[0]] = np.inf
    steps = len(xs)
    log = RouteLog(dev, 64, H)
    try:
        if path == "layer_forward":
            xd, od = dev.DeviceBuffer(4 * H), dev.DeviceBuffer(4 * H)
            for s in range(steps):
                xd.write(xs[s])
                dev.check(L.ds_hip_layer_forward(hs[0], od.ptr, xd.ptr, dev.ROUTE_CFG, 0, None, None), "forward")
            dev.check(L.ds_hip_sync(), "sync")
            expect = steps
        else:
            lm_w = B.normal_bf16(5000 * H, 3401, 0.02)
            lm = dev.DeviceBuffer.from_array(lm_w)
            run_stack(dev, hs, lm, 5000, xs, dev.ROUTE_CFG, kernels=1 if path == "stack1" else 2)
            expect = nl * steps
        idx, w, flags, tags, lx = log.entries()
        assert len(idx) == expect, (len(idx), expect)
        n_nan = n_empty = 0
        for j in range(len(idx)):
            W = routers[int(tags[j]) if path != "layer_forward" else 0]
            sc = np.empty(E, np.float32)
            B.oracle().or_linear_f32(sc, np.ascontiguousarray(lx[j]), W, H, E)
            ri, rw = np.empty(K, np.int32), np.empty(K, np.float32)
            B.oracle().or_moe_top_k(ri, rw, sc, E, K)
            assert np.array_equal(idx[j, :K], ri), (path, j, idx[j, :K], ri, int(flags[j]))
            nan = np.isnan(rw)
            n_nan += int(nan.any())
            n_empty += int(not np.isnan(sc).all() and (rw == 0).any() and ri[0] == 0)
            assert np.array_equal(np.isnan(w[j, :K]), nan), (path, j, w[j, :K], rw)
            assert np.allclose(w[j, :K][~nan], rw[~nan], rtol=2e-5, atol=1e-7), (path, j, w[j, :K], rw)
        print(f"{path}: {len(idx)} routings with non-finite inputs equal to the reference's "
              f"({n_nan} with NaN weights, {n_empty} with expert 0 selected and empty slots)")
        assert n_nan >= 2 and n_empty >= 1
    finally:
        log.close()
        for h in hs:
            L.ds_hip_layer_destroy(h)
