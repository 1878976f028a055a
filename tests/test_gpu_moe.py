"""GPU parity of the device-resident MoE layer and the decode stack (include/ds_hip.h) against the
oracle: small shapes first, then the DeepSeek-OCR shapes (config 2: one 64-expert layer; config 5:
11 layers + the 129280-row argmax LM head)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import golden_cases as G  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-3


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def rel_err(a, ref):
    a, ref = np.asarray(a, np.float64), np.asarray(ref, np.float64)
    return np.abs(a - ref).max() / max(np.abs(ref).max(), 1e-30)


def upload_layer(dev, lay):
    """A device layer holding the host layer's INT8 blocks and routers."""
    L = dev.load()
    h = L.ds_hip_layer_create(lay.hidden, lay.inter, lay.n_experts, lay.top_k, lay.shared_inter)
    assert h, L.ds_hip_last_error()
    dev.check(L.ds_hip_layer_set_router(h, lay.router_f32.ctypes.data, lay.router_bf16.ctypes.data), "router")
    keep = []
    for e in range(lay.n_experts):
        g, d = lay.gu[e], lay.dn[e]
        gb, db = dev.block_from_arrays(g.q, g.scale, g.offset), dev.block_from_arrays(d.q, d.scale, d.offset)
        keep.append((gb, db))
        dev.check(L.ds_hip_layer_set_expert(h, e, C.byref(gb), C.byref(db)), "expert")
    gb = dev.block_from_arrays(lay.sgu.q, lay.sgu.scale, lay.sgu.offset)
    db = dev.block_from_arrays(lay.sdn.q, lay.sdn.scale, lay.sdn.offset)
    dev.check(L.ds_hip_layer_set_expert(h, -1, C.byref(gb), C.byref(db)), "shared")
    return h


def layer_forward(dev, h, x, mode, residual=0, K=6):
    L = dev.load()
    xd = dev.DeviceBuffer.from_array(x)
    od = dev.DeviceBuffer(x.nbytes)
    idd = dev.DeviceBuffer(4 * K)
    wd = dev.DeviceBuffer(4 * K)
    dev.check(L.ds_hip_layer_forward(h, od.ptr, xd.ptr, mode, residual, idd.ptr, wd.ptr), "forward")
    return od.to_array(np.float32), idd.to_array(np.int32), wd.to_array(np.float32)


@pytest.mark.parametrize("sim", [0, 1])
@pytest.mark.parametrize("mode", [0, 1])
def test_small_layer_vs_oracle(dev, B, mode, sim):
    L = dev.load()
    lay = G.small_layer()
    h = upload_layer(dev, lay)
    orl = lay.or_layer()
    try:
        dev.set_bf16sim(sim)
        for s in range(3):
            x = B.normal_f32(lay.hidden, 900 + s)
            out, idx, w = layer_forward(dev, h, x, mode)
            ro = np.empty(lay.hidden, np.float32)
            ri = np.empty(6, np.int32)
            rw = np.empty(6, np.float32)
            B.oracle().or_moe_layer_decode(ro, x, C.byref(orl), mode, sim, 1, ri, rw)
            assert np.array_equal(idx, ri)
            if mode == 0:
                assert np.array_equal(bits(w), bits(rw))  # bit-exact bf16 router + fast-exp softmax
            else:
                assert np.abs(w - rw).max() < 1e-5
            err = rel_err(out, ro)
            print(f"small layer mode={mode} sim={sim} seed={s}: {err:.2e}")
            outr, _, _ = layer_forward(dev, h, x, mode, residual=1)
            if sim and np.array_equal(bits(w), bits(rw)):  # every rounded value in the reference's order
                assert np.array_equal(bits(out), bits(ro))
                assert np.array_equal(bits(outr), bits(x + ro))
            elif sim:  # CFG: glibc's expf 1 ulp off the correctly rounded weight (8.7e-5 of arguments)
                assert err < 1e-6
            else:
                assert err < TOL
                assert rel_err(outr, x + ro) < TOL
    finally:
        dev.set_bf16sim(0)
        L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("threads", [6, 5, 3, 16])
def test_decode_routing_over_thread_chunks(dev, B, threads):
    """DECODE-mode router scores follow the reference's row chunking over its threads: with these
    counts some rows take the 2-row and the single-row AVX-512 paths. Expert ids and weights must be
    bit-identical to the oracle run with the same thread count."""
    L = dev.load()
    lay = B.make_moe_layer(71, hidden=512, inter=128, n_experts=18, top_k=6, n_shared=2)
    h = upload_layer(dev, lay)
    orl = lay.or_layer()
    try:
        L.ds_set_threads(threads)
        for s in range(3):
            x = B.normal_f32(lay.hidden, 7100 + s)
            out, idx, w = layer_forward(dev, h, x, dev.ROUTE_DECODE)
            ro = np.empty(lay.hidden, np.float32)
            ri = np.empty(6, np.int32)
            rw = np.empty(6, np.float32)
            B.oracle().or_moe_layer_decode(ro, x, C.byref(orl), 0, 0, threads, ri, rw)
            assert np.array_equal(idx, ri)
            assert np.array_equal(bits(w), bits(rw))
            assert rel_err(out, ro) < TOL
    finally:
        L.ds_set_threads(1)
        L.ds_hip_layer_destroy(h)


def test_layer_rejects_unsupported_shape(dev):
    L = dev.load()
    assert not L.ds_hip_layer_create(256, 100, 16, 6, 200)
    assert b"not supported" in L.ds_hip_last_error()


def make_device_layer(dev, seed, H=1280, I=896, E=64, K=6, SI=1792):
    """Config-2 layer generated and quantized on the device (seeded N(0, 0.02) bf16 weights)."""
    L = dev.load()
    h = L.ds_hip_layer_create(H, I, E, K, SI)
    assert h, L.ds_hip_last_error()
    gu = dev.DeviceBuffer(2 * SI * H * 2)
    dn = dev.DeviceBuffer(H * SI * 2)
    rb = dev.DeviceBuffer(E * H * 2)
    rf = dev.DeviceBuffer(E * H * 4)
    base = seed * 1000
    for e in range(E):
        dev.check(L.ds_hip_fill_normal_bf16(gu.ptr, 2 * I * H, base + 10 + 2 * e, 0.02), "fill")
        dev.check(L.ds_hip_fill_normal_bf16(dn.ptr, H * I, base + 11 + 2 * e, 0.02), "fill")
        dev.check(L.ds_hip_layer_quantize_expert(h, e, gu.ptr, dn.ptr), "quantize")
    dev.check(L.ds_hip_fill_normal_bf16(gu.ptr, 2 * SI * H, base + 900, 0.02), "fill")
    dev.check(L.ds_hip_fill_normal_bf16(dn.ptr, H * SI, base + 901, 0.02), "fill")
    dev.check(L.ds_hip_layer_quantize_expert(h, -1, gu.ptr, dn.ptr), "quantize")
    dev.check(L.ds_hip_fill_normal_f32(rf.ptr, E * H, base + 1, 0.0, 0.02), "fill")
    dev.check(L.ds_hip_fill_normal_bf16(rb.ptr, E * H, base + 1, 0.02), "fill")
    dev.check(L.ds_hip_layer_set_router_dev(h, rf.ptr, rb.ptr), "router")
    dev.check(L.ds_hip_sync(), "sync")
    return h, rf, rb


def export_layer(dev, B, h, rf, rb, H=1280, I=896, E=64, K=6, SI=1792):
    L = dev.load()

    def blk(e, shared):
        ii = SI if shared else I
        gq = np.empty((2 * ii, H), np.int8)
        gs = np.empty(2 * ii, np.float32)
        go = np.empty(2 * ii, np.float32)
        dq = np.empty((H, ii), np.int8)
        ds = np.empty(H, np.float32)
        do = np.empty(H, np.float32)
        dev.check(L.ds_hip_layer_export_expert(h, e, gq.ctypes.data, gs.ctypes.data, go.ctypes.data, dq.ctypes.data,
                                               ds.ctypes.data, do.ctypes.data), "export")
        return B.QBlock(gq, gs, go), B.QBlock(dq, ds, do)

    gu, dn = [], []
    for e in range(E):
        g, d = blk(e, False)
        gu.append(g)
        dn.append(d)
    sg, sd = blk(-1, True)
    return B.MoELayer(H, I, E, K, SI, rf.to_array(np.float32), rb.to_array(np.uint16), gu, dn, sg, sd)


def test_config2_layer_vs_oracle(dev, B):
    """Config 2: one DeepSeek3B-MoE layer (64 experts + 2 shared, INT8), batch 1, both routers."""
    L = dev.load()
    h, rf, rb = make_device_layer(dev, 31)
    try:
        lay = export_layer(dev, B, h, rf, rb)
        # the device quantizer agrees with the oracle on a sample expert of the arena
        W = dev.DeviceBuffer(2 * 896 * 1280 * 2)
        dev.check(L.ds_hip_fill_normal_bf16(W.ptr, 2 * 896 * 1280, 31 * 1000 + 10 + 2 * 5, 0.02), "fill")
        ref = B.or_quantize_bf16(W.to_array(np.uint16).reshape(1792, 1280))
        assert np.array_equal(ref.q, lay.gu[5].q) and np.array_equal(bits(ref.scale), bits(lay.gu[5].scale))
        orl = lay.or_layer()
        for mode in (1, 0):
            for s in range(2):
                x = B.normal_f32(1280, 950 + s)
                out, idx, w = layer_forward(dev, h, x, mode)
                ro = np.empty(1280, np.float32)
                ri = np.empty(6, np.int32)
                rw = np.empty(6, np.float32)
                B.oracle().or_moe_layer_decode(ro, x, C.byref(orl), mode, 0, 1, ri, rw)
                assert np.array_equal(idx, ri)
                err = rel_err(out, ro)
                print(f"config-2 layer mode={mode} seed={s}: max|a-b|/max|b| = {err:.2e}")
                assert err < TOL
    finally:
        L.ds_hip_layer_destroy(h)


def test_config2_layer_bf16sim_bit_exact(dev, B):
    """bf16 simulation (the reference library's default mode, ds_ocr.c:27) at the config-2 shape: the
    layer output bit-identical to the oracle's on 40 seeded inputs per routing mode, with and without
    the residual."""
    L = dev.load()
    h, rf, rb = make_device_layer(dev, 33)
    try:
        lay = export_layer(dev, B, h, rf, rb)
        orl = lay.or_layer()
        dev.set_bf16sim(1)
        for mode in (0, 1):
            weights_differ = 0
            for s in range(40):
                x = B.normal_f32(1280, 3300 + 100 * mode + s)
                out, idx, w = layer_forward(dev, h, x, mode)
                outr, _, _ = layer_forward(dev, h, x, mode, residual=1)
                ro = np.empty(1280, np.float32)
                ri = np.empty(6, np.int32)
                rw = np.empty(6, np.float32)
                B.oracle().or_moe_layer_decode(ro, x, C.byref(orl), mode, 1, 1, ri, rw)
                assert np.array_equal(idx, ri), (mode, s)
                if not np.array_equal(bits(w), bits(rw)):
                    # CFG only: the host expf (glibc) is 1 ulp off the correctly rounded weight on
                    # 8.7e-5 of its arguments; the expert outputs are still exact, the combine is not
                    assert mode == 1 and np.abs(w.astype(np.float64) - rw).max() <= 2.0 ** -24, (s, w, rw)
                    assert rel_err(out, ro) < 1e-6
                    weights_differ += 1
                    continue
                assert np.array_equal(bits(out), bits(ro)), (mode, s, rel_err(out, ro))
                assert np.array_equal(bits(outr), bits(x + ro)), (mode, s)
            print(f"config-2 layer, bf16 simulation, mode {mode}: bit-identical on {40 - weights_differ}/40 seeds")
            assert weights_differ <= 2
    finally:
        dev.set_bf16sim(0)
        L.ds_hip_layer_destroy(h)


def run_stack(dev, layers, lm, vocab, xs, mode, graph=True, kernels=None, expect=None, names=None):
    """Runs xs through a stack step by step; kernels = 1 or 2 picks the MoE layer kernels (default:
    the library's choice); expect: the kernels per layer the bound stack must report (default: the
    ones picked); names (a list): receives the step's kernel group names."""
    L = dev.load()
    arr = (C.c_void_p * len(layers))(*layers)
    S = L.ds_hip_stack_create(arr, len(layers), lm.ptr, vocab, mode)
    assert S, L.ds_hip_last_error()
    try:
        n = xs.shape[0]
        xd = dev.DeviceBuffer.from_array(xs)
        td = dev.DeviceBuffer(4 * n)
        if kernels is not None:
            dev.check(L.ds_hip_stack_set_layer_kernels(S, 1 if kernels == 1 else 0), "layer kernels")
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, xs.shape[1], n, td.ptr, n), "bind")
        if kernels is not None:
            assert L.ds_hip_stack_layer_kernels(S) == (expect or (1 if kernels == 1 else 2))
        if names is not None:
            names += [L.ds_hip_stack_kernel_name(S, i).decode() for i in range(L.ds_hip_stack_kernel_count(S))]
        hidden = []
        for _ in range(n):
            dev.check(L.ds_hip_stack_run(S, 1) if graph else L.ds_hip_stack_run_eager(S, 1), "run")
            hx = np.empty(xs.shape[1], np.float32)
            dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
            hidden.append(hx)
        return td.to_array(np.int32), np.stack(hidden)
    finally:
        L.ds_hip_stack_destroy(S)


def oracle_decode(B, lays, lm_w, vocab, xs, mode, threads=1):
    toks, hid = [], []
    orls = [lay.or_layer() for lay in lays]
    for x in xs:
        h = x.copy()
        for orl, lay in zip(orls, lays):
            o = np.empty(lay.hidden, np.float32)
            B.oracle().or_moe_layer_decode(o, h, C.byref(orl), mode, 0, threads, None, None)
            h = h + o
        hid.append(h)
        toks.append(B.oracle().or_argmax_bf16(h, lm_w, h.size, vocab, threads, None))
    return np.array(toks), np.stack(hid)


@pytest.mark.parametrize("mode", [0, 1])
def test_small_stack_vs_oracle(dev, B, mode):
    L = dev.load()
    lays = [B.make_moe_layer(40 + i, hidden=256, inter=128, n_experts=16) for i in range(3)]
    hs = [upload_layer(dev, lay) for lay in lays]
    vocab = 5000
    lm_w = B.normal_bf16(vocab * 256, 77, 0.02)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(256, 300 + s) for s in range(4)])
    try:
        # the two-kernel layers are deterministic: graph, eager and repeated runs agree bit for bit
        toks, hid = run_stack(dev, hs, lm, vocab, xs, mode, kernels=2)
        toks_e, hid_e = run_stack(dev, hs, lm, vocab, xs, mode, graph=False, kernels=2)
        assert np.array_equal(toks, toks_e) and np.array_equal(bits(hid), bits(hid_e))  # graph == eager
        toks2, hid2 = run_stack(dev, hs, lm, vocab, xs, mode, kernels=2)
        assert np.array_equal(toks, toks2) and np.array_equal(bits(hid), bits(hid2))  # replays agree
        rt, rh = oracle_decode(B, lays, lm_w, vocab, xs, mode)
        for s in range(len(xs)):
            err = rel_err(hid[s], rh[s])
            print(f"small stack mode={mode} step {s}: hidden err {err:.2e}, token {toks[s]} vs {rt[s]}")
            assert err < TOL
            # the token from the GPU hidden state equals the reference argmax of that state
            assert toks[s] == B.oracle().or_argmax_bf16(hid[s], lm_w, 256, vocab, 1, None)
        assert np.mean(toks == rt) >= 0.75
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("mode", [0, 1])
def test_small_stack_bf16sim_bit_exact(dev, B, mode):
    """A stack in bf16 simulation (two kernels per layer, every rounded value in the reference's
    order): each step's hidden state bit-identical to the oracle's, tokens equal."""
    L = dev.load()
    lays = [B.make_moe_layer(440 + i, hidden=256, inter=128, n_experts=16) for i in range(3)]
    hs = [upload_layer(dev, lay) for lay in lays]
    vocab = 3000
    lm_w = B.normal_bf16(vocab * 256, 441, 0.02)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(256, 4400 + s) for s in range(4)])
    orls = [lay.or_layer() for lay in lays]
    dev.set_bf16sim(1)
    try:
        toks, hid = run_stack(dev, hs, lm, vocab, xs, mode, kernels=1, expect=2)
        for s, x in enumerate(xs):
            h = x.copy()
            for orl in orls:
                o = np.empty(256, np.float32)
                B.oracle().or_moe_layer_decode(o, h, C.byref(orl), mode, 1, 1, None, None)
                h = h + o
            print(f"bf16-sim stack mode {mode} step {s}: err {rel_err(hid[s], h):.2e}")
            if mode == 0:  # DECODE routing is exact too: every step bit-identical
                assert np.array_equal(bits(hid[s]), bits(h)), s
            else:  # CFG: a glibc expf weight 1 ulp off the correctly rounded one is possible (8.7e-5)
                assert np.array_equal(bits(hid[s]), bits(h)) or rel_err(hid[s], h) < 1e-5, s
            assert toks[s] == B.oracle().or_argmax_bf16(hid[s], lm_w, 256, vocab, 1, None)
    finally:
        dev.set_bf16sim(0)
        for h_ in hs:
            L.ds_hip_layer_destroy(h_)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("n_layers", [1, 2, 4])
def test_one_kernel_layers_vs_oracle(dev, B, n_layers, mode):
    """Stacks with one kernel per MoE layer (down split over intermediate units, the output added up
    in per-XCD copies; CFG: the next router's scores accumulated from precomputed products, DECODE:
    the exact bf16 scores kernel on the summed copies before each layer): every step's hidden state
    against the oracle and against the two-kernel layers; more steps than layers, so the copies
    must be cleared between steps; graph and eager runs agree to f32 rounding (the atomic adds make
    the low bits order-dependent)."""
    L = dev.load()
    lays = [B.make_moe_layer(140 + i, hidden=256, inter=128, n_experts=16) for i in range(n_layers)]
    hs = [upload_layer(dev, lay) for lay in lays]
    vocab = 4000
    lm_w = B.normal_bf16(vocab * 256, 141, 0.02)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(256, 1400 + s) for s in range(6)])
    try:
        toks1, hid1 = run_stack(dev, hs, lm, vocab, xs, mode, kernels=1)
        toks1e, hid1e = run_stack(dev, hs, lm, vocab, xs, mode, graph=False, kernels=1)
        toks2, hid2 = run_stack(dev, hs, lm, vocab, xs, mode, kernels=2)
        rt, rh = oracle_decode(B, lays, lm_w, vocab, xs, mode)
        for s in range(len(xs)):
            err, err2, erre = rel_err(hid1[s], rh[s]), rel_err(hid1[s], hid2[s]), rel_err(hid1e[s], hid1[s])
            print(f"one-kernel layers x{n_layers} mode {mode} step {s}: vs oracle {err:.2e}, vs two-kernel {err2:.2e}, "
                  f"eager vs graph {erre:.2e}; token {toks1[s]} vs {rt[s]}")
            assert err < TOL and err2 < 1e-4 and erre < 1e-4
            assert toks1[s] == B.oracle().or_argmax_bf16(hid1[s], lm_w, 256, vocab, 1, None)
            assert toks1e[s] == B.oracle().or_argmax_bf16(hid1e[s], lm_w, 256, vocab, 1, None)
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("threads,fused", [(1, True), (3, True), (16, True), (6, False), (7, False)])
def test_one_kernel_decode_scores_in_layer(dev, B, threads, fused):
    """DECODE routing in one-kernel layers: where every router row of the reference's thread chunks
    sits in a 4- or 2-row group (18 experts: chunks 18, 6, 2), the routed blocks compute the exact
    scores themselves and no scores kernel runs; an odd chunk (3 rows; 6 and 7 threads) puts rows on
    the single-row path and keeps the scores kernel. Hidden states against the oracle run with the
    same thread count (its selection is the reference's), tokens against its argmax.

    The routing itself is pinned too: every layer's bf16 router gets near ties (pairs of rows one
    ulp apart at a coordinate where the first layer's inputs are tiny, so only the order of the sums
    decides, and a pair of equal rows, where the lower index wins), and each layer's logged
    selection (experts in rank order and weights) must equal or_moe_layer_decode's bit for bit on
    the layer's own logged input."""
    from test_gpu_route_cert import RouteLog
    L = dev.load()
    H, K = 512, 6
    lays = [B.make_moe_layer(180 + i, hidden=H, inter=256, n_experts=18, top_k=K, n_shared=2) for i in range(3)]
    for lay in lays:
        Wb = lay.router_bf16.reshape(18, H)
        for a, col in ((0, 3), (2, 7), (4, 11)):
            Wb[a + 1] = Wb[a]
            Wb[a + 1, col] = Wb[a, col] + 1  # one bf16 ulp (same sign and exponent)
        Wb[17] = Wb[16]
    hs = [upload_layer(dev, lay) for lay in lays]
    vocab = 3000
    lm_w = B.normal_bf16(vocab * H, 181, 0.02)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(H, 1800 + s) for s in range(4)])
    xs[:, [3, 7, 11]] = np.float32(1e-6)
    log = RouteLog(dev, 64, H)
    try:
        L.ds_set_threads(threads)
        names = []
        toks, hid = run_stack(dev, hs, lm, vocab, xs, 0, kernels=1, names=names)
        toks_e, hid_e = run_stack(dev, hs, lm, vocab, xs, 0, graph=False, kernels=1)
        rt, rh = oracle_decode(B, lays, lm_w, vocab, xs, 0, threads)
        assert names.count("layer") == 3 and names.count("scores") == (0 if fused else 3), names
        for s in range(len(xs)):
            err, erre = rel_err(hid[s], rh[s]), rel_err(hid_e[s], hid[s])
            print(f"DECODE threads {threads} ({'in-layer' if fused else 'kernel'} scores) step {s}: err {err:.2e}, "
                  f"eager vs graph {erre:.2e}; token {toks[s]} vs {rt[s]}")
            assert err < TOL and erre < 1e-4
            assert toks[s] == B.oracle().or_argmax_bf16(hid[s], lm_w, H, vocab, threads, None)
        idx, w, flags, tags, xin = log.entries()
        assert len(idx) == 2 * len(xs) * len(lays), len(idx)  # graph and eager runs
        orls = [lay.or_layer() for lay in lays]
        for j in range(len(idx)):
            ri, rw = np.empty(K, np.int32), np.empty(K, np.float32)
            o = np.empty(H, np.float32)
            B.oracle().or_moe_layer_decode(o, np.ascontiguousarray(xin[j]), C.byref(orls[int(tags[j])]), 0, 0,
                                           threads, ri, rw)
            assert np.array_equal(idx[j, :K], ri) and np.array_equal(w[j, :K].view(np.int32), rw.view(np.int32)), \
                (j, int(tags[j]), idx[j, :K], ri, w[j, :K], rw)
        print(f"{len(idx)} DECODE routings equal to the reference's bit for bit")
    finally:
        log.close()
        L.ds_set_threads(1)
        for h in hs:
            L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("shape", [(512, 256, 32, 4, 4), (768, 384, 8, 6, 2), (2048, 64, 16, 6, 2)])
@pytest.mark.parametrize("mode", [0, 1])
def test_one_kernel_layer_shapes(dev, B, shape, mode):
    """Other hidden sizes (other kernel instantiations), expert counts and top-k for the one-kernel
    layers, against the oracle; a shape whose blocks cannot cover the next router's rows (H/8 rows
    of 8 per block) falls back to the two-kernel layers."""
    H, I, E, K, NS = shape
    L = dev.load()
    lays = [B.make_moe_layer(160 + i, hidden=H, inter=I, n_experts=E, top_k=K, n_shared=NS) for i in range(2)]
    hs = [upload_layer(dev, lay) for lay in lays]
    vocab = 1000
    lm_w = B.normal_bf16(vocab * H, 161, 0.02)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(H, 1600 + s) for s in range(3)])
    one = (NS * I + K * I) // 32 >= H // 8
    try:
        toks, hid = run_stack(dev, hs, lm, vocab, xs, mode, kernels=1, expect=1 if one else 2)
        rt, rh = oracle_decode(B, lays, lm_w, vocab, xs, mode)
        for s in range(len(xs)):
            err = rel_err(hid[s], rh[s])
            print(f"shape {shape} mode {mode} ({'one' if one else 'two'} kernels) step {s}: err {err:.2e}")
            assert err < TOL
            assert toks[s] == B.oracle().or_argmax_bf16(hid[s], lm_w, H, vocab, 1, None)
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("mode", [1, 0])
def test_config5_stack(dev, B, mode):
    """Config 5 at full size: 11 config-2 layers + the 129280 x 1280 bf16 argmax head, 3 steps, in
    both routing modes (one kernel per MoE layer). Hidden states vs the oracle within 1e-3; the
    tokens equal the reference argmax of the GPU's own final hidden state (bit-exact LM-head order),
    and the oracle's tokens where its top-2 margin is not a near tie; a second run of the same inputs
    (the one-kernel layers add with atomics in hardware order) gives the same tokens."""
    L = dev.load()
    n_layers, vocab, H = 11, 129280, 1280
    made = [make_device_layer(dev, 100 + l) for l in range(n_layers)]
    hs = [m[0] for m in made]
    lm = dev.DeviceBuffer(vocab * H * 2)
    dev.check(L.ds_hip_fill_normal_bf16(lm.ptr, vocab * H, 4242, 0.02), "fill")
    xs = np.stack([B.normal_f32(H, 700 + s) for s in range(3)])
    try:
        toks, hid = run_stack(dev, hs, lm, vocab, xs, mode, kernels=1, expect=1)
        toks2, hid2 = run_stack(dev, hs, lm, vocab, xs, mode, kernels=1, expect=1)
        lm_w = lm.to_array(np.uint16)
        lays = [export_layer(dev, B, *m) for m in made]
        rt, rh = oracle_decode(B, lays, lm_w, vocab, xs, mode)
        for s in range(len(xs)):
            err = rel_err(hid[s], rh[s])
            assert toks[s] == B.oracle().or_argmax_bf16(hid[s], lm_w, H, vocab, 16, None)
            lg = np.empty(vocab, np.float32)
            B.oracle().or_argmax_logits_avx512(lg, rh[s], lm_w, H, vocab, 1)
            top2 = np.sort(lg)[-2:]
            print(f"config-5 mode {mode} step {s}: hidden err {err:.2e}, token {toks[s]} vs {rt[s]}, margin "
                  f"{top2[1] - top2[0]:.2e}; rerun differs by {rel_err(hid2[s], hid[s]):.1e}")
            assert err < TOL and rel_err(hid2[s], hid[s]) < 1e-5
            if top2[1] - top2[0] > 1e-3 * abs(top2[1]):
                assert toks[s] == rt[s] and toks2[s] == toks[s]
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)


def test_timing_hooks_config1_config2(dev, B):
    """The measurement hooks behind the bench's config-1 and config-2 rows: one expert through the
    per-function kernel and one layer through ds_hip_layer_forward, timed on the device; the expert
    hook's kernel is the one ds_expert_forward_fused_int4 launches, whose output matches the oracle's
    ds_expert_forward_fused_int4 bit for bit (checked here through that API on the same blocks)."""
    L = dev.load()
    h, rf, rb = make_device_layer(dev, 302)
    try:
        lay = export_layer(dev, B, h, rf, rb)
        g, d = lay.gu[0], lay.dn[0]
        gb, db = dev.block_from_arrays(g.q, g.scale, g.offset), dev.block_from_arrays(d.q, d.scale, d.offset)
        x = B.normal_f32(1280, 4712)
        ms = C.c_float(0)
        dev.check(L.ds_hip_time_expert(C.byref(gb), C.byref(db), 1280, 896, x.ctypes.data, 5, C.byref(ms)), "expert")
        assert 0.0 < ms.value < 1.0
        y = np.empty(1280, np.float32)
        L.ds_expert_forward_fused_int4(y, x, C.byref(gb), C.byref(db), 1280, 896, None, None, None, None)
        ref = np.empty(1280, np.float32)
        B.oracle().or_expert_int8(ref, x, C.byref(g.or_block()), C.byref(d.or_block()), 1280, 896, 0)
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
        xd = dev.DeviceBuffer.from_array(x)
        od = dev.DeviceBuffer(1280 * 4)
        dev.check(L.ds_hip_time_layer(h, od.ptr, xd.ptr, dev.ROUTE_CFG, 5, C.byref(ms)), "layer")
        assert 0.0 < ms.value < 1.0
        print(f"timing hooks: expert {1e3 * ms.value:.2f} us per layer call")
    finally:
        L.ds_hip_layer_destroy(h)
