"""GPU parity of the per-function C API (include/ds_quantize.h, include/ds_kernels.h) against the
oracle and the golden fixtures. Integer outputs and [exact] functions are compared bit for bit;
the INT8 dequant-matvec paths within the 1e-3 relative bar (reported as max|a-b|/max|b|)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import golden_cases as G  # noqa: E402

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False)
TOL = 1e-3


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) | np.isnan(b)
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(bits(a)[~nan], bits(b)[~nan])


def rel_err(a, ref):
    a, ref = np.asarray(a, np.float64), np.asarray(ref, np.float64)
    return np.abs(a - ref).max() / max(np.abs(ref).max(), 1e-30)


def quantize_gpu(dev, W):
    L = dev.load()
    blk = dev.Int4Block()
    W = np.ascontiguousarray(W)
    if W.dtype == np.float32:
        rc = L.ds_int4_quantize_f32(C.byref(blk), W, W.shape[0], W.shape[1])
    else:
        rc = L.ds_int4_quantize_bf16(C.byref(blk), W, W.shape[0], W.shape[1])
    assert rc == 0, L.ds_hip_last_error()
    return blk


@pytest.mark.parametrize("name", list(G.QUANT_CASES))
def test_quantize_bit_exact(dev, B, name):
    L = dev.load()
    meta = G.QUANT_CASES[name]
    W = G.quant_input(meta)
    blk = quantize_gpu(dev, W)
    try:
        q, s, o = dev.block_arrays(blk)
        ref = B.or_quantize_f32(W) if meta.get("f32") else B.or_quantize_bf16(W)
        assert np.array_equal(q, ref.q)
        assert np.array_equal(bits(s), bits(ref.scale))
        assert np.array_equal(bits(o), bits(ref.offset))
        assert np.array_equal(bits(s), bits(GOLD[f"{name}.scale"]))
        assert blk.bytes == W.size + 8 * W.shape[0]
    finally:
        L.ds_int4_block_free(C.byref(blk))
    assert not blk.qweight and blk.bytes == 0


def test_quantize_rejects_bad_arguments(dev):
    L = dev.load()
    blk = dev.Int4Block()
    W = np.zeros((4, 4), np.uint16)
    assert L.ds_int4_quantize_bf16(C.byref(blk), W, 0, 4) == -1
    assert L.ds_int4_quantize_bf16(C.byref(blk), W, 4, -1) == -1
    L.ds_int4_block_free(None)  # NULL-safe


@pytest.mark.parametrize("name", list(G.MATVEC_CASES))
def test_int8_matvec_dequant_rms(dev, B, name):
    L = dev.load()
    O = B.oracle()
    meta = G.MATVEC_CASES[name]
    W = B.normal_bf16(meta["out"] * meta["in"], meta["wseed"], 0.02).reshape(meta["out"], meta["in"])
    blk = quantize_gpu(dev, W)
    try:
        ref = B.or_quantize_bf16(W)
        x = B.normal_f32(meta["in"], meta["xseed"])
        y = np.empty(meta["out"], np.float32)
        L.ds_int4_matvec(y, x, C.byref(blk))
        yo = np.empty(meta["out"], np.float32)
        O.or_int8_matvec_rows(yo, x, ref.q, ref.scale, ref.offset, meta["in"], 0, meta["out"])
        # one lane per row in the reference's own sequential order: bit-identical
        assert same_bits(y, yo), rel_err(y, yo)
        assert same_bits(y, GOLD[f"{name}.y"])
        rs, rn = meta["rows"]
        yr = np.empty(rn, np.float32)
        L.ds_int4_matvec_rows(yr, x, C.byref(blk), rs, rn)
        assert same_bits(yr, y[rs:rs + rn])  # test_int4.c:109-127 asks for 1e-5
        d = np.empty((meta["out"], meta["in"]), np.float32)
        L.ds_int4_dequantize_f32(d, C.byref(blk))
        do = np.empty_like(d)
        O.or_dequantize_f32(do, ref.q, ref.scale, ref.offset, meta["out"], meta["in"])
        assert np.array_equal(bits(d), bits(do))
        rms = L.ds_int4_quant_error_rms(C.byref(blk), W)
        assert abs(rms - float(GOLD[f"{name}.rms"])) <= 1e-6 * float(GOLD[f"{name}.rms"])
    finally:
        L.ds_int4_block_free(C.byref(blk))


def test_matvec_rows_out_of_range_is_ignored(dev, B):
    L = dev.load()
    W = B.normal_bf16(16 * 32, 5, 0.02).reshape(16, 32)
    blk = quantize_gpu(dev, W)
    try:
        y = np.full(4, 7.0, np.float32)
        L.ds_int4_matvec_rows(y, np.ones(32, np.float32), C.byref(blk), 14, 4)
        assert (y == 7.0).all()
    finally:
        L.ds_int4_block_free(C.byref(blk))


def test_int4_tolerance_suite(dev, B):
    """test_int4.c tests 1-4 with its LCG inputs and thresholds, on the GPU."""
    L = dev.load()
    for s, (od, idim) in enumerate([(1792, 1280), (1280, 896), (3584, 1280)]):
        W, _ = B.lcg_bf16(od * idim, 42 + s)
        blk = quantize_gpu(dev, W.reshape(od, idim))
        rms = L.ds_int4_quant_error_rms(C.byref(blk), W)
        L.ds_int4_block_free(C.byref(blk))
        assert rms < 0.02
        assert abs(rms - float(GOLD["lcg_suite.rms"][s])) < 1e-6
    W, seed = B.lcg_bf16(1792 * 1280, 12345)
    x, _ = B.lcg_f32(1280, seed)
    yr = (B.bf16_to_f32(W).reshape(1792, 1280).astype(np.float64) @ x.astype(np.float64))
    blk = quantize_gpu(dev, W.reshape(1792, 1280))
    yi = np.empty(1792, np.float32)
    L.ds_int4_matvec(yi, x, C.byref(blk))
    L.ds_int4_block_free(C.byref(blk))
    assert np.linalg.norm(yi - yr) / np.linalg.norm(yr) < 0.02


@pytest.mark.parametrize("sim", [0, 1])
def test_expert_int8(dev, B, sim):
    L = dev.load()
    O = B.oracle()
    lay = G.small_layer()
    x = B.normal_f32(lay.hidden, 501)
    g, d = lay.gu[3], lay.dn[3]
    gb = dev.block_from_arrays(g.q, g.scale, g.offset)
    db = dev.block_from_arrays(d.q, d.scale, d.offset)
    dev.set_bf16sim(sim)
    try:
        out = np.empty(lay.hidden, np.float32)
        L.ds_expert_forward_fused_int4(out, x, C.byref(gb), C.byref(db), lay.hidden, lay.inter, None, None, None, None)
    finally:
        dev.set_bf16sim(0)
    ref = GOLD[f"expert_int8.sim{sim}.out"]
    eo = np.empty(lay.hidden, np.float32)
    O.or_expert_int8(eo, x, C.byref(g.or_block()), C.byref(d.or_block()), lay.hidden, lay.inter, sim)
    assert same_bits(eo, ref)
    print(f"expert int8 sim={sim}: {rel_err(out, ref):.2e}")
    assert same_bits(out, ref)


@pytest.mark.parametrize("sim", [0, 1])
def test_expert_int8_full_shape(dev, B, sim):
    """ds_expert_forward_fused_int4 through the C-ABI at DeepSeek's shapes: routed (gate_up
    1792x1280, down 1280x896) and shared (3584x1280, 1280x1792), bf16 simulation off and on,
    bit-identical to the oracle's restatement of the reference (pinned to the reference build)."""
    L = dev.load()
    O = B.oracle()
    for I, seed in ((896, 610), (1792, 620)):
        gu = B.or_quantize_bf16(B.normal_bf16(2 * I * 1280, seed, 0.02).reshape(2 * I, 1280))
        dn = B.or_quantize_bf16(B.normal_bf16(1280 * I, seed + 1, 0.02).reshape(1280, I))
        gb = dev.block_from_arrays(gu.q, gu.scale, gu.offset)
        db = dev.block_from_arrays(dn.q, dn.scale, dn.offset)
        for xs in range(3):
            x = B.normal_f32(1280, seed + 10 + xs)
            dev.set_bf16sim(sim)
            try:
                out = np.empty(1280, np.float32)
                L.ds_expert_forward_fused_int4(out, x, C.byref(gb), C.byref(db), 1280, I, None, None, None, None)
            finally:
                dev.set_bf16sim(0)
            eo = np.empty(1280, np.float32)
            O.or_expert_int8(eo, x, C.byref(gu.or_block()), C.byref(dn.or_block()), 1280, I, sim)
            print(f"expert int8 I={I} sim={sim} x{xs}: {rel_err(out, eo):.2e}")
            assert same_bits(out, eo)
        L.ds_hip_weights_changed(gu.q.ctypes.data)
        L.ds_hip_weights_changed(dn.q.ctypes.data)


def test_elementwise_bit_exact(dev, B):
    L = dev.load()
    g, u = G.swiglu_inputs()
    o = np.empty_like(g)
    L.ds_swiglu_direct(o, g, u, 1, g.size)
    assert same_bits(o, GOLD["swiglu.out"])
    t = G.trunc_inputs()
    L.ds_bf16_truncate_array(t, t.size)
    assert same_bits(t, GOLD["bf16_truncate.out"])
    a, b = B.normal_f32(1000, 1), B.normal_f32(1000, 2)
    s = np.empty(1000, np.float32)
    L.ds_vec_add(s, a, b, 1000)
    assert np.array_equal(bits(s), bits(a + b))
    eo, w = B.normal_f32(6 * 100, 3), B.normal_f32(6, 4)
    co = np.empty(100, np.float32)
    L.ds_expert_combine(co, eo, None, w, 6, 100)
    cr = np.empty(100, np.float32)
    B.oracle().or_expert_combine(cr, eo, w, 6, 100)
    assert np.array_equal(bits(co), bits(cr))


@pytest.mark.parametrize("name", list(G.BF16_CASES))
def test_bf16_matvec_argmax_dot_exact(dev, name):
    L = dev.load()
    meta = G.BF16_CASES[name]
    W, x = G.bf16_inputs(meta)
    try:
        for T in meta["threads"]:
            L.ds_set_threads(T)
            y = np.empty(meta["out"], np.float32)
            L.ds_bf16_matvec_pub(y, x, W, None, meta["in"], meta["out"])
            assert same_bits(y, GOLD[f"{name}.T{T}.y"]), T
            y2 = np.empty(meta["out"], np.float32)
            L.ds_linear_nobias_bf16(y2, x, W, 1, meta["in"], meta["out"])
            assert same_bits(y2, y)
            am = L.ds_argmax_matvec_bf16(x, W, meta["in"], meta["out"])
            assert am == int(GOLD[f"{name}.T{T}.argmax"]), T
            dots = np.array([L.ds_bf16_dot_row(x, W, meta["in"], r) for r in meta["dot_rows"]], np.float32)
            assert same_bits(dots, GOLD[f"{name}.T{T}.dots"])
    finally:
        L.ds_set_threads(1)


def test_argmax_excluding(dev):
    L = dev.load()
    meta = G.EXCL_CASES["excl_v20000"]
    W, x = G.bf16_inputs(meta)
    try:
        for T in meta["threads"]:
            L.ds_set_threads(T)
            best = L.ds_argmax_matvec_bf16(x, W, meta["in"], meta["out"])
            assert best == int(GOLD[f"excl_v20000.T{T}.best"])
            res = []
            for ex in G.resolve_excl(meta, best):
                ea = np.array(ex if ex else [0], np.int32)
                res.append(L.ds_argmax_matvec_bf16_excluding(x, W, meta["in"], meta["out"], ea.ctypes.data, len(ex)))
            assert res == list(GOLD[f"excl_v20000.T{T}.idx"]), T
    finally:
        L.ds_set_threads(1)


@pytest.mark.parametrize("name", list(G.LINEAR_CASES))
def test_router_f32_and_topk(dev, B, name):
    L = dev.load()
    meta = G.LINEAR_CASES[name]
    W = B.normal_f32(meta["out"] * meta["in"], meta["wseed"], 0.02)
    x = B.normal_f32(meta["in"], meta["xseed"])
    y = np.empty(meta["out"], np.float32)
    L.ds_moe_router(y, x, W, meta["in"], meta["out"])
    assert same_bits(y, GOLD[f"{name}.y"])
    if meta["out"] >= 6:
        idx = np.empty(6, np.int32)
        w = np.empty(6, np.float32)
        L.ds_moe_top_k(idx, w, y, meta["out"], 6)
        assert np.array_equal(idx, GOLD[f"{name}.idx"])
        assert np.abs(w - GOLD[f"{name}.w"]).max() <= 2e-7


def test_topk_ties(dev):
    L = dev.load()
    sc = G.topk_tie_scores()
    idx = np.empty(6, np.int32)
    w = np.empty(6, np.float32)
    L.ds_moe_top_k(idx, w, sc, sc.size, 6)
    assert np.array_equal(idx, GOLD["topk_ties.idx"])
    assert np.abs(w - GOLD["topk_ties.w"]).max() <= 2e-7


def test_topk_nonfinite(dev, B):
    """ds_moe_top_k on the device with NaN, infinite and floor scores, and with fewer selectable
    experts than K (the oracle's restatement is pinned to the reference on the same cases on the
    CPU): indices equal; weights NaN where the oracle's are, else within 2 ulp (the device's expf
    is correctly rounded, glibc's is 1 ulp off on a few arguments)."""
    L = dev.load()
    for i, sc in enumerate(G.topk_nonfinite_cases()):
        idx, w = np.empty(6, np.int32), np.empty(6, np.float32)
        L.ds_moe_top_k(idx, w, sc, 64, 6)
        io, wo = np.empty(6, np.int32), np.empty(6, np.float32)
        B.oracle().or_moe_top_k(io, wo, sc, 64, 6)
        assert np.array_equal(idx, io), (i, idx, io)
        nan = np.isnan(wo)
        assert np.array_equal(np.isnan(w), nan), (i, w, wo)
        ulp = np.abs(w.view(np.int32).astype(np.int64) - wo.view(np.int32).astype(np.int64))[~nan]
        assert ulp.max(initial=0) <= 2, (i, w, wo)


def test_router_bf16_exact(dev, B):
    L = dev.load()
    Wr = B.normal_bf16(64 * 1280, 11, 0.02)
    x = B.normal_f32(1280, 12)
    for T in (1, 6, 16):
        L.ds_set_threads(T)
        s = np.empty(64, np.float32)
        L.ds_moe_router_bf16(s, x, Wr, 1280, 64)
        r = np.empty(64, np.float32)
        B.oracle().or_bf16_matvec_avx512(r, x, Wr, 1280, 64, T)
        assert np.array_equal(bits(s), bits(r)), T
    L.ds_set_threads(1)


@pytest.mark.parametrize("sim", [0, 1])
def test_expert_bf16_exact(dev, sim):
    L = dev.load()
    gub, dnb, xb = G.bf16_expert_inputs()
    dev.set_bf16sim(sim)
    try:
        for T in (1, 4):
            L.ds_set_threads(T)
            ob = np.empty(256, np.float32)
            L.ds_expert_forward_fused(ob, xb, gub, dnb, 256, 128, None, None, None, None)
            assert same_bits(ob, GOLD[f"expert_bf16.sim{sim}.T{T}.out"]), T
    finally:
        dev.set_bf16sim(0)
        L.ds_set_threads(1)


def test_linear_bf16_batched(dev, B):
    L = dev.load()
    M, K, N = 37, 200, 130
    W = B.normal_bf16(N * K, 21, 0.02)
    X = B.normal_f32(M * K, 22)
    Y = np.empty(M * N, np.float32)
    L.ds_linear_nobias_bf16(Y, X, W, M, K, N)
    ref = X.reshape(M, K).astype(np.float64) @ B.bf16_to_f32(W).reshape(N, K).astype(np.float64).T
    assert rel_err(Y.reshape(M, N), ref) < 1e-5
