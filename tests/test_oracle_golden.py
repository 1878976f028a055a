"""The CPU oracle reproduces the reference's outputs recorded in tests/golden (written from the
reference's own code by tests/golden/make_golden.py). Bit-exact comparisons throughout."""
import ctypes as C
import hashlib
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import golden_cases as G  # noqa: E402

GOLD = np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return np.array_equal(bits(a)[~both_nan], bits(b)[~both_nan]) and np.array_equal(np.isnan(a), np.isnan(b))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_generator_streams(B):
    assert np.array_equal(B.normal_f32(64, 12345, 1.0), GOLD["gen_normal_f32.v"])
    assert np.array_equal(B.normal_bf16(64, 777, 0.02), GOLD["gen_normal_bf16.v"])
    assert np.array_equal(B.lcg_bf16(64, 42)[0], GOLD["gen_lcg_bf16.v"])


@pytest.mark.parametrize("name", list(G.QUANT_CASES))
def test_quantizer(B, name):
    meta = G.QUANT_CASES[name]
    W = G.quant_input(meta)
    blk = B.or_quantize_f32(W) if meta.get("f32") else B.or_quantize_bf16(W)
    assert np.array_equal(bits(blk.scale), bits(GOLD[f"{name}.scale"]))
    assert np.array_equal(bits(blk.offset), bits(GOLD[f"{name}.offset"]))
    if f"{name}.q" in GOLD:
        assert np.array_equal(blk.q, GOLD[f"{name}.q"])
    else:
        assert sha(blk.q) == str(GOLD[f"{name}.q_sha"])


@pytest.mark.parametrize("name", list(G.MATVEC_CASES))
def test_int8_matvec_dequant_rms(B, name):
    O = B.oracle()
    meta = G.MATVEC_CASES[name]
    W = B.normal_bf16(meta["out"] * meta["in"], meta["wseed"], 0.02).reshape(meta["out"], meta["in"])
    blk = B.or_quantize_bf16(W)
    x = B.normal_f32(meta["in"], meta["xseed"])
    y = np.empty(meta["out"], np.float32)
    O.or_int8_matvec_rows(y, x, blk.q, blk.scale, blk.offset, meta["in"], 0, meta["out"])
    assert same_bits(y, GOLD[f"{name}.y"])
    rs, rn = meta["rows"]
    yr = np.empty(rn, np.float32)
    O.or_int8_matvec_rows(yr, x, blk.q, blk.scale, blk.offset, meta["in"], rs, rn)
    assert same_bits(yr, GOLD[f"{name}.y_rows"])
    d = np.empty((meta["out"], meta["in"]), np.float32)
    O.or_dequantize_f32(d, blk.q, blk.scale, blk.offset, meta["out"], meta["in"])
    assert sha(d) == str(GOLD[f"{name}.deq_sha"])
    rms = O.or_quant_error_rms(blk.q, blk.scale, blk.offset, W, meta["out"], meta["in"])
    assert np.float32(rms) == GOLD[f"{name}.rms"]


def test_swiglu_and_truncate(B):
    O = B.oracle()
    g, u = G.swiglu_inputs()
    o = np.empty_like(g)
    O.or_swiglu_direct(o, g, u, g.size)
    assert same_bits(o, GOLD["swiglu.out"])
    t = G.trunc_inputs()
    O.or_bf16_truncate(t, t.size)
    assert same_bits(t, GOLD["bf16_truncate.out"])


@pytest.mark.parametrize("name", list(G.BF16_CASES))
def test_bf16_matvec_argmax_order(B, name):
    O = B.oracle()
    meta = G.BF16_CASES[name]
    W, x = G.bf16_inputs(meta)
    for T in meta["threads"]:
        y = np.empty(meta["out"], np.float32)
        O.or_bf16_matvec_avx512(y, x, W, meta["in"], meta["out"], T)
        assert same_bits(y, GOLD[f"{name}.T{T}.y"]), T
        am = O.or_argmax_bf16(x, W, meta["in"], meta["out"], T, None)
        assert am == int(GOLD[f"{name}.T{T}.argmax"]), T
        dots = np.array([O.or_bf16_dot_row(x, W, meta["in"], r) for r in meta["dot_rows"]], np.float32)
        assert same_bits(dots, GOLD[f"{name}.T{T}.dots"])


@pytest.mark.parametrize("name", list(G.LINEAR_CASES))
def test_f32_router_and_topk(B, name):
    O = B.oracle()
    meta = G.LINEAR_CASES[name]
    W = B.normal_f32(meta["out"] * meta["in"], meta["wseed"], 0.02)
    x = B.normal_f32(meta["in"], meta["xseed"])
    y = np.empty(meta["out"], np.float32)
    O.or_linear_f32(y, x, W, meta["in"], meta["out"])
    assert same_bits(y, GOLD[f"{name}.y"])
    if meta["out"] >= 6:
        idx = np.empty(6, np.int32)
        w = np.empty(6, np.float32)
        O.or_moe_top_k(idx, w, y, meta["out"], 6)
        assert np.array_equal(idx, GOLD[f"{name}.idx"])
        assert same_bits(w, GOLD[f"{name}.w"])


def test_topk_ties(B):
    sc = G.topk_tie_scores()
    idx = np.empty(6, np.int32)
    w = np.empty(6, np.float32)
    B.oracle().or_moe_top_k(idx, w, sc, sc.size, 6)
    assert np.array_equal(idx, GOLD["topk_ties.idx"])
    assert idx[0] == 10 and idx[1] == 20 and idx[2] == 30
    assert same_bits(w, GOLD["topk_ties.w"])


@pytest.mark.parametrize("sim", [0, 1])
def test_expert_and_layer(B, sim):
    O = B.oracle()
    L = G.small_layer()
    orl = L.or_layer()
    x = B.normal_f32(L.hidden, 501)
    eo = np.empty(L.hidden, np.float32)
    O.or_expert_int8(eo, x, C.byref(L.gu[3].or_block()), C.byref(L.dn[3].or_block()), L.hidden, L.inter, sim)
    assert same_bits(eo, GOLD[f"expert_int8.sim{sim}.out"])
    for mode in (0, 1):
        for T in (1, 4):
            o = np.empty(L.hidden, np.float32)
            idx = np.empty(L.top_k, np.int32)
            w = np.empty(L.top_k, np.float32)
            O.or_moe_layer_decode(o, x, C.byref(orl), mode, sim, T, idx, w)
            key = f"moe_layer.sim{sim}.mode{mode}.T{T}"
            assert same_bits(o, GOLD[key + ".out"]), key
            assert np.array_equal(idx, GOLD[key + ".idx"]), key
            assert same_bits(w, GOLD[key + ".w"]), key
    gub, dnb, xb = G.bf16_expert_inputs()
    for T in (1, 4):
        ob = np.empty(256, np.float32)
        O.or_expert_bf16(ob, xb, gub, dnb, 256, 128, sim, T)
        assert same_bits(ob, GOLD[f"expert_bf16.sim{sim}.T{T}.out"])


def test_lcg_suite_thresholds(B):
    """test_int4.c test 1 (RMS < 0.02 on LCG U(-1,1) weights) recomputed by the oracle."""
    O = B.oracle()
    rms = []
    for s, (od, idim) in enumerate([(1792, 1280), (1280, 896), (3584, 1280)]):
        W, _ = B.lcg_bf16(od * idim, 42 + s)
        W = W.reshape(od, idim)
        blk = B.or_quantize_bf16(W)
        rms.append(O.or_quant_error_rms(blk.q, blk.scale, blk.offset, W, od, idim))
    rms = np.array(rms, np.float32)
    assert np.array_equal(rms, GOLD["lcg_suite.rms"])
    assert (rms < 0.02).all()
