"""The CPU oracle against the reference's own code (oracle/_ref, built from /root/reference by
oracle/build_ref.sh) on more seeds than the golden fixtures hold. Skipped where the reference build
is absent (the GPU box)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import golden_cases as G  # noqa: E402

sys.path.insert(0, os.path.join(os.path.dirname(HERE), "oracle"))
import bindings as _B  # noqa: E402

pytestmark = pytest.mark.skipif(not _B.ref_available("v4"), reason="oracle/_ref not built (no reference tree)")


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("seed", [1, 2, 3])
@pytest.mark.parametrize("shape", [(64, 1280), (33, 896), (5, 19), (3, 4096)])
def test_quantize_matches_reference(B, seed, shape):
    W = B.normal_bf16(shape[0] * shape[1], 1000 + seed, 0.02 * seed).reshape(shape)
    a = B.or_quantize_bf16(W)
    b, nbytes = B.ref_quantize_bf16(W)
    assert np.array_equal(a.q, b.q)
    assert np.array_equal(bits(a.scale), bits(b.scale))
    assert np.array_equal(bits(a.offset), bits(b.offset))
    assert nbytes == shape[0] * shape[1] + 8 * shape[0]


@pytest.mark.parametrize("seed", [5, 6])
def test_int8_matvec_matches_reference(B, seed):
    R = B.ref()
    R.ds_set_threads(1)
    W = B.normal_bf16(300 * 1792, 2000 + seed, 0.02).reshape(300, 1792)
    blk = B.or_quantize_bf16(W)
    x = B.normal_f32(1792, 3000 + seed)
    y = np.empty(300, np.float32)
    B.oracle().or_int8_matvec_rows(y, x, blk.q, blk.scale, blk.offset, 1792, 0, 300)
    yr = np.empty(300, np.float32)
    rb = B.RefBlock(blk)
    R.ds_int4_matvec(yr, x, rb.ptr)
    assert np.array_equal(bits(y), bits(yr))


@pytest.mark.parametrize("T", [1, 2, 5, 8, 12, 16])
def test_argmax_order_matches_reference(B, T):
    R = B.ref()
    R.ds_set_threads(T)
    V, H = 2051, 1280
    W = B.normal_bf16(V * H, 4000 + T, 0.02)
    x = B.normal_f32(H, 5000 + T)
    y = np.empty(V, np.float32)
    B.oracle().or_bf16_matvec_avx512(y, x, W, H, V, T)
    yr = np.empty(V, np.float32)
    R.ds_bf16_matvec_pub(yr, x, W, None, H, V)
    assert np.array_equal(bits(y), bits(yr))
    assert B.oracle().or_argmax_bf16(x, W, H, V, T, None) == R.ds_argmax_matvec_bf16(x, W, H, V)
    R.ds_set_threads(1)


@pytest.mark.parametrize("seed", [11, 12])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("sim", [0, 1])
def test_moe_layer_matches_reference(B, seed, mode, sim):
    R = B.ref()
    R.ds_set_threads(1)
    R.ref_set_bf16sim(sim)
    try:
        L = B.make_moe_layer(seed, hidden=256, inter=128, n_experts=16)
        x = B.normal_f32(256, 6000 + seed)
        o = np.empty(256, np.float32)
        idx = np.empty(6, np.int32)
        w = np.empty(6, np.float32)
        orl = L.or_layer()
        B.oracle().or_moe_layer_decode(o, x, C.byref(orl), mode, sim, 1, idx, w)
        ro = np.empty(256, np.float32)
        ri = np.empty(6, np.int32)
        rw = np.empty(6, np.float32)
        rl = L.ref_layer()
        R.ref_moe_layer(ro, x, C.addressof(rl), mode, ri, rw)
        assert np.array_equal(bits(o), bits(ro))
        assert np.array_equal(idx, ri)
        assert np.array_equal(bits(w), bits(rw))
    finally:
        R.ref_set_bf16sim(0)


def test_fast_expf_full_sweep(B):
    """Oracle fast-exp vs the reference's SwiGLU on a dense sweep of gate values in [-90, 90]."""
    R = B.ref()
    g = np.linspace(-90.0, 90.0, 200001, dtype=np.float32)
    u = np.ones_like(g)
    o = np.empty_like(g)
    B.oracle().or_swiglu_direct(o, g, u, g.size)
    r = np.empty_like(g)
    R.ds_swiglu_direct(r, g, u, 1, g.size)
    nan = np.isnan(o) | np.isnan(r)
    assert np.array_equal(np.isnan(o), np.isnan(r))
    assert np.array_equal(bits(o)[~nan], bits(r)[~nan])


def test_excluding_matches_reference(B):
    """The reference's exclusion fallbacks recorded in the fixtures are also reproduced live."""
    R = B.ref()
    meta = G.EXCL_CASES["excl_v20000"]
    W, x = G.bf16_inputs(meta)
    gold = np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False)
    for T in meta["threads"]:
        R.ds_set_threads(T)
        best = R.ds_argmax_matvec_bf16(x, W, meta["in"], meta["out"])
        assert best == int(gold[f"excl_v20000.T{T}.best"])
        res = []
        for ex in G.resolve_excl(meta, best):
            ea = np.array(ex if ex else [0], np.int32)
            res.append(R.ds_argmax_matvec_bf16_excluding(x, W, meta["in"], meta["out"], ea.ctypes.data, len(ex)))
        assert res == list(gold[f"excl_v20000.T{T}.idx"])
    R.ds_set_threads(1)


def test_topk_nonfinite_matches_reference(B):
    """ds_moe_top_k on NaN, infinite and floor scores, and with fewer selectable experts than K:
    the oracle's restatement against the reference's own function, indices and weight bits."""
    R = B.ref()
    for i, sc in enumerate(G.topk_nonfinite_cases()):
        ir, wr = np.empty(6, np.int32), np.empty(6, np.float32)
        R.ds_moe_top_k(ir, wr, sc, 64, 6)
        io, wo = np.empty(6, np.int32), np.empty(6, np.float32)
        B.oracle().or_moe_top_k(io, wo, sc, 64, 6)
        assert np.array_equal(ir, io), (i, ir, io)
        assert np.array_equal(np.isnan(wr), np.isnan(wo)), i
        assert np.array_equal(bits(wr)[~np.isnan(wr)], bits(wo)[~np.isnan(wo)]), i
