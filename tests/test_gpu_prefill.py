"""GPU parity of the prefill MoE block (ds_hip_layer_prefill; reference block ds_moe_decoder.c:629-809
run on this layer's INT8 experts) against the oracle.

Routing: DECODE mode (bf16 router) is compared bit for bit with the reference arithmetic of the
decode router (the AVX-512-order bf16 scores, or_bf16_matvec_avx512, then the fast-exp softmax and
top-k, or_softmax_topk_decode). CFG mode (f32 router) computes every score in or_linear_f32's order
(one chain per token and expert): its expert indices (in rank order) equal or_prefill_route's on every
token, and its weights are within 2 ulp (the GPU's softmax uses a correctly rounded expf; glibc's is
off by one ulp on a few arguments).
Outputs: the GPU's own routing is fed to the f64 brute force (or_prefill_moe_f64) and the block
output must be within max|a-b|/max|b| <= 1e-3.
"""
import ctypes as C

import numpy as np
import pytest
from test_gpu_moe import export_layer, make_device_layer, rel_err, upload_layer

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(params=[1, 0], ids=["fused", "two_kernels"])
def path(request, dev):
    """Runs a test on both prefill GEMM paths (the persistent kernel only where the device supports
    it), then restores the automatic choice."""
    L = dev.load()
    if request.param == 1 and L.ds_hip_prefill_path(-1) != 1:
        pytest.skip("persistent prefill kernel not available on this device")
    assert L.ds_hip_prefill_path(request.param) == request.param
    yield request.param
    L.ds_hip_prefill_path(-1)


def gpu_prefill(dev, h, X, mode, residual=0, K=6):
    L = dev.load()
    T = X.shape[0]
    xd = dev.DeviceBuffer.from_array(X)
    od = dev.DeviceBuffer(X.nbytes)
    idd = dev.DeviceBuffer(4 * T * K)
    wd = dev.DeviceBuffer(4 * T * K)
    dev.check(L.ds_hip_layer_prefill(h, od.ptr, xd.ptr, T, mode, residual, idd.ptr, wd.ptr), "prefill")
    dev.check(L.ds_hip_sync(), "sync")
    assert L.ds_hip_prefill_wait_error(h, T) == 0
    return (od.to_array(np.float32).reshape(X.shape), idd.to_array(np.int32).reshape(T, K),
            wd.to_array(np.float32).reshape(T, K))


def check_routing(B, lay, X, idx, w, mode):
    T, K, E, H = X.shape[0], lay.top_k, lay.n_experts, lay.hidden
    if mode == 0:
        for t in range(T):
            sc = np.empty(E, np.float32)
            B.oracle().or_bf16_matvec_avx512(sc, X[t], lay.router_bf16, H, E, 1)
            ri, rw = np.empty(K, np.int32), np.empty(K, np.float32)
            B.oracle().or_softmax_topk_decode(ri, rw, sc, E, K)
            assert np.array_equal(ri, idx[t]), (t, ri, idx[t])
            assert np.array_equal(rw.view(np.uint32), w[t].view(np.uint32)), t
        return
    ri, rw = np.empty((T, K), np.int32), np.empty((T, K), np.float32)
    B.oracle().or_prefill_route(ri, rw, X, T, C.byref(lay.or_layer()), mode)
    for t in range(T):
        assert np.array_equal(ri[t], idx[t]), (t, ri[t], idx[t])
    ulp = np.abs(rw.view(np.int32).astype(np.int64) - w.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2, (int(ulp.max()), int(np.argmax(ulp.max(axis=1))))
    return ri, rw


@pytest.mark.parametrize("T", [1, 5, 64, 130])
@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_small_layer(dev, B, mode, T, path):
    L = dev.load()
    lay = B.make_moe_layer(61, hidden=256, inter=128, n_experts=16)
    h = upload_layer(dev, lay)
    try:
        X = np.stack([B.normal_f32(256, 5000 + t) for t in range(T)])
        out, idx, w = gpu_prefill(dev, h, X, mode)
        check_routing(B, lay, X, idx, w, mode)
        ref = np.empty((T, 256), np.float64)
        B.oracle().or_prefill_moe_f64(ref, X, T, C.byref(lay.or_layer()), idx, w)
        err = rel_err(out, ref)
        print(f"prefill small mode={mode} T={T}: max rel err {err:.2e}")
        assert err < TOL
    finally:
        L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_one_token_equals_decode(dev, B, mode):
    """One token through the prefill block routes exactly like the decode layer and gives the same
    output within the two paths' rounding: the decode layer runs the reference's f32 chains, the
    prefill block puts x and h on a 16-bit grid (2^-15 of the row's largest value; h n-tiles at a
    smaller exponent are rounded twice), about 1e-4 of the output's largest value. The weights are
    the same bits in DECODE mode; in CFG mode the prefill block's come from scores in ds_linear's
    order, the decode layer's from its certified partial sums (within 2e-5 unless it recomputed)."""
    from test_gpu_moe import layer_forward
    L = dev.load()
    lay = B.make_moe_layer(62, hidden=256, inter=128, n_experts=16)
    h = upload_layer(dev, lay)
    try:
        x = B.normal_f32(256, 6001)
        out, idx, w = gpu_prefill(dev, h, x[None, :], mode)
        dout, didx, dw = layer_forward(dev, h, x, mode)
        assert np.array_equal(idx[0], didx)
        if mode == 0:
            assert np.array_equal(w[0].view(np.uint32), dw.view(np.uint32))
        else:
            assert np.allclose(w[0], dw, rtol=2e-5, atol=1e-7)
        err = rel_err(out[0], dout)
        print(f"one-token prefill vs decode mode={mode}: {err:.2e}")
        assert err < 2e-4
    finally:
        L.ds_hip_layer_destroy(h)


def test_prefill_residual(dev, B, path):
    L = dev.load()
    lay = B.make_moe_layer(63, hidden=256, inter=128, n_experts=16)
    h = upload_layer(dev, lay)
    try:
        X = np.stack([B.normal_f32(256, 7000 + t) for t in range(9)])
        o0, i0, w0 = gpu_prefill(dev, h, X, 1, residual=0)
        o1, i1, w1 = gpu_prefill(dev, h, X, 1, residual=1)
        assert np.array_equal(i0, i1)
        assert np.array_equal((X + o0).view(np.uint32), o1.view(np.uint32))
    finally:
        L.ds_hip_layer_destroy(h)


def test_prefill_rejects_unsupported_shape(dev, B):
    L = dev.load()
    lay = B.make_moe_layer(64, hidden=256, inter=64, n_experts=16, n_shared=2)
    h = upload_layer(dev, lay)
    try:
        X = np.stack([B.normal_f32(256, 8000 + t) for t in range(2)])
        xd = dev.DeviceBuffer.from_array(X)
        od = dev.DeviceBuffer(X.nbytes)
        assert L.ds_hip_layer_prefill(h, od.ptr, xd.ptr, 2, 1, 0, None, None) != 0
        assert b"not supported" in L.ds_hip_last_error()
    finally:
        L.ds_hip_layer_destroy(h)


def test_prefill_config3(dev, B, path):
    """Config 3: 662 tokens through one config-2 layer (f32 router, renormalised top-6). Routing is
    checked for every token, the block output against the f64 oracle on 24 sampled tokens."""
    L = dev.load()
    T, H = 662, 1280
    h, rf, rb = make_device_layer(dev, 300)
    try:
        X = np.stack([B.normal_f32(H, 9000 + t) for t in range(T)])
        out, idx, w = gpu_prefill(dev, h, X, 1)
        lay = export_layer(dev, B, h, rf, rb)
        check_routing(B, lay, X, idx, w, 1)
        rows = np.linspace(0, T - 1, 24).astype(int)
        Xs = np.ascontiguousarray(X[rows])
        ref = np.empty((len(rows), H), np.float64)
        B.oracle().or_prefill_moe_f64(ref, Xs, len(rows), C.byref(lay.or_layer()),
                                     np.ascontiguousarray(idx[rows]), np.ascontiguousarray(w[rows]))
        err = rel_err(out[rows], ref)
        print(f"config-3 prefill (T={T}): max rel err {err:.2e} on {len(rows)} tokens")
        assert err < TOL
    finally:
        L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("path_id", ["fused", "two_kernels"])
def test_prefill_h_tiles_at_different_exponents(dev, B, path_id):
    """The down GEMM aligns each 128-unit n-tile of an h row to the row's largest exponent. The up
    rows of n-tiles 1, 2, 3 (routed and shared experts) are scaled by 2^-3, 2^-9 and 2^-40, so the
    alignment shifts by about 3 and 9 bits and, for the last tile, past the 31-bit clamp (its values
    become zero, as on the 16-bit grid of the row); a wrong shift, sign or limb order in tile 1 or 2
    moves the output by far more than the tolerance."""
    L = dev.load()
    want = 1 if path_id == "fused" else 0
    if want == 1 and L.ds_hip_prefill_path(-1) != 1:
        pytest.skip("persistent prefill kernel not available on this device")
    lay = B.make_moe_layer(65, hidden=256, inter=512, n_experts=16)
    for blk, inter in [(g, lay.inter) for g in lay.gu] + [(lay.sgu, lay.shared_inter)]:
        for t, f in [(1, 2.0 ** -3), (2, 2.0 ** -9), (3, 2.0 ** -40)]:
            rows = slice(inter + 128 * t, inter + 128 * (t + 1))
            blk.scale[rows] *= np.float32(f)
            blk.offset[rows] *= np.float32(f)
    h = upload_layer(dev, lay)
    try:
        assert L.ds_hip_prefill_path(want) == want
        T = 70
        X = np.stack([B.normal_f32(256, 11000 + t) for t in range(T)])
        out, idx, w = gpu_prefill(dev, h, X, 1)
        ref = np.empty((T, 256), np.float64)
        B.oracle().or_prefill_moe_f64(ref, X, T, C.byref(lay.or_layer()), idx, w)
        err = rel_err(out, ref)
        print(f"h tiles at 2^0, 2^-3, 2^-9, 2^-40 ({path_id}): max rel err {err:.2e}")
        assert err < TOL
    finally:
        L.ds_hip_prefill_path(-1)
        L.ds_hip_layer_destroy(h)


def test_prefill_config3_outlier_channels(dev, B):
    """x is put on a 16-bit grid relative to each token's largest value, so a few large channels
    coarsen the grid of all the others: config-3 tokens with four channels at 100x the others stay
    within the tolerance of the f64 brute force."""
    L = dev.load()
    T, H = 256, 1280
    h, rf, rb = make_device_layer(dev, 301)
    try:
        X = np.stack([B.normal_f32(H, 12000 + t) for t in range(T)])
        X[:, [7, 300, 811, 1201]] *= np.float32(100.0)
        out, idx, w = gpu_prefill(dev, h, X, 1)
        lay = export_layer(dev, B, h, rf, rb)
        rows = np.linspace(0, T - 1, 16).astype(int)
        ref = np.empty((len(rows), H), np.float64)
        B.oracle().or_prefill_moe_f64(ref, np.ascontiguousarray(X[rows]), len(rows), C.byref(lay.or_layer()),
                                     np.ascontiguousarray(idx[rows]), np.ascontiguousarray(w[rows]))
        err = rel_err(out[rows], ref)
        print(f"config-3 layer, outlier channels x100: max rel err {err:.2e} on {len(rows)} tokens")
        assert err < TOL
    finally:
        L.ds_hip_layer_destroy(h)


def test_prefill_cfg_near_ties(dev, B):
    """Router rows 3 and 5 differ by about 1e-6 of their size and are scaled up, so on every token
    they rank next to each other in the top K with scores far closer than any other order's rounding
    could separate: indices (in rank order) equal or_prefill_route's, weights within 2 ulp."""
    L = dev.load()
    lay = B.make_moe_layer(66, hidden=256, inter=128, n_experts=16)
    R = lay.router_f32.reshape(16, 256)
    rng = np.random.default_rng(66)
    R[3] *= np.float32(4.0)
    R[5] = (R[3] * (1.0 + 1e-6 * rng.standard_normal(256))).astype(np.float32)
    lay.router_bf16[:] = B.f32_to_bf16_rne(lay.router_f32).reshape(lay.router_bf16.shape)
    h = upload_layer(dev, lay)
    try:
        T = 48
        X = np.stack([np.abs(B.normal_f32(256, 13000 + t)) * np.sign(R[3]) for t in range(T)]).astype(np.float32)
        out, idx, w = gpu_prefill(dev, h, X, 1)
        ri, rw = check_routing(B, lay, X, idx, w, 1)
        both = [t for t in range(T) if 3 in ri[t][:2] and 5 in ri[t][:2]]
        assert len(both) == T, "rows 3 and 5 must lead every token"
        # the softmax uses a correctly rounded expf; glibc's is off by one ulp on a few arguments
        ulp = np.abs(rw.view(np.int32).astype(np.int64) - w.view(np.int32).astype(np.int64))
        assert ulp.max() <= 2, ulp.max()
    finally:
        L.ds_hip_layer_destroy(h)


def test_prefill_swiglu_equals_division_on_every_gate_value(dev):
    """The GEMM epilogue's SwiGLU quotient (hardware reciprocal, one Newton step, power-of-two
    rescales at the ends of the range) against the correctly rounded division the decode kernels use
    (ds_swiglu_direct, ds_kernels.c:1771), over all 2^32 gate values: every finite g whose quotient
    is zero or normal gives the same bits; only quotients below 2^-126 may differ."""
    L = dev.load()
    n = (C.c_uint64 * 2)()
    dev.check(L.ds_hip_check_prefill_swiglu(n), "swiglu check")
    assert n[0] == 0, n[0]
    assert n[1] <= 2 ** 25, n[1]  # only among the g with |g| < 2^-125 (2^24 bit patterns per sign)


def test_prefill_wait_expiry_reaches_the_caller(dev, B):
    """The reference's block always returns a complete result (ds_moe_decoder.c:629-809). When the
    persistent kernel's bounded wait for a down tile's gate_up tiles gives up, the caller is told:
    with the wait limit forced from the host so that every such wait gives up at once (each kernel
    still runs to its end), the next ds_hip_sync returns -1 naming the prefill, a later prefill call
    reports a failure left unreported, and once the limit is restored the same call is valid and
    equal to the normal result."""
    L = dev.load()
    if L.ds_hip_prefill_path(-1) != 1:
        pytest.skip("persistent prefill kernel not available on this device")
    lay = B.make_moe_layer(65, hidden=256, inter=128, n_experts=16)
    h = upload_layer(dev, lay)
    T = 64
    X = np.stack([B.normal_f32(256, 9000 + t) for t in range(T)])
    xd = dev.DeviceBuffer.from_array(X)
    od = dev.DeviceBuffer(X.nbytes)
    try:
        assert L.ds_hip_prefill_path(1) == 1
        good, _, _ = gpu_prefill(dev, h, X, 1)
        assert L.ds_hip_prefill_set_wait_limit(-1) == 0
        print("prefill with every wait giving up: ds_hip_sync", flush=True)
        dev.check(L.ds_hip_layer_prefill(h, od.ptr, xd.ptr, T, 1, 0, None, None), "prefill")
        assert L.ds_hip_sync() == -1
        assert b"prefill" in L.ds_hip_last_error() and b"not valid" in L.ds_hip_last_error()
        assert L.ds_hip_sync() == 0  # reported once
        print("prefill with every wait giving up: the next prefill call", flush=True)
        dev.check(L.ds_hip_layer_prefill(h, od.ptr, xd.ptr, T, 1, 0, None, None), "prefill")
        od.to_array(np.float32)  # synchronises without checking the error words
        assert L.ds_hip_prefill_set_wait_limit(L_DEFAULT) == 0
        assert L.ds_hip_layer_prefill(h, od.ptr, xd.ptr, T, 1, 0, None, None) == -1
        assert b"prefill" in L.ds_hip_last_error()
        print("prefill with the default wait limit", flush=True)
        again, _, _ = gpu_prefill(dev, h, X, 1)
        assert L.ds_hip_sync() == 0
        assert np.array_equal(good.view(np.uint32), again.view(np.uint32))
    finally:
        L.ds_hip_prefill_set_wait_limit(L_DEFAULT)
        L.ds_hip_prefill_path(-1)
        L.ds_hip_layer_destroy(h)


L_DEFAULT = -2147483647 - 1  # DS_HIP_PREFILL_WAIT_DEFAULT


@pytest.mark.parametrize("threads", [8, 16])
def test_prefill_decode_scores_both_kernels(dev, B, threads):
    """DECODE routing's scores in the reference's bf16 AVX-512 order from both scores kernels: with
    16 experts, 8 reference threads make chunks of 2 rows (every row on the 2-row group path: the
    kernel that keeps each lane's router columns in registers) and 16 threads chunks of 1 (single
    rows: the kernel that reads the rows per token). Indices and weights bit for bit."""
    L = dev.load()
    lay = B.make_moe_layer(67, hidden=256, inter=128, n_experts=16)
    h = upload_layer(dev, lay)
    old = L.ds_get_threads()
    try:
        L.ds_set_threads(threads)
        T = 37
        X = np.stack([B.normal_f32(256, 14000 + t) for t in range(T)])
        out, idx, w = gpu_prefill(dev, h, X, 0)
        for t in range(T):
            sc = np.empty(16, np.float32)
            B.oracle().or_bf16_matvec_avx512(sc, X[t], lay.router_bf16, 256, 16, threads)
            ri, rw = np.empty(6, np.int32), np.empty(6, np.float32)
            B.oracle().or_softmax_topk_decode(ri, rw, sc, 16, 6)
            assert np.array_equal(ri, idx[t]), (t, ri, idx[t])
            assert np.array_equal(rw.view(np.uint32), w[t].view(np.uint32)), t
    finally:
        L.ds_set_threads(old)
        L.ds_hip_layer_destroy(h)


def test_prefill_config3_decode_routing(dev, B):
    """Config 3 in DECODE routing (the bf16 router in the reference's AVX-512 order; one reference
    thread: all 64 rows in 4-row groups, the register-resident scores kernel): indices and weights
    bit for bit on all 662 tokens, output within the tolerance of the f64 brute force on 24 sampled
    tokens."""
    L = dev.load()
    T, H = 662, 1280
    h, rf, rb = make_device_layer(dev, 303)
    try:
        X = np.stack([B.normal_f32(H, 15000 + t) for t in range(T)])
        out, idx, w = gpu_prefill(dev, h, X, 0)
        lay = export_layer(dev, B, h, rf, rb)
        check_routing(B, lay, X, idx, w, 0)
        rows = np.linspace(0, T - 1, 24).astype(int)
        ref = np.empty((len(rows), H), np.float64)
        B.oracle().or_prefill_moe_f64(ref, np.ascontiguousarray(X[rows]), len(rows), C.byref(lay.or_layer()),
                                     np.ascontiguousarray(idx[rows]), np.ascontiguousarray(w[rows]))
        err = rel_err(out[rows], ref)
        print(f"config-3 prefill, DECODE routing: max rel err {err:.2e} on {len(rows)} tokens")
        assert err < TOL
    finally:
        L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("hidden", [512, 1024, 2048])
@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_hidden_sizes(dev, B, mode, hidden):
    """The routing kernels at other hidden sizes: CFG scores in ds_linear's order (the router staged
    in 128-row chunks: 4, 8 and 16 of them) and DECODE scores with the router columns in registers
    (512, 1024) or streamed per token (2048); indices bit for bit, weights as check_routing asks;
    the block output within the tolerance of the f64 brute force."""
    L = dev.load()
    lay = B.make_moe_layer(68 + hidden // 512, hidden=hidden, inter=128, n_experts=16)
    h = upload_layer(dev, lay)
    try:
        T = 21
        X = np.stack([B.normal_f32(hidden, 16000 + t) for t in range(T)])
        out, idx, w = gpu_prefill(dev, h, X, mode)
        check_routing(B, lay, X, idx, w, mode)
        ref = np.empty((T, hidden), np.float64)
        B.oracle().or_prefill_moe_f64(ref, X, T, C.byref(lay.or_layer()), idx, w)
        err = rel_err(out, ref)
        print(f"prefill hidden={hidden} mode={mode}: max rel err {err:.2e}")
        assert err < TOL
    finally:
        L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_nonfinite_tokens(dev, B, mode, path):
    """Tokens with a +inf, a NaN or a -inf coordinate among ordinary ones. Each token's row is
    computed on its own (the GEMM's exact int32 sums, the per-row limb exponents and sums, the
    per-token combine), so the ordinary tokens' outputs, indices and weights must be bit-identical
    to those of a call where the three tokens are ordinary rows, and no wait may expire. CFG: every
    token's expert indices must be the reference's (ds_moe_top_k never selects a NaN or floor score
    and fills empty slots with expert 0, weight 0), with NaN weights where the oracle's are NaN and
    the others within 2 ulp."""
    L = dev.load()
    T, H = 20, 256
    lay = B.make_moe_layer(67, hidden=H, inter=128, n_experts=16)
    h = upload_layer(dev, lay)
    try:
        X = np.stack([B.normal_f32(H, 6700 + t) for t in range(T)])
        out_ok, idx_ok, w_ok = gpu_prefill(dev, h, X, mode, residual=1)
        Xb = X.copy()
        Xb[3, 17] = np.inf
        Xb[7, 40] = np.nan
        Xb[11, 5] = -np.inf
        out, idx, w = gpu_prefill(dev, h, Xb, mode, residual=1)
        bad = {3, 7, 11}
        for t in range(T):
            if t in bad:
                assert not np.isfinite(out[t]).all(), t
                continue
            assert np.array_equal(out[t].view(np.uint32), out_ok[t].view(np.uint32)), t
            assert np.array_equal(idx[t], idx_ok[t]) and np.array_equal(w[t].view(np.uint32), w_ok[t].view(np.uint32)), t
        if mode == 1:
            ri, rw = np.empty((T, lay.top_k), np.int32), np.empty((T, lay.top_k), np.float32)
            B.oracle().or_prefill_route(ri, rw, Xb, T, C.byref(lay.or_layer()), mode)
            assert np.array_equal(ri, idx), [(t, ri[t], idx[t]) for t in range(T) if not np.array_equal(ri[t], idx[t])]
            nan = np.isnan(rw)
            assert np.array_equal(np.isnan(w), nan)
            assert nan[list(bad)].any()
            ulp = np.abs(rw[~nan].view(np.int32).astype(np.int64) - w[~nan].view(np.int32).astype(np.int64))
            assert ulp.max() <= 2, int(ulp.max())
        print(f"mode {mode}: {T - len(bad)} ordinary tokens bit-identical next to tokens with +inf, NaN, -inf")
    finally:
        L.ds_hip_layer_destroy(h)


@pytest.mark.parametrize("mode", [0, 1])
def test_prefill_zero_h_tile(dev, B, mode, path):
    """The gate rows of units 0-127 of every expert are zero, so each row's h is zero over its first
    128-unit n-tile and small (x scaled by 1/64) over the others. The zero tile must not set the
    exponent to which the down GEMM aligns the row's n-tiles (exponent 0 would shift the small
    tiles' limbs out entirely): the output must stay within 1e-3 of the f64 brute force."""
    L = dev.load()
    T, H, I = 40, 256, 256
    lay = B.make_moe_layer(71, hidden=H, inter=I, n_experts=16)
    for blk in list(lay.gu) + [lay.sgu]:
        blk.q[:128] = -128  # stored code -128: u = 0
        blk.scale[:128] = 0.0
        blk.offset[:128] = 0.0
    h = upload_layer(dev, lay)
    try:
        X = np.stack([B.normal_f32(H, 7100 + t) for t in range(T)]) / 64.0
        out, idx, w = gpu_prefill(dev, h, X, mode)
        ref = np.empty((T, H), np.float64)
        B.oracle().or_prefill_moe_f64(ref, X, T, C.byref(lay.or_layer()), idx, w)
        err = rel_err(out, ref)
        print(f"mode {mode}: zero first h tile, rel err {err:.2e}")
        assert err < TOL, err
    finally:
        L.ds_hip_layer_destroy(h)
