"""GPU: a whole decoder step as one graph (ds_hip_stack_set_attention: per decoder layer the
attention half, then its MLP on the post-attention RMSNorm with the attention output as residual;
then the final RMSNorm and the argmax LM head; ds_moe_decoder.c:339-474, :1000-1041) against the
oracle composed in decoder_layer_forward's order (or_decoder_attn, or_expert_bf16 for the dense
layer, or_moe_layer_decode, the residual adds, or_rms_norm, or_argmax_bf16)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_gpu_attn import make  # noqa: E402
from test_gpu_moe import bits, rel_err, upload_layer  # noqa: E402
from test_oracle_attn import attn_weights, or_attn, rnd  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-3
H, NH, HD, I0, V = 256, 2, 128, 384, 3000


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("rswa", [False, True])
def test_decoder_step_vs_oracle(dev, B, mode, rswa):
    L = dev.load()
    O = B.oracle()
    pos0, steps, max_seq = 5, 6, 32
    pre, win = (pos0, 3) if rswa else (0, 0)
    qd, stride = NH * HD, NH * HD
    # layer 0: dense FFN; layers 1-2: MoE
    g, u, d = (B.normal_bf16(I0 * H, 900 + i, 0.02) for i in range(3))
    D = L.ds_hip_dense_create(H, I0, g.ctypes.data, u.ctypes.data, d.ctypes.data)
    assert D, L.ds_hip_last_error()
    lays = [B.make_moe_layer(90 + i, hidden=H, inter=128, n_experts=16) for i in range(2)]
    hs = [upload_layer(dev, lay) for lay in lays]
    orls = [lay.or_layer() for lay in lays]
    ws = [attn_weights(H, NH, HD, 500 + 20 * i, qk_norm=(i == 1)) for i in range(3)]
    attns = [make(dev, w, H, NH, HD, max_seq) for w in ws]
    oas = [or_attn(w, H, NH, HD, stride) for w in ws]
    caches = []
    for i, A in enumerate(attns):
        kp, vp = rnd(pos0 * qd, 700 + i, 0.3), rnd(pos0 * qd, 710 + i)
        dev.check(L.ds_hip_attn_load_kv(A, kp.ctypes.data, vp.ctypes.data, pos0, qd), "load kv")
        dev.check(L.ds_hip_attn_set_window(A, pre, win), "window")
        Kc, Vc = np.zeros(max_seq * stride, np.float32), np.zeros(max_seq * stride, np.float32)
        Kc[:pos0 * qd], Vc[:pos0 * qd] = kp, vp
        caches.append((Kc, Vc))
    fnorm = rnd(H, 800, 0.1) + 1
    lm_w = B.normal_bf16(V * H, 801, 0.02)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([rnd(H, 810 + s) for s in range(steps)])
    S = None
    try:
        arr = (C.c_void_p * 2)(*hs)
        S = L.ds_hip_stack_create(arr, 2, lm.ptr, V, mode)
        assert S, L.ds_hip_last_error()
        dev.check(L.ds_hip_stack_set_dense(S, D), "dense")
        at = (C.c_void_p * 3)(*attns)
        assert L.ds_hip_stack_set_attention(S, at, 2, fnorm.ctypes.data, 1e-6, pos0, 0) == -1  # wrong count
        dev.check(L.ds_hip_stack_set_attention(S, at, 3, fnorm.ctypes.data, 1e-6, pos0, 0), "attention")
        names = [L.ds_hip_stack_kernel_name(S, i).decode() for i in range(L.ds_hip_stack_kernel_count(S))]
        assert names[0] == "attention" and names[-3] == "final_norm" and names.count("attention") == 3
        xd = dev.DeviceBuffer.from_array(xs)
        td = dev.DeviceBuffer(4 * steps)
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, len(xs), td.ptr, steps), "bind")
        worst = 0.0
        for s in range(steps):
            pos = pos0 + s
            dev.check(L.ds_hip_stack_run(S, 1), "run")
            hx = np.empty(H, np.float32)
            dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
            # oracle, decoder_layer_forward's order
            x = xs[s].copy()
            h, n = np.empty(H, np.float32), np.empty(H, np.float32)
            O.or_decoder_attn(h, n, x, C.byref(oas[0]), caches[0][0], caches[0][1], pos, pre, win, 1)
            out = np.empty(H, np.float32)
            O.or_expert_bf16(out, n, np.concatenate([g, u]), d, H, I0, 0, 1)
            x = h + out
            for i in range(2):
                O.or_decoder_attn(h, n, x, C.byref(oas[i + 1]), caches[i + 1][0], caches[i + 1][1], pos, pre, win, 1)
                O.or_moe_layer_decode(out, n, C.byref(orls[i]), mode, 0, 1, None, None)
                x = h + out
            err = rel_err(hx, x)
            worst = max(worst, err)
            assert err < TOL, (s, err)
            f = np.empty(H, np.float32)
            O.or_rms_norm(f, hx, fnorm, H, 1e-6)  # the GPU's own state: final norm and argmax are exact
            assert td.to_array(np.int32)[s] == O.or_argmax_bf16(f, lm_w, H, V, 1, None), s
        print(f"decoder step mode={mode} rswa={rswa}: worst hidden err {worst:.2e}")
        toks = td.to_array(np.int32)
        # graph == eager on a fresh run of the same steps (caches rewound by re-uploading the prefill)
        for i, A in enumerate(attns):  # the first pos0 rows are still the uploaded prefill
            kp, vp = caches[i][0][:pos0 * qd].copy(), caches[i][1][:pos0 * qd].copy()
            dev.check(L.ds_hip_attn_load_kv(A, kp.ctypes.data, vp.ctypes.data, pos0, qd), "reload")
        dev.check(L.ds_hip_stack_reset(S), "reset")
        dev.check(L.ds_hip_stack_run_eager(S, steps), "eager")
        assert np.array_equal(td.to_array(np.int32), toks)
    finally:
        if S:
            L.ds_hip_stack_destroy(S)
        for A in attns:
            L.ds_hip_attn_destroy(A)
        for h_ in hs:
            L.ds_hip_layer_destroy(h_)
        L.ds_hip_dense_destroy(D)


def test_decoder_step_deepseek_size(dev, B):
    """DeepSeek-OCR's decoder at full size: layer 0 dense (1280 x 6848), layers 1-11 config-2 MoE
    (64 experts + 2 shared, INT8), 12 attention halves (10 heads x 128) after 64 cached positions,
    R-SWA (reference 64 tokens, window 8), final RMSNorm, the 129280 x 1280 head; 3 steps in DECODE
    routing against the oracle composed in the reference's order."""
    from test_gpu_moe import export_layer, make_device_layer
    L = dev.load()
    O = B.oracle()
    Hf, I0f, vocab, pos0, steps = 1280, 6848, 129280, 64, 3
    qd = 10 * 128
    made = [make_device_layer(dev, 130 + l) for l in range(11)]
    hs = [m[0] for m in made]
    g, u, d = (B.normal_bf16(I0f * Hf, 950 + i, 0.02) for i in range(3))
    D = L.ds_hip_dense_create(Hf, I0f, g.ctypes.data, u.ctypes.data, d.ctypes.data)
    assert D, L.ds_hip_last_error()
    ws = [attn_weights(Hf, 10, 128, 1000 + 10 * i) for i in range(12)]
    attns = [make(dev, w, Hf, 10, 128, 128) for w in ws]
    oas = [or_attn(w, Hf, 10, 128, qd) for w in ws]
    caches = []
    for i, A in enumerate(attns):
        kp, vp = rnd(pos0 * qd, 1200 + i, 0.3), rnd(pos0 * qd, 1300 + i)
        dev.check(L.ds_hip_attn_load_kv(A, kp.ctypes.data, vp.ctypes.data, pos0, qd), "load kv")
        dev.check(L.ds_hip_attn_set_window(A, pos0, 8), "window")
        Kc, Vc = np.zeros(128 * qd, np.float32), np.zeros(128 * qd, np.float32)
        Kc[:pos0 * qd], Vc[:pos0 * qd] = kp, vp
        caches.append((Kc, Vc))
    fnorm = rnd(Hf, 1400, 0.1) + 1
    lm = dev.DeviceBuffer(vocab * Hf * 2)
    dev.check(L.ds_hip_fill_normal_bf16(lm.ptr, vocab * Hf, 4343, 0.02), "fill")
    xs = np.stack([rnd(Hf, 1500 + s) for s in range(steps)])
    S = None
    try:
        arr = (C.c_void_p * 11)(*hs)
        S = L.ds_hip_stack_create(arr, 11, lm.ptr, vocab, 0)
        assert S, L.ds_hip_last_error()
        dev.check(L.ds_hip_stack_set_dense(S, D), "dense")
        at = (C.c_void_p * 12)(*attns)
        dev.check(L.ds_hip_stack_set_attention(S, at, 12, fnorm.ctypes.data, 1e-6, pos0, 0), "attention")
        xd = dev.DeviceBuffer.from_array(xs)
        td = dev.DeviceBuffer(4 * steps)
        dev.check(L.ds_hip_stack_bind(S, xd.ptr, Hf, len(xs), td.ptr, steps), "bind")
        hidden = []
        for _ in range(steps):
            dev.check(L.ds_hip_stack_run(S, 1), "run")
            hx = np.empty(Hf, np.float32)
            dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
            hidden.append(hx)
        toks = td.to_array(np.int32)
        lm_w = lm.to_array(np.uint16)
        lays = [export_layer(dev, B, *m) for m in made]
        orls = [lay.or_layer() for lay in lays]
        gu = np.concatenate([g, u])
        for s in range(steps):
            pos = pos0 + s
            x = xs[s].copy()
            h, n = np.empty(Hf, np.float32), np.empty(Hf, np.float32)
            out = np.empty(Hf, np.float32)
            O.or_decoder_attn(h, n, x, C.byref(oas[0]), caches[0][0], caches[0][1], pos, pos0, 8, 1)
            O.or_expert_bf16(out, n, gu, d, Hf, I0f, 0, 1)
            x = h + out
            for i in range(11):
                O.or_decoder_attn(h, n, x, C.byref(oas[i + 1]), caches[i + 1][0], caches[i + 1][1], pos, pos0, 8, 1)
                O.or_moe_layer_decode(out, n, C.byref(orls[i]), 0, 0, 1, None, None)
                x = h + out
            err = rel_err(hidden[s], x)
            f = np.empty(Hf, np.float32)
            O.or_rms_norm(f, hidden[s], fnorm, Hf, 1e-6)
            print(f"DeepSeek-size decoder step {s}: hidden err {err:.2e}, token {toks[s]}")
            assert err < TOL
            assert toks[s] == O.or_argmax_bf16(f, lm_w, Hf, vocab, 1, None)
    finally:
        if S:
            L.ds_hip_stack_destroy(S)
        for A in attns:
            L.ds_hip_attn_destroy(A)
        for h_ in hs:
            L.ds_hip_layer_destroy(h_)
        L.ds_hip_dense_destroy(D)
