"""GPU: the decoder's dense SwiGLU FFN (layer 0; ds_moe_decoder.c:75-105) — ds_hip_dense_forward
against the oracle's BF16 expert (or_expert_bf16 on the fused [gate; up] matrix, i.e. two
ds_linear_nobias_bf16, ds_swiglu_direct, ds_linear_nobias_bf16 in the reference's order), the stack
with a dense layer first (its down kernel also writes the first MoE layer's router partials), and
the checkpoint loader."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import checkpoints as CK  # noqa: E402
from test_gpu_moe import bits, rel_err, run_stack, upload_layer  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 1e-3


def dense_weights(B, H, I, seed):
    g = B.normal_bf16(I * H, seed, 0.02)
    u = B.normal_bf16(I * H, seed + 1, 0.02)
    d = B.normal_bf16(H * I, seed + 2, 0.02)
    return g, u, d


def oracle_dense(B, x, g, u, d, H, I):
    out = np.empty(H, np.float32)
    B.oracle().or_expert_bf16(out, np.ascontiguousarray(x, np.float32), np.concatenate([g, u]), d, H, I, 0, 1)
    return out


def make_dense(dev, H, I, g, u, d):
    L = dev.load()
    D = L.ds_hip_dense_create(H, I, g.ctypes.data, u.ctypes.data, d.ctypes.data)
    assert D, L.ds_hip_last_error()
    return D


@pytest.mark.parametrize("H,I", [(256, 384), (256, 200), (1280, 6848)])
def test_dense_forward_vs_oracle(dev, B, H, I):
    L = dev.load()
    g, u, d = dense_weights(B, H, I, 8100 + I)
    D = make_dense(dev, H, I, g, u, d)
    try:
        for s in range(2):
            x = B.normal_f32(H, 8200 + s)
            ref = oracle_dense(B, x, g, u, d, H, I)
            xd = dev.DeviceBuffer.from_array(x)
            od = dev.DeviceBuffer(x.nbytes)
            dev.check(L.ds_hip_dense_forward(D, od.ptr, xd.ptr, 0), "dense")
            out = od.to_array(np.float32)
            err = rel_err(out, ref)
            print(f"dense H={H} I={I} seed {s}: {err:.2e}")
            assert err < TOL
            dev.check(L.ds_hip_dense_forward(D, xd.ptr, xd.ptr, 1), "dense in place + residual")
            assert rel_err(xd.to_array(np.float32), x + ref) < TOL
    finally:
        L.ds_hip_dense_destroy(D)


def test_dense_rejects_unsupported_shapes(dev, B):
    L = dev.load()
    g = np.zeros(8 * 100, np.uint16)
    assert not L.ds_hip_dense_create(100, 8, g.ctypes.data, g.ctypes.data, g.ctypes.data)  # hidden % 128
    assert not L.ds_hip_dense_create(128, 12, g.ctypes.data, g.ctypes.data, g.ctypes.data)  # inter % 8
    assert b"ds_hip_dense_create" in L.ds_hip_last_error()


@pytest.mark.parametrize("mode", [0, 1])
def test_stack_with_dense_layer_vs_oracle(dev, B, mode):
    L = dev.load()
    H, I0, V = 256, 512, 3000
    g, u, d = dense_weights(B, H, I0, 8300)
    D = make_dense(dev, H, I0, g, u, d)
    lays = [B.make_moe_layer(50 + i, hidden=H, inter=128, n_experts=16) for i in range(2)]
    hs = [upload_layer(dev, lay) for lay in lays]
    lm_w = B.normal_bf16(V * H, 78, 0.02)
    lm = dev.DeviceBuffer.from_array(lm_w)
    xs = np.stack([B.normal_f32(H, 8400 + s) for s in range(3)])
    orls = [lay.or_layer() for lay in lays]
    try:
        # reference: x + FFN(x), then the MoE layers, then the argmax head
        hid_ref = []
        for x in xs:
            h = x + oracle_dense(B, x, g, u, d, H, I0)
            for orl, lay in zip(orls, lays):
                o = np.empty(H, np.float32)
                B.oracle().or_moe_layer_decode(o, h, C.byref(orl), mode, 0, 1, None, None)
                h = h + o
            hid_ref.append(h)
        arr = (C.c_void_p * 2)(*hs)
        S = L.ds_hip_stack_create(arr, 2, lm.ptr, V, mode)
        assert S, L.ds_hip_last_error()
        try:
            dev.check(L.ds_hip_stack_set_dense(S, D), "set dense")
            nk = L.ds_hip_stack_kernel_count(S)
            names = [L.ds_hip_stack_kernel_name(S, i).decode() for i in range(nk)]
            assert names[:2] == ["dense.gate_up", "dense.down"]
            assert ("scores" in names) == (mode == 0)  # CFG: the dense down writes the partials
            xd = dev.DeviceBuffer.from_array(xs)
            td = dev.DeviceBuffer(4 * len(xs))
            dev.check(L.ds_hip_stack_bind(S, xd.ptr, H, len(xs), td.ptr, len(xs)), "bind")
            assert L.ds_hip_stack_set_dense(S, D) == -1  # only before binding
            for s in range(len(xs)):
                dev.check(L.ds_hip_stack_run(S, 1), "run")
                hx = np.empty(H, np.float32)
                dev.check(L.ds_hip_stack_hidden(S, hx), "hidden")
                err = rel_err(hx, hid_ref[s])
                print(f"stack+dense mode={mode} step {s}: {err:.2e}")
                assert err < TOL
            toks = td.to_array(np.int32)
            dev.check(L.ds_hip_stack_reset(S), "reset")
            dev.check(L.ds_hip_stack_run_eager(S, len(xs)), "eager")
            assert np.array_equal(td.to_array(np.int32), toks)  # graph == eager
        finally:
            L.ds_hip_stack_destroy(S)
    finally:
        for h in hs:
            L.ds_hip_layer_destroy(h)
        L.ds_hip_dense_destroy(D)


def test_dense_from_checkpoint(dev, B, tmp_path):
    from safetensors.torch import save_file
    L = dev.load()
    H, I0 = 256, 384
    g, u, d = dense_weights(B, H, I0, 8500)
    path = str(tmp_path / "dense.safetensors")
    save_file({"model.layers.0.mlp.gate_proj.weight": CK._bf16(g, (I0, H)),
               "model.layers.0.mlp.up_proj.weight": CK._bf16(u, (I0, H)),
               "model.layers.0.mlp.down_proj.weight": CK._bf16(d, (H, I0))}, path)
    arr = (C.c_char_p * 1)(path.encode())
    Dp = C.c_void_p()
    dev.check(L.ds_hip_load_dense(arr, 1, 0, C.byref(Dp)), "load dense")
    D2 = make_dense(dev, H, I0, g, u, d)
    try:
        x = B.normal_f32(H, 8600)
        xd = dev.DeviceBuffer.from_array(x)
        o1, o2 = dev.DeviceBuffer(x.nbytes), dev.DeviceBuffer(x.nbytes)
        dev.check(L.ds_hip_dense_forward(Dp.value, o1.ptr, xd.ptr, 1), "dense 1")
        dev.check(L.ds_hip_dense_forward(D2, o2.ptr, xd.ptr, 1), "dense 2")
        assert np.array_equal(bits(o1.to_array(np.float32)), bits(o2.to_array(np.float32)))
        assert L.ds_hip_load_dense(arr, 1, 1, C.byref(C.c_void_p())) == -1  # no layer 1 in the file
    finally:
        L.ds_hip_dense_destroy(Dp.value)
        L.ds_hip_dense_destroy(D2)
