"""GPU: DeepSeek-OCR safetensors shards → device MoE layers (ds_hip_load_moe_layers /
ds_hip_load_lm_head), and the persisted INT8 arena (ds_hip_arena_save / _load).

The checkpoint's layers carry oracle/bindings.py make_moe_layer's weights (tests/checkpoints.py), so
the loaded codes must equal the oracle quantizer's bit for bit (ds_int4_quantize_bf16 restated,
with the reference's gate-then-up fusion), and a loaded or reloaded layer must produce exactly the
outputs of a layer uploaded from those host blocks."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import checkpoints as CK  # noqa: E402
from test_gpu_moe import bits, layer_forward, rel_err, run_stack, upload_layer  # noqa: E402

pytestmark = pytest.mark.gpu
H, I, E, NS, K, V = 256, 128, 16, 2, 6, 5000
SEEDS = [(1, 41, "bf16"), (2, 42, "f32")]


def files_arg(paths):
    return (C.c_char_p * len(paths))(*[p.encode() for p in paths]), len(paths)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt_gpu")
    return CK.write_checkpoint(str(d), SEEDS, hidden=H, inter=I, n_experts=E, n_shared=NS, vocab=V)


def load_layers(L, files, first, n):
    arr, nf = files_arg(files)
    out = (C.c_void_p * n)()
    rc = L.ds_hip_load_moe_layers(arr, nf, first, n, K, out)
    return rc, [out[i] for i in range(n)]


def export(dev, h, e, I_):
    L = dev.load()
    gq = np.empty(2 * I_ * H, np.int8)
    gs, go = np.empty(2 * I_, np.float32), np.empty(2 * I_, np.float32)
    dq = np.empty(H * I_, np.int8)
    ds, do = np.empty(H, np.float32), np.empty(H, np.float32)
    dev.check(L.ds_hip_layer_export_expert(h, e, gq.ctypes.data, gs.ctypes.data, go.ctypes.data, dq.ctypes.data,
                                           ds.ctypes.data, do.ctypes.data), "export")
    return gq, gs, go, dq, ds, do


def same_block(exp, blk_gu, blk_dn):
    gq, gs, go, dq, ds, do = exp
    return (np.array_equal(gq, blk_gu.q.reshape(-1)) and np.array_equal(bits(gs), bits(blk_gu.scale))
            and np.array_equal(bits(go), bits(blk_gu.offset)) and np.array_equal(dq, blk_dn.q.reshape(-1))
            and np.array_equal(bits(ds), bits(blk_dn.scale)) and np.array_equal(bits(do), bits(blk_dn.offset)))


def reference_layer(dev, B, seed, router_dtype):
    """The same layer uploaded from the oracle's host blocks, with the router the checkpoint implies."""
    L = dev.load()
    lay = B.make_moe_layer(seed, hidden=H, inter=I, n_experts=E, top_k=K, n_shared=NS)
    h = upload_layer(dev, lay)
    if router_dtype == "bf16":
        rf = np.ascontiguousarray((lay.router_bf16.astype(np.uint32) << 16).view(np.float32).reshape(E, H))
        dev.check(L.ds_hip_layer_set_router(h, rf.ctypes.data, lay.router_bf16.ctypes.data), "router")
    return lay, h


def test_loaded_layers_match_the_oracle_quantizer_and_forward(dev, B, ckpt):
    L = dev.load()
    rc, hs = load_layers(L, ckpt, 1, 2)
    assert rc == 2, L.ds_hip_last_error()
    refs = []
    try:
        for (l, seed, rdt), h in zip(SEEDS, hs):
            lay, href = reference_layer(dev, B, seed, rdt)
            refs.append(href)
            for e in range(E):
                assert same_block(export(dev, h, e, I), lay.gu[e], lay.dn[e]), (l, e)
            assert same_block(export(dev, h, -1, NS * I), lay.sgu, lay.sdn), (l, "shared")
            modes = [0, 1] if rdt == "bf16" else [1]  # an F32 router gives no bf16 router
            for mode in modes:
                x = B.normal_f32(H, 5000 + l)
                out, idx, w = layer_forward(dev, h, x, mode)
                ro, ri, rw = layer_forward(dev, href, x, mode)
                assert np.array_equal(idx, ri) and np.array_equal(bits(w), bits(rw))
                assert np.array_equal(bits(out), bits(ro)), (l, mode)
            if rdt == "f32":
                x = B.normal_f32(H, 77)
                od = dev.DeviceBuffer(x.nbytes)
                xd = dev.DeviceBuffer.from_array(x)
                assert L.ds_hip_layer_forward(h, od.ptr, xd.ptr, 0, 0, None, None) == -1  # no bf16 router
    finally:
        for h in hs + refs:
            L.ds_hip_layer_destroy(h)


def test_arena_round_trip_and_stack(dev, B, ckpt, tmp_path):
    L = dev.load()
    rc, hs = load_layers(L, ckpt, 1, 2)
    assert rc == 2, L.ds_hip_last_error()
    arr, nf = files_arg(ckpt)
    lm, voc, hid = C.c_void_p(), C.c_int(), C.c_int()
    dev.check(L.ds_hip_load_lm_head(arr, nf, C.byref(lm), C.byref(voc), C.byref(hid)), "lm head")
    assert (voc.value, hid.value) == (V, H)
    lm_ref = CK.lm_head(V, H)
    got = np.empty(V * H, np.uint16)
    dev.check(L.ds_hip_memcpy_d2h(got.ctypes.data, lm.value, got.nbytes), "d2h")
    assert np.array_equal(got, lm_ref)
    path = str(tmp_path / "moe.i8arena")
    hs2, lm2 = [], C.c_void_p()
    try:
        dev.check(L.ds_hip_arena_save(path.encode(), (C.c_void_p * 2)(*hs), 2, lm.value, V), "save")
        out = (C.c_void_p * 4)()
        voc2 = C.c_int()
        assert L.ds_hip_arena_load(path.encode(), out, 4, C.byref(lm2), C.byref(voc2)) == 2, L.ds_hip_last_error()
        hs2 = [out[0], out[1]]
        assert voc2.value == V
        for h, h2 in zip(hs, hs2):
            for e in list(range(E)) + [-1]:
                a, b = export(dev, h, e, I if e >= 0 else NS * I), export(dev, h2, e, I if e >= 0 else NS * I)
                assert all(np.array_equal(u.view(np.uint8), v.view(np.uint8)) for u, v in zip(a, b)), e
        x = B.normal_f32(H, 901)
        for mode in (0, 1):
            o1 = layer_forward(dev, hs[0], x, mode)
            o2 = layer_forward(dev, hs2[0], x, mode)
            assert all(np.array_equal(bits(a), bits(b)) for a, b in zip(o1, o2))
        # the decode stack over the loaded layers and head, before and after the round trip (CFG
        # routing: layer 2 has only the f32 router)
        xs = np.stack([B.normal_f32(H, 930 + s) for s in range(3)])
        lmb = dev.DeviceBuffer(V * H * 2)
        dev.check(L.ds_hip_memcpy_d2d(lmb.ptr, lm2.value, V * H * 2), "d2d")
        # (the two-kernel layers are deterministic; the one-kernel layers agree to f32 rounding)
        t1, hid1 = run_stack(dev, hs, lmb, V, xs, 1, kernels=2)
        t2, hid2 = run_stack(dev, hs2, lmb, V, xs, 1, kernels=2)
        assert np.array_equal(t1, t2) and np.array_equal(bits(hid1), bits(hid2))
        t3, hid3 = run_stack(dev, hs2, lmb, V, xs, 1, kernels=1)
        assert rel_err(hid3, hid1) < 1e-5
        # a flipped byte in the file is caught by the checksum, and nothing is left allocated
        blob = bytearray(open(path, "rb").read())
        blob[256 + 64 + 1000] ^= 0x40
        bad = str(tmp_path / "bad.i8arena")
        open(bad, "wb").write(bytes(blob))
        out3 = (C.c_void_p * 4)()
        assert L.ds_hip_arena_load(bad.encode(), out3, 4, None, None) == -1
        assert b"checksum" in L.ds_hip_last_error()
        assert all(v is None for v in out3)
    finally:
        for h in hs + hs2:
            L.ds_hip_layer_destroy(h)
        L.ds_hip_free(lm.value)
        if lm2.value:
            L.ds_hip_free(lm2.value)


def test_checkpoint_missing_an_expert_fails_cleanly(dev, tmp_path):
    from safetensors.torch import load_file, save_file
    L = dev.load()
    files = CK.write_checkpoint(str(tmp_path), [(1, 43, "bf16")], hidden=H, inter=I, n_experts=E, n_shared=NS,
                                vocab=64)
    t = load_file(files[0])
    del t["model.layers.1.mlp.experts.5.up_proj.weight"]
    save_file(t, files[0])
    rc, hs = load_layers(L, files, 1, 1)
    assert rc == -1 and hs == [None]
    assert b"experts.5.up_proj" in L.ds_hip_last_error()
    rc, hs = load_layers(L, files, 0, 1)  # layer 0 has no MoE weights in this checkpoint
    assert rc == -1 and b"model.layers.0.mlp.gate.weight" in L.ds_hip_last_error()
