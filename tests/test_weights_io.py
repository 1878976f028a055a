"""Host side of the weight formats (no GPU): the safetensors header reader behind
ds_hip_load_moe_layers / ds_hip_load_lm_head, and the persisted-arena header checks of
ds_hip_arena_load (both fail before any device call on a bad file)."""
import ctypes as C
import os
import struct
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import checkpoints as CK  # noqa: E402


def files_arg(paths):
    arr = (C.c_char_p * len(paths))(*[p.encode() for p in paths])
    return arr, len(paths)


def info(L, paths, name):
    arr, n = files_arg(paths)
    dt = C.c_int(-1)
    shape = (C.c_int64 * 8)()
    nd = L.ds_hip_safetensors_info(arr, n, name.encode(), C.byref(dt), shape, 8)
    return nd, dt.value, [shape[i] for i in range(max(nd, 0))]


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    return CK.write_checkpoint(str(d), [(1, 41, "bf16"), (2, 42, "f32")], hidden=256, inter=128, n_experts=4,
                               n_shared=2, vocab=300)


def test_safetensors_shapes_and_dtypes_across_shards(lib, ckpt):
    L = lib.load()
    assert info(L, ckpt, "model.layers.1.mlp.gate.weight") == (2, 0, [4, 256])  # BF16 router
    assert info(L, ckpt, "model.layers.2.mlp.gate.weight") == (2, 1, [4, 256])  # F32 router
    assert info(L, ckpt, "model.layers.2.mlp.experts.3.down_proj.weight") == (2, 0, [256, 128])
    assert info(L, ckpt, "model.layers.1.mlp.shared_experts.up_proj.weight") == (2, 0, [256, 256])
    assert info(L, ckpt, "model.layers.1.input_layernorm.weight") == (1, 1, [256])
    assert info(L, ckpt, "lm_head.weight") == (2, 0, [300, 256])


def test_safetensors_missing_tensor_is_an_error(lib, ckpt):
    L = lib.load()
    assert info(L, ckpt, "model.layers.3.mlp.gate.weight")[0] == -1
    assert b"not found" in L.ds_hip_last_error()


def test_safetensors_malformed_files_are_rejected(lib, tmp_path):
    L = lib.load()
    cases = {
        "short": b"\x01\x02",
        "header_past_end": struct.pack("<Q", 1 << 20) + b"{}",
        "not_json": struct.pack("<Q", 5) + b"hello",
        "offsets_out_of_bounds": None,
        "size_mismatch": None,
    }
    hdr = b'{"t":{"dtype":"F32","shape":[4],"data_offsets":[0,64]}}'
    cases["offsets_out_of_bounds"] = struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16
    hdr2 = b'{"t":{"dtype":"F32","shape":[3],"data_offsets":[0,16]}}'
    cases["size_mismatch"] = struct.pack("<Q", len(hdr2)) + hdr2 + b"\0" * 16
    for name, blob in cases.items():
        p = tmp_path / f"{name}.safetensors"
        p.write_bytes(blob)
        assert info(L, [str(p)], "t")[0] == -1, name
    # a well-formed file with metadata, a nested unknown field and an empty shape (a scalar)
    hdr3 = (b'{"__metadata__":{"format":"pt","note":"a \\"quoted\\" word"},'
            b'"s":{"dtype":"F32","shape":[],"data_offsets":[0,4],"extra":{"k":[1,2,{"z":null}]}},'
            b'"u":{"dtype":"I8","shape":[2,3],"data_offsets":[4,10]}}')
    p = tmp_path / "ok.safetensors"
    p.write_bytes(struct.pack("<Q", len(hdr3)) + hdr3 + b"\0" * 10)
    assert info(L, [str(p)], "s") == (0, 1, [])
    assert info(L, [str(p)], "u") == (2, 3, [2, 3])


def test_arena_load_rejects_other_files_before_touching_the_device(lib, tmp_path):
    L = lib.load()
    layers = (C.c_void_p * 4)()
    lm = C.c_void_p()
    voc = C.c_int()
    p = tmp_path / "junk.bin"
    p.write_bytes(b"\0" * 512)
    assert L.ds_hip_arena_load(str(p).encode(), layers, 4, C.byref(lm), C.byref(voc)) == -1
    assert b"not a packed INT8 arena" in L.ds_hip_last_error()
    hdr = bytearray(256)
    hdr[0:8] = b"DSI8ARNA"
    struct.pack_into("<I", hdr, 8, 99)  # version
    p.write_bytes(bytes(hdr))
    assert L.ds_hip_arena_load(str(p).encode(), layers, 4, C.byref(lm), C.byref(voc)) == -1
    assert b"version 99" in L.ds_hip_last_error()
    struct.pack_into("<IIIIIIII", hdr, 8, 1, 9, 256, 128, 4, 2, 256, 0)  # 9 layers, room for 4
    p.write_bytes(bytes(hdr))
    assert L.ds_hip_arena_load(str(p).encode(), layers, 4, C.byref(lm), C.byref(voc)) == -1
    assert b"room for 4" in L.ds_hip_last_error()
    struct.pack_into("<IIIIIIII", hdr, 8, 1, 2, 256, 128, 4, 2, 256, 0)
    struct.pack_into("<QQ", hdr, 40, 1000, 0)
    p.write_bytes(bytes(hdr))  # header describes 2 layers of 1000 bytes, file has none
    assert L.ds_hip_arena_load(str(p).encode(), layers, 4, C.byref(lm), C.byref(voc)) == -1
    assert b"file size" in L.ds_hip_last_error()
    assert all(v is None for v in layers)
