"""Writes the golden fixtures in this directory from the reference's own code.

The reference hot-path C sources are compiled in place by oracle/build_ref.sh into oracle/_ref/
(only possible where /root/reference exists, i.e. in the build container). This script feeds that
library seeded inputs and stores the outputs:
  - golden.npz: expected outputs (full arrays for small results, SHA-256 of the bytes for large
    ones) keyed by case name,
  - manifest.json: for every case the shapes, seeds, thread counts and modes that regenerate its
    inputs with the oracle's generator (the generator's own stream is pinned by the "gen_*" cases).
Run: python tests/golden/make_golden.py   (rewrites both files)
"""
import ctypes as C
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import bindings as B  # noqa: E402

import golden_cases as G  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    R = B.ref("v4")
    if R is None:
        sys.exit("oracle/_ref/libdsref_v4.so missing: run oracle/build_ref.sh first")
    out = {}
    manifest = {}

    def put(name, meta, **arrays):
        manifest[name] = meta
        for k, v in arrays.items():
            out[f"{name}.{k}"] = v

    # -- generator streams (pin the input generator itself)
    put("gen_normal_f32", {"seed": 12345, "n": 64}, v=B.normal_f32(64, 12345, 1.0))
    put("gen_normal_bf16", {"seed": 777, "n": 64, "std": 0.02}, v=B.normal_bf16(64, 777, 0.02))
    lc, _ = B.lcg_bf16(64, 42)
    put("gen_lcg_bf16", {"seed": 42, "n": 64}, v=lc)

    # -- quantizer
    for name, meta in G.QUANT_CASES.items():
        W = G.quant_input(meta)
        if meta.get("f32"):
            q = np.empty(W.shape, np.int8)
            s = np.empty(W.shape[0], np.float32)
            f = np.empty(W.shape[0], np.float32)
            assert R.ref_quantize_f32_copy(q, s, f, W, W.shape[0], W.shape[1]) == 0
            blk = B.QBlock(q, s, f)
        else:
            blk, _ = B.ref_quantize_bf16(W)
        arrays = {"scale": blk.scale, "offset": blk.offset}
        if blk.q.size <= 65536:
            arrays["q"] = blk.q
        else:
            arrays["q_sha"] = np.array(sha(blk.q))
        put(name, meta, **arrays)

    # -- INT8 matvec, dequantize, RMS (config-1 gate_up shape and an odd in_dim)
    R.ds_set_threads(1)
    for name, meta in G.MATVEC_CASES.items():
        W = B.normal_bf16(meta["out"] * meta["in"], meta["wseed"], 0.02).reshape(meta["out"], meta["in"])
        blk, _ = B.ref_quantize_bf16(W)
        x = B.normal_f32(meta["in"], meta["xseed"])
        rb = B.RefBlock(blk)
        y = np.empty(meta["out"], np.float32)
        R.ds_int4_matvec(y, x, rb.ptr)
        rs, rn = meta["rows"]
        yr = np.empty(rn, np.float32)
        R.ds_int4_matvec_rows(yr, x, rb.ptr, rs, rn)
        d = np.empty((meta["out"], meta["in"]), np.float32)
        R.ds_int4_dequantize_f32(d, rb.ptr)
        rms = np.float32(R.ds_int4_quant_error_rms(rb.ptr, W))
        put(name, meta, y=y, y_rows=yr, deq_sha=np.array(sha(d)), rms=np.array(rms))

    # -- elementwise
    g, u = G.swiglu_inputs()
    o = np.empty_like(g)
    R.ds_swiglu_direct(o, g, u, 1, g.size)
    put("swiglu", {"seed_g": 31, "seed_u": 32}, out=o)
    t = G.trunc_inputs()
    tt = t.copy()
    R.ds_bf16_truncate_array(tt, tt.size)
    put("bf16_truncate", {"seed": 33}, out=tt)

    # -- BF16 matvec / argmax in the AVX-512 order, per thread count
    for name, meta in G.BF16_CASES.items():
        W, x = G.bf16_inputs(meta)
        for T in meta["threads"]:
            R.ds_set_threads(T)
            y = np.empty(meta["out"], np.float32)
            R.ds_bf16_matvec_pub(y, x, W, None, meta["in"], meta["out"])
            am = R.ds_argmax_matvec_bf16(x, W, meta["in"], meta["out"])
            dots = np.array([R.ds_bf16_dot_row(x, W, meta["in"], r) for r in meta["dot_rows"]], np.float32)
            out[f"{name}.T{T}.y"] = y
            out[f"{name}.T{T}.argmax"] = np.array(am, np.int32)
            out[f"{name}.T{T}.dots"] = dots
        manifest[name] = meta
    R.ds_set_threads(1)

    # -- argmax with exclusions (the third set always contains the unconstrained best)
    for name, meta in G.EXCL_CASES.items():
        W, x = G.bf16_inputs(meta)
        for T in meta["threads"]:
            R.ds_set_threads(T)
            best = R.ds_argmax_matvec_bf16(x, W, meta["in"], meta["out"])
            res = []
            for ex in G.resolve_excl(meta, best):
                ea = np.array(ex if ex else [0], np.int32)
                res.append(R.ds_argmax_matvec_bf16_excluding(x, W, meta["in"], meta["out"], ea.ctypes.data, len(ex)))
            out[f"{name}.T{T}.best"] = np.array(best, np.int32)
            out[f"{name}.T{T}.idx"] = np.array(res, np.int32)
        manifest[name] = meta
    R.ds_set_threads(1)

    # -- f32 router (no-BLAS ds_linear order) + ds_moe_top_k
    for name, meta in G.LINEAR_CASES.items():
        W = B.normal_f32(meta["out"] * meta["in"], meta["wseed"], 0.02)
        x = B.normal_f32(meta["in"], meta["xseed"])
        y = np.empty(meta["out"], np.float32)
        R.ds_moe_router(y, x, W, meta["in"], meta["out"])
        arrays = {"y": y}
        if meta["out"] >= 6:
            idx = np.empty(6, np.int32)
            w = np.empty(6, np.float32)
            R.ds_moe_top_k(idx, w, y, meta["out"], 6)
            arrays.update(idx=idx, w=w)
        put(name, meta, **arrays)
    sc = G.topk_tie_scores()
    idx = np.empty(6, np.int32)
    w = np.empty(6, np.float32)
    R.ds_moe_top_k(idx, w, sc, sc.size, 6)
    put("topk_ties", {}, idx=idx, w=w)

    # -- experts and MoE layers (reference composite, ds_moe_decoder.c order)
    for sim in (0, 1):
        R.ref_set_bf16sim(sim)
        L = G.small_layer()
        rl = L.ref_layer()
        x = B.normal_f32(L.hidden, 501)
        e = 3
        rg, rd = B.RefBlock(L.gu[e]), B.RefBlock(L.dn[e])
        bufs = [np.empty(4096, np.float32) for _ in range(4)]
        eo = np.empty(L.hidden, np.float32)
        R.ds_expert_forward_fused_int4(eo, x, rg.ptr, rd.ptr, L.hidden, L.inter, *bufs)
        out[f"expert_int8.sim{sim}.out"] = eo
        for mode in (0, 1):
            for T in (1, 4):
                R.ds_set_threads(T)
                o = np.empty(L.hidden, np.float32)
                idx = np.empty(L.top_k, np.int32)
                w = np.empty(L.top_k, np.float32)
                R.ref_moe_layer(o, x, C.addressof(rl), mode, idx, w)
                key = f"moe_layer.sim{sim}.mode{mode}.T{T}"
                out[key + ".out"] = o
                out[key + ".idx"] = idx
                out[key + ".w"] = w
        R.ds_set_threads(1)
        gub, dnb, xb = G.bf16_expert_inputs()
        for T in (1, 4):
            R.ds_set_threads(T)
            ob = np.empty(256, np.float32)
            R.ds_expert_forward_fused(ob, xb, gub, dnb, 256, 128, *bufs)
            out[f"expert_bf16.sim{sim}.T{T}.out"] = ob
        R.ds_set_threads(1)
    R.ref_set_bf16sim(0)
    manifest["expert_int8"] = {"layer": G.SMALL_LAYER, "x_seed": 501, "expert": 3}
    manifest["moe_layer"] = {"layer": G.SMALL_LAYER, "x_seed": 501}
    manifest["expert_bf16"] = {"hidden": 256, "inter": 128, "seeds": [601, 602, 603]}

    # -- test_int4.c tolerance suite values (LCG inputs), for the record
    vals = G.lcg_suite(R)
    put("lcg_suite", {"source": "test_int4.c:43-127"}, **vals)

    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    size = os.path.getsize(os.path.join(HERE, "golden.npz"))
    print(f"wrote {len(out)} arrays, golden.npz {size / 1024:.1f} KiB")


if __name__ == "__main__":
    main()
