"""Case definitions shared by make_golden.py (writes fixtures from the reference build) and the tests
(regenerate the same inputs with the oracle's generator and compare)."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))
import bindings as B  # noqa: E402


def _bf16_of(vals):
    return B.f32_to_bf16_rne(np.asarray(vals, np.float32))


def quant_edge_rows(in_dim):
    """Rows that probe the quantizer's corner cases (bf16 bit patterns)."""
    rows = []
    rows.append(np.full(in_dim, 0.5, np.float32))                                  # constant -> scale 1e-10
    r = np.zeros(in_dim, np.float32)
    r[1::2] = -0.0
    r[-1] = 1.0
    rows.append(r)                                                                 # +0 first, then -0
    r = np.zeros(in_dim, np.float32)
    r[0::2] = -0.0
    r[-1] = -1.0
    rows.append(r)                                                                 # -0 first
    half = np.array([0.0, 255.0] + [k + 0.5 for k in range(128)], np.float32)
    rows.append(np.resize(half, in_dim))                                           # exact .5 ties
    rows.append(np.resize(np.array([1e-39, -2e-39, 3e-40, 0.0], np.float32), in_dim))  # subnormals
    rows.append(np.resize(np.array([3e38, -3e38, 1.0, -1.0], np.float32), in_dim))     # range overflows
    r = np.resize(np.array([0.1, -0.3, 0.7, 0.2], np.float32), in_dim).copy()
    r[5] = np.nan
    rows.append(r)                                                                 # a NaN element
    rows.append(np.resize(np.array([-0.5, 0.25], np.float32), in_dim))             # two-valued
    return np.stack(rows)


QUANT_CASES = {
    "quant_bf16_small": {"out": 48, "in": 200, "seed": 101, "edge": True},
    "quant_bf16_odd": {"out": 7, "in": 37, "seed": 102, "edge": True},
    "quant_bf16_cfg1_gate_up": {"out": 1792, "in": 1280, "seed": 103, "edge": False},
    "quant_bf16_cfg1_down": {"out": 1280, "in": 896, "seed": 104, "edge": False},
    "quant_f32": {"out": 16, "in": 100, "seed": 105, "edge": False, "f32": True},
}


def quant_input(meta):
    if meta.get("f32"):
        return B.normal_f32(meta["out"] * meta["in"], meta["seed"], 0.02).reshape(meta["out"], meta["in"])
    W = B.normal_bf16(meta["out"] * meta["in"], meta["seed"], 0.02).reshape(meta["out"], meta["in"])
    if meta.get("edge"):
        W = np.concatenate([W, _bf16_of(quant_edge_rows(meta["in"]))])
    return np.ascontiguousarray(W)


MATVEC_CASES = {
    "matvec_cfg1": {"out": 1792, "in": 1280, "wseed": 201, "xseed": 202, "rows": [0, 896]},
    "matvec_odd": {"out": 33, "in": 77, "wseed": 203, "xseed": 204, "rows": [5, 20]},
}


def swiglu_inputs():
    g = B.normal_f32(2000, 31, 3.0)
    u = B.normal_f32(2000, 32, 1.0)
    specials = np.array([0.0, -0.0, 88.0, -88.0, 87.99, -87.99, 88.01, -88.01, 100.0, -100.0, 1e-40, -1e-40,
                         1e-30, 20.0, -20.0, 0.5], np.float32)
    g[: specials.size] = specials
    return g, u


def trunc_inputs():
    t = B.normal_f32(1000, 33, 10.0)
    t[:8] = np.array([0.0, -0.0, 1.0, 3.4e38, -3.4e38, 1e-40, np.inf, 65504.0], np.float32)
    return t


BF16_CASES = {
    "bf16_h1280": {"out": 301, "in": 1280, "wseed": 301, "xseed": 302, "threads": [1, 3, 16],
                   "dot_rows": [0, 150, 300]},
    "bf16_h200": {"out": 97, "in": 200, "wseed": 303, "xseed": 304, "threads": [1, 4, 6],
                  "dot_rows": [0, 50, 96]},
    "bf16_h40": {"out": 13, "in": 40, "wseed": 305, "xseed": 306, "threads": [1, 2],
                 "dot_rows": [0, 12]},
    "bf16_dup_nan": {"out": 64, "in": 64, "wseed": 307, "xseed": 308, "threads": [1, 4], "dup": True,
                     "dot_rows": [0, 63]},
}


def bf16_inputs(meta):
    W = B.normal_bf16(meta["out"] * meta["in"], meta["wseed"], 0.02)
    x = B.normal_f32(meta["in"], meta["xseed"])
    if meta.get("dup"):
        # copy the best row to the last row (equal maxima: the lower index must win) and make row 1
        # all-NaN (never chosen)
        best = B.oracle().or_argmax_bf16(x, W, meta["in"], meta["out"], 1, None)
        W = W.reshape(meta["out"], meta["in"]).copy()
        W[meta["out"] - 1] = W[best]
        W[1] = 0x7FC0
        W = W.reshape(-1)
    return np.ascontiguousarray(W), x


EXCL_CASES = {
    "excl_v20000": {"out": 20000, "in": 128, "wseed": 401, "xseed": 402, "threads": [1, 4],
                    "excl_sets": [[], [5], None]},
}


def resolve_excl(meta, best):
    """Exclusion sets: [] (none), a set not containing the best, and one containing it."""
    sets = []
    for s in meta["excl_sets"]:
        if s is None:
            sets.append([best, 3, 7])
        else:
            sets.append(list(s))
    return sets


LINEAR_CASES = {
    "linear_f32_h1280": {"out": 64, "in": 1280, "wseed": 701, "xseed": 702},
    "linear_f32_h7": {"out": 5, "in": 7, "wseed": 703, "xseed": 704},
    "linear_f32_h15": {"out": 5, "in": 15, "wseed": 705, "xseed": 706},
    "linear_f32_h23": {"out": 5, "in": 23, "wseed": 707, "xseed": 708},
    "linear_f32_h24": {"out": 5, "in": 24, "wseed": 709, "xseed": 710},
    "linear_f32_h40": {"out": 8, "in": 40, "wseed": 711, "xseed": 712},
}


def topk_tie_scores():
    s = B.normal_f32(64, 801, 1.0)
    s[10] = s[20] = s[30] = np.float32(5.0)   # three-way tie at the top: lowest index first
    s[40] = np.float32(-0.0)
    s[41] = np.float32(0.0)
    return s


def topk_nonfinite_cases():
    """Score vectors (64 experts) for the selection's edge cases: NaN scores (never selected:
    every comparison with NaN is false), -inf and +inf (+inf is selected; its softmax weight is
    exp(inf - inf) = NaN), scores at or below the -1e30 floor (not selectable: the comparison is
    strict), fewer selectable experts than K (the remaining slots are index 0, weight 0), all NaN,
    and ties."""
    base = B.normal_f32(64, 803, 1.0)
    cases = []
    s = base.copy(); s[[3, 17, 40]] = np.nan; cases.append(s)
    s = base.copy(); s[[5, 9]] = -np.inf; cases.append(s)
    s = base.copy(); s[11] = np.inf; s[12] = -np.inf; cases.append(s)
    s = np.full(64, np.float32(-2e30)); s[[2, 30, 50]] = base[[2, 30, 50]]; cases.append(s)
    s = base.copy(); s[::2] = np.float32(-1e30); cases.append(s)
    s = np.full(64, np.float32(np.nan)); cases.append(s)
    s = base.copy(); s[[1, 2, 7]] = s[0]; s[8] = np.nan; cases.append(s)
    return [c.astype(np.float32) for c in cases]


SMALL_LAYER = {"hidden": 256, "inter": 128, "n_experts": 16, "top_k": 6, "n_shared": 2, "seed": 9}


def small_layer():
    m = SMALL_LAYER
    return B.make_moe_layer(m["seed"], hidden=m["hidden"], inter=m["inter"], n_experts=m["n_experts"],
                            top_k=m["top_k"], n_shared=m["n_shared"])


def bf16_expert_inputs():
    gub = B.normal_bf16(256 * 256, 601, 0.02)
    dnb = B.normal_bf16(256 * 128, 602, 0.02)
    x = B.normal_f32(256, 603)
    return gub, dnb, x


def lcg_suite(R):
    """test_int4.c tests 1-4 on the reference (values recorded; thresholds are 0.02 / 1e-5)."""
    out = {}
    R.ds_set_threads(1)
    rms = []
    for s, (od, idim) in enumerate([(1792, 1280), (1280, 896), (3584, 1280)]):
        W, _ = B.lcg_bf16(od * idim, 42 + s)
        blk, _ = B.ref_quantize_bf16(W.reshape(od, idim))
        rb = B.RefBlock(blk)  # keep the wrapper alive for the call
        rms.append(R.ds_int4_quant_error_rms(rb.ptr, W))
    out["rms"] = np.array(rms, np.float32)
    return out
