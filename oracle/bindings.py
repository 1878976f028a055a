"""ctypes bindings for the CPU oracle (liboracle.so) and the reference build (oracle/_ref).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, never by the product library.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


class _Optional:
    """ctypes argument type: a contiguous ndarray of one dtype, or None (NULL)."""

    def __init__(self, nd):
        self.nd = nd

    def from_param(self, obj):
        return None if obj is None else self.nd.from_param(obj)


f32p_opt = _Optional(f32p)
i32p_opt = _Optional(i32p)


class OrBlock(C.Structure):
    _fields_ = [("q", C.c_void_p), ("scale", C.c_void_p), ("offset", C.c_void_p),
                ("out_dim", C.c_int), ("in_dim", C.c_int)]


class OrAttn(C.Structure):
    """or_attn_t (oracle.h)."""
    _fields_ = [("hidden", C.c_int), ("n_heads", C.c_int), ("head_dim", C.c_int), ("kv_stride", C.c_int),
                ("eps", C.c_float), ("theta", C.c_float),
                ("wq", C.c_void_p), ("wk", C.c_void_p), ("wv", C.c_void_p), ("wo", C.c_void_p),
                ("input_norm", C.c_void_p), ("post_norm", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p)]


class OrLayer(C.Structure):
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
                ("shared_inter", C.c_int), ("router_f32", C.c_void_p), ("router_bf16", C.c_void_p),
                ("gu", C.c_void_p), ("dn", C.c_void_p), ("sgu", OrBlock), ("sdn", OrBlock)]


def _load_oracle():
    path = os.path.join(HERE, "liboracle.so")
    if not os.path.exists(path):
        raise RuntimeError(f"oracle library missing: {path} (run __graft_entry__.build())")
    lib = C.CDLL(path)
    sig = {
        "or_fill_normal_f32": (None, [f32p, C.c_size_t, C.c_uint64, C.c_float, C.c_float]),
        "or_fill_normal_bf16": (None, [u16p, C.c_size_t, C.c_uint64, C.c_float]),
        "or_fill_lcg_bf16": (None, [u16p, C.c_size_t, C.POINTER(C.c_uint), C.c_float, C.c_float]),
        "or_fill_lcg_f32": (None, [f32p, C.c_size_t, C.POINTER(C.c_uint), C.c_float, C.c_float]),
        "or_quantize_bf16": (C.c_int, [i8p, f32p, f32p, u16p, C.c_int, C.c_int]),
        "or_quantize_f32": (C.c_int, [i8p, f32p, f32p, f32p, C.c_int, C.c_int]),
        "or_dequantize_f32": (None, [f32p, i8p, f32p, f32p, C.c_int, C.c_int]),
        "or_quant_error_rms": (C.c_float, [i8p, f32p, f32p, u16p, C.c_int, C.c_int]),
        "or_int8_matvec_rows": (None, [f32p, f32p, i8p, f32p, f32p, C.c_int, C.c_int, C.c_int]),
        "or_int8_matvec_f64": (None, [f64p, f32p, i8p, f32p, f32p, C.c_int, C.c_int]),
        "or_fast_expf": (C.c_float, [C.c_float]),
        "or_swiglu_direct": (None, [f32p, f32p, f32p, C.c_int]),
        "or_bf16_truncate": (None, [f32p, C.c_int]),
        "or_bf16_matvec_avx512": (None, [f32p, f32p, u16p, C.c_int, C.c_int, C.c_int]),
        "or_argmax_logits_avx512": (None, [f32p, f32p, u16p, C.c_int, C.c_int, C.c_int]),
        "or_argmax_bf16": (C.c_int, [f32p, u16p, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float)]),
        "or_bf16_dot_row": (C.c_float, [f32p, u16p, C.c_int, C.c_int]),
        "or_rms_norm": (None, [f32p, f32p, f32p, C.c_int, C.c_float]),
        "or_residual_rms_norm": (None, [f32p, f32p, f32p, f32p, f32p, C.c_int, C.c_float]),
        "or_rope_row": (None, [f32p, f32p, C.c_int, C.c_int, C.c_float]),
        "or_apply_rope": (None, [f32p, f32p, f32p, C.c_int, C.c_int]),
        "or_rms_norm_per_head": (None, [f32p, f32p, C.c_int, C.c_int, C.c_float]),
        "or_dot_f32": (C.c_float, [f32p, f32p, C.c_int]),
        "or_attn_ranges": (C.c_int, [i32p, C.c_int, C.c_int, C.c_int]),
        "or_attention_decode": (None, [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_float, C.c_int, i32p, C.c_int]),
        "or_qkv": (None, [f32p, f32p, f32p, f32p, u16p, u16p, u16p, C.c_int, C.c_int, C.c_int, C.c_int]),
        "or_decoder_attn": (None, [f32p, f32p, f32p, C.c_void_p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]),
        "or_lm_sample_greedy": (C.c_int, [f32p, u16p, C.c_int, C.c_int, i32p_opt, C.c_int, C.c_float, C.c_int,
                                           C.c_int, C.c_void_p]),
        "or_linear_f32": (None, [f32p, f32p, f32p, C.c_int, C.c_int]),
        "or_moe_top_k": (None, [i32p, f32p, f32p, C.c_int, C.c_int]),
        "or_softmax_topk_decode": (None, [i32p, f32p, f32p, C.c_int, C.c_int]),
        "or_expert_int8": (None, [f32p, f32p, C.POINTER(OrBlock), C.POINTER(OrBlock), C.c_int, C.c_int, C.c_int]),
        "or_expert_bf16": (None, [f32p, f32p, u16p, u16p, C.c_int, C.c_int, C.c_int, C.c_int]),
        "or_expert_combine": (None, [f32p, f32p, f32p, C.c_int, C.c_int]),
        "or_moe_layer_decode": (None, [f32p, f32p, C.POINTER(OrLayer), C.c_int, C.c_int, C.c_int, i32p_opt,
                                       f32p_opt]),
        "or_prefill_route": (None, [i32p, f32p, f32p, C.c_int, C.POINTER(OrLayer), C.c_int]),
        "or_prefill_moe_f64": (None, [f64p, f32p, C.c_int, C.POINTER(OrLayer), i32p, f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_oracle = None


def oracle():
    global _oracle
    if _oracle is None:
        _oracle = _load_oracle()
    return _oracle


def ref_path(variant="v4"):
    return os.path.join(HERE, "_ref", f"libdsref_{variant}.so")


def ref_available(variant="v4"):
    return os.path.exists(ref_path(variant))


_ref = {}


def ref(variant="v4"):
    """The reference's own hot-path code built by oracle/build_ref.sh (None if not built)."""
    if variant in _ref:
        return _ref[variant]
    path = ref_path(variant)
    if not os.path.exists(path):
        return None
    lib = C.CDLL(path)
    vp = C.c_void_p
    sig = {
        "ref_set_bf16sim": (None, [C.c_int]),
        "ref_quantize_bf16_copy": (C.c_int, [i8p, f32p, f32p, u16p, C.c_int, C.c_int, C.POINTER(C.c_size_t)]),
        "ref_quantize_f32_copy": (C.c_int, [i8p, f32p, f32p, f32p, C.c_int, C.c_int]),
        "ref_block_wrap": (None, [vp, i8p, f32p, f32p, C.c_int, C.c_int]),
        "ref_block_sizeof": (C.c_size_t, []),
        "ref_layer_sizeof": (C.c_size_t, []),
        "ref_layer_init": (None, [vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp]),
        "ref_layer_set_expert": (None, [vp, C.c_int, i8p, f32p, f32p, i8p, f32p, f32p]),
        "ref_moe_layer": (None, [f32p, f32p, vp, C.c_int, i32p_opt, f32p_opt]),
        "ref_decode_steps": (C.c_double, [vp, C.c_int, u16p, C.c_int, f32p, C.c_int, C.c_int, i32p]),
        "ref_decode_hidden": (None, [f32p, vp, C.c_int, f32p, C.c_int]),
        "ds_set_threads": (None, [C.c_int]),
        "ds_rms_norm": (None, [f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]),
        "ds_residual_rms_norm": (None, [f32p, f32p, f32p, f32p, f32p, C.c_int, C.c_float]),
        "ds_compute_rope_neox": (None, [f32p, f32p, i32p, C.c_int, C.c_int, C.c_float]),
        "ds_apply_rope_neox": (None, [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int]),
        "ds_rms_norm_per_head": (None, [f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_float]),
        "ds_linear_nobias_bf16_qkv": (None, [f32p, f32p, f32p, f32p, u16p, u16p, u16p, C.c_int, C.c_int, C.c_int]),
        "ds_linear_nobias_bf16": (None, [f32p, f32p, u16p, C.c_int, C.c_int, C.c_int]),
        "ds_causal_attention_aligned": (None, [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                               C.c_float, C.c_int, C.c_int]),
        "ds_rswa_attention_aligned": (None, [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                             C.c_int, C.c_int, C.c_int, C.c_int]),
        "ds_set_threads": (None, [C.c_int]),
        "ds_get_threads": (C.c_int, []),
        "ds_int4_dequantize_f32": (None, [f32p, vp]),
        "ds_int4_quant_error_rms": (C.c_float, [vp, u16p]),
        "ds_int4_matvec": (None, [f32p, f32p, vp]),
        "ds_int4_matvec_rows": (None, [f32p, f32p, vp, C.c_int, C.c_int]),
        "ds_expert_forward_fused_int4": (None, [f32p, f32p, vp, vp, C.c_int, C.c_int, f32p, f32p, f32p, f32p]),
        "ds_expert_forward_fused": (None, [f32p, f32p, u16p, u16p, C.c_int, C.c_int, f32p, f32p, f32p, f32p]),
        "ds_swiglu_direct": (None, [f32p, f32p, f32p, C.c_int, C.c_int]),
        "ds_bf16_truncate_array": (None, [f32p, C.c_int]),
        "ds_bf16_matvec_pub": (None, [f32p, f32p, u16p, vp, C.c_int, C.c_int]),
        "ds_argmax_matvec_bf16": (C.c_int, [f32p, u16p, C.c_int, C.c_int]),
        "ds_argmax_matvec_bf16_excluding": (C.c_int, [f32p, u16p, C.c_int, C.c_int, vp, C.c_int]),
        "ds_bf16_dot_row": (C.c_float, [f32p, u16p, C.c_int, C.c_int]),
        "ds_moe_router": (None, [f32p, f32p, f32p, C.c_int, C.c_int]),
        "ds_moe_router_bf16": (None, [f32p, f32p, u16p, C.c_int, C.c_int]),
        "ds_moe_top_k": (None, [i32p, f32p, f32p, C.c_int, C.c_int]),
        "ds_expert_combine": (None, [f32p, f32p, i32p, f32p, C.c_int, C.c_int]),
        "ds_vec_add": (None, [f32p, f32p, f32p, C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _ref[variant] = lib
    return lib


# ----------------------------------------------------------------------------- helpers

def normal_f32(n, seed, std=1.0, mean=0.0):
    out = np.empty(n, dtype=np.float32)
    oracle().or_fill_normal_f32(out, n, seed, mean, std)
    return out


def normal_bf16(n, seed, std):
    out = np.empty(n, dtype=np.uint16)
    oracle().or_fill_normal_bf16(out, n, seed, std)
    return out


def lcg_bf16(n, seed, lo=-1.0, hi=1.0):
    s = C.c_uint(seed)
    out = np.empty(n, dtype=np.uint16)
    oracle().or_fill_lcg_bf16(out, n, C.byref(s), lo, hi)
    return out, s.value


def lcg_f32(n, seed, lo=-1.0, hi=1.0):
    s = C.c_uint(seed)
    out = np.empty(n, dtype=np.float32)
    oracle().or_fill_lcg_f32(out, n, C.byref(s), lo, hi)
    return out, s.value


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(f):
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(f, dtype=np.float32))
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


class QBlock:
    """INT8 per-row block as three numpy arrays (codes are the stored int8 = u - 128)."""

    def __init__(self, q, scale, offset):
        self.q = np.ascontiguousarray(q, dtype=np.int8)
        self.scale = np.ascontiguousarray(scale, dtype=np.float32)
        self.offset = np.ascontiguousarray(offset, dtype=np.float32)
        self.out_dim, self.in_dim = self.q.shape

    def or_block(self):
        return OrBlock(self.q.ctypes.data, self.scale.ctypes.data, self.offset.ctypes.data,
                       self.out_dim, self.in_dim)


def or_quantize_bf16(W):
    W = np.ascontiguousarray(W, dtype=np.uint16)
    o, i = W.shape
    q = np.empty((o, i), np.int8)
    s = np.empty(o, np.float32)
    f = np.empty(o, np.float32)
    rc = oracle().or_quantize_bf16(q, s, f, W, o, i)
    assert rc == 0
    return QBlock(q, s, f)


def or_quantize_f32(W):
    W = np.ascontiguousarray(W, dtype=np.float32)
    o, i = W.shape
    q = np.empty((o, i), np.int8)
    s = np.empty(o, np.float32)
    f = np.empty(o, np.float32)
    rc = oracle().or_quantize_f32(q, s, f, W, o, i)
    assert rc == 0
    return QBlock(q, s, f)


def ref_quantize_bf16(W, variant="v4"):
    lib = ref(variant)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    o, i = W.shape
    q = np.empty((o, i), np.int8)
    s = np.empty(o, np.float32)
    f = np.empty(o, np.float32)
    nb = C.c_size_t(0)
    rc = lib.ref_quantize_bf16_copy(q, s, f, W, o, i, C.byref(nb))
    assert rc == 0
    return QBlock(q, s, f), nb.value


class RefBlock:
    """A reference ds_int4_block_t borrowing a QBlock's arrays."""

    def __init__(self, qb, variant="v4"):
        lib = ref(variant)
        self.qb = qb
        self.buf = C.create_string_buffer(lib.ref_block_sizeof())
        lib.ref_block_wrap(C.addressof(self.buf), qb.q, qb.scale, qb.offset, qb.out_dim, qb.in_dim)

    @property
    def ptr(self):
        return C.addressof(self.buf)


class MoELayer:
    """One MoE layer's weights on the host: INT8 experts + routers (f32 and bf16)."""

    def __init__(self, hidden, inter, n_experts, top_k, shared_inter, router_f32, router_bf16, gu, dn, sgu, sdn):
        self.hidden, self.inter, self.n_experts, self.top_k, self.shared_inter = (
            hidden, inter, n_experts, top_k, shared_inter)
        self.router_f32 = np.ascontiguousarray(router_f32, dtype=np.float32)
        self.router_bf16 = np.ascontiguousarray(router_bf16, dtype=np.uint16)
        self.gu, self.dn, self.sgu, self.sdn = gu, dn, sgu, sdn
        self._keep = []

    def or_layer(self):
        gu_arr = (OrBlock * self.n_experts)(*[b.or_block() for b in self.gu])
        dn_arr = (OrBlock * self.n_experts)(*[b.or_block() for b in self.dn])
        self._keep = [gu_arr, dn_arr]
        return OrLayer(self.hidden, self.inter, self.n_experts, self.top_k, self.shared_inter,
                       self.router_f32.ctypes.data, self.router_bf16.ctypes.data,
                       C.addressof(gu_arr), C.addressof(dn_arr), self.sgu.or_block(), self.sdn.or_block())

    def ref_layer(self, variant="v4"):
        lib = ref(variant)
        buf = C.create_string_buffer(lib.ref_layer_sizeof())
        lib.ref_layer_init(C.addressof(buf), self.hidden, self.inter, self.n_experts, self.top_k,
                           self.shared_inter, self.router_f32.ctypes.data, self.router_bf16.ctypes.data)
        for e in range(self.n_experts):
            g, d = self.gu[e], self.dn[e]
            lib.ref_layer_set_expert(C.addressof(buf), e, g.q, g.scale, g.offset, d.q, d.scale, d.offset)
        lib.ref_layer_set_expert(C.addressof(buf), -1, self.sgu.q, self.sgu.scale, self.sgu.offset,
                                 self.sdn.q, self.sdn.scale, self.sdn.offset)
        return buf


def make_moe_layer(seed, hidden=1280, inter=896, n_experts=64, top_k=6, n_shared=2, std=0.02):
    """Seeded synthetic MoE layer: every weight N(0, std) in bf16, experts quantized by the oracle.

    Seeds: router f32 = seed*1000+1, router bf16 = bf16 RNE of the same samples, expert e gate_up =
    seed*1000+10+2e, down = seed*1000+11+2e, shared gate_up = seed*1000+900, shared down = +901.
    """
    si = n_shared * inter
    base = seed * 1000
    rf = normal_f32(n_experts * hidden, base + 1, std).reshape(n_experts, hidden)
    rb = f32_to_bf16_rne(rf)
    gu, dn = [], []
    for e in range(n_experts):
        gu.append(or_quantize_bf16(normal_bf16(2 * inter * hidden, base + 10 + 2 * e, std).reshape(2 * inter, hidden)))
        dn.append(or_quantize_bf16(normal_bf16(hidden * inter, base + 11 + 2 * e, std).reshape(hidden, inter)))
    sgu = or_quantize_bf16(normal_bf16(2 * si * hidden, base + 900, std).reshape(2 * si, hidden))
    sdn = or_quantize_bf16(normal_bf16(hidden * si, base + 901, std).reshape(hidden, si))
    return MoELayer(hidden, inter, n_experts, top_k, si, rf, rb, gu, dn, sgu, sdn)
