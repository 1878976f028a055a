"""ctypes bindings of libds_ocr_hip.so — the MI355X build of ds-ocr's INT8 MoE decode path.

The library is C-ABI (include/ds_quantize.h, include/ds_kernels.h, include/ds_hip.h). This module
only loads it from this directory and declares the signatures; it never falls back to another
implementation: if the library is missing, load() raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libds_ocr_hip.so")

ROUTE_DECODE = 0
ROUTE_CFG = 1

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
vp = C.c_void_p


class Int4Block(C.Structure):
    """ds_int4_block_t (include/ds_quantize.h)."""
    _fields_ = [("qweight", vp), ("scale", vp), ("offset", vp), ("out_dim", C.c_int), ("in_dim", C.c_int),
                ("bytes", C.c_size_t)]


# name -> (restype, argtypes); the exported C-ABI surface.
SIGNATURES = {
    # ds_quantize.h
    "ds_int4_quantize_bf16": (C.c_int, [C.POINTER(Int4Block), u16p, C.c_int, C.c_int]),
    "ds_int4_quantize_f32": (C.c_int, [C.POINTER(Int4Block), f32p, C.c_int, C.c_int]),
    "ds_int4_block_free": (None, [C.POINTER(Int4Block)]),
    "ds_int4_dequantize_f32": (None, [f32p, C.POINTER(Int4Block)]),
    "ds_int4_matvec": (None, [f32p, f32p, C.POINTER(Int4Block)]),
    "ds_int4_matvec_rows": (None, [f32p, f32p, C.POINTER(Int4Block), C.c_int, C.c_int]),
    "ds_expert_forward_fused_int4": (None, [f32p, f32p, C.POINTER(Int4Block), C.POINTER(Int4Block), C.c_int,
                                            C.c_int, vp, vp, vp, vp]),
    "ds_int4_quant_error_rms": (C.c_float, [C.POINTER(Int4Block), u16p]),
    # ds_kernels.h
    "ds_linear_nobias_bf16": (None, [f32p, f32p, u16p, C.c_int, C.c_int, C.c_int]),
    "ds_vec_add": (None, [f32p, f32p, f32p, C.c_int]),
    "ds_swiglu_direct": (None, [f32p, f32p, f32p, C.c_int, C.c_int]),
    "ds_moe_router": (None, [f32p, f32p, f32p, C.c_int, C.c_int]),
    "ds_moe_router_bf16": (None, [f32p, f32p, u16p, C.c_int, C.c_int]),
    "ds_moe_top_k": (None, [i32p, f32p, f32p, C.c_int, C.c_int]),
    "ds_expert_forward_fused": (None, [f32p, f32p, u16p, u16p, C.c_int, C.c_int, vp, vp, vp, vp]),
    "ds_expert_combine": (None, [f32p, f32p, vp, f32p, C.c_int, C.c_int]),
    "ds_argmax_matvec_bf16": (C.c_int, [f32p, u16p, C.c_int, C.c_int]),
    "ds_argmax_matvec_bf16_excluding": (C.c_int, [f32p, u16p, C.c_int, C.c_int, vp, C.c_int]),
    "ds_bf16_dot_row": (C.c_float, [f32p, u16p, C.c_int, C.c_int]),
    "ds_bf16_matvec_pub": (None, [f32p, f32p, u16p, vp, C.c_int, C.c_int]),
    "ds_bf16_truncate_array": (None, [f32p, C.c_int]),
    "ds_set_threads": (None, [C.c_int]),
    "ds_get_threads": (C.c_int, []),
    "ds_get_num_cpus": (C.c_int, []),
    "ds_dispatch_ensure_init": (None, []),
    "ds_parallel_for": (None, [vp, vp]),
    # ds_hip.h
    "ds_hip_init": (C.c_int, []),
    "ds_hip_last_error": (C.c_char_p, []),
    "ds_hip_malloc": (vp, [C.c_size_t]),
    "ds_hip_free": (None, [vp]),
    "ds_hip_memcpy_h2d": (C.c_int, [vp, vp, C.c_size_t]),
    "ds_hip_memcpy_d2h": (C.c_int, [vp, vp, C.c_size_t]),
    "ds_hip_time_stream_read": (C.c_int, [vp, C.c_size_t, C.c_int, C.POINTER(C.c_float)]),
    "ds_hip_time_expert": (C.c_int, [C.POINTER(Int4Block), C.POINTER(Int4Block), C.c_int, C.c_int, vp, C.c_int,
                                     C.POINTER(C.c_float)]),
    "ds_hip_memcpy_d2d": (C.c_int, [vp, vp, C.c_size_t]),
    "ds_hip_sync": (C.c_int, []),
    "ds_hip_fill_normal_bf16": (C.c_int, [vp, C.c_size_t, C.c_uint64, C.c_float]),
    "ds_hip_fill_normal_f32": (C.c_int, [vp, C.c_size_t, C.c_uint64, C.c_float, C.c_float]),
    "ds_hip_quantize_bf16": (C.c_int, [vp, vp, vp, vp, C.c_int, C.c_int]),
    "ds_hip_int8_matvec": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int]),
    "ds_hip_argmax_bf16": (C.c_int, [vp, vp, vp, C.c_int, C.c_int]),
    "ds_hip_layer_create": (vp, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "ds_hip_layer_destroy": (None, [vp]),
    "ds_hip_layer_bytes": (C.c_size_t, [vp]),
    "ds_hip_layer_set_router": (C.c_int, [vp, vp, vp]),
    "ds_hip_layer_set_router_dev": (C.c_int, [vp, vp, vp]),
    "ds_hip_layer_set_expert": (C.c_int, [vp, C.c_int, C.POINTER(Int4Block), C.POINTER(Int4Block)]),
    "ds_hip_layer_quantize_expert": (C.c_int, [vp, C.c_int, vp, vp]),
    "ds_hip_layer_export_expert": (C.c_int, [vp, C.c_int, vp, vp, vp, vp, vp, vp]),
    "ds_hip_layer_forward": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, vp, vp]),
    "ds_hip_layer_prefill": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, vp]),
    "ds_hip_time_prefill": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float)]),
    "ds_hip_time_layer": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.POINTER(C.c_float)]),
    "ds_hip_prefill_path": (C.c_int, [C.c_int]),
    "ds_hip_stack_set_graph_steps": (C.c_int, [C.c_void_p, C.c_int]),
    "ds_hip_prefill_wait_error": (C.c_int, [vp, C.c_int]),
    "ds_hip_prefill_set_wait_limit": (C.c_int, [C.c_int]),
    "ds_hip_route_stats": (C.c_int, [vp, C.c_int]),
    "ds_hip_set_route_log": (C.c_int, [vp, C.c_int]),
    "ds_hip_check_prefill_swiglu": (C.c_int, [vp]),
    "ds_hip_stack_create": (vp, [vp, C.c_int, vp, C.c_int, C.c_int]),
    "ds_hip_stack_destroy": (None, [vp]),
    "ds_hip_stack_bind": (C.c_int, [vp, vp, C.c_int, C.c_int, vp, C.c_int]),
    "ds_hip_stack_set_embedding": (C.c_int, [vp, vp, C.c_int]),
    "ds_hip_stack_capacity": (C.c_int, [vp]),
    "ds_hip_argmax_bf16_noalloc": (C.c_int, [vp, vp, vp, C.c_int, C.c_int]),
    "ds_hip_weights_changed": (C.c_int, [vp]),
    "ds_hip_argmax_int8_copy": (C.c_int, [vp]),
    "ds_hip_register_block": (C.c_int, [C.POINTER(Int4Block)]),
    "ds_hip_register_weights": (C.c_int, [vp, C.c_size_t]),
    "ds_hip_stack_steps_left": (C.c_int, [vp]),
    "ds_hip_stack_capacity_for": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "ds_hip_steps_fit": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "ds_hip_time_stack_each": (C.c_int, [vp, C.c_int, f32p]),
    "ds_hip_time_stack_span": (C.c_int, [vp, C.c_int, C.c_int, C.c_int, f32p]),
    "ds_hip_stack_reset": (C.c_int, [vp]),
    "ds_hip_stack_run": (C.c_int, [vp, C.c_int]),
    "ds_hip_stack_run_eager": (C.c_int, [vp, C.c_int]),
    "ds_hip_stack_hidden": (C.c_int, [vp, f32p]),
    "ds_hip_stack_bytes_per_step": (C.c_size_t, [vp]),
    "ds_hip_time_stack": (C.c_int, [vp, C.c_int, C.POINTER(C.c_float)]),
    "ds_hip_time_lm_head": (C.c_int, [vp, C.c_int, C.POINTER(C.c_float)]),
    "ds_hip_stack_kernel_count": (C.c_int, [vp]),
    "ds_hip_attn_create": (vp, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, vp, vp, vp, vp, vp, vp,
                                vp, vp]),
    "ds_hip_attn_destroy": (None, [vp]),
    "ds_hip_attn_set_window": (C.c_int, [vp, C.c_int, C.c_int]),
    "ds_hip_attn_kv": (C.c_int, [vp, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), C.POINTER(C.c_int)]),
    "ds_hip_attn_load_kv": (C.c_int, [vp, vp, vp, C.c_int, C.c_int]),
    "ds_hip_attn_forward": (C.c_int, [vp, vp, vp, vp, C.c_int]),
    "ds_hip_stack_set_attention": (C.c_int, [vp, vp, C.c_int, vp, C.c_float, C.c_int, C.c_int]),
    "ds_hip_stack_set_sampling": (C.c_int, [vp, C.c_float, C.c_int, C.c_int]),
    "ds_hip_lm_head_sample": (C.c_int, [vp, vp, C.c_int, C.c_int, vp, C.c_int, C.c_float, C.c_int, vp]),
    "ds_hip_stack_kernel_name": (C.c_char_p, [vp, C.c_int]),
    "ds_hip_profile_stack": (C.c_int, [vp, C.c_int, f32p]),
    "ds_hip_dense_create": (vp, [C.c_int, C.c_int, vp, vp, vp]),
    "ds_hip_dense_destroy": (None, [vp]),
    "ds_hip_dense_forward": (C.c_int, [vp, vp, vp, C.c_int]),
    "ds_hip_stack_set_dense": (C.c_int, [vp, vp]),
    "ds_hip_stack_set_layer_kernels": (C.c_int, [vp, C.c_int]),
    "ds_hip_stack_layer_kernels": (C.c_int, [vp]),
    "ds_hip_stack_set_lm_certified": (C.c_int, [vp, C.c_int]),
    "ds_hip_stack_lm_certified": (C.c_int, [vp]),
    "ds_hip_load_dense": (C.c_int, [C.POINTER(C.c_char_p), C.c_int, C.c_int, C.POINTER(vp)]),
    "ds_hip_safetensors_info": (C.c_int, [C.POINTER(C.c_char_p), C.c_int, C.c_char_p, C.POINTER(C.c_int),
                                          C.POINTER(C.c_int64), C.c_int]),
    "ds_hip_load_moe_layers": (C.c_int, [C.POINTER(C.c_char_p), C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.POINTER(vp)]),
    "ds_hip_load_lm_head": (C.c_int, [C.POINTER(C.c_char_p), C.c_int, C.POINTER(vp), C.POINTER(C.c_int),
                                      C.POINTER(C.c_int)]),
    "ds_hip_arena_save": (C.c_int, [C.c_char_p, C.POINTER(vp), C.c_int, vp, C.c_int]),
    "ds_hip_arena_load": (C.c_int, [C.c_char_p, C.POINTER(vp), C.c_int, C.POINTER(vp), C.POINTER(C.c_int)]),
}

# Data symbols (mode globals).
GLOBALS = ["ds_verbose", "ds_bf16_simulate_python"]

_lib = None


def load():
    """Loads the in-tree libds_ocr_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class HipError(RuntimeError):
    pass


def check(rc, what=""):
    if rc != 0:
        msg = load().ds_hip_last_error().decode(errors="replace")
        raise HipError(f"{what}: {msg}")


def set_bf16sim(on):
    C.c_int.in_dll(load(), "ds_bf16_simulate_python").value = 1 if on else 0


def get_bf16sim():
    return C.c_int.in_dll(load(), "ds_bf16_simulate_python").value


class DeviceBuffer:
    """A device allocation owned by Python (freed on close/GC)."""

    def __init__(self, nbytes):
        lib = load()
        self.nbytes = int(nbytes)
        self.ptr = lib.ds_hip_malloc(max(self.nbytes, 16))
        if not self.ptr:
            raise HipError("ds_hip_malloc: " + lib.ds_hip_last_error().decode())

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        check(load().ds_hip_memcpy_h2d(b.ptr, arr.ctypes.data, arr.nbytes), "h2d")
        return b

    def to_array(self, dtype, count=None):
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(n, dtype=dtype)
        check(load().ds_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def write(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(load().ds_hip_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes), "h2d")

    def close(self):
        if self.ptr:
            load().ds_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def block_from_arrays(q, scale, offset):
    """A ds_int4_block_t borrowing numpy arrays (keep them alive while the block is used). Converted
    copies (non-contiguous or other dtypes) are held by the block itself."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(scale, np.float32)
    o = np.ascontiguousarray(offset, np.float32)
    b = Int4Block(q.ctypes.data, s.ctypes.data, o.ctypes.data, q.shape[0], q.shape[1], q.size + 8 * q.shape[0])
    b._arrays = (q, s, o)
    return b


def block_arrays(b):
    """Copies a library-owned block's host arrays into numpy (codes, scales, offsets)."""
    n = b.out_dim * b.in_dim
    q = np.ctypeslib.as_array(C.cast(b.qweight, C.POINTER(C.c_int8)), shape=(n,)).copy().reshape(b.out_dim, b.in_dim)
    s = np.ctypeslib.as_array(C.cast(b.scale, C.POINTER(C.c_float)), shape=(b.out_dim,)).copy()
    o = np.ctypeslib.as_array(C.cast(b.offset, C.POINTER(C.c_float)), shape=(b.out_dim,)).copy()
    return q, s, o
