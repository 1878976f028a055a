"""The C-ABI library loads without a GPU and exports every function include/*.h declares (no
compute calls here)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)  # header-inline helpers
        for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\([^;{]*\)\s*;", text):
            name = m.group(1)
            if name.startswith("ds_"):
                names.add(name)
    return sorted(names)


def test_headers_declare_the_reference_boundary():
    names = declared_functions()
    for n in ["ds_int4_quantize_bf16", "ds_int4_matvec", "ds_int4_matvec_rows", "ds_expert_forward_fused_int4",
              "ds_expert_forward_fused", "ds_argmax_matvec_bf16", "ds_moe_router", "ds_moe_top_k",
              "ds_hip_stack_create"]:
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    L = lib.load()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing
    for g in lib.GLOBALS:
        C.c_int.in_dll(L, g)


def test_binding_signatures_cover_headers(lib):
    assert set(declared_functions()) <= set(lib.SIGNATURES), sorted(set(declared_functions()) - set(lib.SIGNATURES))


def test_product_library_links_no_oracle(lib):
    """The shipped library must not depend on the test oracle."""
    data = open(lib.LIB_PATH, "rb").read()
    assert b"liboracle" not in data and b"libdsref" not in data
    assert b"or_quantize_bf16" not in data
