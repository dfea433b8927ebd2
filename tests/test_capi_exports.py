"""CPU: the C-ABI library loads, and exports every function that include/*.h
declares (no compute calls: there is no GPU here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from cogito_amd import capi

ROOT = Path(__file__).resolve().parents[1]
HEADERS = ["cg_tensor.h", "cg_quantize.h", "cg_speculative.h", "cg_flash_attn.h",
           "cg_serialization.h", "cg_mi355x.h"]


def declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = (ROOT / "include" / h).read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"static inline[^{]*\{[^}]*\}", "", text, flags=re.S)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(", text):
            name = m.group(1)
            if name.startswith(("cg_", "cgx_")) and name != "cg_backward_fn":
                names.add(name)
    return names


def test_headers_and_bindings_agree():
    decl = declared_functions()
    missing_in_bindings = decl - set(capi.SIGNATURES)
    extra_in_bindings = set(capi.SIGNATURES) - decl
    assert not missing_in_bindings, sorted(missing_in_bindings)
    assert not extra_in_bindings, sorted(extra_in_bindings)


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_cg_tensor_struct_size():
    # the reference struct on x86-64: pointers 8, ints 4, bools padded
    import ctypes as C
    assert C.sizeof(capi.CgTensor) == 168
    assert C.sizeof(capi.CgTensorQuant) == 56
    assert C.sizeof(capi.CgKvCacheInt4) == 56


def test_host_tensor_api_without_gpu(lib):
    import ctypes as C
    shape = (C.c_int * 2)(3, 4)
    t = lib.cg_tensor_full(shape, 2, 2.5, False)
    assert t and t.contents.size == 12 and t.contents.strides[0] == 4
    assert t.contents.data[11] == 2.5
    t2 = lib.cg_tensor_clone(t)
    new_shape = (C.c_int * 1)(12)
    lib.cg_tensor_reshape(t2, new_shape, 1)
    assert t2.contents.ndim == 1 and t2.contents.ref_count == 1
    assert not lib.cg_tensor_shape_equal(t, t2)
    lib.cg_tensor_free(t)
    lib.cg_tensor_free(t2)


def test_declared_only_functions_report_errors(lib):
    lib.cgx_clear_error()
    assert not lib.cg_quantize_gptq(None, None, 128, 4)
    assert "not implemented" in capi.last_error(lib)


def test_device_draws_reject_bad_arguments_without_gpu(lib):
    """The device-row draw entry points check their arguments before any
    device call: null pointers and empty rows are errors, on any host."""
    lib.cgx_clear_error()
    assert lib.cgx_sample_temperature_dev(None, 32000, 1.0, 0.5, None) == -1
    assert "invalid argument" in capi.last_error(lib)
    lib.cgx_clear_error()
    assert lib.cgx_sample_temperature_rows_dev(None, 4, 32000, 1.0, None, None, 32000) == -1
    assert "invalid argument" in capi.last_error(lib)
    lib.cgx_clear_error()
    buf = ctypes.create_string_buffer(16)
    p = ctypes.addressof(buf)
    assert lib.cgx_sample_temperature_rows_dev(p, 0, 32000, 1.0, p, p, 32000) == -1
    assert "invalid argument" in capi.last_error(lib)
    assert lib.cgx_sample_row_certified(-1) in (0, 1)
