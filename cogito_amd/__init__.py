"""cogito_amd -- MI355X-native implementation of cogito's speculative-decoding
verify path (acceptance sampling, INT4 GEMV, flash attention over an INT4 KV
cache) behind cogito's C API.

The product is the shared library ``lib/libcogito_mi355x.so`` (HIP kernels
for gfx950 plus the C implementation of cg_speculative.h / cg_quantize.h /
cg_flash_attn.h).  This Python package only locates and loads it; there is
no Python or CPU compute path.  :func:`load` raises when the library has not
been built.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libcogito_mi355x.so"

_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library (once).  Raises if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(hipcc, gfx950); there is no fallback path")
        _lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
        from . import capi
        capi.declare(_lib)
    return _lib


__all__ = ["load", "LIB_PATH"]
