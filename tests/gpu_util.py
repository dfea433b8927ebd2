"""Helpers for GPU tests: product-library tensors from numpy and back."""
from __future__ import annotations

import ctypes as C

import numpy as np

from cogito_amd.capi import CgTensorQuant, host_quant_from_arrays, last_error  # noqa: F401


def host_tensor(lib, arr: np.ndarray):
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    shape = (C.c_int * arr.ndim)(*arr.shape)
    t = lib.cg_tensor_new(shape, arr.ndim, False)
    assert t, last_error(lib)
    C.memmove(t.contents.data, arr.ctypes.data, arr.nbytes)
    return t


def device_tensor(lib, arr: np.ndarray):
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    shape = (C.c_int * arr.ndim)(*arr.shape)
    t = lib.cgx_tensor_device_new(shape, arr.ndim)
    assert t, last_error(lib)
    assert lib.cgx_memcpy_h2d(C.cast(t.contents.data, C.c_void_p), arr.ctypes.data,
                              arr.nbytes) == 0, last_error(lib)
    return t


def tensor_np(lib, t) -> np.ndarray:
    n = t.contents.size
    shape = tuple(t.contents.shape[i] for i in range(t.contents.ndim))
    out = np.empty(n, np.float32)
    assert lib.cgx_tensor_to_host(t, out.ctypes.data_as(C.POINTER(C.c_float))) == 0, \
        last_error(lib)
    return out.reshape(shape)


def quant_host_arrays(q) -> tuple[np.ndarray, np.ndarray]:
    n = q.contents.size
    ng = q.contents.num_groups
    data = np.ctypeslib.as_array(q.contents.data, shape=((n + 1) // 2,)).copy()
    scales = np.ctypeslib.as_array(q.contents.scales, shape=(ng,)).copy()
    return data, scales


def rel_err_rows(y: np.ndarray, ref: np.ndarray) -> float:
    """max over rows of max|y - ref| / max|ref| (the 1e-3 metric)."""
    y = y.reshape(ref.shape[0], -1).astype(np.float64)
    r = ref.reshape(ref.shape[0], -1).astype(np.float64)
    worst = 0.0
    for a, b in zip(y, r):
        scale = np.max(np.abs(b))
        worst = max(worst, float(np.max(np.abs(a - b)) / (scale if scale > 0 else 1.0)))
    return worst
