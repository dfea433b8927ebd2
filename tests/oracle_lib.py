"""ctypes access to the CPU checkers (test infrastructure only):

* ``load_oracle()`` -- oracle/_build/liboracle.so, the C restatement;
* ``load_ref()``    -- oracle/_ref/libcgref.so, cogito's own sources compiled
  from the reference tree (None when it was not built).

Plus numpy-facing wrappers used by the tests and by bench.py's CPU baseline.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "_build" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libcgref.so"

F = C.c_float
I = C.c_int
VP = C.c_void_p

_ORACLE_SIGS = {
    "orc_lcg_next_state": (C.c_uint32, [C.c_uint32]),
    "orc_lcg_uniform": (F, [C.POINTER(C.c_uint32)]),
    "orc_acceptance_prob": (F, [F, F]),
    "orc_sample_temperature": (I, [VP, I, F, F]),
    "orc_temperature_probs": (None, [VP, I, F, VP]),
    "orc_top_k_list": (None, [VP, I, I, VP, VP]),
    "orc_sample_top_k": (I, [VP, I, I, F]),
    "orc_top_p_sorted": (I, [VP, I, F, VP, VP, C.POINTER(F)]),
    "orc_sample_top_p": (I, [VP, I, F, F]),
    "orc_sample_corrected": (I, [VP, VP, I, F]),
    "orc_filtered_dist": (I, [VP, I, F, I, F, VP]),
    "orc_sample_filtered": (I, [VP, I, F, I, F, F]),
    "orc_verify_chain": (I, [VP, VP, VP, VP, I, I, F, I, F, VP, VP]),
    "orc_verify_chain_many": (None, [VP, VP, VP, VP, I, I, I, F, I, F, VP, VP]),
    "orc_typ_log": (C.c_double, [F]),
    "orc_typical_sorted": (I, [VP, I, F, VP, VP, C.POINTER(F)]),
    "orc_sample_typical": (I, [VP, I, F, F]),
    "orc_typical_dist": (None, [VP, I, F, VP]),
    "orc_quantize_int4": (None, [VP, I, I, VP, VP]),
    "orc_dequantize_int4": (None, [VP, VP, I, I, VP]),
    "orc_matmul_int4": (None, [VP, I, I, VP, VP, I, I, VP]),
    "orc_kv_append": (None, [VP, VP, VP, VP, I, I, I, I, VP, VP]),
    "orc_kv_get": (None, [VP, VP, VP, VP, I, I, I, I, VP, VP]),
    "orc_flash_fwd": (None, [VP, VP, VP, VP, VP, I, I, I, I, I, I, F, I, I, VP]),
    "orc_apply_rope": (None, [VP, I, I, I, I, F]),
    "orc_rope_freqs": (None, [VP, VP, I, I, F]),
    "orc_alibi_slopes": (None, [VP, I]),
    "orc_fill_key": (C.c_uint32, [C.c_uint64, C.c_uint32]),
    "orc_fill_normal": (None, [VP, C.c_size_t, C.c_uint64, C.c_uint32, F]),
    "orc_alibi_bias": (None, [VP, I, I, I, VP]),
    "orc_rmsnorm": (None, [VP, VP, VP, I, I, F]),
    "orc_swiglu": (None, [VP, VP, VP, I]),
    "orc_softmax_rows": (None, [VP, VP, I, I]),
    "orc_tree_mask_chain": (None, [VP, I, I]),
    "orc_topk_lists": (None, [VP, I, I, F, VP, VP]),
    "orc_tree_accept": (I, [VP, I, I, VP, VP, VP, VP, VP, VP]),
}

_oracle = None
_ref = None


def _open_oracle(path: Path) -> C.CDLL:
    if not path.exists():
        raise RuntimeError(f"{path} missing: run `make -C oracle`")
    lib = C.CDLL(str(path), mode=C.RTLD_LOCAL)
    for name, (res, args) in _ORACLE_SIGS.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def load_oracle() -> C.CDLL:
    global _oracle
    if _oracle is None:
        _oracle = _open_oracle(ORACLE_SO)
    return _oracle


def load_oracle_mutant(n: int) -> C.CDLL:
    """The oracle built with planted mistake n (ORC_MUTANT in cg_oracle.c)."""
    return _open_oracle(ORACLE_SO.with_name(f"liboracle_mut{n}.so"))


class RefTensor(C.Structure):
    """Layout of the reference's cg_tensor (identical to ours)."""


RefTensor._fields_ = [
    ("data", C.POINTER(F)), ("grad", C.POINTER(F)),
    ("shape", I * 8), ("strides", I * 8), ("ndim", I), ("size", I),
    ("requires_grad", C.c_bool), ("backward_fn", VP),
    ("parents", C.POINTER(RefTensor) * 4), ("num_parents", I),
    ("backward_ctx", VP), ("ref_count", I), ("is_view", C.c_bool), ("arena", VP),
]


class RefQuant(C.Structure):
    _fields_ = [
        ("data", C.POINTER(C.c_uint8)), ("scales", C.POINTER(F)),
        ("zeros", C.POINTER(F)), ("shape", C.POINTER(I)), ("ndim", I),
        ("size", I), ("quant_type", I), ("group_size", I), ("num_groups", I),
        ("symmetric", C.c_bool),
    ]


class RefKv(C.Structure):
    _fields_ = [
        ("k_cache", C.POINTER(C.c_uint8)), ("v_cache", C.POINTER(C.c_uint8)),
        ("k_scales", C.POINTER(F)), ("v_scales", C.POINTER(F)),
        ("current_len", I), ("max_seq_len", I), ("num_layers", I),
        ("n_heads", I), ("head_dim", I), ("group_size", I),
    ]


_REF_SIGS = {
    "cg_tensor_new": (C.POINTER(RefTensor), [C.POINTER(I), I, C.c_bool]),
    "cg_tensor_free": (None, [C.POINTER(RefTensor)]),
    "cg_quantize_int4": (C.POINTER(RefQuant), [C.POINTER(RefTensor), I]),
    "cg_dequantize": (C.POINTER(RefTensor), [C.POINTER(RefQuant)]),
    "cg_tensor_quant_free": (None, [C.POINTER(RefQuant)]),
    "cg_matmul_int4": (None, [C.POINTER(RefTensor), C.POINTER(RefQuant),
                              C.POINTER(RefTensor)]),
    "cg_kv_cache_int4_new": (C.POINTER(RefKv), [I, I, I, I, I]),
    "cg_kv_cache_int4_append": (None, [C.POINTER(RefKv), I, C.POINTER(RefTensor),
                                       C.POINTER(RefTensor)]),
    "cg_kv_cache_int4_get": (None, [C.POINTER(RefKv), I, C.POINTER(RefTensor),
                                    C.POINTER(RefTensor)]),
    "cg_kv_cache_int4_free": (None, [C.POINTER(RefKv)]),
    "cg_sample_temperature": (I, [VP, I, F]),
    "cg_sample_top_p": (I, [VP, I, F]),
    "cg_sample_top_k": (I, [VP, I, I]),
    "cg_sample_corrected": (I, [VP, VP, I]),
    "cg_acceptance_prob": (F, [F, F]),
    "cg_tree_attention_mask": (C.POINTER(RefTensor), [VP, I]),
    "cg_token_tree_new": (VP, [I]),
    "cg_token_tree_free": (None, [VP]),
    "cg_token_tree_to_tensor": (C.POINTER(RefTensor), [VP]),
    "cg_flash_attention_forward_cuda": (None, [VP]),
    "cg_flash_attention_forward_cpu": (None, [VP]),
    "cg_apply_rope": (None, [VP, VP, I, I, I, I, F]),
    "cg_rope_precompute_freqs": (None, [VP, VP, I, I, F]),
    "cg_alibi_slopes": (None, [VP, I]),
    "cg_alibi_bias": (None, [VP, I, I, I, VP]),
    "cg_kv_cache_int4_reset": (None, [C.POINTER(RefKv)]),
    "cg_cuda_rmsnorm_forward": (None, [C.POINTER(RefTensor), C.POINTER(RefTensor),
                                       C.POINTER(RefTensor), F]),
    "cg_cuda_softmax_forward": (None, [C.POINTER(RefTensor), C.POINTER(RefTensor), I]),
    "cg_swiglu_forward_split": (C.POINTER(RefTensor), [C.POINTER(RefTensor)]),
}


def load_ref():
    global _ref
    if _ref is None and REF_SO.exists():
        lib = C.CDLL(str(REF_SO), mode=C.RTLD_LOCAL)
        for name, (res, args) in _REF_SIGS.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _ref = lib
    return _ref


# ---------------------------------------------------------------- helpers

def ptr(a: np.ndarray) -> C.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


def ref_tensor(lib, arr: np.ndarray):
    """A reference cg_tensor holding a copy of `arr` (float32)."""
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    shape = (I * arr.ndim)(*arr.shape)
    t = lib.cg_tensor_new(shape, arr.ndim, False)
    C.memmove(t.contents.data, arr.ctypes.data, arr.nbytes)
    return t


def ref_tensor_np(t) -> np.ndarray:
    n = t.contents.size
    shape = tuple(t.contents.shape[i] for i in range(t.contents.ndim))
    return np.ctypeslib.as_array(t.contents.data, shape=(n,)).copy().reshape(shape)


class LCG:
    """Mirror of the reference's global LCG stream (seed 42)."""

    def __init__(self, state: int = 42):
        self.state = C.c_uint32(state)

    def draw(self, orc) -> float:
        return orc.orc_lcg_uniform(C.byref(self.state))


def oracle_quantize(orc, x: np.ndarray, gs: int):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    n = x.size
    data = np.zeros((n + 1) // 2, np.uint8)
    scales = np.zeros((n + gs - 1) // gs, np.float32)
    orc.orc_quantize_int4(ptr(x), n, gs, ptr(data), ptr(scales))
    return data, scales


def oracle_matmul(orc, x: np.ndarray, data, scales, K: int, N: int, gs: int):
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.zeros((M, N), np.float32)
    orc.orc_matmul_int4(ptr(x), M, K, ptr(data), ptr(scales), N, gs, ptr(y))
    return y
