"""ctypes declarations of the C ABI (include/*.h) for tests and the bench.

The structs mirror the C layouts field for field; `declare` sets argtypes and
restypes on a loaded library so that calls are type-checked.
"""
from __future__ import annotations

import ctypes as C

from typing import Iterable

CG_MAX_DIMS = 8
CG_MAX_PARENTS = 4


class CgTensor(C.Structure):
    pass


CgTensor._fields_ = [
    ("data", C.POINTER(C.c_float)),
    ("grad", C.POINTER(C.c_float)),
    ("shape", C.c_int * CG_MAX_DIMS),
    ("strides", C.c_int * CG_MAX_DIMS),
    ("ndim", C.c_int),
    ("size", C.c_int),
    ("requires_grad", C.c_bool),
    ("backward_fn", C.c_void_p),
    ("parents", C.POINTER(CgTensor) * CG_MAX_PARENTS),
    ("num_parents", C.c_int),
    ("backward_ctx", C.c_void_p),
    ("ref_count", C.c_int),
    ("is_view", C.c_bool),
    ("arena", C.c_void_p),
]


class CgTensorQuant(C.Structure):
    _fields_ = [
        ("data", C.POINTER(C.c_uint8)),
        ("scales", C.POINTER(C.c_float)),
        ("zeros", C.POINTER(C.c_float)),
        ("shape", C.POINTER(C.c_int)),
        ("ndim", C.c_int),
        ("size", C.c_int),
        ("quant_type", C.c_int),
        ("group_size", C.c_int),
        ("num_groups", C.c_int),
        ("symmetric", C.c_bool),
    ]


class CgKvCacheInt4(C.Structure):
    _fields_ = [
        ("k_cache", C.POINTER(C.c_uint8)),
        ("v_cache", C.POINTER(C.c_uint8)),
        ("k_scales", C.POINTER(C.c_float)),
        ("v_scales", C.POINTER(C.c_float)),
        ("current_len", C.c_int),
        ("max_seq_len", C.c_int),
        ("num_layers", C.c_int),
        ("n_heads", C.c_int),
        ("head_dim", C.c_int),
        ("group_size", C.c_int),
    ]


class CgTokenTree(C.Structure):
    _fields_ = [
        ("tokens", C.POINTER(C.c_int)),
        ("draft_probs", C.POINTER(C.c_float)),
        ("target_probs", C.POINTER(C.c_float)),
        ("accepted", C.POINTER(C.c_bool)),
        ("hidden_states", C.POINTER(CgTensor)),
        ("depth", C.c_int),
        ("branch_points", C.POINTER(C.c_int)),
        ("num_branches", C.c_int),
    ]


class CgSpeculativeDecoder(C.Structure):
    _fields_ = [
        ("draft_model", C.c_void_p),
        ("target_model", C.c_void_p),
        ("gamma", C.c_int),
        ("temperature", C.c_float),
        ("top_p", C.c_float),
        ("top_k", C.c_int),
        ("accept_threshold", C.c_float),
        ("use_typical_sampling", C.c_bool),
        ("total_draft_tokens", C.c_int),
        ("accepted_draft_tokens", C.c_int),
        ("avg_acceptance_rate", C.c_float),
        ("num_steps", C.c_int),
        ("draft_kv_cache", C.c_void_p),
        ("target_kv_cache", C.c_void_p),
    ]


class CgFlashAttnParams(C.Structure):
    _fields_ = [
        ("Q", C.c_void_p), ("K", C.c_void_p), ("V", C.c_void_p), ("O", C.c_void_p),
        ("mask", C.c_void_p), ("dropout_mask", C.c_void_p),
        ("batch_size", C.c_int), ("seqlen_q", C.c_int), ("seqlen_k", C.c_int),
        ("n_heads", C.c_int), ("n_heads_k", C.c_int), ("d_head", C.c_int),
        ("scale", C.c_float), ("dropout_prob", C.c_float),
        ("mask_type", C.c_int), ("window_size", C.c_int),
        ("is_training", C.c_bool), ("softmax_lse", C.c_void_p),
        ("dO", C.c_void_p), ("dQ", C.c_void_p), ("dK", C.c_void_p), ("dV", C.c_void_p),
    ]


class CgFlashAttnConfig(C.Structure):
    _fields_ = [
        ("block_m", C.c_int), ("block_n", C.c_int), ("split_k", C.c_int),
        ("use_persistent", C.c_bool), ("use_register_tile", C.c_bool),
        ("num_warps", C.c_int), ("sm_count", C.c_int),
    ]


class CgxModelConfig(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("d_model", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("d_ff", C.c_int),
        ("vocab", C.c_int), ("group_size", C.c_int), ("kv_group_size", C.c_int),
        ("max_seq", C.c_int), ("max_tokens", C.c_int), ("rope_theta", C.c_float),
        ("norm_eps", C.c_float), ("init_std", C.c_float), ("max_batch", C.c_int),
    ]


PT = C.POINTER(CgTensor)
PQ = C.POINTER(CgTensorQuant)
PKV = C.POINTER(CgKvCacheInt4)
PTREE = C.POINTER(CgTokenTree)
PDEC = C.POINTER(CgSpeculativeDecoder)
PPARAMS = C.POINTER(CgFlashAttnParams)
VP = C.c_void_p
I = C.c_int
F = C.c_float
SZ = C.c_size_t

# name -> (restype, argtypes).  Every symbol declared in include/*.h.
SIGNATURES: dict[str, tuple] = {
    # cg_tensor.h
    "cg_tensor_new": (PT, [C.POINTER(I), I, C.c_bool]),
    "cg_tensor_zeros": (PT, [C.POINTER(I), I, C.c_bool]),
    "cg_tensor_ones": (PT, [C.POINTER(I), I, C.c_bool]),
    "cg_tensor_full": (PT, [C.POINTER(I), I, F, C.c_bool]),
    "cg_tensor_from_data": (PT, [C.POINTER(F), C.POINTER(I), I, C.c_bool]),
    "cg_tensor_clone": (PT, [PT]),
    "cg_tensor_retain": (None, [PT]),
    "cg_tensor_release": (None, [PT]),
    "cg_tensor_free": (None, [PT]),
    "cg_tensor_reshape": (None, [PT, C.POINTER(I), I]),
    "cg_tensor_shape_equal": (C.c_bool, [PT, PT]),
    # cg_quantize.h
    "cg_quantize_int4": (PQ, [PT, I]),
    "cg_quantize_gptq": (PQ, [PT, PT, I, I]),
    "cg_quantize_awq": (PQ, [PT, PT, I]),
    "cg_quantize_nf4": (PQ, [PT, I]),
    "cg_dequantize": (PT, [PQ]),
    "cg_tensor_quant_free": (None, [PQ]),
    "cg_matmul_int4": (None, [PT, PQ, PT]),
    "cg_gemv_int4": (None, [PT, PQ, PT]),
    "cg_attention_int4_kv": (None, [PT, PKV, I, PT]),
    "cg_kv_cache_int4_new": (PKV, [I, I, I, I, I]),
    "cg_kv_cache_int4_append": (None, [PKV, I, PT, PT]),
    "cg_kv_cache_int4_get": (None, [PKV, I, PT, PT]),
    "cg_kv_cache_int4_reset": (None, [PKV]),
    "cg_kv_cache_int4_free": (None, [PKV]),
    "cg_calibration_new": (VP, [I]),
    "cg_calibration_update": (None, [VP, PT]),
    "cg_calibration_compute_scales": (None, [VP, C.POINTER(F), C.POINTER(F), I]),
    "cg_calibration_free": (None, [VP]),
    # cg_speculative.h
    "cg_speculative_decoder_new": (PDEC, [VP, VP, I]),
    "cg_speculative_generate": (PT, [PDEC, PT, I, F, F]),
    "cg_speculative_step": (I, [PDEC, PT, PTREE]),
    "cg_draft_generate": (PTREE, [PDEC, PT]),
    "cg_target_verify": (I, [PDEC, PT, PTREE]),
    "cg_speculative_decoder_free": (None, [PDEC]),
    "cg_token_tree_new": (PTREE, [I]),
    "cg_token_tree_add_token": (None, [PTREE, I, C.POINTER(F)]),
    "cg_token_tree_to_tensor": (PT, [PTREE]),
    "cg_token_tree_free": (None, [PTREE]),
    "cg_tree_attention_mask": (PT, [PTREE, I]),
    "cg_forward_tree_attention": (PT, [VP, PT, PT]),
    "cg_eagle_draft_new": (VP, [VP]),
    "cg_eagle_generate_tree": (PTREE, [VP, PT, I]),
    "cg_eagle_compute_branching": (C.POINTER(I), [VP, PT]),
    "cg_eagle_draft_free": (None, [VP]),
    "cg_sample_temperature": (I, [VP, I, F]),
    "cg_sample_top_p": (I, [VP, I, F]),
    "cg_sample_top_k": (I, [VP, I, I]),
    "cg_sample_typical": (I, [VP, I, F]),
    "cg_acceptance_prob": (F, [F, F]),
    "cg_sample_corrected": (I, [VP, VP, I]),
    # cg_flash_attn.h
    "cg_flash_attention_forward": (None, [PPARAMS]),
    "cg_flash_attention_forward_cpu": (None, [PPARAMS]),
    "cg_flash_attention_backward": (None, [PPARAMS]),
    "cg_flash_attention_backward_cpu": (None, [PPARAMS]),
    "cg_flash_attention_mqa": (None, [PPARAMS]),
    "cg_flash_attention_gqa": (None, [PPARAMS, I]),
    "cg_flash_attn_params_new": (PPARAMS, [PT, PT, PT, I, F]),
    "cg_flash_attn_autotune": (CgFlashAttnConfig, [I, I, I, I]),
    "cg_flash_attn_shared_mem": (SZ, [I, I, I]),
    "cg_flash_attn_params_free": (None, [PPARAMS]),
    "cg_apply_rope": (None, [VP, VP, I, I, I, I, F]),
    "cg_rope_precompute_freqs": (None, [VP, VP, I, I, F]),
    "cg_alibi_bias": (None, [VP, I, I, I, VP]),
    "cg_alibi_slopes": (None, [VP, I]),
    # cg_serialization.h
    "cg_save_model": (None, [C.c_char_p, C.POINTER(PT), C.POINTER(C.c_char_p), I]),
    "cg_load_model": (None, [C.c_char_p, C.POINTER(C.POINTER(PT)),
                             C.POINTER(C.POINTER(C.c_char_p)), C.POINTER(I)]),
    # cg_mi355x.h
    "cgx_init": (I, [I]),
    "cgx_last_error": (C.c_char_p, []),
    "cgx_clear_error": (None, []),
    "cgx_device_count": (I, []),
    "cgx_stream": (VP, []),
    "cgx_synchronize": (I, []),
    "cgx_device_name": (C.c_char_p, []),
    "cgx_malloc": (VP, [SZ]),
    "cgx_free": (I, [VP]),
    "cgx_memcpy_h2d": (I, [VP, VP, SZ]),
    "cgx_memcpy_d2h": (I, [VP, VP, SZ]),
    "cgx_memcpy_d2d": (I, [VP, VP, SZ]),
    "cgx_memset": (I, [VP, I, SZ]),
    "cgx_is_device_ptr": (I, [VP]),
    "cgx_event_record": (I, [I]),
    "cgx_event_elapsed_ms": (F, [I, I]),
    "cgx_stream_read": (I, [VP, SZ, VP]),
    "cgx_tensor_device_new": (PT, [C.POINTER(I), I]),
    "cgx_tensor_to_device": (PT, [PT]),
    "cgx_tensor_to_host": (I, [PT, C.POINTER(F)]),
    "cgx_quant_to_device": (PQ, [PQ]),
    "cgx_quant_to_device_flat": (PQ, [PQ]),
    "cgx_quant_to_device_layout": (PQ, [PQ, I]),
    "cgx_quant_layout": (I, [PQ]),
    "cgx_matmul_int4_dev": (I, [VP, I, PQ, VP]),
    "cgx_matmul_int4_dev_kernel": (I, [VP, I, PQ, VP, I]),
    "cgx_lcg_seed": (None, [C.c_uint32]),
    "cgx_lcg_state": (C.c_uint32, []),
    "cgx_verify_chain": (I, [VP, VP, VP, VP, I, I, F, I, F, VP, VP]),
    "cgx_verify_chain_batch_dev": (I, [VP, VP, VP, VP, I, I, I, F, I, F, VP, VP, VP]),
    "cgx_verify_chain_batch_dev_noalloc": (I, [VP, VP, VP, VP, I, I, I, F, I, F, VP, VP, VP]),
    "cgx_verify_lean_min_blocks": (I, [I]),
    "cgx_graph_begin": (I, []),
    "cgx_graph_end": (VP, []),
    "cgx_graph_launch": (I, [VP]),
    "cgx_graph_free": (I, [VP]),
    "cgx_sample_temperature_u": (I, [VP, I, F, F]),
    "cgx_sample_temperature_dev": (I, [VP, I, F, F, VP]),
    "cgx_sample_temperature_rows_dev": (I, [VP, I, I, F, VP, VP, C.c_size_t]),
    "cgx_sample_top_k_u": (I, [VP, I, I, F]),
    "cgx_sample_top_p_u": (I, [VP, I, F, F]),
    "cgx_sample_corrected_u": (I, [VP, VP, I, F]),
    "cgx_filtered_dist": (I, [VP, I, F, I, F, VP]),
    "cgx_sample_typical_u": (I, [VP, I, F, F]),
    "cgx_typical_dist": (I, [VP, I, F, VP]),
    "cgx_last_verify_token": (I, []),
    "cgx_tree_attention_mask_parents": (PT, [VP, I, I]),
    "cgx_exact_expf_dev": (I, [VP, VP, I]),
    "cgx_ordered_sum_dev": (I, [VP, I, VP]),
    "cgx_sort_rows_dev": (I, [VP, VP, I, I, I, VP, VP]),
    "cgx_typ_log_dev": (I, [VP, VP, I]),
    "cgx_exp_fast_maxerr_dev": (I, [F, F, VP]),
    "cgx_exp_stat_maxerr_dev": (I, [F, F, VP]),
    "cgx_sample_row_certified": (I, [I]),
    "cgx_sample_row_fallbacks": (C.c_longlong, []),
    "cgx_save_quantized": (I, [C.c_char_p, C.POINTER(PQ), C.POINTER(C.c_char_p), I]),
    "cgx_load_quantized": (I, [C.c_char_p, C.POINTER(C.POINTER(PQ)),
                               C.POINTER(C.POINTER(C.c_char_p)), C.POINTER(I)]),
    "cgx_kv_cache_int4_truncate": (I, [PKV, I]),
    "cgx_kv_cache_int4_write": (I, [PKV, I, I, VP, VP, I]),
    "cgx_kv_cache_int4_set_len": (I, [PKV, I]),
    "cgx_attention_int4_kv_dev": (I, [VP, I, I, PKV, I, I, VP, VP]),
    "cgx_attention_int4_kv_batch_dev": (I, [VP, I, I, I, PKV, I, VP, I, VP, I, VP]),
    # synthetic decoder and the speculative loop
    "cgx_model_new": (VP, [C.POINTER(CgxModelConfig), C.c_uint64, VP]),
    "cgx_model_free": (None, [VP]),
    "cgx_model_forward": (I, [VP, VP, I, I, VP]),
    "cgx_model_logits": (VP, [VP]),
    "cgx_model_get_config": (I, [VP, C.POINTER(CgxModelConfig)]),
    "cgx_model_len": (I, [VP]),
    "cgx_model_truncate": (I, [VP, I]),
    "cgx_model_forward_batch": (I, [VP, VP, I, I, VP]),
    "cgx_model_batch": (I, [VP]),
    "cgx_model_len_seq": (I, [VP, I]),
    "cgx_model_truncate_seq": (I, [VP, I, I]),
    "cgx_model_kv": (PKV, [VP]),
    "cgx_model_fill_context": (I, [VP, I, C.c_uint64]),
    "cgx_model_export": (I, [VP, I, I, VP, VP]),
    "cgx_model_load": (VP, [C.POINTER(CgxModelConfig), C.c_char_p, VP]),
    "cgx_rope_table_dev": (I, [I, I, I, C.c_float, VP]),
    "cgx_attention_rope_append_dev": (I, [VP, I, VP, I, I, VP, I, I, VP]),
    "cgx_decoder_fused_attention": (I, [I]),
    "cgx_decoder_attention_stats": (I, [I]),
    "cgx_gemv_stream_min_units": (I, [I]),
    "cgx_gemm_reduce4_min_blocks": (I, [I]),
    "cgx_gemm_swiglu_here": (I, [I]),
    "cgx_model_save": (I, [VP, C.c_char_p, I]),
    "cgx_fill_normal_dev": (I, [VP, SZ, C.c_uint64, C.c_uint32, F]),
    "cgx_spec_new": (VP, [VP, VP, I, F, I, F]),
    "cgx_spec_free": (None, [VP]),
    "cgx_spec_prefill": (I, [VP, VP, I]),
    "cgx_spec_set_last": (I, [VP, I]),
    "cgx_spec_step": (I, [VP, VP, VP, VP]),
    "cgx_spec_stats": (None, [VP, C.POINTER(C.c_longlong), C.POINTER(C.c_longlong),
                              C.POINTER(C.c_longlong)]),
    "cgx_spec_batch_new": (VP, [VP, VP, I, F]),
    "cgx_spec_batch_free": (None, [VP]),
    "cgx_spec_batch_set_last": (I, [VP, VP, VP]),
    "cgx_spec_batch_step": (I, [VP, VP, VP, VP, VP]),
    "cgx_spec_batch_stats": (None, [VP, C.POINTER(C.c_longlong), C.POINTER(C.c_longlong),
                                    C.POINTER(C.c_longlong)]),
    "cgx_model_forward_tree_rows": (I, [VP, VP, I, VP, VP, I, VP]),
    "cgx_tree_spec_new": (VP, [VP, VP, I, I, F, I, F]),
    "cgx_tree_spec_free": (None, [VP]),
    "cgx_tree_spec_nodes": (I, [VP]),
    "cgx_tree_spec_depth": (I, [VP]),
    "cgx_tree_spec_set_root": (I, [VP, VP]),
    "cgx_tree_spec_step": (I, [VP, VP, VP, VP]),
    "cgx_tree_spec_stats": (None, [VP, C.POINTER(C.c_longlong), C.POINTER(C.c_longlong),
                                   C.POINTER(C.c_longlong)]),
    "cgx_tree_shape_get": (I, [I, I, VP, VP, VP]),
    "cgx_topk_lists_dev": (I, [VP, I, I, I, F, VP, VP]),
    "cgx_tree_accept_dev": (I, [VP, I, I, I, VP, VP, VP, VP, VP, VP, VP]),
}

# The subset implemented so far; the rest are declared in the headers and
# are added here as their kernels land.
def declare(lib: C.CDLL, names: Iterable[str] | None = None) -> list[str]:
    """Set prototypes on `lib`.  Returns the names that are missing."""
    missing = []
    for name in (names or SIGNATURES):
        res, args = SIGNATURES[name]
        try:
            fn = getattr(lib, name)
        except AttributeError:
            missing.append(name)
            continue
        fn.restype = res
        fn.argtypes = args
    return missing


def last_error(lib: C.CDLL) -> str:
    msg = lib.cgx_last_error()
    return msg.decode() if msg else ""


class DeviceArray:
    """A device allocation made through the C ABI (cgx_malloc), with numpy
    copies in and out.  Plumbing for tests and the bench."""

    def __init__(self, lib: C.CDLL, nbytes: int):
        self.lib = lib
        self.nbytes = int(nbytes)
        self.ptr = lib.cgx_malloc(max(1, self.nbytes))
        if not self.ptr:
            raise RuntimeError(f"cgx_malloc({nbytes}) failed: {last_error(lib)}")

    @classmethod
    def from_numpy(cls, lib: C.CDLL, arr) -> "DeviceArray":
        import numpy as np
        arr = np.ascontiguousarray(arr)
        d = cls(lib, arr.nbytes)
        d.upload(arr)
        return d

    def upload(self, arr) -> None:
        import numpy as np
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        if self.lib.cgx_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes):
            raise RuntimeError(last_error(self.lib))

    def numpy(self, dtype, shape) -> "np.ndarray":
        import numpy as np
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        if self.lib.cgx_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes):
            raise RuntimeError(last_error(self.lib))
        return out

    def free(self) -> None:
        if self.ptr:
            self.lib.cgx_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def host_quant_from_arrays(data, scales, K: int, N: int, gs: int):
    """A host cg_tensor_quant over numpy arrays in cogito's layout (owned by
    Python; never pass it to cg_tensor_quant_free)."""
    import numpy as np
    keep = {
        "data": np.ascontiguousarray(data, np.uint8),
        "scales": np.ascontiguousarray(scales, np.float32),
        "zeros": np.zeros_like(scales, np.float32),
        "shape": (C.c_int * 2)(K, N),
    }
    q = CgTensorQuant()
    q.data = keep["data"].ctypes.data_as(C.POINTER(C.c_uint8))
    q.scales = keep["scales"].ctypes.data_as(C.POINTER(C.c_float))
    q.zeros = keep["zeros"].ctypes.data_as(C.POINTER(C.c_float))
    q.shape = C.cast(keep["shape"], C.POINTER(C.c_int))
    q.ndim = 2
    q.size = K * N
    q.quant_type = 2
    q.group_size = gs
    q.num_groups = (K * N + gs - 1) // gs
    q.symmetric = True
    return q, keep
