/*
 * cg_mi355x.h -- MI355X extensions to cogito's verify-path C API.
 *
 * These entry points have no counterpart in cogito's headers.  They add what
 * a GPU drop-in needs and the reference has no way to express:
 *   - device memory and the library's HIP stream (as plain C types);
 *   - device-resident INT4 weights in the tiled HBM layout;
 *   - verification and sampling with PRE-DRAWN uniforms instead of the
 *     global LCG (the north-star requirement for reproducible parity);
 *   - KV-cache rollback after a rejected draft.
 * Every function returns 0 on success and -1 on failure with the reason in
 * cgx_last_error(), unless documented otherwise.  Like the reference, the
 * library is not thread-safe.
 */
#ifndef CG_MI355X_H
#define CG_MI355X_H

#include <stddef.h>
#include <stdint.h>
#include "cg_tensor.h"
#include "cg_quantize.h"
#include "cg_speculative.h"
#include "cg_flash_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ runtime */
int cgx_init(int device);            /* idempotent; API entries call it */
const char* cgx_last_error(void);    /* "" when no error is pending      */
void cgx_clear_error(void);
int cgx_device_count(void);
void* cgx_stream(void);              /* the hipStream_t all kernels use   */
int cgx_synchronize(void);
const char* cgx_device_name(void);

void* cgx_malloc(size_t bytes);
int cgx_free(void* dptr);
int cgx_memcpy_h2d(void* dst, const void* src, size_t bytes);
int cgx_memcpy_d2h(void* dst, const void* src, size_t bytes);
int cgx_memcpy_d2d(void* dst, const void* src, size_t bytes);
int cgx_memset(void* dst, int byte_value, size_t bytes);
int cgx_is_device_ptr(const void* p);  /* 1 device, 0 host */

/* Timing with HIP events on the library stream (milliseconds). */
int cgx_event_record(int slot);      /* slot 0..7 */
float cgx_event_elapsed_ms(int slot_begin, int slot_end);

/* ------------------------------------------------- device-resident data */
/* Tensor whose data lives in HBM (zero-filled).  Free with cg_tensor_free. */
cg_tensor* cgx_tensor_device_new(int* shape, int ndim);
cg_tensor* cgx_tensor_to_device(cg_tensor* host);
int cgx_tensor_to_host(cg_tensor* t, float* host_out);

/* Uploads a quantized 2-D weight W[K,N] (reference layout, host or device)
 * into HBM.  When K % 256 == 0, N % 16 == 0, group_size % 16 == 0 and
 * N % group_size == 0 the data is re-tiled for the GEMV kernel (layout 2);
 * otherwise it is kept in the reference layout (layout 1).  Free with
 * cg_tensor_quant_free. */
cg_tensor_quant* cgx_quant_to_device(cg_tensor_quant* q);
/* Same, always keeping the reference layout (for the generic kernel). */
cg_tensor_quant* cgx_quant_to_device_flat(cg_tensor_quant* q);
int cgx_quant_layout(cg_tensor_quant* q);   /* 0 host, 1 device flat, 2 device tiled */

/* ------------------------------------------------------ INT4 GEMV (raw) */
/* y[M,N] = x[M,K] @ W; x and y are device pointers, w a device handle. */
int cgx_matmul_int4_dev(const float* x, int M, cg_tensor_quant* w, float* y);
/* Same with the kernel forced: 0 auto, 1 tiled VALU GEMV, 2 generic. */
int cgx_matmul_int4_dev_kernel(const float* x, int M, cg_tensor_quant* w,
                               float* y, int kernel);

/* ------------------------------------------------------------ sampling */
void cgx_lcg_seed(uint32_t state);   /* the reference starts at 42 */
uint32_t cgx_lcg_state(void);

/* Chain verification with explicit uniforms (u[k] is draw k: accept tests
 * use u[0..j], the final token u[j+1], or u[gamma] when all are accepted).
 * target_logits [gamma+1][V], draft_logits [gamma][V], draft_tokens[gamma],
 * u[gamma+1]: host or device pointers.  out_tokens[gamma+1] and
 * accept_prob[gamma] (optional) are host pointers.  Returns n_accepted
 * (0..gamma), or -1 on error. */
int cgx_verify_chain(const float* target_logits, const float* draft_logits,
                     const int* draft_tokens, const float* u, int gamma, int V,
                     float temperature, int top_k, float top_p,
                     int* out_tokens, float* accept_prob);

/* Batched form: `batch` independent chains laid out back to back
 * (target [batch][gamma+1][V], draft [batch][gamma][V], tokens
 * [batch][gamma], u [batch][gamma+1]); all pointers are DEVICE pointers.
 * out_tokens [batch][gamma+1] and n_accepted [batch] are device pointers.
 * Asynchronous on the library stream. */
int cgx_verify_chain_batch_dev(const float* target_logits,
                               const float* draft_logits,
                               const int* draft_tokens, const float* u,
                               int batch, int gamma, int V, float temperature,
                               int top_k, float top_p, int* out_tokens,
                               int* n_accepted, float* accept_prob);

/* Single samplers with an explicit uniform (same arithmetic as the
 * reference samplers; logits host or device). */
int cgx_sample_temperature_u(const float* logits, int V, float T, float u);
int cgx_sample_top_k_u(const float* logits, int V, int k, float u);
int cgx_sample_top_p_u(const float* logits, int V, float top_p, float u);
int cgx_sample_corrected_u(const float* draft_probs, const float* target_probs,
                           int V, float u);

/* Probability vector the verify composition uses for one row (host or
 * device logits; dist_out host or device, V floats). */
int cgx_filtered_dist(const float* logits, int V, float T, int top_k,
                      float top_p, float* dist_out);

/* Test hooks for the two exactness building blocks (device pointers):
 * glibc-identical expf, and the exact left-to-right fp32 sum of
 * non-negative values. */
int cgx_exact_expf_dev(const float* x, float* y, int n);
int cgx_ordered_sum_dev(const float* x, int n, float* out_dev);

/* ----------------------------------------------------------- KV cache */
/* Drops positions >= new_len (rollback after a rejected draft). */
int cgx_kv_cache_int4_truncate(cg_kv_cache_int4* cache, int new_len);
/* Writes T tokens ([T, n_heads, head_dim], host or device) of one layer at
 * positions pos..pos+T-1 without touching current_len. */
int cgx_kv_cache_int4_write(cg_kv_cache_int4* cache, int layer_idx, int pos,
                            const float* k, const float* v, int T);
int cgx_kv_cache_int4_set_len(cg_kv_cache_int4* cache, int len);

/* INT4-KV attention with an explicit mask (device Q/O [Nq][H][D]):
 * mask_kind 0: chain (query i sees [0, len - Nq + i]);
 * mask_kind 1: tree, parents[Nq] (device or host, -1 = root): query i sees
 * [0, len - Nq) plus its ancestors and itself among the last Nq positions. */
int cgx_attention_int4_kv_dev(const float* Q, int Nq, int H,
                              cg_kv_cache_int4* cache, int layer_idx,
                              int mask_kind, const int* parents, float* O);

#ifdef __cplusplus
}
#endif

#endif /* CG_MI355X_H */
