/*
 * cg_flash_attn.h -- flash attention parameters, forward entry points and
 * RoPE (cogito's include/cg_flash_attn.h, same declarations).
 *
 * Layouts (reference :52-88): Q/O [batch, seqlen_q, n_heads, d_head];
 * K/V [batch, seqlen_k, n_heads_k, d_head]; GQA maps query head h to KV head
 * h * n_heads_k / n_heads (reference src/cuda/flash_attn_kernels.c:278).
 *
 * MI355X implementation: cg_flash_attention_forward (and its _cpu-named
 * twin, kept for source compatibility) run a HIP split-KV flash kernel on
 * the GPU.  Mask types:
 *   ATTN_MASK_NONE, ATTN_MASK_SLIDING_WINDOW -- as the reference;
 *   ATTN_MASK_CAUSAL -- bottom-right aligned: query i sees keys
 *     [0, seqlen_k - seqlen_q + i].  For seqlen_q == seqlen_k this is the
 *     reference's rule (k_idx > q_idx masked, src/attention/flash_attn.c:82);
 *     for verify (seqlen_q < seqlen_k) the reference rule would mask the
 *     cached context, so the aligned form is used;
 *   ATTN_MASK_CUSTOM -- `mask` is an additive fp32 [seqlen_q, seqlen_k] mask
 *     (e.g. the rows of cg_tree_attention_mask for the new tokens).
 * Backward passes are training-only and not provided (set the last error).
 */
#ifndef CG_FLASH_ATTN_H
#define CG_FLASH_ATTN_H

#include "cg_tensor.h"
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLASH_BLOCK_M_DEFAULT 64
#define FLASH_BLOCK_N_DEFAULT 64
#define FLASH_BLOCK_K 64
#define FLASH_WARPS 4

typedef struct {
    int block_m;
    int block_n;
    int split_k;
    bool use_persistent;
    bool use_register_tile;
    int num_warps;
    int sm_count;
} cg_flash_attn_config;

#define FLASH_BLOCK_M FLASH_BLOCK_M_DEFAULT
#define FLASH_BLOCK_N FLASH_BLOCK_N_DEFAULT

typedef enum {
    ATTN_MASK_NONE = 0,
    ATTN_MASK_CAUSAL,
    ATTN_MASK_SLIDING_WINDOW,
    ATTN_MASK_CUSTOM
} cg_attention_mask_type;

typedef struct {
    float* Q;
    float* K;
    float* V;
    float* O;
    float* mask;
    float* dropout_mask;
    int batch_size;
    int seqlen_q;
    int seqlen_k;
    int n_heads;
    int n_heads_k;
    int d_head;
    float scale;
    float dropout_prob;
    cg_attention_mask_type mask_type;
    int window_size;
    bool is_training;
    float* softmax_lse;
    float* dO;
    float* dQ;
    float* dK;
    float* dV;
} cg_flash_attn_params;

void cg_flash_attention_forward(cg_flash_attn_params* params);
void cg_flash_attention_forward_cpu(cg_flash_attn_params* params);
void cg_flash_attention_backward(cg_flash_attn_params* params);
void cg_flash_attention_backward_cpu(cg_flash_attn_params* params);
void cg_flash_attention_mqa(cg_flash_attn_params* params);
void cg_flash_attention_gqa(cg_flash_attn_params* params, int num_kv_groups);

cg_flash_attn_params* cg_flash_attn_params_new(
    cg_tensor* Q, cg_tensor* K, cg_tensor* V,
    cg_attention_mask_type mask_type, float dropout_prob
);
cg_flash_attn_config cg_flash_attn_autotune(int seqlen_q, int seqlen_k,
                                              int d_head, int sm_count);
size_t cg_flash_attn_shared_mem(int block_m, int block_n, int d_head);
void cg_flash_attn_params_free(cg_flash_attn_params* params);

/* RoPE, rotate-half form (reference src/attention/flash_attn.c:318-362):
 * pairs (i, i + d/2), freq_i = 1 / theta^(2i/d), angle = pos * freq_i.
 * Q and K are [seqlen, n_heads, d_head]; both are rotated in place. */
void cg_apply_rope(float* Q, float* K, int seqlen, int n_heads,
                   int d_head, int position_offset, float rope_theta);
void cg_rope_precompute_freqs(float* cos_cache, float* sin_cache,
                              int max_seqlen, int d_head, float theta);

/* ALiBi (reference src/attention/flash_attn.c:368-388). */
void cg_alibi_bias(float* bias, int seqlen_q, int seqlen_k,
                   int n_heads, float* slopes);
void cg_alibi_slopes(float* slopes, int n_heads);

#ifdef __cplusplus
}
#endif

#endif /* CG_FLASH_ATTN_H */
