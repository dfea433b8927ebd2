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
#include "cg_serialization.h"

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

/* HIP graphs of the library stream (no counterpart in the reference; for
 * callers that replay a fixed-shape call, such as a serving loop's verify,
 * without its launch cost).  Calls issued between cgx_graph_begin and
 * cgx_graph_end are captured, not run; cgx_graph_end returns the executable
 * graph (NULL on error) and cgx_graph_launch replays it on the library
 * stream, reading and writing the same device addresses each time.  Only
 * calls that allocate and set no memory may be captured: the verify through
 * cgx_verify_chain_batch_dev_noalloc is the one this build tests. */
int cgx_graph_begin(void);
void* cgx_graph_end(void);
int cgx_graph_launch(void* graph);
int cgx_graph_free(void* graph);

/* Timing with HIP events on the library stream (milliseconds). */
int cgx_event_record(int slot);      /* slot 0..7 */
float cgx_event_elapsed_ms(int slot_begin, int slot_end);

/* A plain streaming read of `bytes` (a multiple of 16, 16-byte aligned) of
 * device memory, the floor of any kernel that reads the same bytes: out
 * (device, 4 * ceil(bytes / 8192) words) receives, for block b and wave w,
 * the XOR of the 32-bit words of the 16-byte words b*512 + 64w + l and
 * b*512 + 256 + 64w + l, l = 0..63.  No counterpart in the reference: a
 * measurement aid for bench.py's roofline figures. */
int cgx_stream_read(const void* buf, size_t bytes, unsigned int* out);

/* ------------------------------------------------- device-resident data */
/* Tensor whose data lives in HBM (zero-filled).  Free with cg_tensor_free. */
cg_tensor* cgx_tensor_device_new(int* shape, int ndim);
cg_tensor* cgx_tensor_to_device(cg_tensor* host);
int cgx_tensor_to_host(cg_tensor* t, float* host_out);

/* Uploads a quantized 2-D weight W[K,N] (reference layout, host or device)
 * into HBM.  When K % 256 == 0, N % 16 == 0, group_size % 16 == 0 and
 * N % group_size == 0 the data is re-tiled for the MFMA GEMV (layout 3);
 * otherwise it is kept in the reference layout (layout 1).  Free with
 * cg_tensor_quant_free. */
cg_tensor_quant* cgx_quant_to_device(cg_tensor_quant* q);
/* Same, always keeping the reference layout (for the generic kernel). */
cg_tensor_quant* cgx_quant_to_device_flat(cg_tensor_quant* q);
/* Same with the layout chosen: 1 reference, 2 VALU-GEMV strips, 3 MFMA
 * tiles (2 and 3 fall back to 1 for shapes outside the rule above). */
cg_tensor_quant* cgx_quant_to_device_layout(cg_tensor_quant* q, int layout);
/* 0 host, 1 device flat, 2 device VALU tiles, 3 device MFMA tiles */
int cgx_quant_layout(cg_tensor_quant* q);

/* ------------------------------------------------------ INT4 GEMV (raw) */
/* y[M,N] = x[M,K] @ W; x and y are device pointers, w a device handle. */
int cgx_matmul_int4_dev(const float* x, int M, cg_tensor_quant* w, float* y);
/* Same with the kernel forced: 0 auto (by layout), 1 VALU GEMV (layout 2),
 * 2 generic reference-order kernel (layout 1), 3 MFMA GEMV (layout 3),
 * 4 MFMA GEMM with a shared activation tile (layout 3, N % 128 == 0,
 * group % 128 == 0; the batched and tree verify shapes, M >= 16). */
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

/* Without accept_prob (NULL) only the emitted tokens and counts are asked
 * for, and a large call (at least `blocks` pass-1 workgroups: 4096-value
 * segments times the 2 gamma + 1 rows of every chain; 2048 at load) settles
 * most accept tests from certified bounds of the row sums, summing exactly
 * only the rows its outcome still depends on.  The results are the same
 * either way.  Sets the threshold (blocks >= 0) and returns the previous one;
 * no counterpart in the reference (a tuning and test hook). */
int cgx_verify_lean_min_blocks(int blocks);

/* Allocation-free form of cgx_verify_chain_batch_dev.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as cgx_verify_chain_batch_dev for
 * unfiltered verification (top_k <= 0 or >= V, top_p >= 1, temperature > 0);
 * filtered calls are rejected.  The workspace is a static 32 MiB device array
 * per GPU, held from library load until the process ends, which covers
 * 16 chains of gamma 4 at V = 32000 or 4 chains at V = 128256; larger calls
 * fail with an error naming the bytes needed.  Nothing is allocated or
 * freed (the array's address is resolved once per device by cgx_init).
 * Every call on one GPU uses the same array and leaves its contents behind;
 * calls issued on the library stream run in order, but calls that overlap on
 * one GPU (graph replays or other threads running concurrently) race. */
int cgx_verify_chain_batch_dev_noalloc(const float* target_logits,
                                       const float* draft_logits,
                                       const int* draft_tokens, const float* u,
                                       int batch, int gamma, int V,
                                       float temperature, int top_k, float top_p,
                                       int* out_tokens, int* n_accepted,
                                       float* accept_prob);

/* Single samplers with an explicit uniform (same arithmetic as the
 * reference samplers; logits host or device). */
int cgx_sample_temperature_u(const float* logits, int V, float T, float u);
/* The same draw from a device logits row into *out_dev (device int), queued
 * on the library's stream without synchronising: the loops' draft draw
 * (rows of up to 32768 values on one workgroup, longer rows through the
 * chunk-parallel pipeline). */
int cgx_sample_temperature_dev(const float* logits, int V, float T, float u, int* out_dev);
/* The same on `rows` device rows at once (row r at logits + r * ld, its
 * draw u_dev[r] on the device, token to out_dev[r]), queued without
 * synchronising: the batched loop's draft draws (rows of up to 32768 values
 * one workgroup each in one launch, longer rows through the pipeline). */
int cgx_sample_temperature_rows_dev(const float* logits, int rows, int V, float T,
                                    const float* u_dev, int* out_dev, size_t ld);
int cgx_sample_top_k_u(const float* logits, int V, int k, float u);
int cgx_sample_top_p_u(const float* logits, int V, float top_p, float u);
int cgx_sample_corrected_u(const float* draft_probs, const float* target_probs,
                           int V, float u);

/* Typical sampling with an explicit uniform, and its distribution (logits
 * host or device; dist_out host or device, V floats): see cg_sample_typical. */
int cgx_sample_typical_u(const float* logits, int V, float typical_p, float u);
int cgx_typical_dist(const float* logits, int V, float typical_p, float* dist_out);

/* The token that followed the accepted drafts (correction or bonus) in the
 * last cg_target_verify / cg_speculative_step; -1 before any. */
int cgx_last_verify_token(void);

/* cg_tree_attention_mask for a tree: nodes[0..nodes) with parents[i] < i
 * (-1: child of the prefix); node i sees the prefix, itself and its
 * ancestors.  New host tensor [1, 1, seqlen + nodes, seqlen + nodes]. */
cg_tensor* cgx_tree_attention_mask_parents(const int* parents, int nodes, int seqlen);

/* Probability vector the verify composition uses for one row (host or
 * device logits; dist_out host or device, V floats). */
int cgx_filtered_dist(const float* logits, int V, float T, int top_k,
                      float top_p, float* dist_out);

/* Test hooks for the two exactness building blocks (device pointers):
 * glibc-identical expf, and the exact left-to-right fp32 sum of
 * non-negative values. */
int cgx_exact_expf_dev(const float* x, float* y, int n);
int cgx_ordered_sum_dev(const float* x, int n, float* out_dev);
/* Test hook: the typical sampler's binary64 log of positive floats
 * (device pointers), the same bits as the CPU restatement's. */
int cgx_typ_log_dev(const float* x, double* y, int n);
/* Test hook of the samplers' row sort: rows [rows][n] of 32-bit keys sorted
 * stably (descending when `descending`), payloads carried along when
 * payload_out is given (payload NULL: each key's index in its row).  Device
 * pointers; synchronous. */
int cgx_sort_rows_dev(const uint32_t* keys, const uint32_t* payload, int rows, int n,
                      int descending, uint32_t* keys_out, uint32_t* payload_out);
/* Largest relative distance between the samplers' fast exponential and the
 * exact one over every fp32 in [lo, hi] (-104 <= lo < hi <= 0), folded with
 * an unsigned max into *out_dev as the float's bits (caller zeroes it).  The
 * certified sampler paths assume it stays within 2^-20 on [-87, 0]. */
int cgx_exp_fast_maxerr_dev(float lo, float hi, unsigned int* out_dev);
/* The same for the cheaper exponential of the acceptance pipeline's
 * segment statistics, whose sums feed only bounds (kExpFastMin = -87 <= lo <
 * hi <= 0); the bounds assume it stays within 2^-16 on [-87, 0].  No
 * counterpart in the reference (a test of a certified bound). */
int cgx_exp_stat_maxerr_dev(float lo, float hi, unsigned int* out_dev);
/* The single-row draws (cgx_sample_temperature_u and the loops' draft draws
 * on rows of up to 32768 values) first decide the token from certified
 * approximations and run the exact sums only where u lies within the bounds
 * of a CDF step (the same token either way).  cgx_sample_row_certified turns
 * that decision off (0) or on (1, the default) and returns the previous
 * setting (-1 only reads it); cgx_sample_row_fallbacks counts the draws since
 * the library loaded that the exact sums decided (synchronises).  No
 * counterpart in the reference (test hooks of a certified decision). */
int cgx_sample_row_certified(int on);
long long cgx_sample_row_fallbacks(void);

/* ------------------------------------------------ INT4 tensors on disk */
/* COG1 files (cg_serialization.h) holding INT4 tensors: each tensor is an
 * entry "<name>" of the reference's INT4 dtype 2 (shape[0..ndim) the logical
 * shape, shape[7] the group size, data the reference's packed nibbles) and
 * an fp32 entry "<name>.scales" of num_groups values.  Tensors may be host
 * or flat device tensors (cgx_quant_to_device_flat); names up to 56
 * characters.  The loader returns host tensors (free each with
 * cg_tensor_quant_free, the arrays and names with free()); other entries of
 * the file are skipped. */
int cgx_save_quantized(const char* filename, cg_tensor_quant* const* tensors,
                       const char* const* names, int count);
int cgx_load_quantized(const char* filename, cg_tensor_quant*** out_tensors,
                       char*** out_names, int* out_count);

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

/* The batched decode/verify attention of the decoder (test hook): B
 * sequences, sequence b's keys in cache layer slot slot0 + b (the batched
 * models' layout), nk[b] keys each (host array), Q/O [B][Nq][H][D] device.
 * mask_kind 0: chain (query i sees keys < nk[b] - Nq + i + 1); 1: tree, the
 * last tw keys (Nq <= tw <= 64) visible to query i where bit j of anc[i]
 * (host array of Nq masks) is set.  Needs group_size == head_dim. */
/* The decoder's attention step in one launch (no reference counterpart: it
 * fuses cg_apply_rope, src/attention/flash_attn.c:335-360, the INT4 append of
 * src/quantize/int4.c:155-231 and cg_attention_int4_kv): qkv [Nq][ldq] are
 * the raw projections of Nq rows (q heads, then k heads, then v heads) at
 * positions pos .. pos + Nq - 1; their K is rotated and quantised with V into
 * those positions of `layer` (one scale per head row), Q is rotated, and O
 * [Nq][H][head_dim] receives attention over positions 0 .. pos + Nq - 1 under
 * the chain mask.  rope [Nq][head_dim / 2][2]: (cos, sin) of the rows'
 * positions, from cgx_rope_table_dev(Nq, head_dim, pos, theta, rope).  Nq <= 64;
 * device pointers, 16-byte aligned, ldq % 4 == 0.  The cache's current_len is
 * left to the caller. */
int cgx_rope_table_dev(int rows, int head_dim, int pos0, float theta, float* cs);
int cgx_attention_rope_append_dev(const float* qkv, int ldq, const float* rope, int Nq, int H,
                                  cg_kv_cache_int4* c, int layer, int pos, float* O);
/* Test hook, no reference counterpart: 1 (default) runs the decoder's RoPE and
 * cache append inside the attention launch, 0 as launches of their own (the
 * same cache contents); returns the previous setting (-1 only reads it). */
int cgx_decoder_fused_attention(int on);
/* Test hook, no reference counterpart: 1 (default) has the decoder's
 * attention (head_dim 128, 16+ rows) write the row statistics of its output
 * for the O projection's GEMM, 0 leaves them to a pass of the GEMM's own (the
 * same row factors, so the same outputs); returns the previous setting (-1
 * only reads it). */
int cgx_decoder_attention_stats(int on);
/* Test hook, no reference counterpart: the INT4 GEMV takes the persistent
 * streaming kernel for K = 4096 and up to 5 rows once the busiest CU gets at
 * least this many 32-column units (default 8: a 64k- or 128k-vocabulary
 * lm_head; 0 never, 1 every product it supports); returns the previous value
 * (-1 only reads it). */
int cgx_gemv_stream_min_units(int units);
/* Test hook, no reference counterpart: the GEMM (16+ rows) sums its K splits
 * with four outputs a thread once that launch has at least this many
 * 256-thread blocks (default 512; 0 always, a large value never); returns
 * the previous value (-1 only reads it). */
int cgx_gemm_reduce4_min_blocks(int blocks);
/* Test hook, no reference counterpart: 1 (default) applies SwiGLU inside the
 * GEMM when a gate|up product has one K split, 0 stores its partial sums for
 * the separate reduction pass (the same outputs, bit for bit); returns the
 * previous setting (-1 only reads it). */
int cgx_gemm_swiglu_here(int on);
int cgx_attention_int4_kv_batch_dev(const float* Q, int B, int Nq, int H,
                                    cg_kv_cache_int4* cache, int slot0, const int* nk,
                                    int mask_kind, const unsigned long long* anc, int tw,
                                    float* O);

/* ------------------------------------------------- synthetic decoder */
/* Decoder-only transformer with INT4 weights resident in HBM, the model the
 * verify stack runs (reference src/layers/transformer.c:26-149 block order,
 * src/layers/linear.c:53-98 layout y = x @ W with W [in, out]):
 *   x = embed[token]
 *   per layer: x += attn(rope(rmsnorm(x) @ Wqkv)) @ Wo
 *              x += (silu(h @ Wg) * (h @ Wu)) @ Wd,  h = rmsnorm(x)
 *   logits = rmsnorm(x) @ Wlm
 * RMSNorm weights are 1, eps = norm_eps; RoPE rotate-half with rope_theta;
 * INT4 KV cache with kv_group_size; attention scale 1/sqrt(head_dim).
 *
 * Seeded weights: every matrix is filled by cgx_fill_normal semantics
 * (Irwin-Hall of four 16-bit uniforms from a lowbias32 counter hash, unit
 * variance, times init_std), row-major, then quantized with
 * cg_quantize_int4's rule (groups of group_size along the flat index).
 * Stream ids: embedding [V][d] 1; lm_head [d][V] 2; layer l:
 * Wqkv [d][(H + 2 Hk) hd] 16 l + 3 (columns q | k | v), Wo [H hd][d]
 * 16 l + 4, Wgate|up [d][2 ff] 16 l + 5 (columns gate | up), Wd [ff][d]
 * 16 l + 6.  A model built with `share_from` uses that model's embedding
 * and lm_head (a draft head over the target's vocabulary projection). */
typedef struct {
    int n_layers;
    int d_model;
    int n_heads;
    int n_kv_heads;
    int head_dim;
    int d_ff;
    int vocab;
    int group_size;       /* INT4 weight group along the flat index */
    int kv_group_size;    /* INT4 KV-cache group along head_dim */
    int max_seq;          /* KV-cache capacity (positions) */
    int max_tokens;       /* largest number of tokens per forward */
    float rope_theta;
    float norm_eps;
    float init_std;
    int max_batch;        /* sequences held, each with its own KV cache (0: 1) */
} cgx_model_config;

typedef struct cgx_model cgx_model;

cgx_model* cgx_model_new(const cgx_model_config* cfg, uint64_t seed,
                         cgx_model* share_from);
void cgx_model_free(cgx_model* m);
/* Forward of M tokens (host or device ids) at positions len..len+M-1: KV
 * rows appended, len advanced by M.  Logits of the last `n_logits` tokens
 * go to logits [n_logits][V] (device pointer, or NULL for the model's own
 * buffer, see cgx_model_logits).  Asynchronous on the library stream when
 * `tokens` is a device pointer. */
int cgx_model_forward(cgx_model* m, const int* tokens, int M, int n_logits,
                      float* logits);
float* cgx_model_logits(cgx_model* m);
int cgx_model_get_config(const cgx_model* m, cgx_model_config* out);
int cgx_model_len(const cgx_model* m);
int cgx_model_truncate(cgx_model* m, int len);
/* Batch of max_batch sequences: each forward advances every sequence by M
 * tokens (tokens [B][M], host or device); logits of the last n_logits tokens
 * of each sequence go to logits [B][n_logits][V].  The single-sequence
 * functions above act on sequence 0. */
int cgx_model_forward_batch(cgx_model* m, const int* tokens, int M, int n_logits,
                            float* logits);
int cgx_model_batch(const cgx_model* m);
int cgx_model_len_seq(const cgx_model* m, int seq);
int cgx_model_truncate_seq(cgx_model* m, int seq, int len);
cg_kv_cache_int4* cgx_model_kv(cgx_model* m);
/* Synthetic context: K/V rows of positions [0, len) of every layer filled
 * with seeded values (std 1) and len set, as if a prompt had been run. */
int cgx_model_fill_context(cgx_model* m, int len, uint64_t seed);
/* Weight export for checkers: the reference layout (flat nibbles, scales)
 * of one matrix: which = 0 Wqkv, 1 Wo, 2 Wgate|up, 3 Wd (of `layer`),
 * 4 lm_head.  data: K*N/2 bytes, scales: K*N/group_size floats (host). */
int cgx_model_export(cgx_model* m, int layer, int which, uint8_t* data,
                     float* scales);
/* Model files ("COG1", reference src/core/serialization.c:9-77; INT4
 * entries as cgx_save_quantized writes them).  Entry names are the fields of
 * the reference's transformer block (include/cg_transformer.h:41-50):
 *   embed [V, d] (fp32), norm [d] (final RMSNorm), lm_head [d, V];
 *   layers.<l>.norm1, layers.<l>.norm2 [d];
 *   layers.<l>.attn_qkv_proj [d, (H + 2 Hk) hd] (columns q | k | v), or
 *     its blocks attn_q_proj [d, H hd], attn_k_proj, attn_v_proj [d, Hk hd];
 *   layers.<l>.attn_o_proj [H hd, d];
 *   layers.<l>.mlp_gate_up [d, 2 ff] (columns gate | up), or its blocks
 *     mlp_gate, mlp_up [d, ff];
 *   layers.<l>.mlp_down [ff, d].
 * Matrices are fp32 entries, quantized at load by cg_quantize_int4's rule
 * (groups of cfg->group_size along the flat index of the whole matrix), or
 * INT4 entries of that group size, copied (split blocks must then hold whole
 * groups of their rows).  Missing norms are 1.  cgx_model_load builds the
 * decoder of `cfg` from such a file (every entry is checked before anything
 * is allocated; a missing or malformed one is named in cgx_last_error); with
 * `share_from`, embed and lm_head come from that model and the file's are not
 * read.  cgx_model_save writes every entry the model holds (embed and lm_head
 * unless shared): INT4 entries (fp32 = 0), or, for a seeded model, the fp32
 * values before quantization (fp32 = 1), which load back to the same INT4
 * weights. */
cgx_model* cgx_model_load(const cgx_model_config* cfg, const char* path,
                          cgx_model* share_from);
int cgx_model_save(cgx_model* m, const char* path, int fp32);
/* The fill rule of the seeded weights, into device memory. */
int cgx_fill_normal_dev(float* out, size_t n, uint64_t seed, uint32_t stream_id,
                        float stddev);

/* ------------------------------------------ chain speculative decoding */
/* Draft / target pair stepping gamma-token chains entirely on the GPU: the
 * draft proposes gamma tokens (one forward and one filtered draw each), the
 * target scores [last, d_1..d_gamma] in one forward, the verify kernels
 * accept a prefix, and both KV caches roll back to the accepted tokens. */
typedef struct cgx_spec cgx_spec;

cgx_spec* cgx_spec_new(cgx_model* draft, cgx_model* target, int gamma,
                       float temperature, int top_k, float top_p);
void cgx_spec_free(cgx_spec* s);
/* Runs both models over the prompt (host ids) and makes its last token the
 * next input.  The target and draft must be empty or at the same length. */
int cgx_spec_prefill(cgx_spec* s, const int* prompt, int n);
/* Continues from a filled context (cgx_model_fill_context at the same
 * length on both models) with `last_token` as the next input. */
int cgx_spec_set_last(cgx_spec* s, int last_token);
/* One step.  u_draft[gamma]: draws of the draft samplers; u_verify[gamma+1]
 * (D6 order) for the verify.  Host arrays.  Writes the n+1 emitted tokens
 * to out_tokens (host, gamma+1 entries) and returns n (0..gamma). */
int cgx_spec_step(cgx_spec* s, const float* u_draft, const float* u_verify,
                  int* out_tokens);
/* totals since cgx_spec_new: steps, drafted tokens, accepted tokens */
void cgx_spec_stats(const cgx_spec* s, long long* steps, long long* drafted,
                    long long* accepted);

/* Batched loop: B = max_batch sequences of both models in lockstep (each
 * with its own caches), unfiltered sampling.  set_last gives, per sequence,
 * the token at the target's last cached position (prev) and the next token
 * (last, not cached yet).  A step takes draws u_draft [B][gamma] and
 * u_verify [B][gamma + 1], writes out_tokens [B][gamma + 1] (-1 past the
 * emitted ones) and n_accepted [B], and returns the total accepted. */
typedef struct cgx_spec_batch cgx_spec_batch;
cgx_spec_batch* cgx_spec_batch_new(cgx_model* draft, cgx_model* target, int gamma,
                                   float temperature);
void cgx_spec_batch_free(cgx_spec_batch* s);
int cgx_spec_batch_set_last(cgx_spec_batch* s, const int* prev, const int* last);
int cgx_spec_batch_step(cgx_spec_batch* s, const float* u_draft, const float* u_verify,
                        int* out_tokens, int* n_accepted);
void cgx_spec_batch_stats(const cgx_spec_batch* s, long long* steps, long long* drafted,
                          long long* accepted);

/* Tree forward of every sequence (M <= 64 rows each, tokens [B][M]): row i
 * goes to cache slot len + i with rotary position len + rel[i]; of the keys,
 * the last tw (M <= tw <= 64: the tree's nodes cached so far, these rows
 * last) are visible to row i only where bit j of anc[i] is set (key
 * len + M - tw + j).  Logits of every row at logits ([B][M][vocab]) or in the
 * model's own buffer (logits NULL). */
int cgx_model_forward_tree_rows(cgx_model* m, const int* tokens, int M, const int* rel,
                                const unsigned long long* anc, int tw, float* logits);

/* Tree speculation (EAGLE-style), B = max_batch sequences in lockstep.  The
 * draft tree has `nodes` nodes (node 0 the root: the last emitted token, not
 * cached yet) to the given depth, chosen best-first with at most 4 children
 * a node and numbered breadth-first (cgx_tree_shape_get).  A step drafts the
 * tree level by level (a node's children: the top-c tokens of the draft's
 * logits at that node), verifies every node in one target forward under the
 * tree mask, and walks it: at the current node the target distribution p
 * (top_k list at temperature T, then top_p) accepts candidate x with
 * probability w[x] / W, a rejected candidate's mass is removed (w[x] = 0),
 * and when all are rejected (or at a leaf) the next token is drawn from w / W.
 * No reference counterpart: cogito's EAGLE builder is a stub
 * (src/inference/speculative.c:244-262).  u: [B][depth + 1][5] draws (slot r
 * < 4: candidate r's test at that depth, slot 4: the final draw); out_tokens
 * [B][depth + 2] (the accepted tokens, then the drawn one; -1 after);
 * n_accepted [B]; returns the total accepted.  Requires max_tokens >= nodes
 * in both models, 1 <= top_k <= 64. */
typedef struct cgx_tree_spec cgx_tree_spec;
cgx_tree_spec* cgx_tree_spec_new(cgx_model* draft, cgx_model* target, int nodes, int depth,
                                 float temperature, int top_k, float top_p);
void cgx_tree_spec_free(cgx_tree_spec* s);
int cgx_tree_spec_nodes(const cgx_tree_spec* s);
int cgx_tree_spec_depth(const cgx_tree_spec* s);
int cgx_tree_spec_set_root(cgx_tree_spec* s, const int* root);
int cgx_tree_spec_step(cgx_tree_spec* s, const float* u, int* out_tokens, int* n_accepted);
void cgx_tree_spec_stats(const cgx_tree_spec* s, long long* steps, long long* drafted,
                         long long* accepted);
/* The default tree's parent, depth and sibling rank per node; returns the
 * node count. */
int cgx_tree_shape_get(int nodes, int depth, int* parent, int* node_depth, int* rank);
/* Device pieces of the step (device pointers): top-k lists of `rows` rows
 * of z (index and probability per entry, cg_sample_top_k's order), and the
 * acceptance walk over a tree given by parents (breadth-first, parent[0] =
 * -1, siblings in rank order) with lists [B * nodes][K], node tokens
 * [B][nodes] and draws as in cgx_tree_spec_step; out [B][depth + 2], nacc
 * [B], path [B][depth] (node index of each accepted node). */
int cgx_topk_lists_dev(const float* z, int rows, int V, int top_k, float top_p, int* lidx,
                       float* lp);
int cgx_tree_accept_dev(const int* parent, int nodes, int B, int K, const int* lidx,
                        const float* lp, const int* tok, const float* u, int* out, int* nacc,
                        int* path);

#ifdef __cplusplus
}
#endif

#endif /* CG_MI355X_H */
