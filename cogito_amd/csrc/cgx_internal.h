/*
 * cgx_internal.h -- the C-ABI seam between the host C code (the cogito API
 * implementation, *.c) and the HIP side (*.hip).  Plain C types only: device
 * pointers, sizes, ints and floats.  Every cgk_* launcher enqueues work on
 * the library stream and returns 0, or -1 with the last error set.
 */
#ifndef CGX_INTERNAL_H
#define CGX_INTERNAL_H

#include <stddef.h>
#include <stdint.h>
#include "cg_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ----------------------------------------------------------- runtime */
void cgx_set_error(const char* fmt, ...);
int cgx_ensure_init(void);
/* Grow-only device scratch buffers for staging host arguments.  Slots are
 * reused by later calls, so their contents live until the next call that
 * names the same slot. */
enum { CGX_SLOT_IN0 = 0, CGX_SLOT_IN1, CGX_SLOT_IN2, CGX_SLOT_IN3,
       CGX_SLOT_OUT0, CGX_SLOT_OUT1, CGX_SLOT_WS0, CGX_SLOT_WS1,
       CGX_SLOT_WS2, CGX_SLOT_WS3, CGX_SLOT_WS4, CGX_SLOT_WS5, CGX_SLOT_WS6,
       CGX_NUM_SLOTS };
void* cgx_scratch(int slot, size_t bytes);
/* Zero-initialised counters that kernels reset themselves after use. */
unsigned int* cgx_counters(size_t count);
/* Device view of a host-or-device argument: returns p itself when it is a
 * device pointer, else copies `bytes` into scratch `slot`. */
const void* cgx_dev_in(const void* p, size_t bytes, int slot);

/* ------------------------------------------------ quantized-weight registry */
enum { CGX_LAYOUT_HOST = 0, CGX_LAYOUT_FLAT = 1, CGX_LAYOUT_TILED = 2, CGX_LAYOUT_MFMA = 3 };
typedef struct {
    int layout;
    int K, N, group_size;
    int paired;          /* layout 3: gate|up tiles interleaved (SwiGLU) */
    float smax;          /* layout 3: max |scale| (the GEMM's row-scaling bound) */
} cgx_qinfo;
int cgx_quant_lookup(const cg_tensor_quant* q, cgx_qinfo* info);
void cgx_quant_register(const cg_tensor_quant* q, const cgx_qinfo* info);
void cgx_quant_unregister(const cg_tensor_quant* q);

/* ------------------------------------------------------- INT4 kernels */
int cgk_int4_quantize(const float* x, int n, int gs, uint8_t* data,
                      float* scales);
int cgk_int4_dequantize_flat(const uint8_t* data, const float* scales, int n,
                             int gs, float* out);
int cgk_int4_repack_tiled(const uint8_t* flat, const float* scales, int K,
                          int N, int gs, uint8_t* tiled, float* scales_t);
int cgk_int4_dequantize_tiled(const uint8_t* tiled, const float* scales_t,
                              int K, int N, int gs, float* out);
int cgk_int4_gemv_tiled(const float* x, int M, int K, int N, int gs,
                        const uint8_t* tiled, const float* scales_t, float* y);
/* GEMV with the decoder's fusions: pro 0 none, 1 RMSNorm of the rows
 * (weights norm_w[K], eps) before the product, 2 SwiGLU of the gate|up rows
 * (x row = [g | u], ldx >= 2K); accumulate: y += result. */
int cgk_int4_gemv_fused(const float* x, int ldx, int M, int K, int N, int gs,
                        const uint8_t* tiled, const float* scales_t, float* y, int pro,
                        const float* norm_w, float eps, int accumulate);
int cgk_int4_transpose_scales(const float* scales, int K, int G, float* scales_t);
/* MFMA GEMV (gemv.hip), weight layout 3: fp16 matrix cores, exact nibble
 * operands, activations x * scale as two fp16 terms.  pro 0 none / 1
 * RMSNorm; epi 0 store, 1 accumulate, 2 SwiGLU of a paired gate|up weight
 * (y [M][N/2]).  M any (launches of 16 rows, 8 for SwiGLU). */
int cgk_int4_repack_mfma(const uint8_t* flat, const float* scales, int K, int N, int gs,
                         int paired, uint8_t* w, float* scales_t);
int cgk_int4_dequantize_mfma(const uint8_t* w, const float* scales_t, int K, int N, int gs,
                             int paired, float* out);
/* The inverse of cgk_int4_repack_mfma: layout 3 back to the reference's
 * flat nibbles (K*N/2 bytes) and flat scales [K][N/gs]. */
int cgk_int4_unpack_mfma(const uint8_t* w, const float* scales_t, int K, int N, int gs,
                         int paired, uint8_t* flat, float* scales);
/* INT4 GEMM for M >= 16 rows over layout 3 (gemv.hip): same arguments and
 * epilogues as cgk_gemv_mfma plus smax >= every |scale| of the weight.
 * stats_in ([M][nstat_in][2] partial max|x*nw| and sum x^2, from the
 * producer's stats_out) replaces the row-statistics pass over x; stats_out
 * ([M][Nout/128][2]) receives those of the output, per 128 columns, with
 * nw_next the consumer's RMSNorm weights (NULL: 1). */
int cgk_gemm_int4_supported(int M, int K, int N, int gs, int paired);
int cgk_gemm_int4(const float* x, int ldx, int M, int K, int N, int gs, const uint8_t* w,
                  const float* scales_t, float smax, float* y, int ldy, int pro,
                  const float* nw, float eps, int epi, const float* stats_in, int nstat_in,
                  float* stats_out, const float* nw_next);
int cgk_absmax(const float* s, size_t n, float* out_host);
int cgk_gemv_mfma(const float* x, int ldx, int M, int K, int N, int gs, const uint8_t* w,
                  const float* scales_t, float* y, int ldy, int pro, const float* nw, float eps,
                  int epi);
int cgk_gemv_mfma_tiles(int N, int gs, int paired);
int cgk_int4_matmul_generic(const float* x, int M, int K, int N, int gs,
                            const uint8_t* flat, const float* scales, float* y);

/* ------------------------------------------- acceptance and filters */
int cgk_exact_expf(const float* x, float* y, int n);
int cgk_verify_pipe_supported(int batch, int gamma, int V, float T);
int cgk_verify_pipe(const float* target, const float* draft, const int* tokens, const float* u,
                    int batch, int gamma, int V, float T, float* accept_prob, int* out_tokens,
                    int* n_accepted);
int cgk_sample_temperature_pipe(const float* logits, int rows, int V, float T, const float* u,
                                int* out, size_t ld);
/* The verify pipeline on the static workspace of `device` (verify.hip): no
 * allocation; the address is resolved once per device by
 * cgk_verify_static_init (cgx_init calls it). */
int cgk_verify_static_init(int device);
int cgk_verify_pipe_static(int device, const float* target, const float* draft,
                           const int* tokens, const float* u, int batch, int gamma, int V,
                           float T, float* accept_prob, int* out_tokens, int* n_accepted);
/* The device the library is bound to (-1 before cgx_init). */
int cgx_device_id(void);
/* The loop's token rows: ttok[b] = last_b, d_1 .. d_gamma and vtok[b] = d_1 .. d_gamma from
 * feed [B][2] (prev, last) and the drafted tokens dtok [gamma][B]. */
int cgk_spec_tokens(const int* feed, const int* dtok, int B, int gamma, int* ttok, int* vtok);
/* Batched model forward with the logits rows of each sequence ld floats apart
 * (host/model.c; the loop writes draft logits straight into [B][gamma][V]). */
int cgx_model_forward_batch_ld(struct cgx_model* m, const int* tokens, int M, int n_logits,
                               float* logits, size_t ld);
int cgk_exp_fast_maxerr(float lo, float hi, unsigned int* out_dev);
int cgk_exp_stat_maxerr(float lo, float hi, unsigned int* out_dev);
int cgk_ordered_sum(const float* x, int n, float* out);
int cgk_sample_temperature(const float* logits, int V, float T, float u, int* out);
/* the same on `rows` rows (row r at logits + r * ld, draw u[r] on the
 * device, token to out[r]), one workgroup per row */
int cgk_sample_temperature_rows(const float* logits, int rows, int V, float T, const float* u,
                                int* out, size_t ld);
int cgk_sample_corrected(const float* q, const float* p, int V, float u, int* out);
int cgk_temperature_probs(const float* logits, int V, float T, float* probs);
int cgk_verify_chain(const float* target, const float* draft, const int* tokens,
                     const float* u, int batch, int gamma, int V, float T,
                     float* accept_prob, int* correction, int* bonus,
                     int* out_tokens, int* n_accepted);
/* Verify over dense (filtered) distributions: p [batch][gamma + 1][V]
 * target (row gamma unused), q [batch][gamma][V] draft; bonus[batch] drawn
 * beforehand. */
int cgk_verify_chain_dist(const float* p, const float* q, const int* tokens, const float* u,
                          int batch, int gamma, int V, const int* bonus, float* accept_prob,
                          int* correction, int* out_tokens, int* n_accepted);
/* One token from a device logits row with the verify filters (host/sampling.c):
 * draw at du (device), the same value uh on the host; z: V-float workspace.
 * With top-k / top-p, dist (device, V floats, or NULL) also receives the
 * row's filtered distribution from the same launches. */
int cgx_sample_row_dev(const float* row, int V, float T, int top_k, float top_p,
                       const float* du, float uh, float* z, int* out, float* dist);
/* cgx_verify_chain_batch_dev with the draft's filtered distributions
 * already computed (qdist [batch][gamma][V], device, as cgx_sample_row_dev
 * writes them; NULL: computed from draft_logits). */
int cgx_verify_chain_dev_q(const float* target_logits, const float* draft_logits,
                           const float* qdist, const int* draft_tokens, const float* u,
                           int batch, int gamma, int V, float temperature, int top_k,
                           float top_p, int* out_tokens, int* n_accepted, float* accept_prob);
/* The global LCG of the drop-in samplers (host/speculative.c). */
float cgx_lcg_draw(void);
/* Typical sampling (decision D16) over rows of logits at T = 1: tokens drawn
 * with u (device), or dense distributions.  Uses scratch slot WS0. */
int cgk_typical_rows(const float* logits, int rows, int V, float typical_p, const float* u,
                     int* tokens, float* dist);
/* The typical sampler's binary64 log of positive floats, elementwise. */
int cgk_typ_log(const float* x, double* y, int n);
/* Stable radix sort of rows of 32-bit keys (rowsort.hip), descending or
 * ascending; with pout, payloads travel with their keys (pin NULL: the key's
 * index in its row).  ws: cgk_row_sort_ws(rows, n, pout != NULL) bytes. */
size_t cgk_row_sort_ws(int rows, int n, int with_payload);
int cgk_row_sort(const uint32_t* kin, const uint32_t* pin, int rows, int n, int desc,
                 uint32_t* kout, uint32_t* pout, void* ws, size_t ws_bytes);
/* z = x / T elementwise. */
int cgk_scale(const float* x, float* z, size_t n, float T);
/* Top-k (0 < top_k < V) or top-p over rows of z [rows][V]: a token per row
 * drawn with u[row] (tokens != NULL), or dense filtered distributions
 * (dist != NULL).  Uses scratch slot WS0. */
int cgk_filter_rows(const float* z, int rows, int V, int top_k, float top_p, const float* u,
                    int* tokens, float* dist);
/* The same with both outputs from one pass: distributions of every row
 * (dist != NULL) and tokens of the rows r with (r + 1) % tok_every == 0
 * (tokens[r / tok_every], drawn with u[(r / tok_every) * u_stride]). */
int cgk_filter_rows_ex(const float* z, int rows, int V, int top_k, float top_p,
                       const float* u, int u_stride, int* tokens, int tok_every, float* dist);
/* The same over rows of x at temperature T (z = x / T, computed as read;
 * zbuf [rows][V] holds z for the top-k path when T != 1). */
int cgk_filter_rows_t(const float* x, float T, float* zbuf, int rows, int V, int top_k,
                      float top_p, const float* u, int u_stride, int* tokens, int tok_every,
                      float* dist);

/* ---------------------------------------- KV cache, attention, RoPE */
/* attention mask kinds of cgk_attention */
enum {
    CGK_MASK_NONE = 0,
    CGK_MASK_CAUSAL_ALIGNED = 1, /* query q sees keys <= Nk - Nq + q */
    CGK_MASK_WINDOW = 2,         /* |key - q| <= window */
    CGK_MASK_CUSTOM = 3,         /* additive fp32 [Nq][Nk] */
    CGK_MASK_TREE = 4,           /* keys < Nk - tw, plus ancestor bits over the last tw */
    CGK_MASK_CAUSAL = 5          /* query q sees keys <= q */
};
int cgk_kv_append(const float* k, const float* v, int T, int H, int D, int gs, int pos,
                  uint8_t* kc, uint8_t* vc, float* ks, float* vs);
int cgk_kv_get(const uint8_t* kc, const uint8_t* vc, const float* ks, const float* vs,
               int len, int H, int D, int gs, float* ko, float* vo);
/* Q [B][Nq][H][D]; INT4 cache slice (int4 != 0, B must be 1) or fp32
 * K/V [B][Nk][Hk][D]; O [B][Nq][H][D]; lse optional [B][H][Nq].  anc: HOST
 * array of Nq <= 64 ancestor bitmasks (tree mask only), passed by value. */
int cgk_attention(const float* Q, int int4, const uint8_t* kc, const uint8_t* vc,
                  const float* ks, const float* vs, int gs, const float* K, const float* V,
                  int B, int Nq, int Nk, int H, int Hk, int D, float scale, int mask_kind,
                  int window, const float* mask, const unsigned long long* anc, float* O,
                  float* lse);
/* MFMA decode/verify attention over an INT4 cache slice with one scale per
 * head row (attn_dec.hip); cgk_attention routes here when supported. */
int cgk_attn_dec_supported(int D, int gs, int B, int mask_kind);
int cgk_attn_dec(const float* Q, const uint8_t* kc, const uint8_t* vc, const float* ks,
                 const float* vs, int Nq, int Nk, int H, int Hk, int D, float scale,
                 int mask_kind, const unsigned long long* anc, float* O);
/* Batched decode attention: B sequences of Nq query rows, sequence b's cache
 * at kc + b * seq_kbytes (scales + b * seq_groups) with nk[b] keys.  Tree
 * mask: the last tw keys (Nq <= tw <= 64; the tree's nodes so far, the query
 * rows last) are visible to query row i only where bit j of anc[i] is set.
 * stats (D == 128; NULL: none) receives the row statistics of O for the GEMM
 * that reads it: (max|o|, sum o^2) per output row and head, [B][Nq][H][2]. */
int cgk_attn_dec_batch(const float* Q, const uint8_t* kc, const uint8_t* vc, const float* ks,
                       const float* vs, int B, const int* nk, size_t seq_kbytes,
                       size_t seq_groups, int Nq, int H, int Hk, int D, float scale,
                       int mask_kind, const unsigned long long* anc, int tw, float* O,
                       float* stats);

/* Rows of a tree forward (cgx_model_forward_tree): row i sits at cache slot
 * len + i and rotary position len + rel[i]; the last tw cached keys are the
 * tree's nodes, visible to row i through anc[i]. */
typedef struct {
    int rel[64];
    unsigned long long anc[64];
    int tw;
} cgx_tree_rows;
int cgx_model_forward_tree(cgx_model* m, const int* tokens, int M, const cgx_tree_rows* tr,
                           float* logits, size_t ldl);
/* The same for sequence 0 only (tokens [M]; every row's logits, or none). */
int cgx_model_forward_tree1(cgx_model* m, const int* tokens, int M, const cgx_tree_rows* tr,
                            float* logits);
/* The model behind a void* handle, or NULL when p is no live model. */
cgx_model* cgx_model_from_handle(const void* p);
/* Changes with every forward, truncation, context fill or compaction. */
uint64_t cgx_model_epoch(const cgx_model* m);
/* The driver (host/driver.c) drops what it knows about a freed model. */
void cgx_driver_forget_model(const cgx_model* m);

/* A COG1 file opened for a decoder's weights (host/model_file.c).  Entry
 * indices come from cgx_wfile_find (-1: absent).  A matrix [K, N] is nb
 * column blocks (entries idx[b] of widths[b]); cgx_wfile_matrix_kind checks
 * their directory entries and returns 0 (fp32) or 2 (INT4 of group gs), or
 * -1 with the error set; the readers then fill host buffers: fp32 [K][N], or
 * flat nibbles [K][N/2] and scales [K][N/gs].  cgx_wfile_vector returns the
 * index of an fp32 vector of n values, -1 when absent, -2 (error set) when
 * malformed. */
typedef struct cgx_wfile cgx_wfile;
cgx_wfile* cgx_wfile_open(const char* path, const char* who);
void cgx_wfile_close(cgx_wfile* w);
int cgx_wfile_find(const cgx_wfile* w, const char* name);
int cgx_wfile_vector(const cgx_wfile* w, const char* name, int n, const char* who);
int cgx_wfile_matrix_kind(const cgx_wfile* w, const int* idx, const int* widths, int nb, int K,
                          int gs, const char* who);
int cgx_wfile_read_vector(const cgx_wfile* w, int i, float* out, int n);
int cgx_wfile_read_f32(const cgx_wfile* w, const int* idx, const int* widths, int nb, int K,
                       float* out);
int cgx_wfile_read_int4(const cgx_wfile* w, const int* idx, const int* widths, int nb, int K,
                        int gs, uint8_t* data, float* scales);

/* Static draft tree (tree.hip, host/tree.c): node 0 is the verified root;
 * nodes are in breadth-first order; kids[i][0..nkids[i]) the children of
 * node i in rank order (rank r = the draft's (r+1)-th most likely token). */
typedef struct {
    int nodes, depth;
    int parent[64], node_depth[64];
    int nkids[64];
    int kids[64][4];
    int rank[64];
} cgx_tree_shape;
int cgk_tree_accept(const cgx_tree_shape* t, int B, int K, const int* lidx, const float* lp,
                    const int* tok, const float* u, int* out, int* nacc, int* path);
int cgk_kv_compact(const cgx_tree_shape* t, int B, const int* len0, const int* nacc,
                   const int* path, int layers, int nb, uint8_t* kc, uint8_t* vc, float* ks,
                   float* vs, int row_bytes, int row_groups, size_t layer_bytes,
                   size_t layer_groups);
int cgk_topk_lists(const float* z, int rows, int V, int top_k, float top_p, int* lidx,
                   float* lp);
int cgk_tree_children(const cgx_tree_shape* t, int B, int K, int first, int count, int pfirst,
                      int pcount, const int* parent_dev, const int* rank_dev, const int* lidx,
                      int* tok);
int cgk_tree_gather(int B, int R, int first, int count, const int* tok, int* out);
/* Moves the accepted path's cache rows (tree.hip k_kv_compact) in every layer
 * and sets sequence b's length to len0[b] + 1 + nacc_host[b]. */
int cgx_model_compact_tree(cgx_model* m, const cgx_tree_shape* t, const int* len0,
                           const int* nacc_dev, const int* path_dev, const int* nacc_host);
/* The default draft tree: nodes (root included) chosen best-first by a path
 * score (the product of fixed per-rank weights), at most 4 children and the
 * given depth; breadth-first numbering. */
int cgx_tree_shape_default(cgx_tree_shape* t, int nodes, int depth);
/* A tree from parents (breadth-first, parent[i] < i, parent[0] = -1) and the
 * rank of each node among its siblings (0 .. 3, distinct, in order). */
int cgx_tree_shape_from_parents(cgx_tree_shape* t, const int* parent, int nodes);
int cgk_rope(float* x, int S, int H, int D, int pos0, float theta);
/* (cos, sin) of positions pos0 .. pos0 + rows - 1 times each RoPE frequency:
 * cs [rows][D/2][2] (decoder.hip; the arithmetic of the cache append). */
int cgk_rope_table(int rows, int D, int pos0, float theta, float* cs);
/* Fused RoPE, INT4 cache append of the Nq new keys and attention (attn_dec.hip). */
int cgk_attn_dec_rope(const float* qkv, int ldq, const float* rope, uint8_t* kc, uint8_t* vc,
                      float* ks, float* vs, int B, const int* nk, size_t seq_kbytes,
                      size_t seq_groups, int Nq, int H, int Hk, int D, float scale,
                      int mask_kind, const unsigned long long* anc, int tw, float* O,
                      float* stats);
int cgk_rope_freqs(float* cs, float* sn, int S, int D, float theta);
int cgk_alibi_slopes(float* slopes, int H);
int cgk_alibi_bias(float* bias, int Sq, int Sk, int H, const float* slopes);

#ifdef __cplusplus
}
#endif

#endif /* CGX_INTERNAL_H */
