/*
 * pending.c -- entry points whose GPU kernels are not wired yet.  Each one
 * records "not implemented yet" in the last error and returns an error
 * value; none computes anything on the CPU.  Entries move out of this file
 * as their kernels land.
 */
#include <stddef.h>

#include "cg_mi355x.h"
#include "cgx_internal.h"

#define PENDING(name) cgx_set_error("%s: not implemented yet", name)

/* cg_quantize.h: KV cache and attention */
void cg_attention_int4_kv(cg_tensor* Q, cg_kv_cache_int4* kv, int layer, cg_tensor* out) {
    (void)Q; (void)kv; (void)layer; (void)out; PENDING("cg_attention_int4_kv");
}
cg_kv_cache_int4* cg_kv_cache_int4_new(int L, int S, int H, int D, int gs) {
    (void)L; (void)S; (void)H; (void)D; (void)gs; PENDING("cg_kv_cache_int4_new"); return NULL;
}
void cg_kv_cache_int4_append(cg_kv_cache_int4* c, int l, cg_tensor* k, cg_tensor* v) {
    (void)c; (void)l; (void)k; (void)v; PENDING("cg_kv_cache_int4_append");
}
void cg_kv_cache_int4_get(cg_kv_cache_int4* c, int l, cg_tensor* k, cg_tensor* v) {
    (void)c; (void)l; (void)k; (void)v; PENDING("cg_kv_cache_int4_get");
}
void cg_kv_cache_int4_reset(cg_kv_cache_int4* c) { (void)c; PENDING("cg_kv_cache_int4_reset"); }
void cg_kv_cache_int4_free(cg_kv_cache_int4* c) { (void)c; }
int cgx_kv_cache_int4_truncate(cg_kv_cache_int4* c, int n) { (void)c; (void)n; PENDING("cgx_kv_cache_int4_truncate"); return -1; }
int cgx_kv_cache_int4_write(cg_kv_cache_int4* c, int l, int p, const float* k, const float* v, int T) {
    (void)c; (void)l; (void)p; (void)k; (void)v; (void)T; PENDING("cgx_kv_cache_int4_write"); return -1;
}
int cgx_kv_cache_int4_set_len(cg_kv_cache_int4* c, int n) { (void)c; (void)n; PENDING("cgx_kv_cache_int4_set_len"); return -1; }
int cgx_attention_int4_kv_dev(const float* Q, int Nq, int H, cg_kv_cache_int4* c, int l,
                              int mk, const int* par, float* O) {
    (void)Q; (void)Nq; (void)H; (void)c; (void)l; (void)mk; (void)par; (void)O;
    PENDING("cgx_attention_int4_kv_dev"); return -1;
}

/* cg_flash_attn.h */
void cg_flash_attention_forward(cg_flash_attn_params* p) { (void)p; PENDING("cg_flash_attention_forward"); }
void cg_flash_attention_forward_cpu(cg_flash_attn_params* p) { (void)p; PENDING("cg_flash_attention_forward_cpu"); }
void cg_flash_attention_backward(cg_flash_attn_params* p) { (void)p; PENDING("cg_flash_attention_backward"); }
void cg_flash_attention_backward_cpu(cg_flash_attn_params* p) { (void)p; PENDING("cg_flash_attention_backward_cpu"); }
void cg_flash_attention_mqa(cg_flash_attn_params* p) { (void)p; PENDING("cg_flash_attention_mqa"); }
void cg_flash_attention_gqa(cg_flash_attn_params* p, int g) { (void)p; (void)g; PENDING("cg_flash_attention_gqa"); }
cg_flash_attn_params* cg_flash_attn_params_new(cg_tensor* Q, cg_tensor* K, cg_tensor* V,
                                               cg_attention_mask_type m, float d) {
    (void)Q; (void)K; (void)V; (void)m; (void)d; PENDING("cg_flash_attn_params_new"); return NULL;
}
cg_flash_attn_config cg_flash_attn_autotune(int sq, int sk, int d, int sm) {
    cg_flash_attn_config c = {0};
    (void)sq; (void)sk; (void)d; (void)sm; PENDING("cg_flash_attn_autotune");
    return c;
}
size_t cg_flash_attn_shared_mem(int bm, int bn, int d) { (void)bm; (void)bn; (void)d; return 0; }
void cg_flash_attn_params_free(cg_flash_attn_params* p) { (void)p; }
void cg_apply_rope(float* Q, float* K, int s, int h, int d, int off, float th) {
    (void)Q; (void)K; (void)s; (void)h; (void)d; (void)off; (void)th; PENDING("cg_apply_rope");
}
void cg_rope_precompute_freqs(float* c, float* s, int m, int d, float th) {
    (void)c; (void)s; (void)m; (void)d; (void)th; PENDING("cg_rope_precompute_freqs");
}
void cg_alibi_bias(float* b, int sq, int sk, int h, float* sl) {
    (void)b; (void)sq; (void)sk; (void)h; (void)sl; PENDING("cg_alibi_bias");
}
void cg_alibi_slopes(float* s, int h) { (void)s; (void)h; PENDING("cg_alibi_slopes"); }

/* cg_speculative.h: sampling and verification */
int cg_sample_top_p(float* l, int V, float p) { (void)l; (void)V; (void)p; PENDING("cg_sample_top_p"); return -1; }
int cg_sample_top_k(float* l, int V, int k) { (void)l; (void)V; (void)k; PENDING("cg_sample_top_k"); return -1; }
int cg_sample_typical(float* l, int V, float p) { (void)l; (void)V; (void)p; PENDING("cg_sample_typical"); return -1; }
int cg_target_verify(cg_speculative_decoder* d, cg_tensor* ids, cg_token_tree* t) {
    (void)d; (void)ids; (void)t; PENDING("cg_target_verify"); return -1;
}
int cg_speculative_step(cg_speculative_decoder* d, cg_tensor* ids, cg_token_tree* t) {
    (void)d; (void)ids; (void)t; PENDING("cg_speculative_step"); return -1;
}
cg_tensor* cg_speculative_generate(cg_speculative_decoder* d, cg_tensor* ids, int n, float T, float p) {
    (void)d; (void)ids; (void)n; (void)T; (void)p; PENDING("cg_speculative_generate"); return NULL;
}
cg_token_tree* cg_draft_generate(cg_speculative_decoder* d, cg_tensor* ids) {
    (void)d; (void)ids; PENDING("cg_draft_generate"); return NULL;
}
cg_tensor* cg_forward_tree_attention(void* m, cg_tensor* in, cg_tensor* mask) {
    (void)m; (void)in; (void)mask; PENDING("cg_forward_tree_attention"); return NULL;
}
cg_token_tree* cg_eagle_generate_tree(cg_eagle_draft* e, cg_tensor* in, int d) {
    (void)e; (void)in; (void)d; PENDING("cg_eagle_generate_tree"); return NULL;
}
int* cg_eagle_compute_branching(cg_eagle_draft* e, cg_tensor* f) {
    (void)e; (void)f; PENDING("cg_eagle_compute_branching"); return NULL;
}
int cgx_sample_top_k_u(const float* l, int V, int k, float u) { (void)l; (void)V; (void)k; (void)u; PENDING("x"); return -1; }
int cgx_sample_top_p_u(const float* l, int V, float p, float u) { (void)l; (void)V; (void)p; (void)u; PENDING("x"); return -1; }
