/*
 * kvcache.c -- cogito's INT4 KV cache (include/cg_quantize.h:52-64,126-146;
 * reference src/quantize/int4.c:116-289) held in HBM, and attention over it
 * (cg_attention_int4_kv, declared only in the reference at
 * include/cg_quantize.h:116-117).
 *
 * Layout as the reference: K/V bytes [layers][max_seq][n_heads][head_dim/2],
 * scales [layers][max_seq][n_heads][head_dim/group_size] fp32.
 * current_len advances once per token position, on the append of the last
 * layer (the reference advances once per call, int4.c:233).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "cg_mi355x.h"
#include "cg_quantize.h"
#include "cgx_internal.h"

static size_t layer_bytes(const cg_kv_cache_int4* c) {
    return (size_t)c->max_seq_len * c->n_heads * (c->head_dim / 2);
}

static size_t layer_groups(const cg_kv_cache_int4* c) {
    return (size_t)c->max_seq_len * c->n_heads * (c->head_dim / c->group_size);
}

cg_kv_cache_int4* cg_kv_cache_int4_new(int num_layers, int max_seq_len, int n_heads,
                                        int head_dim, int group_size) {
    if (num_layers <= 0 || max_seq_len <= 0 || n_heads <= 0 || head_dim <= 0 ||
        (head_dim & 1) || group_size <= 0 || (group_size & 1) || head_dim % group_size) {
        cgx_set_error("cg_kv_cache_int4_new: invalid dimensions (head_dim and group_size "
                      "must be even, group_size must divide head_dim)");
        return NULL;
    }
    if (cgx_ensure_init()) return NULL;
    cg_kv_cache_int4* c = (cg_kv_cache_int4*)calloc(1, sizeof(*c));
    if (!c) return NULL;
    c->num_layers = num_layers;
    c->max_seq_len = max_seq_len;
    c->n_heads = n_heads;
    c->head_dim = head_dim;
    c->group_size = group_size;
    size_t bytes = layer_bytes(c) * num_layers;
    size_t groups = layer_groups(c) * num_layers;
    c->k_cache = (uint8_t*)cgx_malloc(bytes);
    c->v_cache = (uint8_t*)cgx_malloc(bytes);
    c->k_scales = (float*)cgx_malloc(groups * 4);
    c->v_scales = (float*)cgx_malloc(groups * 4);
    if (!c->k_cache || !c->v_cache || !c->k_scales || !c->v_scales ||
        cgx_memset(c->k_cache, 0, bytes) || cgx_memset(c->v_cache, 0, bytes) ||
        cgx_memset(c->k_scales, 0, groups * 4) || cgx_memset(c->v_scales, 0, groups * 4)) {
        cg_kv_cache_int4_free(c);
        return NULL;
    }
    return c;
}

void cg_kv_cache_int4_free(cg_kv_cache_int4* c) {
    if (!c) return;
    cgx_free(c->k_cache);
    cgx_free(c->v_cache);
    cgx_free(c->k_scales);
    cgx_free(c->v_scales);
    free(c);
}

void cg_kv_cache_int4_reset(cg_kv_cache_int4* c) {
    if (c) c->current_len = 0;
}

int cgx_kv_cache_int4_set_len(cg_kv_cache_int4* c, int len) {
    if (!c || len < 0 || len > c->max_seq_len) {
        cgx_set_error("cgx_kv_cache_int4_set_len: length out of range");
        return -1;
    }
    c->current_len = len;
    return 0;
}

int cgx_kv_cache_int4_truncate(cg_kv_cache_int4* c, int new_len) {
    if (!c || new_len < 0 || new_len > c->current_len) {
        cgx_set_error("cgx_kv_cache_int4_truncate: new length out of range");
        return -1;
    }
    c->current_len = new_len;
    return 0;
}

int cgx_kv_cache_int4_write(cg_kv_cache_int4* c, int layer, int pos, const float* k,
                            const float* v, int T) {
    if (!c || !k || !v || layer < 0 || layer >= c->num_layers || pos < 0 || T < 0 ||
        pos + T > c->max_seq_len) {
        cgx_set_error("cgx_kv_cache_int4_write: invalid layer/position/length");
        return -1;
    }
    if (!T) return 0;
    if (cgx_ensure_init()) return -1;
    size_t n = (size_t)T * c->n_heads * c->head_dim;
    const float* dk = (const float*)cgx_dev_in(k, n * 4, CGX_SLOT_IN0);
    const float* dv = (const float*)cgx_dev_in(v, n * 4, CGX_SLOT_IN1);
    if (!dk || !dv) return -1;
    if (cgk_kv_append(dk, dv, T, c->n_heads, c->head_dim, c->group_size, pos,
                      c->k_cache + layer_bytes(c) * layer, c->v_cache + layer_bytes(c) * layer,
                      c->k_scales + layer_groups(c) * layer,
                      c->v_scales + layer_groups(c) * layer))
        return -1;
    /* host inputs were staged: finish before the caller may reuse them */
    if (dk != k || dv != v) return cgx_synchronize();
    return 0;
}

void cg_kv_cache_int4_append(cg_kv_cache_int4* c, int layer, cg_tensor* new_k,
                             cg_tensor* new_v) {
    if (!c || !new_k || !new_v || !new_k->data || !new_v->data || layer < 0 ||
        layer >= c->num_layers) {
        cgx_set_error("cg_kv_cache_int4_append: invalid argument");
        return;
    }
    int per_tok = c->n_heads * c->head_dim;
    if (new_k->size % per_tok || new_v->size != new_k->size) {
        cgx_set_error("cg_kv_cache_int4_append: K/V size %d is not T x %d", new_k->size,
                      per_tok);
        return;
    }
    int T = new_k->size / per_tok;
    if (c->current_len + T > c->max_seq_len) {
        /* the reference returns silently when full (int4.c:153) */
        cgx_set_error("cg_kv_cache_int4_append: cache full (%d + %d > %d)", c->current_len,
                      T, c->max_seq_len);
        return;
    }
    if (cgx_kv_cache_int4_write(c, layer, c->current_len, new_k->data, new_v->data, T))
        return;
    if (layer == c->num_layers - 1) c->current_len += T;
}

void cg_kv_cache_int4_get(cg_kv_cache_int4* c, int layer, cg_tensor* k_out,
                          cg_tensor* v_out) {
    if (!c || !k_out || !v_out || !k_out->data || !v_out->data || layer < 0 ||
        layer >= c->num_layers) {
        cgx_set_error("cg_kv_cache_int4_get: invalid argument");
        return;
    }
    int len = c->current_len;
    size_t n = (size_t)len * c->n_heads * c->head_dim;
    if ((size_t)k_out->size < n || (size_t)v_out->size < n) {
        cgx_set_error("cg_kv_cache_int4_get: outputs hold fewer than %zu values", n);
        return;
    }
    if (!n) return;
    if (cgx_ensure_init()) return;
    int kd = cgx_is_device_ptr(k_out->data), vd = cgx_is_device_ptr(v_out->data);
    float* ko = kd ? k_out->data : (float*)cgx_scratch(CGX_SLOT_OUT0, n * 4);
    float* vo = vd ? v_out->data : (float*)cgx_scratch(CGX_SLOT_OUT1, n * 4);
    if (!ko || !vo) return;
    if (cgk_kv_get(c->k_cache + layer_bytes(c) * layer, c->v_cache + layer_bytes(c) * layer,
                   c->k_scales + layer_groups(c) * layer,
                   c->v_scales + layer_groups(c) * layer, len, c->n_heads, c->head_dim,
                   c->group_size, ko, vo))
        return;
    if (!kd) cgx_memcpy_d2h(k_out->data, ko, n * 4);
    if (!vd) cgx_memcpy_d2h(v_out->data, vo, n * 4);
    if (kd && vd) cgx_synchronize();
}

/* ------------------------------------------------------------ attention */

int cgx_attention_int4_kv_batch_dev(const float* Q, int B, int Nq, int H, cg_kv_cache_int4* c,
                                    int slot0, const int* nk, int mask_kind,
                                    const unsigned long long* anc, int tw, float* O) {
    if (!Q || !O || !c || !nk || B < 1 || Nq <= 0 || H <= 0 || slot0 < 0 ||
        slot0 + B > c->num_layers || (mask_kind != 0 && mask_kind != 1) ||
        (mask_kind == 1 && !anc)) {
        cgx_set_error("cgx_attention_int4_kv_batch_dev: invalid argument");
        return -1;
    }
    for (int b = 0; b < B; b++)
        if (nk[b] < Nq || nk[b] > c->max_seq_len) {
            cgx_set_error("cgx_attention_int4_kv_batch_dev: sequence %d has %d keys (need %d.."
                          "%d)", b, nk[b], Nq, c->max_seq_len);
            return -1;
        }
    if (c->group_size != c->head_dim) {
        cgx_set_error("cgx_attention_int4_kv_batch_dev: the batched kernel needs one scale per "
                      "head row (group_size == head_dim)");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const size_t lb = layer_bytes(c), lg = layer_groups(c);
    return cgk_attn_dec_batch(Q, c->k_cache + lb * slot0, c->v_cache + lb * slot0,
                              c->k_scales + lg * slot0, c->v_scales + lg * slot0, B, nk, lb, lg,
                              Nq, H, c->n_heads, c->head_dim, 1.0f / sqrtf((float)c->head_dim),
                              mask_kind == 1 ? CGK_MASK_TREE : CGK_MASK_CAUSAL_ALIGNED, anc, tw,
                              O, NULL);
}

int cgx_rope_table_dev(int rows, int head_dim, int pos0, float theta, float* cs) {
    if (!cs || rows <= 0 || head_dim < 2 || (head_dim & 1) || pos0 < 0) {
        cgx_set_error("cgx_rope_table_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    return cgk_rope_table(rows, head_dim, pos0, theta, cs);
}

int cgx_attention_rope_append_dev(const float* qkv, int ldq, const float* rope, int Nq, int H,
                                  cg_kv_cache_int4* c, int layer, int pos, float* O) {
    if (!qkv || !rope || !O || !c || Nq <= 0 || Nq > 64 || H <= 0 || layer < 0 ||
        layer >= c->num_layers || pos < 0 || pos + Nq > c->max_seq_len) {
        cgx_set_error("cgx_attention_rope_append_dev: invalid argument (%d rows at position "
                      "%d, at most 64 rows)", Nq, pos);
        return -1;
    }
    if (c->group_size != c->head_dim) {
        cgx_set_error("cgx_attention_rope_append_dev: needs one scale per head row "
                      "(group_size == head_dim)");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const size_t lb = layer_bytes(c), lg = layer_groups(c);
    const int nk = pos + Nq;
    return cgk_attn_dec_rope(qkv, ldq, rope, c->k_cache + lb * layer, c->v_cache + lb * layer,
                             c->k_scales + lg * layer, c->v_scales + lg * layer, 1, &nk, 0, 0,
                             Nq, H, c->n_heads, c->head_dim, 1.0f / sqrtf((float)c->head_dim),
                             CGK_MASK_CAUSAL_ALIGNED, NULL, Nq, O, NULL);
}

int cgx_attention_int4_kv_dev(const float* Q, int Nq, int H, cg_kv_cache_int4* c,
                              int layer, int mask_kind, const int* parents, float* O) {
    if (!Q || !O || !c || Nq <= 0 || H <= 0 || layer < 0 || layer >= c->num_layers) {
        cgx_set_error("cgx_attention_int4_kv_dev: invalid argument");
        return -1;
    }
    int len = c->current_len;
    if (Nq > len) {
        cgx_set_error("cgx_attention_int4_kv_dev: %d queries but only %d cached tokens "
                      "(append the new tokens first)", Nq, len);
        return -1;
    }
    if (H < c->n_heads) {
        cgx_set_error("cgx_attention_int4_kv_dev: %d query heads < %d KV heads", H, c->n_heads);
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    int kind = CGK_MASK_CAUSAL_ALIGNED;    /* chain */
    if (mask_kind == 1) {
        if (!parents || Nq > 64) {
            cgx_set_error("cgx_attention_int4_kv_dev: tree mask needs parents[] and <= 64 nodes");
            return -1;
        }
        int par[64];
        if (cgx_is_device_ptr(parents)) {
            if (cgx_memcpy_d2h(par, parents, (size_t)Nq * sizeof(int))) return -1;
        } else {
            memcpy(par, parents, (size_t)Nq * sizeof(int));
        }
        unsigned long long anc[64];
        for (int i = 0; i < Nq; i++) {
            if (par[i] >= i || par[i] < -1) {
                cgx_set_error("cgx_attention_int4_kv_dev: parents[%d] = %d must be -1 or a "
                              "preceding node", i, par[i]);
                return -1;
            }
            anc[i] = (1ull << i) | (par[i] >= 0 ? anc[par[i]] : 0ull);
        }
        kind = CGK_MASK_TREE;
        return cgk_attention(Q, 1, c->k_cache + layer_bytes(c) * layer,
                             c->v_cache + layer_bytes(c) * layer,
                             c->k_scales + layer_groups(c) * layer,
                             c->v_scales + layer_groups(c) * layer, c->group_size, NULL, NULL, 1,
                             Nq, len, H, c->n_heads, c->head_dim,
                             1.0f / sqrtf((float)c->head_dim), kind, 0, NULL, anc, O, NULL);
    } else if (mask_kind != 0) {
        cgx_set_error("cgx_attention_int4_kv_dev: mask_kind must be 0 (chain) or 1 (tree)");
        return -1;
    }
    size_t lb = layer_bytes(c), lg = layer_groups(c);
    float scale = 1.0f / sqrtf((float)c->head_dim);
    return cgk_attention(Q, 1, c->k_cache + lb * layer, c->v_cache + lb * layer,
                         c->k_scales + lg * layer, c->v_scales + lg * layer, c->group_size,
                         NULL, NULL, 1, Nq, len, H, c->n_heads, c->head_dim, scale, kind, 0,
                         NULL, NULL, O, NULL);
}

void cg_attention_int4_kv(cg_tensor* Q, cg_kv_cache_int4* c, int layer, cg_tensor* output) {
    if (!Q || !c || !output || !Q->data || !output->data) {
        cgx_set_error("cg_attention_int4_kv: invalid argument");
        return;
    }
    int D = c->head_dim;
    int H, Nq;
    if (Q->ndim >= 3) {
        H = Q->shape[Q->ndim - 2];
        if (Q->shape[Q->ndim - 1] != D) {
            cgx_set_error("cg_attention_int4_kv: Q head_dim %d != cache %d",
                          Q->shape[Q->ndim - 1], D);
            return;
        }
        Nq = Q->size / (H * D);
    } else if (Q->ndim == 2 && Q->shape[1] % D == 0) {
        Nq = Q->shape[0];
        H = Q->shape[1] / D;
    } else {
        cgx_set_error("cg_attention_int4_kv: Q must be [Nq, H, D] or [1, Nq, H, D]");
        return;
    }
    if (output->size < Q->size) {
        cgx_set_error("cg_attention_int4_kv: output smaller than Q");
        return;
    }
    if (cgx_ensure_init()) return;
    size_t n = (size_t)Q->size;
    const float* dq = (const float*)cgx_dev_in(Q->data, n * 4, CGX_SLOT_IN2);
    int od = cgx_is_device_ptr(output->data);
    float* dout = od ? output->data : (float*)cgx_scratch(CGX_SLOT_OUT0, n * 4);
    if (!dq || !dout) return;
    if (cgx_attention_int4_kv_dev(dq, Nq, H, c, layer, 0, NULL, dout)) return;
    if (!od) cgx_memcpy_d2h(output->data, dout, n * 4);
    else cgx_synchronize();
}
