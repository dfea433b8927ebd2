/*
 * flash.c -- cogito's flash-attention API (include/cg_flash_attn.h; reference
 * src/attention/flash_attn.c and src/cuda/flash_attn_kernels.c:261-396,
 * 582-598), RoPE and ALiBi, on the GPU.
 *
 * Every entry point takes host or device pointers.  Host arrays are staged
 * through the library's scratch buffers; results are copied back before the
 * call returns.  All-device calls return after the GPU finished.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "cg_flash_attn.h"
#include "cg_mi355x.h"
#include "cgx_internal.h"

/* Device view of an input array: the pointer itself, or a scratch copy. */
static const float* dev_view(const float* p, size_t n, int slot) {
    return (const float*)cgx_dev_in(p, n * sizeof(float), slot);
}

/* Runs attention for params with KV head count Hk and kernel mask kind. */
static void flash_run(const char* who, cg_flash_attn_params* p, int Hk, int kind) {
    if (!p || !p->Q || !p->K || !p->V || !p->O) {
        cgx_set_error("%s: params, Q, K, V and O are required", who);
        return;
    }
    int B = p->batch_size, Nq = p->seqlen_q, Nk = p->seqlen_k, H = p->n_heads, D = p->d_head;
    if (B <= 0 || Nq <= 0 || Nk <= 0 || H <= 0 || Hk <= 0 || D <= 0) {
        cgx_set_error("%s: invalid shape B=%d Nq=%d Nk=%d H=%d Hk=%d D=%d", who, B, Nq, Nk, H,
                      Hk, D);
        return;
    }
    if (kind == CGK_MASK_CUSTOM && !p->mask) kind = CGK_MASK_NONE;
    if (cgx_ensure_init()) return;
    size_t nq = (size_t)B * Nq * H * D, nk = (size_t)B * Nk * Hk * D;
    const float* dq = dev_view(p->Q, nq, CGX_SLOT_IN0);
    const float* dk = dev_view(p->K, nk, CGX_SLOT_IN1);
    const float* dv = dev_view(p->V, nk, CGX_SLOT_IN2);
    const float* dm = kind == CGK_MASK_CUSTOM ? dev_view(p->mask, (size_t)Nq * Nk, CGX_SLOT_IN3)
                                              : NULL;
    if (!dq || !dk || !dv || (kind == CGK_MASK_CUSTOM && !dm)) return;
    int od = cgx_is_device_ptr(p->O);
    float* dout = od ? p->O : (float*)cgx_scratch(CGX_SLOT_OUT0, nq * sizeof(float));
    size_t nl = (size_t)B * H * Nq;
    int ld = p->softmax_lse ? cgx_is_device_ptr(p->softmax_lse) : 1;
    float* dlse = NULL;
    if (p->softmax_lse) dlse = ld ? p->softmax_lse : (float*)cgx_scratch(CGX_SLOT_OUT1, nl * 4);
    if (!dout || (p->softmax_lse && !dlse)) return;
    if (cgk_attention(dq, 0, NULL, NULL, NULL, NULL, 0, dk, dv, B, Nq, Nk, H, Hk, D, p->scale,
                      kind, p->window_size, dm, NULL, dout, dlse))
        return;
    if (!od && cgx_memcpy_d2h(p->O, dout, nq * sizeof(float))) return;
    if (p->softmax_lse && !ld && cgx_memcpy_d2h(p->softmax_lse, dlse, nl * 4)) return;
    if (od && ld) cgx_synchronize();
}

static int mask_kind_of(const cg_flash_attn_params* p) {
    switch (p->mask_type) {
        case ATTN_MASK_CAUSAL: return CGK_MASK_CAUSAL;
        case ATTN_MASK_SLIDING_WINDOW: return CGK_MASK_WINDOW;
        case ATTN_MASK_CUSTOM: return CGK_MASK_CUSTOM;
        default: return CGK_MASK_NONE;
    }
}

/* Forward with GQA (n_heads_k), causal / sliding-window masks as the
 * reference (flash_attn_kernels.c:317-329) and an additive custom mask. */
void cg_flash_attention_forward(cg_flash_attn_params* params) {
    if (!params) {
        cgx_set_error("cg_flash_attention_forward: params is NULL");
        return;
    }
    flash_run("cg_flash_attention_forward", params, params->n_heads_k, mask_kind_of(params));
}

/* The reference's CPU forward (flash_attn.c:17-149): K/V have n_heads heads
 * (n_heads_k is ignored) and only the causal mask is applied. */
void cg_flash_attention_forward_cpu(cg_flash_attn_params* params) {
    if (!params) {
        cgx_set_error("cg_flash_attention_forward_cpu: params is NULL");
        return;
    }
    flash_run("cg_flash_attention_forward_cpu", params, params->n_heads,
              params->mask_type == ATTN_MASK_CAUSAL ? CGK_MASK_CAUSAL : CGK_MASK_NONE);
}

/* flash_attn_kernels.c:582-592: MQA sets n_heads_k = 1, GQA sets it to the
 * number of KV groups, then the forward runs. */
void cg_flash_attention_mqa(cg_flash_attn_params* params) {
    if (!params) {
        cgx_set_error("cg_flash_attention_mqa: params is NULL");
        return;
    }
    params->n_heads_k = 1;
    cg_flash_attention_forward(params);
}

void cg_flash_attention_gqa(cg_flash_attn_params* params, int num_kv_groups) {
    if (!params) {
        cgx_set_error("cg_flash_attention_gqa: params is NULL");
        return;
    }
    params->n_heads_k = num_kv_groups;
    cg_flash_attention_forward(params);
}

void cg_flash_attention_backward(cg_flash_attn_params* params) {
    (void)params;
    cgx_set_error("cg_flash_attention_backward: not implemented (inference-only library)");
}

void cg_flash_attention_backward_cpu(cg_flash_attn_params* params) {
    (void)params;
    cgx_set_error("cg_flash_attention_backward_cpu: not implemented (inference-only library)");
}

/* ------------------------------------------------------------- params */

/* Output buffers allocated by cg_flash_attn_params_new, freed with the
 * params (the reference leaks them, flash_attn.c:416-420). */
#define MAX_OWNED 256
static struct {
    cg_flash_attn_params* p;
    float* o;
    int dev;
} owned[MAX_OWNED];

cg_flash_attn_params* cg_flash_attn_params_new(cg_tensor* Q, cg_tensor* K, cg_tensor* V,
                                               cg_attention_mask_type mask_type,
                                               float dropout_prob) {
    if (!Q || !K || !V || Q->ndim != 4 || K->ndim != 4 || V->ndim != 4) {
        cgx_set_error("cg_flash_attn_params_new: Q, K, V must be 4-D [batch, seq, heads, d]");
        return NULL;
    }
    cg_flash_attn_params* p = (cg_flash_attn_params*)calloc(1, sizeof(*p));
    if (!p) return NULL;
    p->Q = Q->data;
    p->K = K->data;
    p->V = V->data;
    p->batch_size = Q->shape[0];
    p->seqlen_q = Q->shape[1];
    p->n_heads = Q->shape[2];
    p->d_head = Q->shape[3];
    p->seqlen_k = K->shape[1];
    p->n_heads_k = K->shape[2];
    p->scale = 1.0f / sqrtf((float)p->d_head);
    p->dropout_prob = dropout_prob;
    p->mask_type = mask_type;
    size_t n = (size_t)p->batch_size * p->seqlen_q * p->n_heads * p->d_head;
    int dev = Q->data && cgx_is_device_ptr(Q->data);
    float* o = dev ? (float*)cgx_malloc(n * sizeof(float)) : (float*)calloc(n ? n : 1, sizeof(float));
    if (!o || (dev && cgx_memset(o, 0, n * sizeof(float)))) {
        if (dev) cgx_free(o); else free(o);
        free(p);
        cgx_set_error("cg_flash_attn_params_new: cannot allocate the output");
        return NULL;
    }
    p->O = o;
    int slot = -1;
    for (int i = 0; i < MAX_OWNED && slot < 0; i++)
        if (!owned[i].p) slot = i;
    if (slot < 0) {
        if (dev) cgx_free(o); else free(o);
        free(p);
        cgx_set_error("cg_flash_attn_params_new: more than %d live params", MAX_OWNED);
        return NULL;
    }
    owned[slot].p = p;
    owned[slot].o = o;
    owned[slot].dev = dev;
    return p;
}

void cg_flash_attn_params_free(cg_flash_attn_params* params) {
    if (!params) return;
    for (int i = 0; i < MAX_OWNED; i++) {
        if (owned[i].p == params) {
            if (owned[i].dev) cgx_free(owned[i].o); else free(owned[i].o);
            owned[i].p = NULL;
            owned[i].o = NULL;
        }
    }
    free(params);
}

/* The launch shape of the GPU forward for one (batch, KV head): 32 query
 * rows per workgroup, 4 waves x 32 keys in flight, key splits chosen to
 * give >= 512 workgroups with >= 128 keys per split. */
cg_flash_attn_config cg_flash_attn_autotune(int seqlen_q, int seqlen_k, int d_head,
                                            int sm_count) {
    cg_flash_attn_config c;
    memset(&c, 0, sizeof(c));
    c.block_m = 32;
    c.block_n = 128;
    c.num_warps = 4;
    c.use_register_tile = true;
    c.sm_count = sm_count > 0 ? sm_count : 256;
    int chunks = seqlen_q > 0 ? (seqlen_q + 31) / 32 : 1;
    int splits = (512 + chunks - 1) / chunks;
    int max_splits = seqlen_k > 0 ? (seqlen_k + 127) / 128 : 1;
    if (splits > max_splits) splits = max_splits;
    c.split_k = splits < 1 ? 1 : splits;
    c.use_persistent = false;
    (void)d_head;
    return c;
}

/* LDS bytes of the GPU forward's workgroup for a (block_m query rows,
 * block_n keys in flight) tile: Q and V tiles padded to a multiple of 32
 * columns plus one, the score tile and three per-key statistics. */
size_t cg_flash_attn_shared_mem(int block_m, int block_n, int d_head) {
    if (block_m <= 0 || block_n <= 0 || d_head <= 0) return 0;
    size_t dp = (size_t)(d_head + 31) / 32 * 32 + 1;
    return ((size_t)block_m * dp + (size_t)block_n * dp + (size_t)block_n * 33 +
            3 * (size_t)block_n) * sizeof(float);
}

/* --------------------------------------------------------------- RoPE */

static int rope_one(float* x, int seqlen, int n_heads, int d_head, int off, float theta,
                    int slot) {
    size_t n = (size_t)seqlen * n_heads * d_head;
    if (cgx_is_device_ptr(x)) return cgk_rope(x, seqlen, n_heads, d_head, off, theta);
    float* d = (float*)cgx_scratch(slot, n * sizeof(float));
    if (!d || cgx_memcpy_h2d(d, x, n * sizeof(float)) ||
        cgk_rope(d, seqlen, n_heads, d_head, off, theta) ||
        cgx_memcpy_d2h(x, d, n * sizeof(float)))
        return -1;
    return 0;
}

void cg_apply_rope(float* Q, float* K, int seqlen, int n_heads, int d_head,
                   int position_offset, float rope_theta) {
    if (seqlen < 0 || n_heads < 0 || d_head < 0) {
        cgx_set_error("cg_apply_rope: negative size");
        return;
    }
    if (!seqlen || !n_heads || d_head < 2) return;
    if (cgx_ensure_init()) return;
    if (Q && rope_one(Q, seqlen, n_heads, d_head, position_offset, rope_theta, CGX_SLOT_IN0))
        return;
    if (K && rope_one(K, seqlen, n_heads, d_head, position_offset, rope_theta, CGX_SLOT_IN1))
        return;
    cgx_synchronize();
}

void cg_rope_precompute_freqs(float* cos_cache, float* sin_cache, int max_seqlen, int d_head,
                              float theta) {
    if (!cos_cache || !sin_cache || max_seqlen < 0 || d_head < 0) {
        cgx_set_error("cg_rope_precompute_freqs: invalid argument");
        return;
    }
    size_t n = (size_t)max_seqlen * (d_head / 2);
    if (!n) return;
    if (cgx_ensure_init()) return;
    int cd = cgx_is_device_ptr(cos_cache), sd = cgx_is_device_ptr(sin_cache);
    float* dc = cd ? cos_cache : (float*)cgx_scratch(CGX_SLOT_OUT0, n * 4);
    float* ds = sd ? sin_cache : (float*)cgx_scratch(CGX_SLOT_OUT1, n * 4);
    if (!dc || !ds || cgk_rope_freqs(dc, ds, max_seqlen, d_head, theta)) return;
    if (!cd && cgx_memcpy_d2h(cos_cache, dc, n * 4)) return;
    if (!sd && cgx_memcpy_d2h(sin_cache, ds, n * 4)) return;
    cgx_synchronize();
}

/* -------------------------------------------------------------- ALiBi */

void cg_alibi_slopes(float* slopes, int n_heads) {
    if (!slopes || n_heads < 0) {
        cgx_set_error("cg_alibi_slopes: invalid argument");
        return;
    }
    if (!n_heads) return;
    if (cgx_ensure_init()) return;
    int sd = cgx_is_device_ptr(slopes);
    float* d = sd ? slopes : (float*)cgx_scratch(CGX_SLOT_OUT0, (size_t)n_heads * 4);
    if (!d || cgk_alibi_slopes(d, n_heads)) return;
    if (!sd) cgx_memcpy_d2h(slopes, d, (size_t)n_heads * 4);
    else cgx_synchronize();
}

void cg_alibi_bias(float* bias, int seqlen_q, int seqlen_k, int n_heads, float* slopes) {
    if (!bias || !slopes || seqlen_q < 0 || seqlen_k < 0 || n_heads < 0) {
        cgx_set_error("cg_alibi_bias: invalid argument");
        return;
    }
    size_t n = (size_t)n_heads * seqlen_q * seqlen_k;
    if (!n) return;
    if (cgx_ensure_init()) return;
    const float* dsl = dev_view(slopes, (size_t)n_heads, CGX_SLOT_IN0);
    int bd = cgx_is_device_ptr(bias);
    float* db = bd ? bias : (float*)cgx_scratch(CGX_SLOT_OUT0, n * 4);
    if (!dsl || !db || cgk_alibi_bias(db, seqlen_q, seqlen_k, n_heads, dsl)) return;
    if (!bd) cgx_memcpy_d2h(bias, db, n * 4);
    else cgx_synchronize();
}
