/*
 * model.c -- the synthetic decoder stack of the verify path (INT4 weights
 * and KV cache in HBM).  Layer order and layouts follow the reference
 * (src/layers/transformer.c:26-149, src/layers/linear.c:53-98); every
 * linear layer is one MFMA GEMV launch with the RMSNorm / SwiGLU / residual
 * work fused around it (gemv.hip: RMSNorm folded into the activation side,
 * SwiGLU computed in the epilogue of the gate|up product, whose gate and up
 * column tiles are interleaved), attention reads the INT4 cache directly
 * (attn_dec.hip).  Per layer: 4 GEMVs and attention (+ split combine), with
 * RoPE and the KV append inside the attention launch (or, for tree forwards
 * of more than 16 rows, a launch of their own before it).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "cg_mi355x.h"
#include "cg_serialization.h"
#include "cgx_internal.h"

int cgk_embed_rope(const float* table, const int* tokens, int B, int M, int d, int V, float* x,
                   const int* pos0, const int* rel, int D, float theta, float* cs);
int cgk_attn_dec_rope(const float* qkv, int ldq, const float* rope, uint8_t* kc, uint8_t* vc,
                      float* ks, float* vs, int B, const int* nk, size_t seq_kbytes,
                      size_t seq_groups, int Nq, int H, int Hk, int D, float scale,
                      int mask_kind, const unsigned long long* anc, int tw, float* O,
                      float* stats);
int cgk_rope_append_batch(const float* qkv, int ld, int B, int M, int H, int Hk, int D, int gs,
                          const int* pos0, const int* rel, float theta, const float* cs,
                          float* q_out, uint8_t* kc, uint8_t* vc, float* ks, float* vs,
                          size_t seq_kbytes, size_t seq_groups);
int cgk_fill_normal(float* out, size_t n, uint64_t seed, uint32_t stream_id, float stddev);

enum { PRO_NONE = 0, PRO_RMSNORM = 1 };
enum { EPI_STORE = 0, EPI_ACCUMULATE = 1, EPI_SWIGLU = 2 };
enum { W_QKV = 0, W_O = 1, W_GU = 2, W_DOWN = 3, W_LM = 4 };

typedef struct {
    uint8_t* tiled;
    float* scales_t;
    int K, N;
    uint32_t sid;
    float smax;              /* max |scale|: the GEMM's row-scaling bound */
} lin_t;

typedef struct {
    lin_t w[4];
} layer_t;

#define CGX_MAX_BATCH 16

struct cgx_model {
    cgx_model_config c;
    uint64_t epoch;          /* bumped by every change of the cached positions */
    int nb;                  /* sequences (max_batch, at least 1) */
    int len[CGX_MAX_BATCH];  /* KV length of each sequence */
    uint64_t seed;
    float* embed;
    lin_t lm;
    int shared;              /* embed / lm_head borrowed from another model */
    int from_file;           /* weights read from a file (no seed behind them) */
    float* ones;             /* d_ff ones: the RMSNorm weights of a seeded model */
    float* nw;               /* [2 n_layers + 1][d]: each layer's attention and MLP
                              * RMSNorm weights, then the final one; NULL: all 1 */
    layer_t* layers;
    cg_kv_cache_int4* kv;
    int* tok;
    float *x, *qkv, *q, *attn, *gu, *logits;
    float* rope;             /* [rows][head_dim / 2] (cos, sin) of the step's positions */
    float *stats_x, *stats_g;  /* row statistics of x and of the SwiGLU output */
    float* stats_a;          /* of the attention output (head_dim 128: per head) */
};

static int nqkv(const cgx_model_config* c) { return (c->n_heads + 2 * c->n_kv_heads) * c->head_dim; }

static void lin_shape(const cgx_model_config* c, int which, int* K, int* N) {
    int d = c->d_model, hq = c->n_heads * c->head_dim;
    switch (which) {
        case W_QKV: *K = d; *N = nqkv(c); break;
        case W_O: *K = hq; *N = d; break;
        case W_GU: *K = d; *N = 2 * c->d_ff; break;
        case W_DOWN: *K = c->d_ff; *N = d; break;
        default: *K = d; *N = c->vocab; break;
    }
}

static uint32_t lin_sid(int layer, int which) {
    return which == W_LM ? 2u : (uint32_t)(16 * layer + 3 + which);
}

/* RMSNorm weights: i = 2 l (before attention of layer l), 2 l + 1 (before
 * its MLP), 2 n_layers (before the lm_head). */
static const float* norm_w(const cgx_model* m, int i) {
    return m->nw ? m->nw + (size_t)i * m->c.d_model : m->ones;
}

/* Seeded fp32 values -> reference-layout INT4 (flat) in tmp buffers. */
static int gen_flat(const cgx_model* m, uint32_t sid, int K, int N, float* tf, uint8_t* tq,
                    float* ts) {
    size_t n = (size_t)K * N;
    if (cgk_fill_normal(tf, n, m->seed, sid, m->c.init_std)) return -1;
    return cgk_int4_quantize(tf, (int)n, m->c.group_size, tq, ts);
}

/* ---------------------------------------------------------- model files */
/* Entry names (the fields of the reference's transformer block,
 * include/cg_transformer.h:41-50):
 *   embed [V, d] fp32;  norm [d] (final RMSNorm);  lm_head [d, V]
 *   layers.<l>.norm1, layers.<l>.norm2 [d]            RMSNorm weights
 *   layers.<l>.attn_qkv_proj [d, (H + 2 Hk) hd]      or attn_q_proj,
 *                                                    attn_k_proj, attn_v_proj
 *   layers.<l>.attn_o_proj [H hd, d]
 *   layers.<l>.mlp_gate_up [d, 2 ff]                 or mlp_gate, mlp_up
 *   layers.<l>.mlp_down [ff, d]
 * Matrices are fp32 (quantized at load with cg_quantize_int4's rule) or INT4
 * entries (host/model_file.c).  Missing norms are 1. */
static const char* const kQkvParts[3] = {"attn_q_proj", "attn_k_proj", "attn_v_proj"};
static const char* const kGuParts[2] = {"mlp_gate", "mlp_up"};

static void lin_name(int which, int layer, char* out) {
    static const char* const whole[4] = {"attn_qkv_proj", "attn_o_proj", "mlp_gate_up",
                                         "mlp_down"};
    if (which == W_LM)
        snprintf(out, 64, "lm_head");
    else
        snprintf(out, 64, "layers.%d.%s", layer, whole[which]);
}

/* The entries of matrix `which` of `layer`: the whole matrix, else its column
 * blocks.  Returns the block count (idx, widths filled; *kind 0 fp32 / 2
 * INT4), or -1 with the error set. */
static int lin_entries(const cgx_wfile* f, const cgx_model_config* c, int which, int layer,
                       int idx[3], int widths[3], int* kind, const char* who) {
    int K, N, nb = 1;
    lin_shape(c, which, &K, &N);
    char whole[64], parts[3][64];
    int np = 0, pw[3] = {0, 0, 0};
    lin_name(which, layer, whole);
    if (which == W_QKV) {
        np = 3;
        pw[0] = c->n_heads * c->head_dim;
        pw[1] = pw[2] = c->n_kv_heads * c->head_dim;
        for (int b = 0; b < 3; b++) snprintf(parts[b], 64, "layers.%d.%s", layer, kQkvParts[b]);
    } else if (which == W_GU) {
        np = 2;
        pw[0] = pw[1] = c->d_ff;
        for (int b = 0; b < 2; b++) snprintf(parts[b], 64, "layers.%d.%s", layer, kGuParts[b]);
    }
    idx[0] = cgx_wfile_find(f, whole);
    widths[0] = N;
    if (idx[0] < 0) {
        nb = np;
        for (int b = 0; b < np; b++) {
            idx[b] = cgx_wfile_find(f, parts[b]);
            widths[b] = pw[b];
            if (idx[b] < 0) nb = 0;
        }
        if (!nb) {
            if (np)
                cgx_set_error("%s: no entry %s, nor all of its blocks (%s, %s%s%s)", who, whole,
                              parts[0], parts[1], np > 2 ? ", " : "", np > 2 ? parts[2] : "");
            else
                cgx_set_error("%s: no entry %s", who, whole);
            return -1;
        }
    }
    *kind = cgx_wfile_matrix_kind(f, idx, widths, nb, K, c->group_size, who);
    return *kind < 0 ? -1 : nb;
}

/* Matrix `which` of `layer` from the file into the flat INT4 buffers tq, ts
 * (device): INT4 entries are copied, fp32 entries quantized on the device. */
static int file_flat(const cgx_wfile* f, const cgx_model_config* c, int which, int layer,
                     float* tf, uint8_t* tq, float* ts) {
    int idx[3], widths[3], kind, K, N;
    const int nb = lin_entries(f, c, which, layer, idx, widths, &kind, "cgx_model_load");
    if (nb < 0) return -1;
    lin_shape(c, which, &K, &N);
    const size_t n = (size_t)K * N, gs = (size_t)c->group_size;
    int rc;
    if (kind == 0) {
        float* h = (float*)malloc(n * 4);
        rc = !h || cgx_wfile_read_f32(f, idx, widths, nb, K, h) || cgx_memcpy_h2d(tf, h, n * 4) ||
             cgk_int4_quantize(tf, (int)n, c->group_size, tq, ts);
        free(h);
    } else {
        uint8_t* hd = (uint8_t*)malloc(n / 2);
        float* hs = (float*)malloc(n / gs * 4);
        rc = !hd || !hs || cgx_wfile_read_int4(f, idx, widths, nb, K, c->group_size, hd, hs) ||
             cgx_memcpy_h2d(tq, hd, n / 2) || cgx_memcpy_h2d(ts, hs, n / gs * 4);
        free(hd);
        free(hs);
    }
    if (rc && !cgx_last_error()[0]) cgx_set_error("cgx_model_load: out of memory");
    return rc ? -1 : 0;
}

static void norm_name(int i, int n_layers, char* out) {
    if (i == 2 * n_layers)
        snprintf(out, 64, "norm");
    else
        snprintf(out, 64, "layers.%d.norm%d", i / 2, 1 + (i & 1));
}

/* Every entry the model needs is present and well formed (directory only). */
static int check_file(const cgx_wfile* f, const cgx_model_config* c, int shared) {
    const char* who = "cgx_model_load";
    int idx[3], widths[3], kind;
    if (!shared) {
        const int ei = cgx_wfile_find(f, "embed");
        int ew = c->d_model;
        if (ei < 0) {
            cgx_set_error("%s: no entry embed", who);
            return -1;
        }
        const int kind_e = cgx_wfile_matrix_kind(f, &ei, &ew, 1, c->vocab, c->group_size, who);
        if (kind_e < 0) return -1;
        if (kind_e != 0) {
            cgx_set_error("%s: entry embed must be fp32 [%d, %d]", who, c->vocab, c->d_model);
            return -1;
        }
        if (lin_entries(f, c, W_LM, 0, idx, widths, &kind, who) < 0) return -1;
    }
    for (int l = 0; l < c->n_layers; l++)
        for (int w = 0; w < 4; w++)
            if (lin_entries(f, c, w, l, idx, widths, &kind, who) < 0) return -1;
    for (int i = 0; i <= 2 * c->n_layers; i++) {
        char nm[64];
        norm_name(i, c->n_layers, nm);
        if (cgx_wfile_vector(f, nm, c->d_model, who) == -2) return -1;
    }
    return 0;
}

static int make_lin(cgx_model* m, lin_t* L, int which, int layer, float* tf, uint8_t* tq,
                    float* ts, const cgx_wfile* f) {
    lin_shape(&m->c, which, &L->K, &L->N);
    L->sid = lin_sid(layer, which);
    size_t n = (size_t)L->K * L->N;
    L->tiled = (uint8_t*)cgx_malloc(n / 2);
    L->scales_t = (float*)cgx_malloc(n / m->c.group_size * 4);
    if (!L->tiled || !L->scales_t) return -1;
    if (f ? file_flat(f, &m->c, which, layer, tf, tq, ts)
          : gen_flat(m, L->sid, L->K, L->N, tf, tq, ts))
        return -1;
    if (cgk_int4_repack_mfma(tq, ts, L->K, L->N, m->c.group_size, which == W_GU, L->tiled,
                             L->scales_t))
        return -1;
    return cgk_absmax(L->scales_t, n / m->c.group_size, &L->smax);
}

static void free_lin(lin_t* L) {
    cgx_free(L->tiled);
    cgx_free(L->scales_t);
    L->tiled = NULL;
    L->scales_t = NULL;
}

static int check_config(const cgx_model_config* c) {
    int gs = c->group_size;
    if (c->n_layers < 1 || c->d_model < 1 || c->n_heads < 1 || c->n_kv_heads < 1 ||
        c->n_heads % c->n_kv_heads || c->head_dim < 2 || c->head_dim > 128 ||
        (c->head_dim & 1) || c->d_ff < 1 || c->vocab < 2 || gs < 16 || gs % 16 ||
        c->kv_group_size < 2 || (c->kv_group_size & 1) || c->head_dim % c->kv_group_size ||
        c->max_seq < 1 || c->max_tokens < 1 || c->max_tokens > c->max_seq ||
        c->max_batch < 0 || c->max_batch > CGX_MAX_BATCH) {
        cgx_set_error("cgx_model_new: invalid configuration");
        return -1;
    }
    for (int w = 0; w <= W_LM; w++) {
        int K, N;
        lin_shape(c, w, &K, &N);
        if (K % 256 || N % 16 || N % gs) {
            cgx_set_error("cgx_model_new: linear %d is %d x %d; the GEMV layout needs K %% 256 "
                          "== 0 and N a multiple of 16 and of group_size %d", w, K, N, gs);
            return -1;
        }
    }
    return 0;
}

/* ------------------------------------------------------ live handles */
/* The reference's decoder holds its models as void* (cg_speculative.h:33-34);
 * the driver accepts a pointer as a model only when it is a live handle. */
static cgx_model** g_live;
static int g_nlive, g_cap_live;

static int live_add(cgx_model* m) {
    if (g_nlive == g_cap_live) {
        int cap = g_cap_live ? 2 * g_cap_live : 16;
        cgx_model** p = (cgx_model**)realloc(g_live, (size_t)cap * sizeof(*p));
        if (!p) return -1;
        g_live = p;
        g_cap_live = cap;
    }
    g_live[g_nlive++] = m;
    return 0;
}

static void live_remove(const cgx_model* m) {
    for (int i = 0; i < g_nlive; i++)
        if (g_live[i] == m) {
            g_live[i] = g_live[--g_nlive];
            return;
        }
}

cgx_model* cgx_model_from_handle(const void* p) {
    for (int i = 0; p && i < g_nlive; i++)
        if (g_live[i] == p) return g_live[i];
    return NULL;
}

uint64_t cgx_model_epoch(const cgx_model* m) { return m ? m->epoch : 0; }

void cgx_model_free(cgx_model* m) {
    if (!m) return;
    live_remove(m);
    cgx_driver_forget_model(m);
    if (m->layers) {
        for (int l = 0; l < m->c.n_layers; l++)
            for (int w = 0; w < 4; w++) free_lin(&m->layers[l].w[w]);
        free(m->layers);
    }
    if (!m->shared) {
        cgx_free(m->embed);
        free_lin(&m->lm);
    }
    cgx_free(m->ones);
    cgx_free(m->nw);
    cg_kv_cache_int4_free(m->kv);
    cgx_free(m->tok);
    cgx_free(m->x);
    cgx_free(m->qkv);
    cgx_free(m->q);
    cgx_free(m->attn);
    cgx_free(m->gu);
    cgx_free(m->logits);
    cgx_free(m->rope);
    cgx_free(m->stats_x);
    cgx_free(m->stats_g);
    cgx_free(m->stats_a);
    free(m);
}

/* The model with seeded weights (f NULL) or the weights of file f. */
static cgx_model* build(const cgx_model_config* cfg, uint64_t seed, cgx_model* share_from,
                        const cgx_wfile* f) {
    if (cgx_ensure_init()) return NULL;
    cgx_model* m = (cgx_model*)calloc(1, sizeof(*m));
    if (!m) return NULL;
    m->c = *cfg;
    m->nb = cfg->max_batch > 0 ? cfg->max_batch : 1;
    m->seed = seed;
    m->from_file = f != NULL;
    const cgx_model_config* c = &m->c;
    int d = c->d_model, V = c->vocab, Mx = c->max_tokens * m->nb;   /* rows per forward */
    size_t maxn = 0;
    for (int w = 0; w <= W_LM; w++) {
        int K, N;
        lin_shape(c, w, &K, &N);
        if ((size_t)K * N > maxn) maxn = (size_t)K * N;
    }
    if ((size_t)V * d > maxn) maxn = (size_t)V * d;
    float* tf = (float*)cgx_malloc(maxn * 4);
    uint8_t* tq = (uint8_t*)cgx_malloc(maxn / 2 + 16);
    float* ts = (float*)cgx_malloc(maxn / c->group_size * 4 + 16);
    m->layers = (layer_t*)calloc((size_t)c->n_layers, sizeof(layer_t));
    int ok = tf && tq && ts && m->layers;
    if (ok && share_from) {
        m->shared = 1;
        m->embed = share_from->embed;
        m->lm = share_from->lm;
    } else if (ok) {
        m->embed = (float*)cgx_malloc((size_t)V * d * 4);
        ok = m->embed != NULL;
        if (ok && f) {
            const int ei = cgx_wfile_find(f, "embed");
            int ew = d;
            float* h = (float*)malloc((size_t)V * d * 4);
            ok = h && !cgx_wfile_read_f32(f, &ei, &ew, 1, V, h) &&
                 !cgx_memcpy_h2d(m->embed, h, (size_t)V * d * 4);
            free(h);
        } else if (ok) {
            ok = !cgk_fill_normal(m->embed, (size_t)V * d, seed, 1u, c->init_std);
        }
        ok = ok && !make_lin(m, &m->lm, W_LM, 0, tf, tq, ts, f);
    }
    for (int l = 0; ok && l < c->n_layers; l++)
        for (int w = 0; ok && w < 4; w++)
            ok = !make_lin(m, &m->layers[l].w[w], w, l, tf, tq, ts, f);
    if (ok) {
        int maxd = d > c->d_ff ? d : c->d_ff;
        const int nn = 2 * c->n_layers + 1;
        int any_norm = 0;
        for (int i = 0; f && i < nn; i++) {
            char nm[64];
            norm_name(i, c->n_layers, nm);
            any_norm |= cgx_wfile_find(f, nm) >= 0;
        }
        m->ones = (float*)cgx_malloc((size_t)maxd * 4);
        const size_t hn = any_norm ? (size_t)nn * d : (size_t)maxd;
        float* h = (float*)malloc(hn * 4);
        ok = m->ones && h;
        for (size_t i = 0; ok && i < hn; i++) h[i] = 1.0f;
        ok = ok && !cgx_memcpy_h2d(m->ones, h, (size_t)maxd * 4);
        if (ok && any_norm) {
            /* the file's norms; those it lacks stay 1 */
            for (int i = 0; ok && i < nn; i++) {
                char nm[64];
                norm_name(i, c->n_layers, nm);
                const int vi = cgx_wfile_find(f, nm);
                ok = vi < 0 || !cgx_wfile_read_vector(f, vi, h + (size_t)i * d, d);
            }
            m->nw = ok ? (float*)cgx_malloc(hn * 4) : NULL;
            ok = m->nw && !cgx_memcpy_h2d(m->nw, h, hn * 4);
        }
        free(h);
    }
    if (ok) {
        /* layer slot l * nb + b holds layer l of sequence b */
        m->kv = cg_kv_cache_int4_new(c->n_layers * m->nb, c->max_seq, c->n_kv_heads,
                                     c->head_dim, c->kv_group_size);
        m->tok = (int*)cgx_malloc((size_t)Mx * 4);
        m->x = (float*)cgx_malloc((size_t)Mx * d * 4);
        m->qkv = (float*)cgx_malloc((size_t)Mx * nqkv(c) * 4);
        m->q = (float*)cgx_malloc((size_t)Mx * c->n_heads * c->head_dim * 4);
        m->attn = (float*)cgx_malloc((size_t)Mx * c->n_heads * c->head_dim * 4);
        m->gu = (float*)cgx_malloc((size_t)Mx * c->d_ff * 4);      /* SwiGLU output */
        m->logits = (float*)cgx_malloc((size_t)Mx * V * 4);
        m->rope = (float*)cgx_malloc((size_t)Mx * c->head_dim * 4);
        m->stats_x = (float*)cgx_malloc((size_t)Mx * (d / 128 + 1) * 2 * 4);
        m->stats_g = (float*)cgx_malloc((size_t)Mx * (c->d_ff / 128 + 1) * 2 * 4);
        m->stats_a = (float*)cgx_malloc((size_t)Mx * c->n_heads * 2 * 4);
        ok = m->kv && m->tok && m->x && m->qkv && m->q && m->attn && m->gu && m->logits &&
             m->rope && m->stats_x && m->stats_g && m->stats_a;
    }
    if (ok) ok = !cgx_synchronize();
    cgx_free(tf);
    cgx_free(tq);
    cgx_free(ts);
    if (ok && live_add(m)) {
        cgx_set_error("cgx_model_new: out of memory");
        ok = 0;
    }
    if (!ok) {
        cgx_model_free(m);
        return NULL;
    }
    return m;
}

static int check_share(const cgx_model_config* cfg, const cgx_model* share_from,
                       const char* who) {
    if (share_from && (share_from->c.d_model != cfg->d_model ||
                       share_from->c.vocab != cfg->vocab ||
                       share_from->c.group_size != cfg->group_size)) {
        cgx_set_error("%s: share_from has another d_model / vocab / group size", who);
        return -1;
    }
    return 0;
}

cgx_model* cgx_model_new(const cgx_model_config* cfg, uint64_t seed, cgx_model* share_from) {
    if (!cfg || check_config(cfg) || check_share(cfg, share_from, "cgx_model_new")) return NULL;
    return build(cfg, seed, share_from, NULL);
}

cgx_model* cgx_model_load(const cgx_model_config* cfg, const char* path, cgx_model* share_from) {
    if (!cfg || !path) {
        cgx_set_error("cgx_model_load: NULL argument");
        return NULL;
    }
    if (check_config(cfg) || check_share(cfg, share_from, "cgx_model_load")) return NULL;
    cgx_wfile* f = cgx_wfile_open(path, "cgx_model_load");
    if (!f) return NULL;
    cgx_model* m = NULL;
    cgx_clear_error();
    if (!check_file(f, cfg, share_from != NULL)) m = build(cfg, 0, share_from, f);
    cgx_wfile_close(f);
    return m;
}

/* Directory entry of a model file being written. */
static void put_entry(cg_tensor_entry* e, int* k, uint64_t* off, const char* name, int ndim,
                      int s0, int s1, int dtype, int gs, uint64_t bytes) {
    cg_tensor_entry* x = &e[(*k)++];
    memset(x, 0, sizeof(*x));
    snprintf(x->name, sizeof(x->name), "%s", name);
    x->ndim = ndim;
    x->shape[0] = s0;
    x->shape[1] = ndim > 1 ? s1 : 0;
    x->shape[7] = gs;
    x->dtype = dtype;
    x->offset = *off;
    x->size_bytes = bytes;
    *off += bytes;
}

/* Matrix `which` (of `layer`) of the model in the reference's flat form:
 * fp32 (the seeded values before quantization; tf) or nibbles and scales. */
static int lin_host(cgx_model* m, const lin_t* L, int which, int fp32, float* tf, uint8_t* tq,
                    float* ts, void* hdata, float* hscales) {
    const size_t n = (size_t)L->K * L->N, gs = (size_t)m->c.group_size;
    if (fp32)
        return cgk_fill_normal(tf, n, m->seed, L->sid, m->c.init_std) ||
               cgx_memcpy_d2h(hdata, tf, n * 4) ? -1 : 0;
    return cgk_int4_unpack_mfma(L->tiled, L->scales_t, L->K, L->N, m->c.group_size,
                                which == W_GU, tq, ts) ||
           cgx_memcpy_d2h(hdata, tq, n / 2) || cgx_memcpy_d2h(hscales, ts, n / gs * 4) ? -1 : 0;
}

int cgx_model_save(cgx_model* m, const char* path, int fp32) {
    if (!m || !path) {
        cgx_set_error("cgx_model_save: NULL argument");
        return -1;
    }
    if (fp32 && m->from_file) {
        cgx_set_error("cgx_model_save: fp32 weights exist only for seeded models (this one was "
                      "loaded from a file; save it as INT4)");
        return -1;
    }
    const cgx_model_config* c = &m->c;
    const int L = c->n_layers, d = c->d_model, V = c->vocab, gs = c->group_size;
    const int nmat = 4 * L + (m->shared ? 0 : 1);
    const int nent = (m->shared ? 0 : 1) + 2 * L + 1 + nmat * (fp32 ? 1 : 2);
    cg_tensor_entry* e = (cg_tensor_entry*)calloc((size_t)nent, sizeof(*e));
    if (!e) {
        cgx_set_error("cgx_model_save: out of memory");
        return -1;
    }
    int k = 0;
    uint64_t off = sizeof(cg_model_header) + (uint64_t)nent * sizeof(cg_tensor_entry);
    size_t maxn = 0;
    if (!m->shared) put_entry(e, &k, &off, "embed", 2, V, d, 0, 0, (uint64_t)V * d * 4);
    for (int i = 0; i <= 2 * L; i++) {
        char nm[64];
        norm_name(i, L, nm);
        put_entry(e, &k, &off, nm, 1, d, 0, 0, 0, (uint64_t)d * 4);
    }
    for (int j = 0; j < nmat; j++) {
        const int which = j < 4 * L ? j % 4 : W_LM, layer = j / 4;
        int K, N;
        char nm[64], sn[80];
        lin_shape(c, which, &K, &N);
        lin_name(which, layer, nm);
        const uint64_t n = (uint64_t)K * N;
        if (n > maxn) maxn = (size_t)n;
        if (fp32) {
            put_entry(e, &k, &off, nm, 2, K, N, 0, 0, n * 4);
        } else {
            put_entry(e, &k, &off, nm, 2, K, N, 2, gs, n / 2);
            snprintf(sn, sizeof(sn), "%s.scales", nm);
            put_entry(e, &k, &off, sn, 1, (int)(n / gs), 0, 0, 0, n / gs * 4);
        }
    }
    FILE* f = fopen(path, "wb");
    if (!f) {
        free(e);
        cgx_set_error("cgx_model_save: cannot open %s", path);
        return -1;
    }
    cg_model_header h;
    memset(&h, 0, sizeof(h));
    h.magic = CG_MODEL_MAGIC;
    h.version = 1;
    h.num_tensors = (uint32_t)nent;
    h.total_size = off;
    int rc = fwrite(&h, sizeof(h), 1, f) == 1 &&
                     fwrite(e, sizeof(*e), (size_t)nent, f) == (size_t)nent ? 0 : -1;
    free(e);
    /* data in directory order */
    const size_t hbytes = maxn * (fp32 ? 4 : 1) > (size_t)V * d * 4 ? maxn * (fp32 ? 4 : 1)
                                                                    : (size_t)V * d * 4;
    void* hd = malloc(hbytes);
    float* hs = (float*)malloc(maxn / (size_t)gs * 4 + 4);
    float* tf = fp32 ? (float*)cgx_malloc(maxn * 4) : NULL;
    uint8_t* tq = fp32 ? NULL : (uint8_t*)cgx_malloc(maxn / 2);
    float* ts = fp32 ? NULL : (float*)cgx_malloc(maxn / (size_t)gs * 4);
    if (!rc && (!hd || !hs || (fp32 ? !tf : (!tq || !ts)))) rc = -1;
    if (!rc && !m->shared)
        rc = cgx_memcpy_d2h(hd, m->embed, (size_t)V * d * 4) ||
             fwrite(hd, 4, (size_t)V * d, f) != (size_t)V * d ? -1 : 0;
    for (int i = 0; !rc && i <= 2 * L; i++)
        rc = cgx_memcpy_d2h(hd, norm_w(m, i), (size_t)d * 4) ||
             fwrite(hd, 4, (size_t)d, f) != (size_t)d ? -1 : 0;
    for (int j = 0; !rc && j < nmat; j++) {
        const int which = j < 4 * L ? j % 4 : W_LM;
        const lin_t* Lw = which == W_LM ? &m->lm : &m->layers[j / 4].w[which];
        const size_t n = (size_t)Lw->K * Lw->N;
        rc = lin_host(m, Lw, which, fp32, tf, tq, ts, hd, hs);
        if (!rc && fp32) rc = fwrite(hd, 4, n, f) == n ? 0 : -1;
        if (!rc && !fp32)
            rc = fwrite(hd, 1, n / 2, f) == n / 2 &&
                         fwrite(hs, 4, n / (size_t)gs, f) == n / (size_t)gs ? 0 : -1;
    }
    free(hd);
    free(hs);
    cgx_free(tf);
    cgx_free(tq);
    cgx_free(ts);
    if (fclose(f) || rc) {
        if (!cgx_last_error()[0] || !rc) cgx_set_error("cgx_model_save: write to %s failed", path);
        return -1;
    }
    return 0;
}

float* cgx_model_logits(cgx_model* m) { return m ? m->logits : NULL; }

int cgx_model_get_config(const cgx_model* m, cgx_model_config* out) {
    if (!m || !out) {
        cgx_set_error("cgx_model_get_config: NULL argument");
        return -1;
    }
    *out = m->c;
    return 0;
}
int cgx_model_len(const cgx_model* m) {
    if (!m) return -1;
    return m->nb == 1 ? m->kv->current_len : m->len[0];
}
int cgx_model_batch(const cgx_model* m) { return m ? m->nb : -1; }
cg_kv_cache_int4* cgx_model_kv(cgx_model* m) { return m ? m->kv : NULL; }

int cgx_model_len_seq(const cgx_model* m, int seq) {
    if (!m || seq < 0 || seq >= m->nb) {
        cgx_set_error("cgx_model_len_seq: invalid sequence");
        return -1;
    }
    return m->len[seq];
}

int cgx_model_truncate_seq(cgx_model* m, int seq, int len) {
    if (!m || seq < 0 || seq >= m->nb || len < 0 || len > m->len[seq]) {
        cgx_set_error("cgx_model_truncate_seq: invalid sequence or length");
        return -1;
    }
    m->len[seq] = len;
    if (seq == 0) m->kv->current_len = len;
    m->epoch++;
    return 0;
}

int cgx_model_truncate(cgx_model* m, int len) {
    if (!m) {
        cgx_set_error("cgx_model_truncate: NULL model");
        return -1;
    }
    if (cgx_kv_cache_int4_truncate(m->kv, len)) return -1;
    m->len[0] = len;
    m->epoch++;
    return 0;
}

static size_t kv_layer_bytes(const cg_kv_cache_int4* c) {
    return (size_t)c->max_seq_len * c->n_heads * (c->head_dim / 2);
}

static size_t kv_layer_groups(const cg_kv_cache_int4* c) {
    return (size_t)c->max_seq_len * c->n_heads * (c->head_dim / c->group_size);
}

/* RoPE and the cache append inside the attention launch (1), or as a launch
 * of their own before it (0; a test hook: both must give the same cache). */
static int g_fused_attention = 1;

/* The attention writes the row statistics of its output for the O GEMM (1),
 * or the GEMM computes them in a pass of its own (0; a test hook: the same
 * row factors, so the same bits). */
static int g_attention_stats = 1;

int cgx_decoder_attention_stats(int on) {
    const int old = g_attention_stats;
    if (on >= 0) g_attention_stats = on != 0;
    return old;
}

int cgx_decoder_fused_attention(int on) {
    const int old = g_fused_attention;
    if (on >= 0) g_fused_attention = on != 0;
    return old;
}

/* Row statistics handed from one GEMM's epilogue to the next GEMM (rows
 * >= GEMM_MIN_ROWS): [rows][width / 128][2] partial (max|y * nw|, sum y^2). */
typedef struct {
    const float* in;      /* statistics of this linear's input, or NULL */
    int nin;
    float* out;           /* statistics of its output for the next linear, or NULL */
    const float* nw_next; /* the next linear's RMSNorm weights */
    int produced;         /* set when `out` was written */
} stats_t;

/* Rows from which a linear layer takes the GEMM: from 16 rows the GEMM's
 * shared activation tiles beat the GEMV, whose 16-row instance needs a hi and
 * a lo MFMA per tile (the tree draft's 16-row levels, 4096 x 128256 lm_head
 * included: tree verify 12.38 -> 12.17 ms a step). */
#define GEMM_MIN_ROWS 16

/* One linear layer over R rows: the GEMM from GEMM_MIN_ROWS rows on (one
 * pass over the weight), the GEMV below (it streams the weight once per 16
 * rows). */
static int linear(const lin_t* L, const float* x, int ldx, int R, float* y, int ldy, int pro,
                  const float* nw, float eps, int epi, int gs, stats_t* st) {
    if (st) st->produced = 0;
    if (R >= GEMM_MIN_ROWS && cgk_gemm_int4_supported(R, L->K, L->N, gs, epi == EPI_SWIGLU)) {
        const int nout = epi == EPI_SWIGLU ? L->N / 2 : L->N;
        float* so = st && st->out && nout % 128 == 0 ? st->out : NULL;
        if (cgk_gemm_int4(x, ldx, R, L->K, L->N, gs, L->tiled, L->scales_t, L->smax, y, ldy,
                          pro, nw, eps, epi, st ? st->in : NULL, st ? st->nin : 0, so,
                          st ? st->nw_next : NULL))
            return -1;
        if (so) st->produced = 1;
        return 0;
    }
    return cgk_gemv_mfma(x, ldx, R, L->K, L->N, gs, L->tiled, L->scales_t, y, ldy, pro, nw,
                         eps, epi);
}

/* Forward of B sequences (0..B-1), M tokens each; tr: the rows are tree
 * nodes (rotary positions and the tree mask of cgx_tree_rows), else a chain. */
static int forward_rows(cgx_model* m, int B, const int* tokens, int M, int n_logits,
                        float* logits, size_t ldl, const cgx_tree_rows* tr) {
    const cgx_model_config* c = &m->c;
    if (!tokens || M < 1 || M > c->max_tokens || n_logits < 0 || n_logits > M) {
        cgx_set_error("cgx_model_forward: invalid argument (M=%d, n_logits=%d)", M, n_logits);
        return -1;
    }
    if (tr && (M > 64 || tr->tw < M || tr->tw > 64)) {
        cgx_set_error("cgx_model_forward_tree: %d rows in a window of %d (at most 64)", M,
                      tr->tw);
        return -1;
    }
    cg_kv_cache_int4* kv = m->kv;
    /* a single-sequence cache may have been moved through cgx_model_kv */
    if (m->nb == 1) m->len[0] = kv->current_len;
    int pos0[CGX_MAX_BATCH], nk[CGX_MAX_BATCH];
    for (int b = 0; b < B; b++) {
        pos0[b] = m->len[b];
        nk[b] = pos0[b] + M;
        if (nk[b] > c->max_seq) {
            cgx_set_error("cgx_model_forward: KV cache full (%d + %d > %d)", pos0[b], M,
                          c->max_seq);
            return -1;
        }
    }
    const int R = B * M;
    const int* dtok = tokens;
    if (!cgx_is_device_ptr(tokens)) {
        if (cgx_memcpy_h2d(m->tok, tokens, (size_t)R * 4)) return -1;
        dtok = m->tok;
    }
    const int d = c->d_model, H = c->n_heads, Hk = c->n_kv_heads, hd = c->head_dim;
    const int hq = H * hd, gs = c->group_size, ff = c->d_ff, nq = nqkv(c);
    const float eps = c->norm_eps, scale = 1.0f / sqrtf((float)hd);
    const size_t lb = kv_layer_bytes(kv), lg = kv_layer_groups(kv);
    int xs_ok = 0;     /* m->stats_x holds the statistics of m->x */
    const int mask = tr ? CGK_MASK_TREE : CGK_MASK_CAUSAL_ALIGNED;
    const int batched = cgk_attn_dec_supported(hd, kv->group_size, 1, mask);
    /* RoPE and the cache append run inside the attention launch for up to 16
     * rows a sequence (chains, draft levels: the new keys are one more key
     * split, staged by its blocks); the 64-row tree forward keeps a launch of
     * its own, since there the extra split and its staging of 128 rows cost
     * more than the launch (C5: 13.6 -> 14.6 ms a step).  The rotary table of
     * the step's positions is filled with the embedding rows either way. */
    const int fused = batched && M <= 16 && g_fused_attention;
    if (cgk_embed_rope(m->embed, dtok, B, M, d, c->vocab, m->x, pos0, tr ? tr->rel : NULL, hd,
                       c->rope_theta, m->rope))
        return -1;
    if (tr && !batched) {
        cgx_set_error("cgx_model_forward_tree: head_dim %d / KV group %d not supported", hd,
                      kv->group_size);
        return -1;
    }
    for (int b = 0; tr && b < B; b++)
        if (pos0[b] + M < tr->tw) {
            cgx_set_error("cgx_model_forward_tree: window %d above the cache length", tr->tw);
            return -1;
        }
    for (int l = 0; l < c->n_layers; l++) {
        const lin_t* w = m->layers[l].w;
        /* layer l of sequence b: slot l * nb + b */
        const size_t slot = (size_t)l * m->nb;
        uint8_t* kc = kv->k_cache + lb * slot;
        uint8_t* vc = kv->v_cache + lb * slot;
        float* ks = kv->k_scales + lg * slot;
        float* vs = kv->v_scales + lg * slot;
        stats_t sq = {xs_ok ? m->stats_x : NULL, d / 128, NULL, NULL, 0};
        if (linear(&w[W_QKV], m->x, d, R, m->qkv, nq, PRO_RMSNORM, norm_w(m, 2 * l), eps,
                   EPI_STORE, gs, &sq))
            return -1;
        /* the attention leaves the O GEMM's row statistics (head_dim 128: one
         * entry per head), which then needs no pass of its own over them */
        float* as =
            batched && hd == 128 && R >= GEMM_MIN_ROWS && g_attention_stats ? m->stats_a : NULL;
        if (fused) {
            if (cgk_attn_dec_rope(m->qkv, nq, m->rope, kc, vc, ks, vs, B, nk, lb, lg, M, H, Hk,
                                  hd, scale, mask, tr ? tr->anc : NULL, tr ? tr->tw : M,
                                  m->attn, as))
                return -1;
        } else if (cgk_rope_append_batch(m->qkv, nq, B, M, H, Hk, hd, kv->group_size, pos0,
                                         tr ? tr->rel : NULL, c->rope_theta, m->rope, m->q, kc,
                                         vc, ks, vs, lb, lg)) {
            return -1;
        } else if (batched) {
            if (cgk_attn_dec_batch(m->q, kc, vc, ks, vs, B, nk, lb, lg, M, H, Hk, hd, scale,
                                   mask, tr ? tr->anc : NULL, tr ? tr->tw : M, m->attn, as))
                return -1;
        } else {
            for (int b = 0; b < B; b++)
                if (cgk_attention(m->q + (size_t)b * M * hq, 1, kc + lb * b, vc + lb * b,
                                  ks + lg * b, vs + lg * b, kv->group_size, NULL, NULL, 1, M,
                                  nk[b], H, Hk, hd, scale, CGK_MASK_CAUSAL_ALIGNED, 0, NULL,
                                  NULL, m->attn + (size_t)b * M * hq, NULL))
                    return -1;
        }
        /* o -> (x) -> gate|up -> (g) -> down -> (x) -> next qkv / lm_head: each
         * reduction leaves the row statistics its consumer needs */
        stats_t so = {as, H, m->stats_x, norm_w(m, 2 * l + 1), 0};
        if (linear(&w[W_O], m->attn, hq, R, m->x, d, PRO_NONE, NULL, 0.0f, EPI_ACCUMULATE,
                   gs, &so))
            return -1;
        stats_t sg = {so.produced ? m->stats_x : NULL, d / 128, m->stats_g, NULL, 0};
        if (linear(&w[W_GU], m->x, d, R, m->gu, ff, PRO_RMSNORM, norm_w(m, 2 * l + 1), eps,
                   EPI_SWIGLU, gs, &sg))
            return -1;
        /* the next consumer of x: layer l + 1's attention norm, or the final one */
        stats_t sd = {sg.produced ? m->stats_g : NULL, ff / 128, m->stats_x,
                      norm_w(m, 2 * l + 2), 0};
        if (linear(&w[W_DOWN], m->gu, ff, R, m->x, d, PRO_NONE, NULL, 0.0f, EPI_ACCUMULATE, gs,
                   &sd))
            return -1;
        xs_ok = sd.produced;
    }
    float* out = logits ? logits : m->logits;
    if (!ldl) ldl = (size_t)n_logits * c->vocab;
    if (n_logits == M && ldl == (size_t)M * c->vocab) {
        /* every row, sequences in order */
        stats_t sl = {xs_ok ? m->stats_x : NULL, d / 128, NULL, NULL, 0};
        if (linear(&m->lm, m->x, d, R, out, c->vocab, PRO_RMSNORM, norm_w(m, 2 * c->n_layers),
                   eps, EPI_STORE, gs, &sl))
            return -1;
    } else if (n_logits == 1) {
        /* the last row of each sequence: rows M-1, 2M-1, ... */
        if (cgk_gemv_mfma(m->x + (size_t)(M - 1) * d, M * d, B, d, c->vocab, gs, m->lm.tiled,
                          m->lm.scales_t, out, (int)ldl, PRO_RMSNORM,
                          norm_w(m, 2 * c->n_layers), eps, EPI_STORE))
            return -1;
    } else if (n_logits > 0) {
        for (int b = 0; b < B; b++)
            if (cgk_gemv_mfma(m->x + ((size_t)b * M + M - n_logits) * d, d, n_logits, d,
                              c->vocab, gs, m->lm.tiled, m->lm.scales_t,
                              out + (size_t)b * ldl, c->vocab, PRO_RMSNORM,
                              norm_w(m, 2 * c->n_layers), eps, EPI_STORE))
                return -1;
    }
    for (int b = 0; b < B; b++) m->len[b] = pos0[b] + M;
    kv->current_len = m->len[0];
    m->epoch++;
    return 0;
}

int cgx_model_forward(cgx_model* m, const int* tokens, int M, int n_logits, float* logits) {
    if (!m) {
        cgx_set_error("cgx_model_forward: NULL model");
        return -1;
    }
    return forward_rows(m, 1, tokens, M, n_logits, logits, 0, NULL);
}

int cgx_model_forward_batch(cgx_model* m, const int* tokens, int M, int n_logits,
                            float* logits) {
    if (!m) {
        cgx_set_error("cgx_model_forward_batch: NULL model");
        return -1;
    }
    return forward_rows(m, m->nb, tokens, M, n_logits, logits, 0, NULL);
}

int cgx_model_forward_batch_ld(cgx_model* m, const int* tokens, int M, int n_logits,
                               float* logits, size_t ld) {
    if (!m) {
        cgx_set_error("cgx_model_forward_batch: NULL model");
        return -1;
    }
    return forward_rows(m, m->nb, tokens, M, n_logits, logits, ld, NULL);
}

/* Tree forward of every sequence: M rows each (device or host tokens
 * [B][M]), logits of every row at logits + (b * M + i) * vocab (ldl 0) or
 * with row stride ... : sequence b's rows at logits + b * ldl. */
int cgx_model_forward_tree(cgx_model* m, const int* tokens, int M, const cgx_tree_rows* tr,
                           float* logits, size_t ldl) {
    if (!m || !tr) {
        cgx_set_error("cgx_model_forward_tree: NULL argument");
        return -1;
    }
    return forward_rows(m, m->nb, tokens, M, logits ? M : 0, logits, ldl, tr);
}

int cgx_model_forward_tree1(cgx_model* m, const int* tokens, int M, const cgx_tree_rows* tr,
                            float* logits) {
    if (!m || !tr) {
        cgx_set_error("cgx_model_forward_tree1: NULL argument");
        return -1;
    }
    return forward_rows(m, 1, tokens, M, logits ? M : 0, logits, 0, tr);
}

int cgx_model_forward_tree_rows(cgx_model* m, const int* tokens, int M, const int* rel,
                                const unsigned long long* anc, int tw, float* logits) {
    if (!m || !rel || !anc || M < 1 || M > 64) {
        cgx_set_error("cgx_model_forward_tree_rows: invalid argument");
        return -1;
    }
    cgx_tree_rows tr;
    memset(&tr, 0, sizeof(tr));
    for (int i = 0; i < M; i++) {
        tr.rel[i] = rel[i];
        tr.anc[i] = anc[i];
    }
    tr.tw = tw;
    return forward_rows(m, m->nb, tokens, M, M, logits, 0, &tr);
}

int cgx_model_compact_tree(cgx_model* m, const cgx_tree_shape* t, const int* len0,
                           const int* nacc_dev, const int* path_dev, const int* nacc_host) {
    if (!m || !t || !len0 || !nacc_host) {
        cgx_set_error("cgx_model_compact_tree: invalid argument");
        return -1;
    }
    m->epoch++;
    cg_kv_cache_int4* kv = m->kv;
    const int B = m->nb;
    for (int b = 0; b < B; b++)
        if (nacc_host[b] < 0 || nacc_host[b] > t->depth || len0[b] + 1 + nacc_host[b] > m->len[b]) {
            cgx_set_error("cgx_model_compact_tree: sequence %d: %d accepted past %d + %d cached",
                          b, nacc_host[b], len0[b], m->len[b] - len0[b]);
            return -1;
        }
    if (cgk_kv_compact(t, B, len0, nacc_dev, path_dev, m->c.n_layers, m->nb, kv->k_cache,
                       kv->v_cache, kv->k_scales, kv->v_scales,
                       kv->n_heads * (kv->head_dim / 2), kv->n_heads * (kv->head_dim / kv->group_size),
                       kv_layer_bytes(kv), kv_layer_groups(kv)))
        return -1;
    for (int b = 0; b < B; b++) m->len[b] = len0[b] + 1 + nacc_host[b];
    kv->current_len = m->len[0];
    return 0;
}

int cgx_model_fill_context(cgx_model* m, int len, uint64_t seed) {
    if (!m || len < 0 || len > m->c.max_seq) {
        cgx_set_error("cgx_model_fill_context: invalid length");
        return -1;
    }
    cg_kv_cache_int4* kv = m->kv;
    m->epoch++;
    if (!len) {
        for (int b = 0; b < m->nb; b++) m->len[b] = 0;
        return cgx_kv_cache_int4_set_len(kv, 0);
    }
    size_t n = (size_t)len * kv->n_heads * kv->head_dim;
    float* k = (float*)cgx_malloc(n * 4);
    float* v = (float*)cgx_malloc(n * 4);
    int rc = (k && v) ? 0 : -1;
    for (int l = 0; !rc && l < kv->num_layers; l++) {
        rc = cgk_fill_normal(k, n, seed, 0x40000000u + 2u * (uint32_t)l, 1.0f) ||
             cgk_fill_normal(v, n, seed, 0x40000001u + 2u * (uint32_t)l, 1.0f) ||
             cgx_kv_cache_int4_write(kv, l, 0, k, v, len);
    }
    if (!rc) rc = cgx_synchronize();
    cgx_free(k);
    cgx_free(v);
    if (!rc) rc = cgx_kv_cache_int4_set_len(kv, len);
    if (!rc)
        for (int b = 0; b < m->nb; b++) m->len[b] = len;
    return rc ? -1 : 0;
}

int cgx_model_export(cgx_model* m, int layer, int which, uint8_t* data, float* scales) {
    if (!m || !data || !scales || which < 0 || which > W_LM ||
        (which != W_LM && (layer < 0 || layer >= m->c.n_layers))) {
        cgx_set_error("cgx_model_export: invalid argument");
        return -1;
    }
    const lin_t* L = which == W_LM ? &m->lm : &m->layers[layer].w[which];
    const size_t n = (size_t)L->K * L->N;
    uint8_t* tq = (uint8_t*)cgx_malloc(n / 2 + 16);
    float* ts = (float*)cgx_malloc(n / m->c.group_size * 4 + 16);
    int rc = (tq && ts) ? 0 : -1;
    if (!rc) rc = lin_host(m, L, which, 0, NULL, tq, ts, data, scales);
    cgx_free(tq);
    cgx_free(ts);
    return rc ? -1 : 0;
}

int cgx_fill_normal_dev(float* out, size_t n, uint64_t seed, uint32_t stream_id,
                        float stddev) {
    if (!out) {
        cgx_set_error("cgx_fill_normal_dev: NULL output");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    if (cgk_fill_normal(out, n, seed, stream_id, stddev)) return -1;
    return cgx_synchronize();
}
