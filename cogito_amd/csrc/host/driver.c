/*
 * driver.c -- cogito's speculative-decoding driver API over device-resident
 * models (cgx_model handles in the decoder's draft_model / target_model):
 *
 *   cg_draft_generate          include/cg_speculative.h:91-94    (declared only)
 *   cg_target_verify           include/cg_speculative.h:99-103   (declared only)
 *   cg_speculative_step        include/cg_speculative.h:82-86    (declared only)
 *   cg_speculative_generate    include/cg_speculative.h:71-77    (declared only)
 *   cg_forward_tree_attention  include/cg_speculative.h:128-130  (declared only)
 *   cg_eagle_generate_tree     src/inference/speculative.c:244-262 (a stub there)
 *   cg_eagle_compute_branching include/cg_speculative.h:160       (declared only)
 *
 * Sequences.  input_ids holds the token ids so far as floats (the form
 * cg_token_tree_to_tensor produces), in host or device memory.  The driver
 * remembers which tokens each model's KV cache holds; before a call it cuts
 * the cache to the longest prefix it shares with input_ids and runs the rest,
 * so any input_ids is served and a growing sequence reuses the cache.  A
 * cache changed behind the driver's back (any cgx_model_* call) is detected
 * by the model's change counter and recomputed from position 0.
 *
 * Randomness.  Every draw comes from the reference's global LCG in the order
 * a sequential implementation makes them (speculative.c:11-12): one per
 * drafted token, then one per accept test and one for the token that follows
 * the accepted drafts (decision D6).  Draws are taken ahead for the kernels
 * and the LCG is set back to the state after the draws actually consumed.
 *
 * Nothing here computes on the CPU: the forwards, the samplers and the
 * verify run in the HIP kernels; host code moves ids, draws and results.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "cg_mi355x.h"
#include "cg_speculative.h"
#include "cgx_internal.h"

/* ------------------------------------------------- what each cache holds */

typedef struct {
    const cgx_model* m;
    uint64_t epoch;    /* the model's change counter when tok[] was last right */
    int* tok;
    int len, cap;
} hist_t;

static hist_t* g_hist;
static int g_nhist, g_caphist;

static hist_t* hist_of(const cgx_model* m) {
    for (int i = 0; i < g_nhist; i++)
        if (g_hist[i].m == m) return &g_hist[i];
    if (g_nhist == g_caphist) {
        int cap = g_caphist ? 2 * g_caphist : 8;
        hist_t* p = (hist_t*)realloc(g_hist, (size_t)cap * sizeof(*p));
        if (!p) {
            cgx_set_error("speculative driver: out of memory");
            return NULL;
        }
        g_hist = p;
        g_caphist = cap;
    }
    hist_t* h = &g_hist[g_nhist++];
    memset(h, 0, sizeof(*h));
    h->m = m;
    h->epoch = ~(uint64_t)0;
    return h;
}

void cgx_driver_forget_model(const cgx_model* m) {
    for (int i = 0; i < g_nhist; i++)
        if (g_hist[i].m == m) {
            free(g_hist[i].tok);
            g_hist[i] = g_hist[--g_nhist];
            return;
        }
}

static int hist_set(hist_t* h, const int* a, int na, const int* b, int nb) {
    if (na + nb > h->cap) {
        int cap = na + nb + 64;
        int* p = (int*)realloc(h->tok, (size_t)cap * sizeof(int));
        if (!p) {
            cgx_set_error("speculative driver: out of memory");
            return -1;
        }
        h->tok = p;
        h->cap = cap;
    }
    if (a && a != h->tok) memmove(h->tok, a, (size_t)na * sizeof(int));
    if (nb) memcpy(h->tok + na, b, (size_t)nb * sizeof(int));
    h->len = na + nb;
    h->epoch = cgx_model_epoch(h->m);
    return 0;
}

/* Cut m's cache to the longest prefix shared with ids[0..n) and run the
 * remaining tokens, so that it holds exactly ids[0..n). */
static int sync_prefix(cgx_model* m, const int* ids, int n) {
    hist_t* h = hist_of(m);
    if (!h) return -1;
    cgx_model_config c;
    cgx_model_get_config(m, &c);
    if (n > c.max_seq) {
        cgx_set_error("speculative driver: %d tokens exceed the KV cache (%d)", n, c.max_seq);
        return -1;
    }
    const int len = cgx_model_len(m);
    if (h->epoch != cgx_model_epoch(m) || h->len != len) h->len = 0;   /* unknown contents */
    int k = 0;
    while (k < h->len && k < n && h->tok[k] == ids[k]) k++;
    if (k != len && cgx_model_truncate(m, k)) return -1;
    for (int i = k; i < n; i += c.max_tokens) {
        const int M = n - i < c.max_tokens ? n - i : c.max_tokens;
        if (cgx_model_forward(m, ids + i, M, 0, NULL)) {
            h->len = 0;
            h->epoch = ~(uint64_t)0;
            return -1;
        }
    }
    return hist_set(h, ids, n, NULL, 0);
}

/* ------------------------------------------------- device work buffers */

enum { B_TOK, B_DL, B_TL, B_U, B_Z, B_N };
static void* g_buf[B_N];
static size_t g_bufsz[B_N];

static void* dbuf(int which, size_t bytes) {
    if (g_bufsz[which] < bytes) {
        cgx_free(g_buf[which]);
        g_buf[which] = cgx_malloc(bytes);
        g_bufsz[which] = g_buf[which] ? bytes : 0;
        if (!g_buf[which]) return NULL;
    }
    return g_buf[which];
}

/* ------------------------------------------------------------- inputs */

static cgx_model* model_of(void* handle, const char* who, const char* role) {
    cgx_model* m = cgx_model_from_handle(handle);
    if (!m) cgx_set_error("%s: decoder->%s is not a cgx_model handle", who, role);
    return m;
}

/* Token ids of a cg_tensor (floats holding integers in [0, V)), host copy. */
static int* read_ids(const cg_tensor* t, int V, int* n_out, const char* who) {
    if (!t || !t->data || t->size < 1) {
        cgx_set_error("%s: input_ids must hold at least one token", who);
        return NULL;
    }
    const int n = t->size;
    float* f = (float*)malloc((size_t)n * sizeof(float));
    int* ids = (int*)malloc((size_t)n * sizeof(int));
    if (!f || !ids) {
        free(f);
        free(ids);
        cgx_set_error("%s: out of memory", who);
        return NULL;
    }
    if (cgx_is_device_ptr(t->data)) {
        if (cgx_memcpy_d2h(f, t->data, (size_t)n * sizeof(float))) {
            free(f);
            free(ids);
            return NULL;
        }
    } else {
        memcpy(f, t->data, (size_t)n * sizeof(float));
    }
    for (int i = 0; i < n; i++) {
        const float v = f[i];
        if (!(v >= 0.0f && v < (float)V) || v != floorf(v)) {
            cgx_set_error("%s: input_ids[%d] = %g is not a token id in [0, %d)", who, i,
                          (double)v, V);
            free(f);
            free(ids);
            return NULL;
        }
        ids[i] = (int)v;
    }
    free(f);
    *n_out = n;
    return ids;
}

/* ------------------------------------------------------------ drafting */

/* g tokens after ids[0..n) from the draft model: tok_out[g] (host), the
 * draft logits [g][V] at *dl (device).  The draft cache then holds ids and
 * the first g - 1 drafted tokens. */
static int draft_chain(const cg_speculative_decoder* dec, cgx_model* dm, const int* ids,
                       int n, int g, int V, int* tok_out, float** dl) {
    cgx_model_config c;
    cgx_model_get_config(dm, &c);
    if (n - 1 + g > c.max_seq) {
        cgx_set_error("speculative driver: draft KV cache full (%d + %d > %d)", n - 1, g,
                      c.max_seq);
        return -1;
    }
    int* dtok = (int*)dbuf(B_TOK, (size_t)(g + 1) * sizeof(int));
    float* dlog = (float*)dbuf(B_DL, (size_t)g * V * sizeof(float));
    float* du = (float*)dbuf(B_U, (size_t)g * sizeof(float));
    float* dz = (float*)dbuf(B_Z, (size_t)V * sizeof(float));
    float* hu = (float*)malloc((size_t)g * sizeof(float));
    if (!dtok || !dlog || !du || !dz || !hu) {
        free(hu);
        if (dtok && dlog && du && dz) cgx_set_error("speculative driver: out of memory");
        return -1;
    }
    int rc = sync_prefix(dm, ids, n - 1);
    for (int i = 0; !rc && i < g; i++) hu[i] = cgx_lcg_draw();
    rc = rc || cgx_memcpy_h2d(du, hu, (size_t)g * sizeof(float)) ||
         cgx_memcpy_h2d(dtok, ids + n - 1, sizeof(int));
    for (int i = 0; !rc && i < g; i++) {
        float* row = dlog + (size_t)i * V;
        rc = cgx_model_forward(dm, dtok + i, 1, 1, row) ||
             cgx_sample_row_dev(row, V, dec->temperature, dec->top_k, dec->top_p, du + i,
                                hu[i], dz, dtok + i + 1, NULL);
    }
    free(hu);
    rc = rc || cgx_memcpy_d2h(tok_out, dtok + 1, (size_t)g * sizeof(int));
    hist_t* h = hist_of(dm);
    if (rc || !h) return -1;
    /* the cache now holds ids[0..n) and the drafts fed back, d_1 .. d_{g-1} */
    if (hist_set(h, ids, n, tok_out, g - 1)) return -1;
    *dl = dlog;
    return 0;
}

/* ----------------------------------------------------------- verifying */

/* The target's logits of [ids[n-1], tok[0..g)] ([g + 1][V], device) after
 * its cache is brought to ids[0..n - 1). */
static int target_rows(cgx_model* tm, const int* ids, int n, const int* tok, int g, int V,
                       float** tl) {
    cgx_model_config c;
    cgx_model_get_config(tm, &c);
    if (n + g > c.max_seq) {
        cgx_set_error("speculative driver: target KV cache full (%d + %d > %d)", n, g,
                      c.max_seq);
        return -1;
    }
    for (int i = 0; i < g; i++)
        if (tok[i] < 0 || tok[i] >= V) {
            cgx_set_error("speculative driver: draft token %d = %d outside [0, %d)", i, tok[i],
                          V);
            return -1;
        }
    int* rows = (int*)malloc((size_t)(g + 1) * sizeof(int));
    float* dlog = (float*)dbuf(B_TL, (size_t)(g + 1) * V * sizeof(float));
    if (!rows || !dlog) {
        free(rows);
        if (dlog) cgx_set_error("speculative driver: out of memory");
        return -1;
    }
    rows[0] = ids[n - 1];
    memcpy(rows + 1, tok, (size_t)g * sizeof(int));
    int rc = sync_prefix(tm, ids, n - 1);
    for (int i = 0; !rc && i <= g; i += c.max_tokens) {
        const int M = g + 1 - i < c.max_tokens ? g + 1 - i : c.max_tokens;
        rc = cgx_model_forward(tm, rows + i, M, M, dlog + (size_t)i * V);
    }
    hist_t* h = hist_of(tm);
    rc = rc || !h || hist_set(h, ids, n, tok, g);
    free(rows);
    if (rc) return -1;
    *tl = dlog;
    return 0;
}

static int g_last_verify_token = -1;

int cgx_last_verify_token(void) { return g_last_verify_token; }

/* The verify kernels with LCG draws (D6 order); returns n accepted. */
static int verify_lcg(const cg_speculative_decoder* dec, const float* tl, const float* dl,
                      const int* tok, int g, int V, int* out) {
    const uint32_t s0 = cgx_lcg_state();
    float* u = (float*)malloc((size_t)(g + 1) * sizeof(float));
    if (!u) {
        cgx_set_error("speculative driver: out of memory");
        return -1;
    }
    for (int i = 0; i <= g; i++) u[i] = cgx_lcg_draw();
    const int n = cgx_verify_chain(tl, dl, tok, u, g, V, dec->temperature, dec->top_k,
                                   dec->top_p, out, NULL);
    free(u);
    cgx_lcg_seed(s0);
    if (n < 0) return -1;
    const int used = n < g ? n + 2 : g + 1;
    for (int i = 0; i < used; i++) cgx_lcg_draw();
    return n;
}

/* accepted[], the token after the accepted drafts, the decoder statistics */
static void record(cg_speculative_decoder* dec, cg_token_tree* tree, const int* out, int n,
                   int g) {
    for (int i = 0; i < g; i++) tree->accepted[i] = i < n;
    if (n < g) tree->tokens[n] = out[n];
    g_last_verify_token = out[n];
    dec->total_draft_tokens += g;
    dec->accepted_draft_tokens += n;
    dec->num_steps += 1;
    dec->avg_acceptance_rate = dec->total_draft_tokens > 0
                                   ? (float)dec->accepted_draft_tokens /
                                         (float)dec->total_draft_tokens
                                   : 0.0f;
}

/* A host copy of device rows into a tree-owned buffer (freed by
 * cg_token_tree_free). */
static int own_rows(float** slot, const float* dev, size_t n) {
    float* h = (float*)malloc(n * sizeof(float));
    if (!h) {
        cgx_set_error("speculative driver: out of memory");
        return -1;
    }
    if (cgx_memcpy_d2h(h, dev, n * sizeof(float))) {
        free(h);
        return -1;
    }
    free(*slot);
    *slot = h;
    return 0;
}

static int check_tree(const cg_token_tree* tree, const char* who) {
    if (!tree || !tree->tokens || !tree->accepted || tree->depth < 1) {
        cgx_set_error("%s: a token tree of depth >= 1 is required", who);
        return -1;
    }
    return 0;
}

int cg_target_verify(cg_speculative_decoder* dec, cg_tensor* input_ids, cg_token_tree* tree) {
    static const char* who = "cg_target_verify";
    if (!dec || check_tree(tree, who)) {
        if (!dec) cgx_set_error("%s: NULL decoder", who);
        return -1;
    }
    if (!tree->draft_probs) {
        cgx_set_error("%s: tree->draft_probs must hold the draft logits [depth][vocab]", who);
        return -1;
    }
    cgx_model* tm = model_of(dec->target_model, who, "target_model");
    if (!tm || cgx_ensure_init()) return -1;
    cgx_model_config c;
    cgx_model_get_config(tm, &c);
    const int V = c.vocab, g = tree->depth;
    int* out = (int*)malloc((size_t)(g + 1) * sizeof(int));
    if (!out) {
        cgx_set_error("%s: out of memory", who);
        return -1;
    }
    int n = -1, nids = 0;
    int* ids = NULL;
    if (tree->target_probs) {
        n = verify_lcg(dec, tree->target_probs, tree->draft_probs, tree->tokens, g, V, out);
    } else {
        /* the target scores [last input token, drafts] and keeps the last
         * input token and the accepted drafts */
        float* tl = NULL;
        ids = read_ids(input_ids, V, &nids, who);
        int rc = !ids || target_rows(tm, ids, nids, tree->tokens, g, V, &tl) ||
                 own_rows(&tree->target_probs, tl, (size_t)(g + 1) * V);
        if (!rc) n = verify_lcg(dec, tl, tree->draft_probs, tree->tokens, g, V, out);
        if (n >= 0) {
            hist_t* h = hist_of(tm);
            if (!h || cgx_model_truncate(tm, nids + n) ||
                hist_set(h, ids, nids, tree->tokens, n))
                n = -1;
        }
    }
    if (n >= 0) record(dec, tree, out, n, g);
    free(ids);
    free(out);
    return n;
}

/* One draft + verify step on ids[0..n): tree->tokens get the drafts (then
 * the correction), out[g + 1] the emitted tokens; with copy, the tree's
 * draft_probs / target_probs get host copies of the logits. */
static int step_ids(cg_speculative_decoder* dec, const int* ids, int n, cg_token_tree* tree,
                    int copy, int* out, const char* who) {
    cgx_model* dm = model_of(dec->draft_model, who, "draft_model");
    cgx_model* tm = dm ? model_of(dec->target_model, who, "target_model") : NULL;
    if (!tm) return -1;
    cgx_model_config cd, ct;
    cgx_model_get_config(dm, &cd);
    cgx_model_get_config(tm, &ct);
    if (dm == tm || cd.vocab != ct.vocab) {
        cgx_set_error("%s: two distinct models with the same vocabulary are required", who);
        return -1;
    }
    const int V = ct.vocab, g = tree->depth;
    float *dl = NULL, *tl = NULL;
    if (draft_chain(dec, dm, ids, n, g, V, tree->tokens, &dl) ||
        target_rows(tm, ids, n, tree->tokens, g, V, &tl))
        return -1;
    if (copy && (own_rows(&tree->draft_probs, dl, (size_t)g * V) ||
                 own_rows(&tree->target_probs, tl, (size_t)(g + 1) * V)))
        return -1;
    const int k = verify_lcg(dec, tl, dl, tree->tokens, g, V, out);
    if (k < 0) return -1;
    /* both caches keep ids and the accepted drafts (the draft never saw d_g) */
    const int dkeep = n + (k < g ? k : g - 1);
    hist_t* hd = hist_of(dm);
    hist_t* ht = hist_of(tm);
    if (!hd || !ht || cgx_model_truncate(tm, n + k) || cgx_model_truncate(dm, dkeep) ||
        hist_set(ht, ids, n, tree->tokens, k) || hist_set(hd, ids, n, tree->tokens, dkeep - n))
        return -1;
    record(dec, tree, out, k, g);
    return k;
}

int cg_speculative_step(cg_speculative_decoder* dec, cg_tensor* input_ids,
                        cg_token_tree* tree) {
    static const char* who = "cg_speculative_step";
    if (!dec || check_tree(tree, who)) {
        if (!dec) cgx_set_error("%s: NULL decoder", who);
        return -1;
    }
    cgx_model* tm = model_of(dec->target_model, who, "target_model");
    if (!tm || cgx_ensure_init()) return -1;
    cgx_model_config c;
    cgx_model_get_config(tm, &c);
    int n = 0;
    int* ids = read_ids(input_ids, c.vocab, &n, who);
    int* out = (int*)malloc((size_t)(tree->depth + 1) * sizeof(int));
    int k = -1;
    if (ids && out) k = step_ids(dec, ids, n, tree, 1, out, who);
    else if (ids) cgx_set_error("%s: out of memory", who);
    free(ids);
    free(out);
    return k;
}

cg_token_tree* cg_draft_generate(cg_speculative_decoder* dec, cg_tensor* input_ids) {
    static const char* who = "cg_draft_generate";
    if (!dec || dec->gamma < 1) {
        cgx_set_error("%s: a decoder with gamma >= 1 is required", who);
        return NULL;
    }
    cgx_model* dm = model_of(dec->draft_model, who, "draft_model");
    if (!dm || cgx_ensure_init()) return NULL;
    cgx_model_config c;
    cgx_model_get_config(dm, &c);
    int n = 0;
    int* ids = read_ids(input_ids, c.vocab, &n, who);
    if (!ids) return NULL;
    cg_token_tree* tree = cg_token_tree_new(dec->gamma);
    float* dl = NULL;
    int rc = !tree || draft_chain(dec, dm, ids, n, dec->gamma, c.vocab, tree->tokens, &dl) ||
             own_rows(&tree->draft_probs, dl, (size_t)dec->gamma * c.vocab);
    free(ids);
    if (rc) {
        cg_token_tree_free(tree);
        return NULL;
    }
    return tree;
}

cg_tensor* cg_speculative_generate(cg_speculative_decoder* dec, cg_tensor* input_ids,
                                   int max_new_tokens, float temperature, float top_p) {
    static const char* who = "cg_speculative_generate";
    if (!dec || dec->gamma < 1 || max_new_tokens < 0) {
        cgx_set_error("%s: a decoder with gamma >= 1 and max_new_tokens >= 0 are required",
                      who);
        return NULL;
    }
    cgx_model* dm = model_of(dec->draft_model, who, "draft_model");
    cgx_model* tm = dm ? model_of(dec->target_model, who, "target_model") : NULL;
    if (!tm || cgx_ensure_init()) return NULL;
    dec->temperature = temperature;
    dec->top_p = top_p;
    cgx_model_config cd, ct;
    cgx_model_get_config(dm, &cd);
    cgx_model_get_config(tm, &ct);
    const int g = dec->gamma;
    const int cap_seq = cd.max_seq < ct.max_seq ? cd.max_seq : ct.max_seq;
    int n0 = 0;
    int* ids0 = read_ids(input_ids, ct.vocab, &n0, who);
    if (!ids0) return NULL;
    int* seq = (int*)malloc(((size_t)n0 + max_new_tokens + g + 1) * sizeof(int));
    int* out = (int*)malloc((size_t)(g + 1) * sizeof(int));
    cg_token_tree* tree = cg_token_tree_new(g);
    int rc = (seq && out && tree) ? 0 : -1;
    if (rc) cgx_set_error("%s: out of memory", who);
    int n = n0;
    if (!rc) memcpy(seq, ids0, (size_t)n0 * sizeof(int));
    free(ids0);
    /* steps until max_new_tokens are out or the caches cannot take a step */
    while (!rc && n - n0 < max_new_tokens && n + g <= cap_seq) {
        const int k = step_ids(dec, seq, n, tree, 0, out, who);
        if (k < 0) {
            rc = -1;
            break;
        }
        for (int i = 0; i <= k && n - n0 < max_new_tokens; i++) seq[n++] = out[i];
    }
    cg_tensor* res = NULL;
    if (!rc) {
        int shape[2] = {1, n};
        res = cg_tensor_new(shape, 2, false);
        if (res)
            for (int i = 0; i < n; i++) res->data[i] = (float)seq[i];
    }
    cg_token_tree_free(tree);
    free(seq);
    free(out);
    return res;
}

/* ------------------------------------------------------ tree attention */

/* The additive mask [S][S] (0 visible; <= -1e4 hidden) as a causal prefix of
 * P rows followed by up to 64 tree rows: row P + i sees every key < P and the
 * tree rows j with bit j of anc[i]; its rotary position is P + depth, depth =
 * (visible tree rows) - 1. */
static int split_mask(const float* mk, int S, int* P_out, cgx_tree_rows* tr) {
    for (size_t i = 0; i < (size_t)S * S; i++)
        if (!(mk[i] == 0.0f || mk[i] <= -1e4f)) {
            cgx_set_error("cg_forward_tree_attention: mask entry %g is neither 0 nor <= -1e4 "
                          "(only visible / hidden keys are supported)", (double)mk[i]);
            return -1;
        }
    int P = 0;
    while (P < S) {
        const float* r = mk + (size_t)P * S;
        int ok = 1;
        for (int j = 0; j < S && ok; j++) ok = (r[j] == 0.0f) == (j <= P);
        if (!ok) break;
        P++;
    }
    for (int changed = 1; changed;) {
        changed = 0;
        for (int r = P; r < S; r++)
            for (int j = 0; j < P; j++)
                if (mk[(size_t)r * S + j] != 0.0f) {
                    P = j;
                    changed = 1;
                    break;
                }
    }
    const int n = S - P;
    if (n > 64) {
        cgx_set_error("cg_forward_tree_attention: %d rows after the causal prefix of %d "
                      "(at most 64 tree rows)", n, P);
        return -1;
    }
    memset(tr, 0, sizeof(*tr));
    tr->tw = n;
    for (int i = 0; i < n; i++) {
        const float* r = mk + (size_t)(P + i) * S + P;
        unsigned long long bits = 0;
        for (int j = 0; j < n; j++)
            if (r[j] == 0.0f) bits |= 1ull << j;
        if (!((bits >> i) & 1)) {
            cgx_set_error("cg_forward_tree_attention: tree row %d does not see itself", P + i);
            return -1;
        }
        tr->anc[i] = bits;
        tr->rel[i] = __builtin_popcountll(bits) - 1;
    }
    *P_out = P;
    return 0;
}

cg_tensor* cg_forward_tree_attention(void* model, cg_tensor* input, cg_tensor* tree_mask) {
    static const char* who = "cg_forward_tree_attention";
    cgx_model* m = cgx_model_from_handle(model);
    if (!m) {
        cgx_set_error("%s: model is not a cgx_model handle", who);
        return NULL;
    }
    if (cgx_ensure_init()) return NULL;
    cgx_model_config c;
    cgx_model_get_config(m, &c);
    int S = 0;
    int* ids = read_ids(input, c.vocab, &S, who);
    if (!ids) return NULL;
    cg_tensor* res = NULL;
    float* mk = NULL;
    float* dlog = NULL;
    const size_t V = (size_t)c.vocab;
    int P = 0;
    cgx_tree_rows tr;
    /* the length first, then the mask size (formed in size_t: S * S can
     * exceed the int range) */
    if (S > c.max_seq) {
        cgx_set_error("%s: %d tokens exceed the KV cache (%d)", who, S, c.max_seq);
        goto done;
    }
    if (!tree_mask || !tree_mask->data || tree_mask->size < 0 ||
        (size_t)tree_mask->size != (size_t)S * (size_t)S) {
        cgx_set_error("%s: tree_mask must hold [S][S] = %d x %d values", who, S, S);
        goto done;
    }
    mk = (float*)malloc((size_t)S * S * sizeof(float));
    if (!mk) {
        cgx_set_error("%s: out of memory", who);
        goto done;
    }
    if (cgx_is_device_ptr(tree_mask->data)) {
        if (cgx_memcpy_d2h(mk, tree_mask->data, (size_t)S * S * sizeof(float))) goto done;
    } else {
        memcpy(mk, tree_mask->data, (size_t)S * S * sizeof(float));
    }
    if (split_mask(mk, S, &P, &tr)) goto done;
    if (tr.tw > c.max_tokens) {
        cgx_set_error("%s: %d tree rows exceed the model's max_tokens (%d)", who, tr.tw,
                      c.max_tokens);
        goto done;
    }
    int shape[3] = {1, S, (int)V};
    res = cg_tensor_new(shape, 3, false);
    dlog = (float*)dbuf(B_TL, (size_t)c.max_tokens * V * sizeof(float));
    if (!res || !dlog) goto fail;
    /* the model's cache is the workspace: every row is recomputed from 0 */
    if (cgx_model_truncate(m, 0)) goto fail;
    for (int i = 0; i < P; i += c.max_tokens) {
        const int M = P - i < c.max_tokens ? P - i : c.max_tokens;
        if (cgx_model_forward(m, ids + i, M, M, dlog) ||
            cgx_memcpy_d2h(res->data + (size_t)i * V, dlog, (size_t)M * V * sizeof(float)))
            goto fail;
    }
    if (tr.tw > 0 &&
        (cgx_model_forward_tree1(m, ids + P, tr.tw, &tr, dlog) ||
         cgx_memcpy_d2h(res->data + (size_t)P * V, dlog, (size_t)tr.tw * V * sizeof(float))))
        goto fail;
    /* the cache keeps the causal prefix */
    if (cgx_model_truncate(m, P)) goto fail;
    hist_t* h = hist_of(m);
    if (!h || hist_set(h, ids, P, NULL, 0)) goto fail;
    goto done;
fail:
    cg_tensor_free(res);
    res = NULL;
done:
    free(mk);
    free(ids);
    return res;
}

/* ---------------------------------------------------------------- EAGLE */

cg_token_tree* cg_eagle_generate_tree(cg_eagle_draft* eagle, cg_tensor* input, int max_depth) {
    static const char* who = "cg_eagle_generate_tree";
    if (!eagle || max_depth < 0) {
        cgx_set_error("%s: an EAGLE draft and max_depth >= 0 are required", who);
        return NULL;
    }
    cgx_model* dm = cgx_model_from_handle(eagle->base_draft);
    cg_token_tree* tree = cg_token_tree_new(max_depth);
    if (!tree) return NULL;
    if (!dm) {
        /* the reference's placeholder tree (speculative.c:244-262): every
         * token 1, for a base_draft that is not a model this library runs */
        for (int i = 0; i < max_depth; i++) tree->tokens[i] = 1;
        return tree;
    }
    if (max_depth == 0) return tree;
    if (cgx_ensure_init()) goto fail;
    cgx_model_config c;
    cgx_model_get_config(dm, &c);
    const int V = c.vocab, g = max_depth;
    int n = 0;
    int* ids = read_ids(input, V, &n, who);
    if (!ids) goto fail;
    if (n - 1 + g > c.max_seq) {
        cgx_set_error("%s: draft KV cache full (%d + %d > %d)", who, n - 1, g, c.max_seq);
        free(ids);
        goto fail;
    }
    /* the draft's most likely token at each depth (ties: the lower index),
     * i.e. the first-ranked path of the draft tree, as a chain */
    int* dtok = (int*)dbuf(B_TOK, (size_t)(g + 1) * sizeof(int));
    float* dlog = (float*)dbuf(B_DL, (size_t)g * V * sizeof(float));
    float* dp = (float*)dbuf(B_Z, (size_t)V * sizeof(float));
    int rc = !dtok || !dlog || !dp || sync_prefix(dm, ids, n - 1) ||
             cgx_memcpy_h2d(dtok, ids + n - 1, sizeof(int));
    for (int i = 0; !rc && i < g; i++) {
        float* row = dlog + (size_t)i * V;
        rc = cgx_model_forward(dm, dtok + i, 1, 1, row) ||
             cgk_topk_lists(row, 1, V, 1, 1.0f, dtok + i + 1, dp);
    }
    rc = rc || cgx_memcpy_d2h(tree->tokens, dtok + 1, (size_t)g * sizeof(int)) ||
         own_rows(&tree->draft_probs, dlog, (size_t)g * V);
    hist_t* h = rc ? NULL : hist_of(dm);
    rc = rc || !h || hist_set(h, ids, n, tree->tokens, g - 1);
    free(ids);
    if (!rc) return tree;
fail:
    cg_token_tree_free(tree);
    return NULL;
}

/* Decision D17: the branching factor of a draft node is the number of its
 * most likely tokens (1..4, cg_sample_top_k's order: probability descending,
 * ties to the lower id) whose probabilities, summed in that order in fp32,
 * first reach kBranchMass; a confident draft branches once, an uncertain one
 * up to four times.  Probabilities are the draft's softmax at T = 1
 * (cg_sample_temperature's). */
static const float kBranchMass = 0.8f;

int* cg_eagle_compute_branching(cg_eagle_draft* eagle, cg_tensor* features) {
    static const char* who = "cg_eagle_compute_branching";
    if (!eagle || !features || !features->data || features->ndim < 1) {
        cgx_set_error("%s: an EAGLE draft and a [rows][vocab] tensor of draft logits are "
                      "required", who);
        return NULL;
    }
    const int V = features->shape[features->ndim - 1];
    cgx_model* dm = cgx_model_from_handle(eagle->base_draft);
    if (dm) {
        cgx_model_config c;
        cgx_model_get_config(dm, &c);
        if (c.vocab != V) {
            cgx_set_error("%s: features have %d columns, the draft's vocabulary is %d", who, V,
                          c.vocab);
            return NULL;
        }
    }
    if (V < 2 || features->size % V) {
        cgx_set_error("%s: features must be [rows][vocab] with vocab >= 2", who);
        return NULL;
    }
    if (cgx_ensure_init()) return NULL;
    const int rows = features->size / V, K = V < 4 ? V - 1 : 4;
    const float* x = (const float*)cgx_dev_in(features->data, (size_t)features->size * 4,
                                              CGX_SLOT_IN0);
    float* probs = (float*)dbuf(B_TL, (size_t)V * sizeof(float));
    int* lidx = (int*)dbuf(B_TOK, 4 * sizeof(int));
    float* lp = (float*)dbuf(B_U, 4 * sizeof(float));
    int* out = (int*)malloc((size_t)rows * sizeof(int));
    if (!x || !probs || !lidx || !lp || !out) {
        free(out);
        if (x && probs && lidx && lp) cgx_set_error("%s: out of memory", who);
        return NULL;
    }
    for (int r = 0; r < rows; r++) {
        int idx[4];
        float pk[4];
        if (cgk_temperature_probs(x + (size_t)r * V, V, 1.0f, probs) ||
            cgk_topk_lists(probs, 1, V, K, 1.0f, lidx, lp) ||
            cgx_memcpy_d2h(idx, lidx, (size_t)K * sizeof(int))) {
            free(out);
            return NULL;
        }
        for (int j = 0; j < K; j++)
            if (cgx_memcpy_d2h(&pk[j], probs + idx[j], sizeof(float))) {
                free(out);
                return NULL;
            }
        int b = K;
        float mass = 0.0f;
        for (int j = 0; j < K; j++) {
            mass += pk[j];
            if (mass >= kBranchMass) {
                b = j + 1;
                break;
            }
        }
        out[r] = b;
    }
    return out;
}
