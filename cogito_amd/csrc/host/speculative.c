/*
 * speculative.c -- host-side objects of cogito's speculative-decoding API
 * (include/cg_speculative.h): the decoder and token-tree containers, the
 * global LCG stream, the acceptance ratio and the tree attention mask.
 * Sampling and verification run in the acceptance kernels (accept.hip) and
 * are wired in sampling.c.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "cg_mi355x.h"
#include "cg_speculative.h"
#include "cgx_internal.h"

/* ---------------------------------------------------------------- LCG */

/* reference src/inference/speculative.c:11-12 */
static uint32_t g_lcg = 42u;

void cgx_lcg_seed(uint32_t state) { g_lcg = state; }
uint32_t cgx_lcg_state(void) { return g_lcg; }

float cgx_lcg_draw(void) {
    g_lcg = g_lcg * 1103515245u + 12345u;
    return (float)(g_lcg % 10000u) / 10000.0f;
}

/* ------------------------------------------------------ acceptance ratio */

float cg_acceptance_prob(float draft_prob, float target_prob) {
    /* reference speculative.c:49-52 */
    if (draft_prob < 1e-10f) return 1.0f;
    return fminf(1.0f, target_prob / draft_prob);
}

/* ------------------------------------------------------------ decoder */

cg_speculative_decoder* cg_speculative_decoder_new(void* draft_model,
                                                   void* target_model, int gamma) {
    /* defaults of reference speculative.c:32-42 */
    cg_speculative_decoder* d = (cg_speculative_decoder*)calloc(1, sizeof(*d));
    if (!d) return NULL;
    d->draft_model = draft_model;
    d->target_model = target_model;
    d->gamma = gamma;
    d->temperature = 1.0f;
    d->top_p = 0.9f;
    d->top_k = 50;
    d->accept_threshold = 0.0f;
    return d;
}

void cg_speculative_decoder_free(cg_speculative_decoder* d) { free(d); }

/* --------------------------------------------------------- token tree */

cg_token_tree* cg_token_tree_new(int depth) {
    if (depth < 0) {
        cgx_set_error("cg_token_tree_new: negative depth");
        return NULL;
    }
    cg_token_tree* t = (cg_token_tree*)calloc(1, sizeof(*t));
    if (!t) return NULL;
    t->depth = depth;
    t->tokens = (int*)calloc((size_t)(depth > 0 ? depth : 1), sizeof(int));
    t->accepted = (bool*)calloc((size_t)(depth > 0 ? depth : 1), sizeof(bool));
    if (!t->tokens || !t->accepted) {
        cg_token_tree_free(t);
        return NULL;
    }
    return t;
}

void cg_token_tree_free(cg_token_tree* t) {
    if (!t) return;
    free(t->tokens);
    free(t->draft_probs);
    free(t->target_probs);
    free(t->accepted);
    free(t->branch_points);
    cg_tensor_free(t->hidden_states);
    free(t);
}

void cg_token_tree_add_token(cg_token_tree* t, int token, float* probs) {
    /* The reference body is empty (speculative.c:184-187).  Here a token is
     * appended as the child of the last node (chain growth); `probs`, when
     * given, is stored as that node's draft row only if the tree already
     * owns a draft_probs buffer. */
    (void)probs;
    if (!t) return;
    int n = t->depth + 1;
    int* tok = (int*)realloc(t->tokens, (size_t)n * sizeof(int));
    bool* acc = (bool*)realloc(t->accepted, (size_t)n * sizeof(bool));
    if (!tok || !acc) {
        if (tok) t->tokens = tok;
        if (acc) t->accepted = acc;
        cgx_set_error("cg_token_tree_add_token: out of memory");
        return;
    }
    t->tokens = tok;
    t->accepted = acc;
    tok[n - 1] = token;
    acc[n - 1] = false;
    if (t->branch_points) {
        int* bp = (int*)realloc(t->branch_points, (size_t)n * sizeof(int));
        if (bp) {
            t->branch_points = bp;
            bp[n - 1] = n - 2;
        }
    }
    t->depth = n;
}

cg_tensor* cg_token_tree_to_tensor(cg_token_tree* t) {
    /* reference speculative.c:189-195: [1, depth] float token ids */
    if (!t || t->depth <= 0) {
        cgx_set_error("cg_token_tree_to_tensor: empty tree");
        return NULL;
    }
    int shape[2] = {1, t->depth};
    cg_tensor* out = cg_tensor_new(shape, 2, false);
    if (!out) return NULL;
    for (int i = 0; i < t->depth; i++) out->data[i] = (float)t->tokens[i];
    return out;
}

cg_tensor* cg_tree_attention_mask(cg_token_tree* t, int seqlen) {
    /* reference speculative.c:197-238: [1,1,S,S] additive mask (0 / -1e9),
     * causal prefix, nodes see the prefix and their ancestors.  The
     * reference assumes a chain; with branch_points (parent per node) the
     * ancestor set follows the tree. */
    if (!t || seqlen < 0) {
        cgx_set_error("cg_tree_attention_mask: invalid argument");
        return NULL;
    }
    int n = t->depth, size = seqlen + n;
    if (size <= 0) {
        cgx_set_error("cg_tree_attention_mask: empty mask");
        return NULL;
    }
    int shape[4] = {1, 1, size, size};
    cg_tensor* m = cg_tensor_new(shape, 4, false);
    if (!m) return NULL;
    for (int i = 0; i < m->size; i++) m->data[i] = -1e9f;
    for (int i = 0; i < seqlen; i++)
        for (int j = 0; j <= i; j++) m->data[(size_t)i * size + j] = 0.0f;
    for (int i = 0; i < n; i++) {
        size_t r = (size_t)(seqlen + i) * size;
        for (int j = 0; j < seqlen; j++) m->data[r + j] = 0.0f;
        if (t->branch_points) {
            for (int a = i, guard = 0; a >= 0 && a < n && guard <= n;
                 a = t->branch_points[a], guard++)
                m->data[r + seqlen + a] = 0.0f;
        } else {
            for (int j = 0; j <= i; j++) m->data[r + seqlen + j] = 0.0f;
        }
    }
    return m;
}

/* ---------------------------------------------------------------- EAGLE */

cg_eagle_draft* cg_eagle_draft_new(void* base_draft) {
    cg_eagle_draft* e = (cg_eagle_draft*)calloc(1, sizeof(*e));
    if (e) e->base_draft = base_draft;
    return e;
}

void cg_eagle_draft_free(cg_eagle_draft* e) {
    if (!e) return;
    free(e->feature_cache);
    free(e);
}
