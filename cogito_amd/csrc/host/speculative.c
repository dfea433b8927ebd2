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
    /* reference speculative.c:22-30: branch_points is not the tree's */
    if (!t) return;
    free(t->tokens);
    free(t->draft_probs);
    free(t->target_probs);
    free(t->accepted);
    cg_tensor_free(t->hidden_states);
    free(t);
}

void cg_token_tree_add_token(cg_token_tree* t, int token, float* probs) {
    /* reference speculative.c:184-187: the body is empty (the tree is a
     * fixed-depth chain filled through tokens[]) */
    (void)t;
    (void)token;
    (void)probs;
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

/* [1,1,S,S] additive mask (0 / -1e9), S = seqlen + nodes: causal prefix;
 * node i sees the prefix and the nodes j with anc(i, j). */
static cg_tensor* tree_mask(int seqlen, int nodes, const int* parents, const char* who) {
    if (seqlen < 0 || nodes < 0 || seqlen + nodes <= 0) {
        cgx_set_error("%s: empty mask", who);
        return NULL;
    }
    const int size = seqlen + nodes;
    int shape[4] = {1, 1, size, size};
    cg_tensor* m = cg_tensor_new(shape, 4, false);
    if (!m) return NULL;
    for (int i = 0; i < m->size; i++) m->data[i] = -1e9f;
    for (int i = 0; i < seqlen; i++)
        for (int j = 0; j <= i; j++) m->data[(size_t)i * size + j] = 0.0f;
    for (int i = 0; i < nodes; i++) {
        size_t r = (size_t)(seqlen + i) * size;
        for (int j = 0; j < seqlen; j++) m->data[r + j] = 0.0f;
        if (parents) {
            for (int a = i; a >= 0; a = parents[a]) m->data[r + seqlen + a] = 0.0f;
        } else {
            for (int j = 0; j <= i; j++) m->data[r + seqlen + j] = 0.0f;
        }
    }
    return m;
}

cg_tensor* cg_tree_attention_mask(cg_token_tree* t, int seqlen) {
    /* reference speculative.c:197-238: the nodes form a chain (the reference
     * reads no parent links); tree parents go through
     * cgx_tree_attention_mask_parents */
    if (!t) {
        cgx_set_error("cg_tree_attention_mask: NULL tree");
        return NULL;
    }
    return tree_mask(seqlen, t->depth, NULL, "cg_tree_attention_mask");
}

cg_tensor* cgx_tree_attention_mask_parents(const int* parents, int nodes, int seqlen) {
    if (!parents || nodes < 1) {
        cgx_set_error("cgx_tree_attention_mask_parents: parents of at least one node required");
        return NULL;
    }
    for (int i = 0; i < nodes; i++)
        if (parents[i] < -1 || parents[i] >= i) {
            cgx_set_error("cgx_tree_attention_mask_parents: node %d has parent %d (need -1 <= "
                          "parent < node)", i, parents[i]);
            return NULL;
        }
    return tree_mask(seqlen, nodes, parents, "cgx_tree_attention_mask_parents");
}

/* ---------------------------------------------------------------- EAGLE */

cg_eagle_draft* cg_eagle_draft_new(void* base_draft) {
    cg_eagle_draft* e = (cg_eagle_draft*)calloc(1, sizeof(*e));
    if (e) e->base_draft = base_draft;
    return e;
}

void cg_eagle_draft_free(cg_eagle_draft* e) {
    /* reference speculative.c:264-267: the struct only (feature_cache is
     * never allocated by the library) */
    free(e);
}
