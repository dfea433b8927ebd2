/* tree.c -- EAGLE-style tree speculation on the device, B sequences in
 * lockstep (cgx_tree_spec_*), and the static draft tree.
 *
 * The reference declares tree verification (include/cg_speculative.h:15-25,
 * 123-130; cg_tree_attention_mask, src/inference/speculative.c:197-238) and
 * leaves the EAGLE builder a stub (speculative.c:244-262).  Here one step is:
 *   1. draft, level by level: the rows of level l (one forward of the draft
 *      model over B * count(l) rows, tree mask over the nodes so far) give
 *      each node's draft logits; a node's children are the top-c tokens of
 *      those logits (ties: lower index), c = its child count in the shape;
 *   2. the target forward over all nodes of every sequence (rotary position
 *      = prefix length + node depth, tree mask over the whole tree);
 *   3. the acceptance walk (tree.hip k_tree_accept) over the target rows'
 *      top-k lists at temperature T;
 *   4. compaction of the accepted path in both caches (the drafted nodes'
 *      rows move to consecutive slots; their rotary positions already are).
 * The drawn token becomes the next step's root (node 0). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "cgx_internal.h"

/* ------------------------------------------------------------ the shape */

int cgx_tree_shape_from_parents(cgx_tree_shape* t, const int* parent, int nodes) {
    if (!t || !parent || nodes < 1 || nodes > 64 || parent[0] != -1) {
        cgx_set_error("tree shape: 1..64 nodes with parent[0] = -1 are required");
        return -1;
    }
    memset(t, 0, sizeof(*t));
    t->nodes = nodes;
    t->parent[0] = -1;
    for (int i = 1; i < nodes; i++) {
        const int p = parent[i];
        if (p < 0 || p >= i) {
            cgx_set_error("tree shape: node %d has parent %d (need 0 <= parent < node)", i, p);
            return -1;
        }
        t->parent[i] = p;
        t->node_depth[i] = t->node_depth[p] + 1;
        if (t->node_depth[i] < t->node_depth[i - 1]) {
            cgx_set_error("tree shape: nodes are not in breadth-first order at %d", i);
            return -1;
        }
        if (t->nkids[p] >= 4) {
            cgx_set_error("tree shape: node %d has more than 4 children", p);
            return -1;
        }
        t->rank[i] = t->nkids[p];
        t->kids[p][t->nkids[p]++] = i;
        if (t->node_depth[i] > t->depth) t->depth = t->node_depth[i];
    }
    return 0;
}

int cgx_tree_shape_default(cgx_tree_shape* t, int nodes, int depth) {
    /* best-first: a candidate's score is the product of the rank weights on
     * its path; the best candidate (ties: the one created first) joins and
     * offers its 4 children; then breadth-first renumbering */
    static const double kW[4] = {0.6, 0.2, 0.12, 0.08};
    if (!t || nodes < 1 || nodes > 64 || depth < 0 || depth > 15) {
        cgx_set_error("tree shape: 1..64 nodes and depth 0..15 are required");
        return -1;
    }
    typedef struct { int parent, rank, depth; double score; } cand_t;
    cand_t sel[64], cand[64 * 4 + 4];
    int nsel = 1, ncand = 0;
    sel[0] = (cand_t){-1, 0, 0, 1.0};
    for (int r = 0; r < 4 && depth > 0; r++) cand[ncand++] = (cand_t){0, r, 1, kW[r]};
    while (nsel < nodes && ncand > 0) {
        int best = 0;
        for (int i = 1; i < ncand; i++)
            if (cand[i].score > cand[best].score) best = i;
        cand_t c = cand[best];
        memmove(cand + best, cand + best + 1, (size_t)(ncand - best - 1) * sizeof(cand_t));
        ncand--;
        const int id = nsel;
        sel[nsel++] = c;
        if (c.depth < depth)
            for (int r = 0; r < 4; r++)
                cand[ncand++] = (cand_t){id, r, c.depth + 1, c.score * kW[r]};
    }
    /* breadth-first order: level by level, each parent's children by rank */
    int order[64], newid[64], parent[64];
    int n = 0;
    order[n++] = 0;
    newid[0] = 0;
    for (int head = 0; head < n; head++) {
        const int old = order[head];
        for (int r = 0; r < 4; r++)
            for (int i = 1; i < nsel; i++)
                if (sel[i].parent == old && sel[i].rank == r) {
                    newid[i] = n;
                    order[n++] = i;
                }
    }
    for (int k = 0; k < n; k++) {
        const int old = order[k];
        parent[k] = k == 0 ? -1 : newid[sel[old].parent];
    }
    /* within a parent the ranks are consecutive from 0, because a candidate
     * of rank r scores below rank r - 1 of the same parent */
    return cgx_tree_shape_from_parents(t, parent, n);
}

int cgx_tree_shape_get(int nodes, int depth, int* parent, int* node_depth, int* rank) {
    cgx_tree_shape t;
    if (cgx_tree_shape_default(&t, nodes, depth)) return -1;
    for (int i = 0; i < t.nodes; i++) {
        if (parent) parent[i] = t.parent[i];
        if (node_depth) node_depth[i] = t.node_depth[i];
        if (rank) rank[i] = t.rank[i];
    }
    return t.nodes;
}

/* ------------------------------------------------ acceptance (tests) */

int cgx_tree_accept_dev(const int* parent, int nodes, int B, int K, const int* lidx,
                        const float* lp, const int* tok, const float* u, int* out, int* nacc,
                        int* path) {
    cgx_tree_shape t;
    if (cgx_tree_shape_from_parents(&t, parent, nodes)) return -1;
    return cgk_tree_accept(&t, B, K, lidx, lp, tok, u, out, nacc, path);
}

int cgx_topk_lists_dev(const float* z, int rows, int V, int top_k, float top_p, int* lidx,
                       float* lp) {
    return cgk_topk_lists(z, rows, V, top_k, top_p, lidx, lp);
}

/* ------------------------------------------------------- the tree loop */

struct cgx_tree_spec {
    cgx_model* draft;
    cgx_model* target;
    cgx_tree_shape t;
    int B, V, K;
    float T, top_p;
    int nlev;
    int lev_first[16], lev_count[16];
    unsigned long long anc[64];
    int* d_parent;           /* shape arrays for k_tree_children */
    int* d_rank;
    int* d_tok;              /* [B][R] node tokens (node 0: the root) */
    int* d_ltok;             /* [B][count] tokens of one level */
    float* d_dlogits;        /* [B][count][V] draft logits of one level */
    int* d_lidx4;            /* [B * count][4] draft top-4 lists */
    float* d_lp4;
    float* d_tlogits;        /* [B][R][V] target logits, then logits / T */
    int* d_lidx;             /* [B * R][K] target lists */
    float* d_lp;
    float* d_u;              /* [B][depth + 1][5] */
    int* d_out;              /* [B][depth + 2] */
    int* d_nacc;             /* [B] */
    int* d_path;             /* [B][depth] */
    int root[16];
    int have_root;
    long long steps, drafted, accepted;
};

void cgx_tree_spec_free(cgx_tree_spec* s) {
    if (!s) return;
    cgx_free(s->d_parent);
    cgx_free(s->d_rank);
    cgx_free(s->d_tok);
    cgx_free(s->d_ltok);
    cgx_free(s->d_dlogits);
    cgx_free(s->d_lidx4);
    cgx_free(s->d_lp4);
    cgx_free(s->d_tlogits);
    cgx_free(s->d_lidx);
    cgx_free(s->d_lp);
    cgx_free(s->d_u);
    cgx_free(s->d_out);
    cgx_free(s->d_nacc);
    cgx_free(s->d_path);
    free(s);
}

cgx_tree_spec* cgx_tree_spec_new(cgx_model* draft, cgx_model* target, int nodes, int depth,
                                 float temperature, int top_k, float top_p) {
    cgx_model_config cd, ct;
    if (!draft || !target || draft == target || cgx_model_get_config(draft, &cd) ||
        cgx_model_get_config(target, &ct)) {
        cgx_set_error("cgx_tree_spec_new: two distinct models are required");
        return NULL;
    }
    const int B = cgx_model_batch(target);
    if (cgx_model_batch(draft) != B || cd.vocab != ct.vocab || !(temperature > 0.0f) ||
        top_k < 1 || top_k > 64 || top_k >= ct.vocab || !(top_p > 0.0f) || top_p > 1.0f) {
        cgx_set_error("cgx_tree_spec_new: the models need the same batch and vocabulary; "
                      "temperature > 0, 1 <= top_k <= 64 and 0 < top_p <= 1 are required");
        return NULL;
    }
    cgx_tree_spec* s = (cgx_tree_spec*)calloc(1, sizeof(*s));
    if (!s) return NULL;
    if (cgx_tree_shape_default(&s->t, nodes, depth)) {
        free(s);
        return NULL;
    }
    const int R = s->t.nodes;
    if (ct.max_tokens < R || cd.max_tokens < R) {
        cgx_set_error("cgx_tree_spec_new: the models take %d / %d rows per sequence, the tree "
                      "has %d nodes", cd.max_tokens, ct.max_tokens, R);
        free(s);
        return NULL;
    }
    s->draft = draft;
    s->target = target;
    s->B = B;
    s->V = ct.vocab;
    s->K = top_k;
    s->T = temperature;
    s->top_p = top_p;
    /* levels and ancestor bits */
    s->nlev = s->t.depth + 1;
    for (int i = 0; i < R; i++) {
        const int d = s->t.node_depth[i];
        if (s->lev_count[d]++ == 0) s->lev_first[d] = i;
        s->anc[i] = (1ull << i) | (i > 0 ? s->anc[s->t.parent[i]] : 0ull);
    }
    int maxc = 0;
    for (int l = 0; l < s->nlev; l++) maxc = s->lev_count[l] > maxc ? s->lev_count[l] : maxc;
    const size_t V = (size_t)s->V, b = (size_t)B, r = (size_t)R, dd = (size_t)s->t.depth;
    s->d_parent = (int*)cgx_malloc(r * 4);
    s->d_rank = (int*)cgx_malloc(r * 4);
    s->d_tok = (int*)cgx_malloc(b * r * 4);
    s->d_ltok = (int*)cgx_malloc(b * (size_t)maxc * 4);
    s->d_dlogits = (float*)cgx_malloc(b * (size_t)maxc * V * 4);
    s->d_lidx4 = (int*)cgx_malloc(b * (size_t)maxc * 4 * 4);
    s->d_lp4 = (float*)cgx_malloc(b * (size_t)maxc * 4 * 4);
    s->d_tlogits = (float*)cgx_malloc(b * r * V * 4);
    s->d_lidx = (int*)cgx_malloc(b * r * (size_t)top_k * 4);
    s->d_lp = (float*)cgx_malloc(b * r * (size_t)top_k * 4);
    s->d_u = (float*)cgx_malloc(b * (dd + 1) * 5 * 4);
    s->d_out = (int*)cgx_malloc(b * (dd + 2) * 4);
    s->d_nacc = (int*)cgx_malloc(b * 4);
    s->d_path = (int*)cgx_malloc(b * (dd > 0 ? dd : 1) * 4);
    if (!s->d_parent || !s->d_rank || !s->d_tok || !s->d_ltok || !s->d_dlogits ||
        !s->d_lidx4 || !s->d_lp4 || !s->d_tlogits || !s->d_lidx || !s->d_lp || !s->d_u ||
        !s->d_out || !s->d_nacc || !s->d_path ||
        cgx_memcpy_h2d(s->d_parent, s->t.parent, r * 4) ||
        cgx_memcpy_h2d(s->d_rank, s->t.rank, r * 4)) {
        cgx_tree_spec_free(s);
        return NULL;
    }
    return s;
}

int cgx_tree_spec_nodes(const cgx_tree_spec* s) { return s ? s->t.nodes : -1; }
int cgx_tree_spec_depth(const cgx_tree_spec* s) { return s ? s->t.depth : -1; }

int cgx_tree_spec_set_root(cgx_tree_spec* s, const int* root) {
    if (!s || !root) {
        cgx_set_error("cgx_tree_spec_set_root: invalid argument");
        return -1;
    }
    for (int b = 0; b < s->B; b++) {
        const int lt = cgx_model_len_seq(s->target, b), ld = cgx_model_len_seq(s->draft, b);
        if (root[b] < 0 || root[b] >= s->V || lt != ld) {
            cgx_set_error("cgx_tree_spec_set_root: sequence %d: token %d, caches hold %d "
                          "(target) / %d (draft) positions", b, root[b], lt, ld);
            return -1;
        }
        s->root[b] = root[b];
    }
    s->have_root = 1;
    return 0;
}

/* Rows of level l in a draft forward: the call appends them at slots
 * L + f .. (L = prefix length, f = the level's first node), so their rotary
 * position L + l is the cache length L + f plus rel = l - f; the window is
 * the f + c nodes appended so far in this step. */
static void level_rows(const cgx_tree_spec* s, int l, cgx_tree_rows* tr) {
    memset(tr, 0, sizeof(*tr));
    const int f = s->lev_first[l], c = s->lev_count[l];
    for (int j = 0; j < c; j++) {
        tr->rel[j] = l - f;
        tr->anc[j] = s->anc[f + j];
    }
    tr->tw = f + c;
}

int cgx_tree_spec_step(cgx_tree_spec* s, const float* u, int* out_tokens, int* n_accepted) {
    if (!s || !u || !out_tokens || !n_accepted) {
        cgx_set_error("cgx_tree_spec_step: invalid argument");
        return -1;
    }
    if (!s->have_root) {
        cgx_set_error("cgx_tree_spec_step: no root token (call cgx_tree_spec_set_root)");
        return -1;
    }
    const int B = s->B, R = s->t.nodes, D = s->t.depth;
    const size_t V = (size_t)s->V;
    cgx_model_config ct, cd;
    cgx_model_get_config(s->target, &ct);
    cgx_model_get_config(s->draft, &cd);
    int L[16];
    for (int b = 0; b < B; b++) {
        L[b] = cgx_model_len_seq(s->target, b);
        if (L[b] != cgx_model_len_seq(s->draft, b) || L[b] + R > ct.max_seq ||
            L[b] + R > cd.max_seq) {
            cgx_set_error("cgx_tree_spec_step: sequence %d: caches out of step or full", b);
            return -1;
        }
    }
    /* node tokens: roots now, the levels on the device */
    int* htok = (int*)calloc((size_t)B * R, sizeof(int));
    if (!htok) return -1;
    for (int b = 0; b < B; b++) htok[(size_t)b * R] = s->root[b];
    int rc = cgx_memcpy_h2d(s->d_tok, htok, (size_t)B * R * sizeof(int)) ||
             cgx_memcpy_h2d(s->d_u, u, (size_t)B * (D + 1) * 5 * sizeof(float));
    free(htok);
    if (rc) return -1;
    /* 1. draft, level by level (the deepest level only for its cache rows) */
    for (int l = 0; l < s->nlev; l++) {
        cgx_tree_rows tr;
        level_rows(s, l, &tr);
        const int f = s->lev_first[l], c = s->lev_count[l];
        const int last = l + 1 == s->nlev;
        if (cgk_tree_gather(B, R, f, c, s->d_tok, s->d_ltok) ||
            cgx_model_forward_tree(s->draft, s->d_ltok, c, &tr, last ? NULL : s->d_dlogits, 0))
            return -1;
        if (last) break;
        if (cgk_topk_lists(s->d_dlogits, B * c, s->V, 4, 1.0f, s->d_lidx4, s->d_lp4) ||
            cgk_tree_children(&s->t, B, 4, s->lev_first[l + 1], s->lev_count[l + 1], f, c,
                              s->d_parent, s->d_rank, s->d_lidx4, s->d_tok))
            return -1;
    }
    /* 2.-3. target forward over every node, lists at T, the walk */
    cgx_tree_rows tt;
    memset(&tt, 0, sizeof(tt));
    for (int i = 0; i < R; i++) {
        tt.rel[i] = s->t.node_depth[i];
        tt.anc[i] = s->anc[i];
    }
    tt.tw = R;
    if (cgx_model_forward_tree(s->target, s->d_tok, R, &tt, s->d_tlogits, 0) ||
        cgk_scale(s->d_tlogits, s->d_tlogits, (size_t)B * R * V, s->T) ||
        cgk_topk_lists(s->d_tlogits, B * R, s->V, s->K, s->top_p, s->d_lidx, s->d_lp) ||
        cgk_tree_accept(&s->t, B, s->K, s->d_lidx, s->d_lp, s->d_tok, s->d_u, s->d_out,
                        s->d_nacc, s->d_path))
        return -1;
    int hn[16];
    int* ho = (int*)malloc((size_t)B * (D + 2) * sizeof(int));
    if (!ho) return -1;
    if (cgx_memcpy_d2h(ho, s->d_out, (size_t)B * (D + 2) * sizeof(int)) ||
        cgx_memcpy_d2h(hn, s->d_nacc, (size_t)B * sizeof(int))) {
        free(ho);
        return -1;
    }
    /* 4. both caches keep the root and the accepted path */
    if (cgx_model_compact_tree(s->target, &s->t, L, s->d_nacc, s->d_path, hn) ||
        cgx_model_compact_tree(s->draft, &s->t, L, s->d_nacc, s->d_path, hn)) {
        free(ho);
        return -1;
    }
    int total = 0;
    for (int b = 0; b < B; b++) {
        const int n = hn[b];
        n_accepted[b] = n;
        for (int i = 0; i <= D + 1; i++)
            out_tokens[(size_t)b * (D + 2) + i] = i <= n ? ho[(size_t)b * (D + 2) + i] : -1;
        s->root[b] = ho[(size_t)b * (D + 2) + n];
        total += n;
        s->accepted += n;
    }
    free(ho);
    s->steps++;
    s->drafted += (long long)(R - 1) * B;
    return total;
}

void cgx_tree_spec_stats(const cgx_tree_spec* s, long long* steps, long long* drafted,
                         long long* accepted) {
    if (steps) *steps = s ? s->steps : 0;
    if (drafted) *drafted = s ? s->drafted : 0;
    if (accepted) *accepted = s ? s->accepted : 0;
}
