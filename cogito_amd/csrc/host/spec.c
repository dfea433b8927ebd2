/*
 * spec.c -- chain speculative decoding over two device-resident models:
 * gamma draft forwards (one token each; every drafted token is sampled on
 * the GPU straight into the target's input row), one target forward over
 * [last, d_1 .. d_gamma], the verify kernels (sampling.c: D4-D6), then KV
 * rollback of both models to the accepted prefix.  One host round trip per
 * step (the emitted tokens and the accepted count).
 *
 * The reference declares the driver (cg_speculative_step / _generate,
 * include/cg_speculative.h:71-94) without defining it.
 */
#include <stdlib.h>
#include <string.h>

#include "cg_mi355x.h"
#include "cg_speculative.h"
#include "cgx_internal.h"

struct cgx_spec {
    cgx_model* draft;
    cgx_model* target;
    int gamma, V;
    float T;
    int top_k;
    float top_p;
    /* one allocation, so that a step's inputs go over in one copy:
     * d_u, then d_pending, then d_tokens */
    uint32_t* d_in;
    int* d_tokens;        /* [gamma + 1]: last, d_1 .. d_gamma */
    int* d_pending;       /* [2]: draft inputs not yet in the draft cache */
    float* d_draft_logits;
    float* d_target_logits;
    float* d_u;           /* [2 gamma + 1]: draft draws, then verify draws */
    float* d_z;           /* [V] scaled draft row for the filtered samplers */
    float* d_draft_dist;  /* [gamma][V] filtered draft distributions (with filters) */
    int* d_out;           /* [gamma + 1] emitted tokens, then n accepted */
    int last;
    int have_last;
    int pend_extra;       /* the draft cache lacks d_gamma of the last step */
    int pend_tok;
    long long steps, drafted, accepted;
};

void cgx_spec_free(cgx_spec* s) {
    if (!s) return;
    cgx_free(s->d_in);
    cgx_free(s->d_draft_logits);
    cgx_free(s->d_target_logits);
    cgx_free(s->d_z);
    cgx_free(s->d_draft_dist);
    cgx_free(s->d_out);
    free(s);
}

cgx_spec* cgx_spec_new(cgx_model* draft, cgx_model* target, int gamma, float temperature,
                       int top_k, float top_p) {
    cgx_model_config cd, ct;
    if (!draft || !target || draft == target || gamma < 1 ||
        cgx_model_get_config(draft, &cd) || cgx_model_get_config(target, &ct)) {
        cgx_set_error("cgx_spec_new: two distinct models and gamma >= 1 are required");
        return NULL;
    }
    if (cd.vocab != ct.vocab || ct.max_tokens < gamma + 1 || cd.max_tokens < 2) {
        cgx_set_error("cgx_spec_new: vocabularies differ or max_tokens too small "
                      "(target needs gamma + 1, draft 2)");
        return NULL;
    }
    cgx_spec* s = (cgx_spec*)calloc(1, sizeof(*s));
    if (!s) return NULL;
    s->draft = draft;
    s->target = target;
    s->gamma = gamma;
    s->V = ct.vocab;
    s->T = temperature;
    s->top_k = top_k;
    s->top_p = top_p;
    size_t V = (size_t)s->V;
    s->d_in = (uint32_t*)cgx_malloc((size_t)(2 * gamma + 1 + 2 + gamma + 1) * 4);
    if (s->d_in) {
        s->d_u = (float*)s->d_in;
        s->d_pending = (int*)(s->d_in + 2 * gamma + 1);
        s->d_tokens = s->d_pending + 2;
    }
    s->d_draft_logits = (float*)cgx_malloc((size_t)gamma * V * 4);
    s->d_target_logits = (float*)cgx_malloc((size_t)(gamma + 1) * V * 4);
    s->d_z = (float*)cgx_malloc(V * 4);
    s->d_out = (int*)cgx_malloc((size_t)(gamma + 2) * 4);
    /* with filters, the draft draws keep their filtered distributions for
     * the verify (the same launches compute both) */
    const int filtered = (top_k > 0 && top_k < s->V) || top_p < 1.0f;
    s->d_draft_dist = filtered ? (float*)cgx_malloc((size_t)gamma * V * 4) : NULL;
    if (!s->d_in || !s->d_draft_logits || !s->d_target_logits || !s->d_z || !s->d_out ||
        (filtered && !s->d_draft_dist)) {
        cgx_spec_free(s);
        return NULL;
    }
    return s;
}

void cgx_spec_stats(const cgx_spec* s, long long* steps, long long* drafted,
                    long long* accepted) {
    if (steps) *steps = s ? s->steps : 0;
    if (drafted) *drafted = s ? s->drafted : 0;
    if (accepted) *accepted = s ? s->accepted : 0;
}

int cgx_spec_set_last(cgx_spec* s, int last_token) {
    if (!s || last_token < 0 || last_token >= s->V) {
        cgx_set_error("cgx_spec_set_last: invalid argument");
        return -1;
    }
    if (cgx_model_len(s->draft) != cgx_model_len(s->target)) {
        cgx_set_error("cgx_spec_set_last: draft and target caches hold %d and %d positions",
                      cgx_model_len(s->draft), cgx_model_len(s->target));
        return -1;
    }
    s->last = last_token;
    s->have_last = 1;
    s->pend_extra = 0;
    return 0;
}

int cgx_spec_prefill(cgx_spec* s, const int* prompt, int n) {
    if (!s || !prompt || n < 1) {
        cgx_set_error("cgx_spec_prefill: invalid argument");
        return -1;
    }
    for (int i = 0; i < n; i++) {
        if (prompt[i] < 0 || prompt[i] >= s->V) {
            cgx_set_error("cgx_spec_prefill: token %d out of range", prompt[i]);
            return -1;
        }
    }
    cgx_model* ms[2] = {s->draft, s->target};
    for (int k = 0; k < 2; k++) {
        cgx_model_config c;
        cgx_model_get_config(ms[k], &c);
        for (int i = 0; i < n - 1; i += c.max_tokens) {
            int M = n - 1 - i < c.max_tokens ? n - 1 - i : c.max_tokens;
            if (cgx_model_forward(ms[k], prompt + i, M, 0, NULL)) return -1;
        }
    }
    if (cgx_synchronize()) return -1;
    return cgx_spec_set_last(s, prompt[n - 1]);
}

/* Draft token i + 1 from the draft logits row i, written to d_tokens[i + 1]. */
static int draft_sample(cgx_spec* s, int i, float u_host) {
    return cgx_sample_row_dev(s->d_draft_logits + (size_t)i * s->V, s->V, s->T, s->top_k,
                              s->top_p, s->d_u + i, u_host, s->d_z, s->d_tokens + i + 1,
                              s->d_draft_dist ? s->d_draft_dist + (size_t)i * s->V : NULL);
}

int cgx_spec_step(cgx_spec* s, const float* u_draft, const float* u_verify, int* out_tokens) {
    if (!s || !u_draft || !u_verify || !out_tokens) {
        cgx_set_error("cgx_spec_step: invalid argument");
        return -1;
    }
    if (!s->have_last) {
        cgx_set_error("cgx_spec_step: no context (call cgx_spec_prefill or cgx_spec_set_last)");
        return -1;
    }
    const int g = s->gamma;
    const int L = cgx_model_len(s->target);
    cgx_model_config ct, cd;
    cgx_model_get_config(s->target, &ct);
    cgx_model_get_config(s->draft, &cd);
    if (L + g + 1 > ct.max_seq || L + g + 1 > cd.max_seq) {
        cgx_set_error("cgx_spec_step: KV cache full (%d + %d)", L, g + 1);
        return -1;
    }
    /* inputs of the step in one copy: the draws, the draft's pending tokens
     * (pend_tok, last; the draft reads the last np of them), the last token */
    uint32_t hu[2 * 64 + 1 + 3];
    const size_t nin = (size_t)(2 * g + 1) + 3;
    uint32_t* hbuf = nin <= sizeof(hu) / sizeof(hu[0]) ? hu : (uint32_t*)malloc(nin * 4);
    if (!hbuf) return -1;
    const int pend[3] = {s->pend_tok, s->last, s->last};
    memcpy(hbuf, u_draft, (size_t)g * sizeof(float));
    memcpy(hbuf + g, u_verify, (size_t)(g + 1) * sizeof(float));
    memcpy(hbuf + 2 * g + 1, pend, sizeof(pend));
    const int np = s->pend_extra ? 2 : 1;
    const int rc = cgx_memcpy_h2d(s->d_in, hbuf, nin * 4);
    if (hbuf != hu) free(hbuf);
    if (rc) return -1;

    /* draft: gamma tokens */
    if (cgx_model_forward(s->draft, s->d_pending + (2 - np), np, 1, s->d_draft_logits) ||
        draft_sample(s, 0, u_draft[0]))
        return -1;
    for (int i = 1; i < g; i++) {
        if (cgx_model_forward(s->draft, s->d_tokens + i, 1, 1,
                              s->d_draft_logits + (size_t)i * s->V) ||
            draft_sample(s, i, u_draft[i]))
            return -1;
    }
    /* target: gamma + 1 rows in one forward, then the verify kernels */
    if (cgx_model_forward(s->target, s->d_tokens, g + 1, g + 1, s->d_target_logits) ||
        cgx_verify_chain_dev_q(s->d_target_logits, s->d_draft_logits, s->d_draft_dist,
                               s->d_tokens + 1, s->d_u + g, 1, g, s->V, s->T, s->top_k,
                               s->top_p, s->d_out, s->d_out + g + 1, NULL))
        return -1;
    int hout[64 + 2];
    int* ho = (g + 2) <= 66 ? hout : (int*)malloc((size_t)(g + 2) * sizeof(int));
    if (!ho) return -1;
    if (cgx_memcpy_d2h(ho, s->d_out, (size_t)(g + 2) * sizeof(int))) {
        if (ho != hout) free(ho);
        return -1;
    }
    const int n = ho[g + 1];
    memcpy(out_tokens, ho, (size_t)(n + 1) * sizeof(int));
    for (int i = n + 1; i <= g; i++) out_tokens[i] = -1;
    /* rollback: the target keeps last, d_1 .. d_n; the draft the same
     * positions it has (it never saw d_gamma) */
    const int keep = L + n + 1;
    const int dlen = cgx_model_len(s->draft);
    if (cgx_model_truncate(s->target, keep) ||
        cgx_model_truncate(s->draft, dlen < keep ? dlen : keep)) {
        if (ho != hout) free(ho);
        return -1;
    }
    s->pend_extra = n == g;
    s->pend_tok = n == g ? ho[g - 1] : 0;
    s->last = ho[n];
    if (ho != hout) free(ho);
    s->steps++;
    s->drafted += g;
    s->accepted += n;
    return n;
}

/* ------------------------------------------------------------ batches */
/*
 * B sequences in lockstep over two models built with max_batch = B (each
 * sequence has its own KV caches).  Every step:
 *   - each draft cache is cut to (target length - 1) and fed (prev, last):
 *     prev is the token at the target's last cached position, recomputed
 *     to the same K/V, so every sequence takes two draft tokens at once;
 *   - gamma - 1 more single-token draft forwards, each draft row sampled on
 *     the GPU into dtok [gamma][B];
 *   - one target forward of gamma + 1 tokens per sequence, the batched
 *     verify (verify.hip), one host round trip for the tokens and counts;
 *   - each target cache keeps last, d_1 .. d_n.
 * Unfiltered sampling only (temperature > 0, no top-k / top-p).
 */
struct cgx_spec_batch {
    cgx_model* draft;
    cgx_model* target;
    int B, gamma, V;
    float T;
    int* d_feed;            /* [B][2] prev, last */
    int* d_dtok;            /* [gamma][B] drafted tokens */
    int* d_ttok;            /* [B][gamma + 1] target input */
    int* d_vtok;            /* [B][gamma] drafted tokens per chain */
    float* d_draft_logits;  /* [B][gamma][V] */
    float* d_target_logits; /* [B][gamma + 1][V] */
    float* d_u;             /* draft draws [gamma][B], then verify draws [B][gamma + 1] */
    int* d_out;             /* [B][gamma + 1] tokens, then [B] accepted counts */
    int prev[16], last[16];
    int have_last;
    long long steps, drafted, accepted;
};

void cgx_spec_batch_free(cgx_spec_batch* s) {
    if (!s) return;
    cgx_free(s->d_feed);
    cgx_free(s->d_dtok);
    cgx_free(s->d_ttok);
    cgx_free(s->d_vtok);
    cgx_free(s->d_draft_logits);
    cgx_free(s->d_target_logits);
    cgx_free(s->d_u);
    cgx_free(s->d_out);
    free(s);
}

cgx_spec_batch* cgx_spec_batch_new(cgx_model* draft, cgx_model* target, int gamma,
                                   float temperature) {
    cgx_model_config cd, ct;
    if (!draft || !target || draft == target || gamma < 1 ||
        cgx_model_get_config(draft, &cd) || cgx_model_get_config(target, &ct)) {
        cgx_set_error("cgx_spec_batch_new: two distinct models and gamma >= 1 are required");
        return NULL;
    }
    const int B = cgx_model_batch(target);
    if (cgx_model_batch(draft) != B || cd.vocab != ct.vocab || ct.max_tokens < gamma + 1 ||
        cd.max_tokens < 2) {
        cgx_set_error("cgx_spec_batch_new: the models need the same batch and vocabulary, "
                      "max_tokens >= gamma + 1 (target) and >= 2 (draft)");
        return NULL;
    }
    if (!cgk_verify_pipe_supported(B, gamma, ct.vocab, temperature)) {
        cgx_set_error("cgx_spec_batch_new: batch %d, gamma %d, vocab %d, temperature %g "
                      "outside the batched verify", B, gamma, ct.vocab, (double)temperature);
        return NULL;
    }
    cgx_spec_batch* s = (cgx_spec_batch*)calloc(1, sizeof(*s));
    if (!s) return NULL;
    s->draft = draft;
    s->target = target;
    s->B = B;
    s->gamma = gamma;
    s->V = ct.vocab;
    s->T = temperature;
    size_t V = (size_t)s->V, g = (size_t)gamma, b = (size_t)B;
    s->d_feed = (int*)cgx_malloc(b * 2 * 4);
    s->d_dtok = (int*)cgx_malloc(g * b * 4);
    s->d_ttok = (int*)cgx_malloc(b * (g + 1) * 4);
    s->d_vtok = (int*)cgx_malloc(b * g * 4);
    s->d_draft_logits = (float*)cgx_malloc(b * g * V * 4);
    s->d_target_logits = (float*)cgx_malloc(b * (g + 1) * V * 4);
    s->d_u = (float*)cgx_malloc(b * (2 * g + 1) * 4);
    s->d_out = (int*)cgx_malloc(b * (g + 2) * 4);
    if (!s->d_feed || !s->d_dtok || !s->d_ttok || !s->d_vtok || !s->d_draft_logits ||
        !s->d_target_logits || !s->d_u || !s->d_out) {
        cgx_spec_batch_free(s);
        return NULL;
    }
    return s;
}

int cgx_spec_batch_set_last(cgx_spec_batch* s, const int* prev, const int* last) {
    if (!s || !prev || !last) {
        cgx_set_error("cgx_spec_batch_set_last: invalid argument");
        return -1;
    }
    for (int b = 0; b < s->B; b++) {
        const int lt = cgx_model_len_seq(s->target, b), ld = cgx_model_len_seq(s->draft, b);
        if (prev[b] < 0 || prev[b] >= s->V || last[b] < 0 || last[b] >= s->V || lt < 1 ||
            ld < lt - 1) {
            cgx_set_error("cgx_spec_batch_set_last: sequence %d: tokens out of range or "
                          "caches hold %d (target) / %d (draft) positions", b, lt, ld);
            return -1;
        }
        s->prev[b] = prev[b];
        s->last[b] = last[b];
    }
    s->have_last = 1;
    return 0;
}

int cgx_spec_batch_step(cgx_spec_batch* s, const float* u_draft, const float* u_verify,
                        int* out_tokens, int* n_accepted) {
    if (!s || !u_draft || !u_verify || !out_tokens || !n_accepted) {
        cgx_set_error("cgx_spec_batch_step: invalid argument");
        return -1;
    }
    if (!s->have_last) {
        cgx_set_error("cgx_spec_batch_step: no context (call cgx_spec_batch_set_last)");
        return -1;
    }
    const int B = s->B, g = s->gamma;
    cgx_model_config ct;
    cgx_model_get_config(s->target, &ct);
    int L[16];
    for (int b = 0; b < B; b++) {
        L[b] = cgx_model_len_seq(s->target, b);
        if (L[b] + g + 1 > ct.max_seq) {
            cgx_set_error("cgx_spec_batch_step: KV cache of sequence %d full", b);
            return -1;
        }
        /* the draft re-takes (prev, last) at positions L - 1, L */
        if (cgx_model_truncate_seq(s->draft, b, L[b] - 1)) return -1;
    }
    /* draws: draft [gamma][B] (transposed), verify [B][gamma + 1]; feed [B][2] */
    size_t nu = (size_t)B * (2 * g + 1);
    float* hu = (float*)malloc(nu * sizeof(float));
    int feed[32];
    if (!hu) return -1;
    for (int i = 0; i < g; i++)
        for (int b = 0; b < B; b++) hu[(size_t)i * B + b] = u_draft[(size_t)b * g + i];
    memcpy(hu + (size_t)g * B, u_verify, (size_t)B * (g + 1) * sizeof(float));
    for (int b = 0; b < B; b++) {
        feed[2 * b] = s->prev[b];
        feed[2 * b + 1] = s->last[b];
    }
    int rc = cgx_memcpy_h2d(s->d_u, hu, nu * sizeof(float)) ||
             cgx_memcpy_h2d(s->d_feed, feed, (size_t)B * 2 * sizeof(int));
    free(hu);
    if (rc) return -1;
    const size_t V = (size_t)s->V, ldd = (size_t)g * V;
    const float* ud = s->d_u;
    const float* uv = s->d_u + (size_t)g * B;
    /* draft: d_1 from (prev, last), then d_2 .. d_gamma */
    if (cgx_model_forward_batch_ld(s->draft, s->d_feed, 2, 1, s->d_draft_logits, ldd) ||
        cgx_sample_temperature_rows_dev(s->d_draft_logits, B, s->V, s->T, ud, s->d_dtok, ldd))
        return -1;
    for (int i = 1; i < g; i++) {
        if (cgx_model_forward_batch_ld(s->draft, s->d_dtok + (size_t)(i - 1) * B, 1, 1,
                                       s->d_draft_logits + (size_t)i * V, ldd) ||
            cgx_sample_temperature_rows_dev(s->d_draft_logits + (size_t)i * V, B, s->V, s->T,
                                            ud + (size_t)i * B, s->d_dtok + (size_t)i * B, ldd))
            return -1;
    }
    /* target over last, d_1 .. d_gamma of every sequence, then the verify */
    int* dn = s->d_out + (size_t)B * (g + 1);
    if (cgk_spec_tokens(s->d_feed, s->d_dtok, B, g, s->d_ttok, s->d_vtok) ||
        cgx_model_forward_batch(s->target, s->d_ttok, g + 1, g + 1, s->d_target_logits) ||
        cgk_verify_pipe(s->d_target_logits, s->d_draft_logits, s->d_vtok, uv, B, g, s->V, s->T,
                        NULL, s->d_out, dn))
        return -1;
    int* ho = (int*)malloc((size_t)B * (g + 2) * sizeof(int));
    if (!ho) return -1;
    if (cgx_memcpy_d2h(ho, s->d_out, (size_t)B * (g + 2) * sizeof(int))) {
        free(ho);
        return -1;
    }
    int total = 0;
    for (int b = 0; b < B; b++) {
        const int n = ho[(size_t)B * (g + 1) + b];
        const int* o = ho + (size_t)b * (g + 1);
        n_accepted[b] = n;
        for (int i = 0; i <= g; i++) out_tokens[(size_t)b * (g + 1) + i] = i <= n ? o[i] : -1;
        /* the target keeps last, d_1 .. d_n */
        if (cgx_model_truncate_seq(s->target, b, L[b] + n + 1)) {
            free(ho);
            return -1;
        }
        s->prev[b] = n > 0 ? o[n - 1] : s->last[b];
        s->last[b] = o[n];
        total += n;
        s->accepted += n;
    }
    free(ho);
    s->steps++;
    s->drafted += (long long)g * B;
    return total;
}

void cgx_spec_batch_stats(const cgx_spec_batch* s, long long* steps, long long* drafted,
                          long long* accepted) {
    if (steps) *steps = s ? s->steps : 0;
    if (drafted) *drafted = s ? s->drafted : 0;
    if (accepted) *accepted = s ? s->accepted : 0;
}
