/*
 * sampling.c -- cogito's samplers and the chain-verification composition on
 * top of the acceptance kernels (accept.hip).
 *
 *   cg_sample_temperature  reference src/inference/speculative.c:54-75
 *   cg_sample_corrected    reference src/inference/speculative.c:148-172
 *   cg_sample_top_p        reference src/inference/speculative.c:77-120
 *   cg_sample_top_k        reference src/inference/speculative.c:122-146
 *   cg_sample_typical      declared only (include/cg_speculative.h:186);
 *                          decision D16
 *   cgx_verify_chain       composition of those with cg_acceptance_prob
 *                          (:49-52); the reference only declares
 *                          cg_target_verify (include/cg_speculative.h:99-103)
 *
 * The drop-in samplers take host or device rows and draw their uniform from
 * the same global LCG as the reference, so a program switching libraries
 * gets the same tokens.  The cgx_*_u / cgx_verify_* forms take pre-drawn
 * uniforms.
 */
#include <stdlib.h>
#include <string.h>

#include "cg_mi355x.h"
#include "cg_speculative.h"
#include "cgx_internal.h"

static int uses_filters(int V, int top_k, float top_p) {
    return (top_k > 0 && top_k < V) || top_p < 1.0f;
}

static int read_token(const int* dev) {
    int tok = -1;
    if (cgx_memcpy_d2h(&tok, dev, sizeof(int))) return -1;
    return tok;
}

/* One token from a device logits row with the verify filters (D5): the
 * reference sampler of that filter (A3 / A4 / A5, or the kept-list scan when
 * both filters are on) over z = row / T.  The draw is at du (device); uh is
 * the same value on the host, for the single-block sampler.  z is a V-float
 * device workspace; out a device int. */
int cgx_sample_row_dev(const float* row, int V, float T, int top_k, float top_p,
                       const float* du, float uh, float* z, int* out, float* dist) {
    if (!uses_filters(V, top_k, top_p)) {
        /* one row of up to 32768 values: the single-workgroup sampler (one
         * launch, the row in registers; a certified decision first on rows
         * peaked enough for it, the exact sums otherwise) beats the
         * chunk-parallel pipeline's nine launches (C4's draft draws: 3.07 ->
         * 2.93 ms a step); longer rows take the pipeline */
        if (V > 32768 && cgk_verify_pipe_supported(1, 0, V, T))
            return cgk_sample_temperature_pipe(row, 1, V, T, du, out, (size_t)V);
        return cgk_sample_temperature(row, V, T, uh, out);
    }
    return cgk_filter_rows_t(row, T, z, 1, V, top_k, top_p, du, 1, out, 1, dist);
}

/* ------------------------------------------------ explicit-uniform forms */

int cgx_sample_temperature_u(const float* logits, int V, float T, float u) {
    if (!logits || V <= 0) {
        cgx_set_error("cgx_sample_temperature_u: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const float* d = (const float*)cgx_dev_in(logits, (size_t)V * 4, CGX_SLOT_IN0);
    int* out = (int*)cgx_scratch(CGX_SLOT_OUT1, 2 * sizeof(int));
    if (!d || !out) return -1;
    /* the loops' dispatch (cgx_sample_row_dev); the draw goes to the device
     * next to the token */
    float* du = (float*)(out + 1);
    if (cgx_memcpy_h2d(du, &u, sizeof(float)) ||
        cgx_sample_row_dev(d, V, T, 0, 1.0f, du, u, NULL, out, NULL))
        return -1;
    return read_token(out);
}

int cgx_sample_temperature_dev(const float* logits, int V, float T, float u, int* out_dev) {
    if (!logits || !out_dev || V <= 0) {
        cgx_set_error("cgx_sample_temperature_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    if (V > 32768 && cgk_verify_pipe_supported(1, 0, V, T)) {
        float* du = (float*)cgx_scratch(CGX_SLOT_OUT1, sizeof(float));
        if (!du || cgx_memcpy_h2d(du, &u, sizeof(float))) return -1;
        return cgx_sample_row_dev(logits, V, T, 0, 1.0f, du, u, NULL, out_dev, NULL);
    }
    return cgx_sample_row_dev(logits, V, T, 0, 1.0f, NULL, u, NULL, out_dev, NULL);
}

int cgx_sample_temperature_rows_dev(const float* logits, int rows, int V, float T,
                                    const float* u_dev, int* out_dev, size_t ld) {
    if (!logits || !u_dev || !out_dev || rows < 1 || V <= 0) {
        cgx_set_error("cgx_sample_temperature_rows_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    /* rows of up to 32768 values: one workgroup per row, all in one launch
     * (the rows in registers, the certified decision first); longer rows:
     * the chunk-parallel pipeline over all of them */
    if (V > 32768 && cgk_verify_pipe_supported(rows, 0, V, T))
        return cgk_sample_temperature_pipe(logits, rows, V, T, u_dev, out_dev, ld);
    return cgk_sample_temperature_rows(logits, rows, V, T, u_dev, out_dev, ld);
}

int cgx_sample_corrected_u(const float* draft_probs, const float* target_probs,
                           int V, float u) {
    if (!draft_probs || !target_probs || V <= 0) {
        cgx_set_error("cgx_sample_corrected_u: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const float* q = (const float*)cgx_dev_in(draft_probs, (size_t)V * 4, CGX_SLOT_IN0);
    const float* p = (const float*)cgx_dev_in(target_probs, (size_t)V * 4, CGX_SLOT_IN1);
    int* out = (int*)cgx_scratch(CGX_SLOT_OUT1, sizeof(int));
    if (!q || !p || !out || cgk_sample_corrected(q, p, V, u, out)) return -1;
    return read_token(out);
}

int cgx_filtered_dist(const float* logits, int V, float T, int top_k, float top_p,
                      float* dist_out) {
    if (!logits || !dist_out || V <= 0) {
        cgx_set_error("cgx_filtered_dist: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const float* d = (const float*)cgx_dev_in(logits, (size_t)V * 4, CGX_SLOT_IN0);
    int out_dev = cgx_is_device_ptr(dist_out);
    float* o = out_dev ? dist_out : (float*)cgx_scratch(CGX_SLOT_OUT0, (size_t)V * 4);
    if (!d || !o) return -1;
    if (uses_filters(V, top_k, top_p)) {
        float* z = (float*)cgx_scratch(CGX_SLOT_WS3, (size_t)V * 4);
        if (!z || cgk_filter_rows_t(d, T, z, 1, V, top_k, top_p, NULL, 0, NULL, 0, o))
            return -1;
    } else if (cgk_temperature_probs(d, V, T, o)) {
        return -1;
    }
    if (!out_dev) return cgx_memcpy_d2h(dist_out, o, (size_t)V * 4);
    return cgx_synchronize();
}

int cgx_exact_expf_dev(const float* x, float* y, int n) {
    if (!x || !y || n < 0) {
        cgx_set_error("cgx_exact_expf_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    return n ? cgk_exact_expf(x, y, n) : 0;
}

int cgx_typ_log_dev(const float* x, double* y, int n) {
    if (!x || !y || n < 0) {
        cgx_set_error("cgx_typ_log_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    return n ? cgk_typ_log(x, y, n) : 0;
}

int cgx_exp_fast_maxerr_dev(float lo, float hi, unsigned int* out_dev) {
    if (!out_dev) {
        cgx_set_error("cgx_exp_fast_maxerr_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    return cgk_exp_fast_maxerr(lo, hi, out_dev);
}

int cgx_exp_stat_maxerr_dev(float lo, float hi, unsigned int* out_dev) {
    if (!out_dev) {
        cgx_set_error("cgx_exp_stat_maxerr_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    return cgk_exp_stat_maxerr(lo, hi, out_dev);
}

int cgx_sort_rows_dev(const uint32_t* keys, const uint32_t* payload, int rows, int n,
                      int descending, uint32_t* keys_out, uint32_t* payload_out) {
    if (!keys || !keys_out || rows <= 0 || n <= 0) {
        cgx_set_error("cgx_sort_rows_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const size_t wb = cgk_row_sort_ws(rows, n, payload_out != NULL);
    void* ws = cgx_scratch(CGX_SLOT_WS5, wb);
    if (!ws || cgk_row_sort(keys, payload, rows, n, descending, keys_out, payload_out, ws, wb))
        return -1;
    return cgx_synchronize();
}

int cgx_ordered_sum_dev(const float* x, int n, float* out_dev) {
    if (!x || !out_dev || n <= 0) {
        cgx_set_error("cgx_ordered_sum_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    return cgk_ordered_sum(x, n, out_dev);
}

/* ------------------------------------------------------ drop-in samplers */

int cg_sample_temperature(float* logits, int vocab_size, float temperature) {
    float u = cgx_lcg_draw();
    return cgx_sample_temperature_u(logits, vocab_size, temperature, u);
}

int cg_sample_corrected(float* draft_probs, float* target_probs, int vocab_size) {
    float u = cgx_lcg_draw();
    return cgx_sample_corrected_u(draft_probs, target_probs, vocab_size, u);
}

/* cg_sample_top_k (speculative.c:122-146): k >= V is cg_sample_temperature
 * at T = 1; k <= 0 is rejected (the reference indexes top_vals[-1]). */
int cgx_sample_top_k_u(const float* logits, int V, int top_k, float u) {
    if (!logits || V <= 0 || top_k <= 0) {
        cgx_set_error("cgx_sample_top_k_u: invalid argument (logits, V > 0, top_k > 0)");
        return -1;
    }
    if (top_k >= V) return cgx_sample_temperature_u(logits, V, 1.0f, u);
    if (cgx_ensure_init()) return -1;
    const float* d = (const float*)cgx_dev_in(logits, (size_t)V * 4, CGX_SLOT_IN0);
    float* du = (float*)cgx_scratch(CGX_SLOT_IN1, sizeof(float));
    int* out = (int*)cgx_scratch(CGX_SLOT_OUT1, sizeof(int));
    if (!d || !du || !out || cgx_memcpy_h2d(du, &u, sizeof(float)) ||
        cgk_filter_rows(d, 1, V, top_k, 1.0f, du, out, NULL))
        return -1;
    return read_token(out);
}

/* cg_sample_top_p (speculative.c:77-120), for any top_p. */
int cgx_sample_top_p_u(const float* logits, int V, float top_p, float u) {
    if (!logits || V <= 0) {
        cgx_set_error("cgx_sample_top_p_u: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const float* d = (const float*)cgx_dev_in(logits, (size_t)V * 4, CGX_SLOT_IN0);
    float* du = (float*)cgx_scratch(CGX_SLOT_IN1, sizeof(float));
    int* out = (int*)cgx_scratch(CGX_SLOT_OUT1, sizeof(int));
    if (!d || !du || !out || cgx_memcpy_h2d(du, &u, sizeof(float)) ||
        cgk_filter_rows(d, 1, V, 0, top_p, du, out, NULL))
        return -1;
    return read_token(out);
}

/* cg_sample_typical (declared only in the reference, include/
 * cg_speculative.h:186): decision D16, the typical kernels of filter.hip. */
int cgx_sample_typical_u(const float* logits, int V, float typical_p, float u) {
    if (!logits || V <= 0) {
        cgx_set_error("cgx_sample_typical_u: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const float* d = (const float*)cgx_dev_in(logits, (size_t)V * 4, CGX_SLOT_IN0);
    float* du = (float*)cgx_scratch(CGX_SLOT_IN1, sizeof(float));
    int* out = (int*)cgx_scratch(CGX_SLOT_OUT1, sizeof(int));
    if (!d || !du || !out || cgx_memcpy_h2d(du, &u, sizeof(float)) ||
        cgk_typical_rows(d, 1, V, typical_p, du, out, NULL))
        return -1;
    return read_token(out);
}

int cg_sample_typical(float* logits, int vocab_size, float typical_p) {
    float u = cgx_lcg_draw();
    return cgx_sample_typical_u(logits, vocab_size, typical_p, u);
}

int cgx_typical_dist(const float* logits, int V, float typical_p, float* dist_out) {
    if (!logits || !dist_out || V <= 0) {
        cgx_set_error("cgx_typical_dist: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const float* d = (const float*)cgx_dev_in(logits, (size_t)V * 4, CGX_SLOT_IN0);
    int out_dev = cgx_is_device_ptr(dist_out);
    float* o = out_dev ? dist_out : (float*)cgx_scratch(CGX_SLOT_OUT0, (size_t)V * 4);
    if (!d || !o || cgk_typical_rows(d, 1, V, typical_p, NULL, NULL, o)) return -1;
    if (!out_dev) return cgx_memcpy_d2h(dist_out, o, (size_t)V * 4);
    return cgx_synchronize();
}

int cg_sample_top_k(float* logits, int vocab_size, int top_k) {
    float u = cgx_lcg_draw();
    return cgx_sample_top_k_u(logits, vocab_size, top_k, u);
}

int cg_sample_top_p(float* logits, int vocab_size, float top_p) {
    float u = cgx_lcg_draw();
    return cgx_sample_top_p_u(logits, vocab_size, top_p, u);
}

/* ------------------------------------------------------------- verify */

/* D5 verify: filtered distributions of every row, then the same accept /
 * correction composition over them; the bonus token is the filtered
 * sampler's draw from target row gamma, taken in the same launches as the
 * target rows' distributions.  qdist: the draft rows' distributions when the
 * caller has them (the loop's draft draws write them), else NULL. */
static int verify_filtered(const float* target, const float* draft, const float* qdist,
                           const int* tokens, const float* u, int batch, int gamma, int V,
                           float T, int top_k, float top_p, float* ap, int* corr, int* bonus,
                           int* out_tokens, int* n_accepted) {
    size_t rt = (size_t)batch * (gamma + 1), rd = qdist ? 0 : (size_t)batch * gamma;
    float* z = (float*)cgx_scratch(CGX_SLOT_WS3, (rt + rd) * V * 4);
    float* dist = (float*)cgx_scratch(CGX_SLOT_WS2, (rt + rd) * V * 4);
    if (!z || !dist) return -1;
    float* zt = z;
    float* zd = z + rt * V;
    float* p = dist;
    float* q = dist + rt * V;
    if (cgk_filter_rows_t(target, T, zt, (int)rt, V, top_k, top_p, u + gamma, gamma + 1, bonus,
                          gamma + 1, p))
        return -1;
    if (!qdist && cgk_filter_rows_t(draft, T, zd, (int)rd, V, top_k, top_p, NULL, 0, NULL, 0, q))
        return -1;
    return cgk_verify_chain_dist(p, qdist ? qdist : q, tokens, u, batch, gamma, V, bonus, ap,
                                 corr, out_tokens, n_accepted);
}


int cgx_verify_chain_batch_dev(const float* target_logits, const float* draft_logits,
                               const int* draft_tokens, const float* u, int batch,
                               int gamma, int V, float temperature, int top_k,
                               float top_p, int* out_tokens, int* n_accepted,
                               float* accept_prob) {
    return cgx_verify_chain_dev_q(target_logits, draft_logits, NULL, draft_tokens, u, batch,
                                  gamma, V, temperature, top_k, top_p, out_tokens, n_accepted,
                                  accept_prob);
}

int cgx_verify_chain_dev_q(const float* target_logits, const float* draft_logits,
                           const float* qdist, const int* draft_tokens, const float* u,
                           int batch, int gamma, int V, float temperature, int top_k,
                           float top_p, int* out_tokens, int* n_accepted, float* accept_prob) {
    if (!target_logits || !draft_logits || !draft_tokens || !u || !out_tokens ||
        !n_accepted || batch <= 0 || gamma <= 0 || V <= 0) {
        cgx_set_error("cgx_verify_chain_batch_dev: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    size_t na = (size_t)batch * gamma;
    char* ws = (char*)cgx_scratch(CGX_SLOT_WS1, na * 4 * 2 + (size_t)batch * 4 + 256);
    if (!ws) return -1;
    float* ap = accept_prob ? accept_prob : (float*)ws;
    int* corr = (int*)(ws + na * 4);
    int* bonus = (int*)(ws + na * 8);
    if (uses_filters(V, top_k, top_p))
        return verify_filtered(target_logits, draft_logits, qdist, draft_tokens, u, batch,
                               gamma, V, temperature, top_k, top_p, ap, corr, bonus,
                               out_tokens, n_accepted);
    if (cgk_verify_pipe_supported(batch, gamma, V, temperature))
        return cgk_verify_pipe(target_logits, draft_logits, draft_tokens, u, batch, gamma, V,
                               temperature, accept_prob, out_tokens, n_accepted);
    return cgk_verify_chain(target_logits, draft_logits, draft_tokens, u, batch, gamma, V,
                            temperature, ap, corr, bonus, out_tokens, n_accepted);
}

int cgx_verify_chain_batch_dev_noalloc(const float* target_logits, const float* draft_logits,
                                       const int* draft_tokens, const float* u, int batch,
                                       int gamma, int V, float temperature, int top_k,
                                       float top_p, int* out_tokens, int* n_accepted,
                                       float* accept_prob) {
    if (!target_logits || !draft_logits || !draft_tokens || !u || !out_tokens ||
        !n_accepted || batch <= 0 || gamma <= 0 || V <= 0) {
        cgx_set_error("cgx_verify_chain_batch_dev_noalloc: invalid argument");
        return -1;
    }
    if (uses_filters(V, top_k, top_p)) {
        cgx_set_error("cgx_verify_chain_batch_dev_noalloc: top-k / top-p verification needs "
                      "cgx_verify_chain_batch_dev");
        return -1;
    }
    if (!cgk_verify_pipe_supported(batch, gamma, V, temperature)) {
        cgx_set_error("cgx_verify_chain_batch_dev_noalloc: batch %d, gamma %d, V %d, "
                      "temperature %g outside the verify pipeline", batch, gamma, V,
                      (double)temperature);
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    return cgk_verify_pipe_static(cgx_device_id(), target_logits, draft_logits, draft_tokens, u,
                                  batch, gamma, V, temperature, accept_prob, out_tokens,
                                  n_accepted);
}

int cgx_verify_chain(const float* target_logits, const float* draft_logits,
                     const int* draft_tokens, const float* u, int gamma, int V,
                     float temperature, int top_k, float top_p, int* out_tokens,
                     float* accept_prob) {
    if (!target_logits || !draft_logits || !draft_tokens || !u || !out_tokens ||
        gamma <= 0 || V <= 0) {
        cgx_set_error("cgx_verify_chain: invalid argument");
        return -1;
    }
    if (cgx_ensure_init()) return -1;
    const float* t = (const float*)cgx_dev_in(target_logits, (size_t)(gamma + 1) * V * 4,
                                              CGX_SLOT_IN0);
    const float* d = (const float*)cgx_dev_in(draft_logits, (size_t)gamma * V * 4,
                                              CGX_SLOT_IN1);
    const int* x = (const int*)cgx_dev_in(draft_tokens, (size_t)gamma * 4, CGX_SLOT_IN2);
    const float* uu = (const float*)cgx_dev_in(u, (size_t)(gamma + 1) * 4, CGX_SLOT_IN3);
    char* o = (char*)cgx_scratch(CGX_SLOT_OUT1, (size_t)(gamma + 1) * 4 + (size_t)gamma * 4 + 64);
    if (!t || !d || !x || !uu || !o) return -1;
    int* dtok = (int*)o;
    float* dap = (float*)(o + (size_t)(gamma + 1) * 4);
    int* dn = (int*)(o + (size_t)(gamma + 1) * 4 + (size_t)gamma * 4);
    /* the ratios only when asked for: without them the pipeline settles most
     * accept tests from its segment statistics (same tokens) */
    if (cgx_verify_chain_batch_dev(t, d, x, uu, 1, gamma, V, temperature, top_k, top_p,
                                   dtok, dn, accept_prob ? dap : NULL))
        return -1;
    int n = -1;
    if (cgx_memcpy_d2h(out_tokens, dtok, (size_t)(gamma + 1) * 4) ||
        cgx_memcpy_d2h(&n, dn, 4))
        return -1;
    if (accept_prob && cgx_memcpy_d2h(accept_prob, dap, (size_t)gamma * 4)) return -1;
    return n;
}
