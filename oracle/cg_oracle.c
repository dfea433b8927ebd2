/*
 * cg_oracle.c -- CPU restatement of cogito's verify-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see cg_oracle.h).  Built with
 *   gcc -O2 -ffp-contract=off -fPIC -shared  (no -march=native)
 * so that every float expression rounds exactly where the reference's does.
 * Loops keep the reference's operation order; where the reference allocates
 * per call, so does this file, because the CPU baseline times it as the
 * reference's algorithm.
 */
#include "cg_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Planted mistakes for the tests that prove the law checks have power
 * (tests/test_verify_law.py builds one library per value; the product
 * oracle is built with 0):
 *   1  the correction draw reuses the accept test's uniform u[i];
 *   2  the acceptance ratio takes p and q swapped;
 *   3  top-p keeps the cut probabilities without renormalising them;
 *   4  the bonus draw reuses the last accept test's uniform u[gamma-1]. */
#ifndef ORC_MUTANT
#define ORC_MUTANT 0
#endif

/* ---------------------------------------------------------------- A1, A2 */

uint32_t orc_lcg_next_state(uint32_t state) {
    /* speculative.c:12: spec_seed = spec_seed * 1103515245 + 12345 (uint) */
    return state * 1103515245u + 12345u;
}

float orc_lcg_uniform(uint32_t* state) {
    *state = orc_lcg_next_state(*state);
    return (float)(*state % 10000u) / 10000.0f;
}

float orc_acceptance_prob(float draft_prob, float target_prob) {
    /* speculative.c:49-52 */
    if (draft_prob < 1e-10f) return 1.0f;
    return fminf(1.0f, target_prob / draft_prob);
}

/* -------------------------------------------------------------------- A3 */

void orc_temperature_probs(const float* logits, int V, float T, float* probs) {
    /* speculative.c:55-64: max scan, expf((l - max) / T), running sum,
     * then every entry divided by the sum. */
    float max_logit = logits[0];
    for (int i = 1; i < V; i++)
        if (logits[i] > max_logit) max_logit = logits[i];
    float sum = 0.0f;
    for (int i = 0; i < V; i++) {
        probs[i] = expf((logits[i] - max_logit) / T);
        sum += probs[i];
    }
    for (int i = 0; i < V; i++) probs[i] /= sum;
}

int orc_sample_temperature(const float* logits, int V, float T, float u) {
    float* probs = (float*)malloc((size_t)V * sizeof(float));
    orc_temperature_probs(logits, V, T, probs);
    /* speculative.c:66-72: first i with r < cumsum, default V - 1 */
    float r = u;
    float cumsum = 0.0f;
    int token = V - 1;
    for (int i = 0; i < V; i++) {
        cumsum += probs[i];
        if (r < cumsum) { token = i; break; }
    }
    free(probs);
    return token;
}

/* -------------------------------------------------------------------- A4 */

void orc_top_k_list(const float* logits, int V, int k, float* vals, int* idx) {
    /* speculative.c:128-139: insertion into a descending list; strict '>'
     * keeps the earlier index ahead of a later equal value. */
    for (int i = 0; i < k; i++) { vals[i] = -1e30f; idx[i] = 0; }
    for (int i = 0; i < V; i++) {
        if (logits[i] > vals[k - 1]) {
            vals[k - 1] = logits[i];
            idx[k - 1] = i;
            for (int j = k - 1; j > 0 && vals[j] > vals[j - 1]; j--) {
                float tv = vals[j]; vals[j] = vals[j - 1]; vals[j - 1] = tv;
                int ti = idx[j]; idx[j] = idx[j - 1]; idx[j - 1] = ti;
            }
        }
    }
}

int orc_sample_top_k(const float* logits, int V, int k, float u) {
    /* speculative.c:122-146 */
    if (k >= V) return orc_sample_temperature(logits, V, 1.0f, u);
    float* vals = (float*)malloc((size_t)k * sizeof(float));
    int* idx = (int*)malloc((size_t)k * sizeof(int));
    orc_top_k_list(logits, V, k, vals, idx);
    int t = orc_sample_temperature(vals, k, 1.0f, u);
    int result = idx[t];
    free(vals);
    free(idx);
    return result;
}

/* -------------------------------------------------------------------- A5 */

int orc_top_p_sorted(const float* logits, int V, float top_p,
                     float* probs, int* indices, float* cum_at_cutoff) {
    /* speculative.c:81-90: softmax at T = 1 (no division by T) */
    float max_logit = logits[0];
    for (int i = 1; i < V; i++)
        if (logits[i] > max_logit) max_logit = logits[i];
    float sum = 0.0f;
    for (int i = 0; i < V; i++) {
        probs[i] = expf(logits[i] - max_logit);
        indices[i] = i;
        sum += probs[i];
    }
    for (int i = 0; i < V; i++) probs[i] /= sum;
    /* speculative.c:93-100: selection sort that swaps on every strictly
     * larger element (not stable) */
    for (int i = 0; i < V - 1; i++) {
        for (int j = i + 1; j < V; j++) {
            if (probs[j] > probs[i]) {
                float tp = probs[i]; probs[i] = probs[j]; probs[j] = tp;
                int ti = indices[i]; indices[i] = indices[j]; indices[j] = ti;
            }
        }
    }
    /* speculative.c:102-107: inclusive cutoff */
    float cumsum = 0.0f;
    int cutoff = V;
    for (int i = 0; i < V; i++) {
        cumsum += probs[i];
        if (cumsum >= top_p) { cutoff = i + 1; break; }
    }
    *cum_at_cutoff = cumsum;
    return cutoff;
}

int orc_sample_top_p(const float* logits, int V, float top_p, float u) {
    float* probs = (float*)malloc((size_t)V * sizeof(float));
    int* indices = (int*)malloc((size_t)V * sizeof(int));
    float cumsum;
    int cutoff = orc_top_p_sorted(logits, V, top_p, probs, indices, &cumsum);
    /* speculative.c:109-115 */
    float r = u * cumsum;
    cumsum = 0.0f;
    int token = indices[0];
    for (int i = 0; i < cutoff; i++) {
        cumsum += probs[i];
        if (r < cumsum) { token = indices[i]; break; }
    }
    free(probs);
    free(indices);
    return token;
}

/* -------------------------------------------------------------------- A6 */

int orc_sample_corrected(const float* draft_probs, const float* target_probs,
                         int V, float u) {
    /* speculative.c:148-172 */
    float* adjusted = (float*)malloc((size_t)V * sizeof(float));
    float sum = 0.0f;
    for (int i = 0; i < V; i++) {
        adjusted[i] = fmaxf(0.0f, target_probs[i] - draft_probs[i]);
        sum += adjusted[i];
    }
    if (sum < 1e-10f) {
        free(adjusted);
        /* :157-160 the target probabilities are passed as logits */
        return orc_sample_temperature(target_probs, V, 1.0f, u);
    }
    float r = u * sum;
    float cumsum = 0.0f;
    int token = 0;
    for (int i = 0; i < V; i++) {
        cumsum += adjusted[i];
        if (r < cumsum) { token = i; break; }
    }
    free(adjusted);
    return token;
}

/* ------------------------------------------------- verify composition (A7) */

static int use_top_k(int top_k, int V) { return top_k > 0 && top_k < V; }
static int use_top_p(float top_p) { return top_p < 1.0f; }

/* Cutoff rule of speculative.c:102-107 applied to an already descending
 * list (the top-k list). */
static int list_cutoff(const float* pr, int n, float top_p, float* mass) {
    float cumsum = 0.0f;
    int cutoff = n;
    for (int i = 0; i < n; i++) {
        cumsum += pr[i];
        if (cumsum >= top_p) { cutoff = i + 1; break; }
    }
    *mass = cumsum;
    return cutoff;
}

int orc_filtered_dist(const float* logits, int V, float T, int top_k,
                      float top_p, float* dist) {
    int uk = use_top_k(top_k, V), up = use_top_p(top_p);
    int nz = 0;
    if (!uk && !up) {
        orc_temperature_probs(logits, V, T, dist);
        for (int i = 0; i < V; i++) nz += dist[i] != 0.0f;
        return nz;
    }
    float* z = (float*)malloc((size_t)V * sizeof(float));
    for (int i = 0; i < V; i++) z[i] = logits[i] / T;
    memset(dist, 0, (size_t)V * sizeof(float));
    if (uk) {
        float* vals = (float*)malloc((size_t)top_k * sizeof(float));
        int* idx = (int*)malloc((size_t)top_k * sizeof(int));
        float* pr = (float*)malloc((size_t)top_k * sizeof(float));
        orc_top_k_list(z, V, top_k, vals, idx);
        orc_temperature_probs(vals, top_k, 1.0f, pr);
        int keep = top_k;
        float mass = 1.0f;
        if (up) keep = list_cutoff(pr, top_k, top_p, &mass);
#if ORC_MUTANT == 3
        mass = 1.0f;
#endif
        for (int j = 0; j < keep; j++) {
            float v = up ? pr[j] / mass : pr[j];
            if (v != 0.0f) { dist[idx[j]] = v; nz++; }
        }
        free(vals); free(idx); free(pr);
    } else {
        float* sp = (float*)malloc((size_t)V * sizeof(float));
        int* si = (int*)malloc((size_t)V * sizeof(int));
        float mass;
        int keep = orc_top_p_sorted(z, V, top_p, sp, si, &mass);
#if ORC_MUTANT == 3
        mass = 1.0f;
#endif
        for (int j = 0; j < keep; j++) {
            float v = sp[j] / mass;
            if (v != 0.0f) { dist[si[j]] = v; nz++; }
        }
        free(sp); free(si);
    }
    free(z);
    return nz;
}

int orc_sample_filtered(const float* logits, int V, float T, int top_k,
                        float top_p, float u) {
    int uk = use_top_k(top_k, V), up = use_top_p(top_p);
    if (!uk && !up) return orc_sample_temperature(logits, V, T, u);
    float* z = (float*)malloc((size_t)V * sizeof(float));
    for (int i = 0; i < V; i++) z[i] = logits[i] / T;
    int token;
    if (uk && !up) {
        token = orc_sample_top_k(z, V, top_k, u);
    } else if (!uk) {
        token = orc_sample_top_p(z, V, top_p, u);
    } else {
        float* vals = (float*)malloc((size_t)top_k * sizeof(float));
        int* idx = (int*)malloc((size_t)top_k * sizeof(int));
        float* pr = (float*)malloc((size_t)top_k * sizeof(float));
        orc_top_k_list(z, V, top_k, vals, idx);
        orc_temperature_probs(vals, top_k, 1.0f, pr);
        float mass;
        int keep = list_cutoff(pr, top_k, top_p, &mass);
        /* the scan of speculative.c:109-115 over the kept list */
        float r = u * mass, cumsum = 0.0f;
        token = idx[0];
        for (int j = 0; j < keep; j++) {
            cumsum += pr[j];
            if (r < cumsum) { token = idx[j]; break; }
        }
        free(vals); free(idx); free(pr);
    }
    free(z);
    return token;
}

int orc_verify_chain(const float* target_logits, const float* draft_logits,
                     const int* draft_tokens, const float* u, int gamma, int V,
                     float T, int top_k, float top_p,
                     int* out_tokens, float* accept_prob) {
    float* p = (float*)malloc((size_t)V * sizeof(float));
    float* q = (float*)malloc((size_t)V * sizeof(float));
    int n = -1;
    for (int i = 0; i < gamma; i++) {
        orc_filtered_dist(target_logits + (size_t)i * V, V, T, top_k, top_p, p);
        orc_filtered_dist(draft_logits + (size_t)i * V, V, T, top_k, top_p, q);
        int x = draft_tokens[i];
#if ORC_MUTANT == 2
        float a = orc_acceptance_prob(p[x], q[x]);
#else
        float a = orc_acceptance_prob(q[x], p[x]);
#endif
        if (accept_prob) accept_prob[i] = a;
        if (n >= 0) continue;              /* decisions stop at the first reject */
        if (u[i] < a) {
            out_tokens[i] = x;
        } else {
#if ORC_MUTANT == 1
            out_tokens[i] = orc_sample_corrected(q, p, V, u[i]);
#else
            out_tokens[i] = orc_sample_corrected(q, p, V, u[i + 1]);
#endif
            n = i;
        }
    }
    if (n < 0) {
        n = gamma;
#if ORC_MUTANT == 4
        float ub = u[gamma - 1];
#else
        float ub = u[gamma];
#endif
        out_tokens[gamma] = orc_sample_filtered(
            target_logits + (size_t)gamma * V, V, T, top_k, top_p, ub);
    }
    free(p);
    free(q);
    return n;
}

void orc_verify_chain_many(const float* target_logits, const float* draft_logits,
                           const int* draft_tokens, const float* u, int N, int gamma,
                           int V, float T, int top_k, float top_p, int* out_tokens,
                           int* n_accepted) {
    /* N independent calls of orc_verify_chain on the same logits: draw set k
     * is draft_tokens[k][gamma] and u[k][gamma + 1].  A loop only, so that
     * the law tests can afford 10^5 draws per case. */
    for (int k = 0; k < N; k++)
        n_accepted[k] = orc_verify_chain(target_logits, draft_logits,
                                         draft_tokens + (size_t)k * gamma,
                                         u + (size_t)k * (gamma + 1), gamma, V, T, top_k,
                                         top_p, out_tokens + (size_t)k * (gamma + 1), NULL);
}

/* ------------------------------------------------------ typical sampling */

/* Natural log of a positive finite float in binary64 by a fixed sequence of
 * IEEE operations (no FMA), the same bits on any conforming host or device:
 * x = m 2^k with m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(s) with
 * s = (m - 1) / (m + 1), |s| <= 0.1716, and atanh(s) = s (1 + s^2/3 + s^4/5
 * + ... + s^24/25) (truncation below 2^-60). */
double orc_typ_log(float x) {
    static const double kLn2 = 0x1.62e42fefa39efp-1;
    static const double kSqrt2 = 0x1.6a09e667f3bcdp+0;
    static const double kC[13] = {1.0,        1.0 / 3.0,  1.0 / 5.0,  1.0 / 7.0,  1.0 / 9.0,
                                  1.0 / 11.0, 1.0 / 13.0, 1.0 / 15.0, 1.0 / 17.0, 1.0 / 19.0,
                                  1.0 / 21.0, 1.0 / 23.0, 1.0 / 25.0};
    double d = (double)x;
    uint64_t b;
    memcpy(&b, &d, sizeof(b));
    int k = (int)((b >> 52) & 0x7ff) - 1023;
    b = (b & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m;
    memcpy(&m, &b, sizeof(m));
    if (m > kSqrt2) {
        m = m * 0.5;
        k += 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double q = kC[12];
    for (int j = 11; j >= 0; j--) q = kC[j] + s2 * q;
    return (double)k * kLn2 + 2.0 * (s * q);
}

typedef struct {
    float score;
    int idx;
} typ_key;

static int typ_cmp(const void* a, const void* b) {
    const typ_key* x = (const typ_key*)a;
    const typ_key* y = (const typ_key*)b;
    if (x->score < y->score) return -1;
    if (x->score > y->score) return 1;
    return (x->idx > y->idx) - (x->idx < y->idx);
}

int orc_typical_sorted(const float* logits, int V, float typical_p, float* probs, int* order,
                       float* mass) {
    /* Decision D16 (cg_sample_typical is declared only in the reference,
     * include/cg_speculative.h:186; locally typical sampling, Meister et al.
     * 2023), written in the reference samplers' style: the softmax of
     * cg_sample_top_p (speculative.c:81-90); L_i = (float)log p_i;
     * H = sum_i fl(p_i * -L_i) left to right in fp32 (p_i = 0 adds 0);
     * score_i = |fl(-L_i - H)| (+inf for p_i = 0); tokens ordered by (score
     * ascending, index ascending); the first `cutoff` of that order with the
     * cumsum >= typical_p rule of speculative.c:102-107. */
    orc_temperature_probs(logits, V, 1.0f, probs);
    float* L = (float*)malloc((size_t)V * sizeof(float));
    float H = 0.0f;
    for (int i = 0; i < V; i++) {
        L[i] = probs[i] > 0.0f ? (float)orc_typ_log(probs[i]) : 0.0f;
        if (probs[i] > 0.0f) H += probs[i] * -L[i];
    }
    typ_key* key = (typ_key*)malloc((size_t)V * sizeof(typ_key));
    for (int i = 0; i < V; i++) {
        key[i].score = probs[i] > 0.0f ? fabsf(-L[i] - H) : INFINITY;
        key[i].idx = i;
    }
    qsort(key, (size_t)V, sizeof(typ_key), typ_cmp);
    float cumsum = 0.0f;
    int cutoff = V;
    for (int j = 0; j < V; j++) {
        order[j] = key[j].idx;
        if (cutoff == V) {
            cumsum += probs[key[j].idx];
            if (cumsum >= typical_p) cutoff = j + 1;
        }
    }
    *mass = cumsum;
    free(L);
    free(key);
    return cutoff;
}

int orc_sample_typical(const float* logits, int V, float typical_p, float u) {
    float* probs = (float*)malloc((size_t)V * sizeof(float));
    int* order = (int*)malloc((size_t)V * sizeof(int));
    float mass;
    const int cutoff = orc_typical_sorted(logits, V, typical_p, probs, order, &mass);
    /* the draw of speculative.c:109-115 over the kept tokens */
    float r = u * mass, cumsum = 0.0f;
    int token = order[0];
    for (int j = 0; j < cutoff; j++) {
        cumsum += probs[order[j]];
        if (r < cumsum) {
            token = order[j];
            break;
        }
    }
    free(probs);
    free(order);
    return token;
}

void orc_typical_dist(const float* logits, int V, float typical_p, float* dist) {
    float* probs = (float*)malloc((size_t)V * sizeof(float));
    int* order = (int*)malloc((size_t)V * sizeof(int));
    float mass;
    const int cutoff = orc_typical_sorted(logits, V, typical_p, probs, order, &mass);
    memset(dist, 0, (size_t)V * sizeof(float));
    for (int j = 0; j < cutoff; j++) dist[order[j]] = probs[order[j]] / mass;
    free(probs);
    free(order);
}

/* ------------------------------------------------------------ A9 .. A12 */

static uint8_t orc_pack(int8_t a, int8_t b) {
    return (uint8_t)((a & 0x0F) | ((b & 0x0F) << 4));
}

static void orc_unpack(uint8_t packed, int8_t* a, int8_t* b) {
    /* include/cg_quantize.h:162-168: low nibble first, sign-extend bit 3 */
    *a = (int8_t)(packed & 0x0F);
    *b = (int8_t)((packed >> 4) & 0x0F);
    if (*a & 0x08) *a |= (int8_t)0xF0;
    if (*b & 0x08) *b |= (int8_t)0xF0;
}

void orc_quantize_int4(const float* x, int n, int gs, uint8_t* data,
                       float* scales) {
    /* int4.c:19-39: absmax / 7 per flat group, floor 1e-10 -> 1 */
    int ng = (n + gs - 1) / gs;
    for (int g = 0; g < ng; g++) {
        int start = g * gs, end = start + gs;
        if (end > n) end = n;
        float absmax = 0.0f;
        for (int i = start; i < end; i++) {
            float a = fabsf(x[i]);
            if (a > absmax) absmax = a;
        }
        scales[g] = absmax / 7.0f;
        if (scales[g] < 1e-10f) scales[g] = 1.0f;
    }
    /* int4.c:42-56: roundf(x / scale), clamp to [-8, 7], pack pairs */
    for (int i = 0; i < n; i += 2) {
        float s = scales[i / gs];
        int8_t v0 = (int8_t)roundf(x[i] / s);
        if (v0 > 7) v0 = 7;
        if (v0 < -8) v0 = -8;
        int8_t v1 = 0;
        if (i + 1 < n) {
            v1 = (int8_t)roundf(x[i + 1] / s);
            if (v1 > 7) v1 = 7;
            if (v1 < -8) v1 = -8;
        }
        data[i / 2] = orc_pack(v0, v1);
    }
}

void orc_dequantize_int4(const uint8_t* data, const float* scales, int n,
                         int gs, float* out) {
    /* int4.c:64-76 with zeros = 0: ((float)v - 0) * scale */
    for (int i = 0; i < n; i += 2) {
        float s = scales[i / gs];
        int8_t v0, v1;
        orc_unpack(data[i / 2], &v0, &v1);
        out[i] = ((float)v0 - 0.0f) * s;
        if (i + 1 < n) out[i + 1] = ((float)v1 - 0.0f) * s;
    }
}

void orc_matmul_int4(const float* x, int M, int K, const uint8_t* data,
                     const float* scales, int N, int gs, float* y) {
    /* int4.c:90-114: sequential k, w_idx = k*N + j, zeros ignored */
    memset(y, 0, (size_t)M * N * sizeof(float));
    for (int i = 0; i < M; i++) {
        for (int j = 0; j < N; j++) {
            float sum = 0.0f;
            for (int k = 0; k < K; k++) {
                int w_idx = k * N + j;
                float scale = scales[w_idx / gs];
                int8_t v0, v1;
                orc_unpack(data[w_idx / 2], &v0, &v1);
                int8_t w = (w_idx % 2 == 0) ? v0 : v1;
                sum += x[i * K + k] * (float)w * scale;
            }
            y[i * N + j] = sum;
        }
    }
}

/* -------------------------------------------------------------------- A14 */

void orc_kv_append(uint8_t* kc, uint8_t* vc, float* ks, float* vs,
                   int pos, int H, int D, int gs,
                   const float* k_tok, const float* v_tok) {
    /* int4.c:155-231 for one token at `pos` of one layer slice */
    int ngh = D / gs;
    uint8_t* kp = kc + (size_t)pos * H * (D / 2);
    uint8_t* vp = vc + (size_t)pos * H * (D / 2);
    float* ksp = ks + (size_t)pos * H * ngh;
    float* vsp = vs + (size_t)pos * H * ngh;
    for (int h = 0; h < H; h++) {
        for (int g = 0; g < ngh; g++) {
            float mk = 0.0f, mv = 0.0f;
            int start = g * gs;
            for (int i = 0; i < gs; i++) {
                float ak = fabsf(k_tok[h * D + start + i]);
                if (ak > mk) mk = ak;
                float av = fabsf(v_tok[h * D + start + i]);
                if (av > mv) mv = av;
            }
            float sk = mk / 7.0f;
            if (sk < 1e-8f) sk = 1.0f;
            ksp[h * ngh + g] = sk;
            float sv = mv / 7.0f;
            if (sv < 1e-8f) sv = 1.0f;
            vsp[h * ngh + g] = sv;
            for (int i = 0; i < gs; i += 2) {
                int d = start + i;
                int8_t k0 = (int8_t)roundf(k_tok[h * D + d] / sk);
                int8_t k1 = (int8_t)roundf(k_tok[h * D + d + 1] / sk);
                if (k0 > 7) k0 = 7;
                if (k0 < -8) k0 = -8;
                if (k1 > 7) k1 = 7;
                if (k1 < -8) k1 = -8;
                kp[h * (D / 2) + d / 2] = orc_pack(k0, k1);
                int8_t v0 = (int8_t)roundf(v_tok[h * D + d] / sv);
                int8_t v1 = (int8_t)roundf(v_tok[h * D + d + 1] / sv);
                if (v0 > 7) v0 = 7;
                if (v0 < -8) v0 = -8;
                if (v1 > 7) v1 = 7;
                if (v1 < -8) v1 = -8;
                vp[h * (D / 2) + d / 2] = orc_pack(v0, v1);
            }
        }
    }
}

void orc_kv_get(const uint8_t* kc, const uint8_t* vc, const float* ks,
                const float* vs, int len, int H, int D, int gs,
                float* k_out, float* v_out) {
    /* int4.c:255-288: (float)v * scale into [len][H][D] */
    int ng = D / gs;
    for (int t = 0; t < len; t++) {
        size_t toff = (size_t)t * H * (D / 2), soff = (size_t)t * H * ng;
        for (int h = 0; h < H; h++) {
            for (int g = 0; g < ng; g++) {
                float sk = ks[soff + h * ng + g], sv = vs[soff + h * ng + g];
                int start = g * gs;
                for (int i = 0; i < gs; i += 2) {
                    int8_t k0, k1, v0, v1;
                    orc_unpack(kc[toff + h * (D / 2) + (start + i) / 2], &k0, &k1);
                    orc_unpack(vc[toff + h * (D / 2) + (start + i) / 2], &v0, &v1);
                    size_t o = ((size_t)t * H + h) * D + start + i;
                    k_out[o] = (float)k0 * sk;
                    k_out[o + 1] = (float)k1 * sk;
                    v_out[o] = (float)v0 * sv;
                    v_out[o + 1] = (float)v1 * sv;
                }
            }
        }
    }
}

/* -------------------------------------------------------------------- A17 */

void orc_flash_fwd(const float* Q, const float* K, const float* Vv, float* O,
                   float* lse, int B, int Nq, int Nk, int H, int Hk, int D,
                   float scale, int mask_type, int window, const float* mask) {
    /* flash_attn_kernels.c:261-396, Br = Bc = 64, K-tile outer loop */
    const int Br = 64, Bc = 64;
    for (int b = 0; b < B; b++) {
        for (int h = 0; h < H; h++) {
            int hk = h * Hk / H;
            float* m = (float*)malloc((size_t)Nq * sizeof(float));
            float* l = (float*)malloc((size_t)Nq * sizeof(float));
            float* acc = (float*)calloc((size_t)Nq * D, sizeof(float));
            for (int i = 0; i < Nq; i++) { m[i] = -FLT_MAX; l[i] = 0.0f; }
            for (int ks0 = 0; ks0 < Nk; ks0 += Bc) {
                int ke = ks0 + Bc < Nk ? ks0 + Bc : Nk, kt = ke - ks0;
                for (int qs0 = 0; qs0 < Nq; qs0 += Br) {
                    int qe = qs0 + Br < Nq ? qs0 + Br : Nq, qt = qe - qs0;
                    float* S = (float*)malloc((size_t)qt * kt * sizeof(float));
                    for (int qi = 0; qi < qt; qi++) {
                        int q = qs0 + qi;
                        for (int ki = 0; ki < kt; ki++) {
                            int k = ks0 + ki;
                            float dot = 0.0f;
                            for (int d = 0; d < D; d++)
                                dot += Q[(((size_t)b * Nq + q) * H + h) * D + d] *
                                       K[(((size_t)b * Nk + k) * Hk + hk) * D + d];
                            dot *= scale;
                            if (mask_type == 1 && k > q) dot = -FLT_MAX;
                            if (mask_type == 2 && abs(k - q) > window) dot = -FLT_MAX;
                            if (mask_type == 3) dot = dot + mask[(size_t)q * Nk + k];
                            if (mask_type == 4 && k > Nk - Nq + q) dot = -FLT_MAX;
                            S[qi * kt + ki] = dot;
                        }
                    }
                    for (int qi = 0; qi < qt; qi++) {
                        int q = qs0 + qi;
                        float mn = m[q];
                        for (int ki = 0; ki < kt; ki++)
                            if (S[qi * kt + ki] > mn) mn = S[qi * kt + ki];
                        float ln = l[q] * expf(m[q] - mn);
                        for (int ki = 0; ki < kt; ki++) ln += expf(S[qi * kt + ki] - mn);
                        float so = expf(m[q] - mn);
                        for (int d = 0; d < D; d++) acc[q * D + d] *= so;
                        for (int d = 0; d < D; d++) {
                            for (int ki = 0; ki < kt; ki++) {
                                int k = ks0 + ki;
                                float pr = expf(S[qi * kt + ki] - mn);
                                acc[q * D + d] +=
                                    pr * Vv[(((size_t)b * Nk + k) * Hk + hk) * D + d];
                            }
                        }
                        m[q] = mn;
                        l[q] = ln;
                    }
                    free(S);
                }
            }
            for (int q = 0; q < Nq; q++) {
                for (int d = 0; d < D; d++)
                    O[(((size_t)b * Nq + q) * H + h) * D + d] = acc[q * D + d] / l[q];
                if (lse) lse[((size_t)b * H + h) * Nq + q] = m[q] + logf(l[q]);
            }
            free(m); free(l); free(acc);
        }
    }
}

/* ---------------------------------------------------------- A18 .. A22 */

void orc_rope_freqs(float* cos_c, float* sin_c, int max_s, int D, float theta) {
    /* flash_attn.c:318-328 */
    for (int pos = 0; pos < max_s; pos++) {
        for (int i = 0; i < D / 2; i++) {
            float freq = 1.0f / powf(theta, (float)(2 * i) / D);
            float angle = pos * freq;
            cos_c[pos * (D / 2) + i] = cosf(angle);
            sin_c[pos * (D / 2) + i] = sinf(angle);
        }
    }
}

void orc_apply_rope(float* x, int S, int H, int D, int pos0, float theta) {
    /* flash_attn.c:335-360 (one tensor; the reference rotates Q and K with
     * the same loop) */
    int half = D / 2;
    for (int pos = 0; pos < S; pos++) {
        int ap = pos0 + pos;
        for (int h = 0; h < H; h++) {
            float* v = x + ((size_t)pos * H + h) * D;
            for (int i = 0; i < half; i++) {
                float freq = 1.0f / powf(theta, (float)(2 * i) / D);
                float angle = ap * freq;
                float c = cosf(angle), s = sinf(angle);
                float x0 = v[i], x1 = v[i + half];
                v[i] = x0 * c - x1 * s;
                v[i + half] = x0 * s + x1 * c;
            }
        }
    }
}

static uint32_t lowbias32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

uint32_t orc_fill_key(uint64_t seed, uint32_t stream_id) {
    uint32_t k = (uint32_t)seed ^ (uint32_t)(seed >> 32) * 0x9E3779B9u;
    k = k * 0x85EBCA6Bu + stream_id * 0xC2B2AE35u;
    k ^= k >> 15;
    k *= 0x2C1B3C6Du;
    k ^= k >> 12;
    return k;
}

void orc_fill_normal(float* out, size_t n, uint64_t seed, uint32_t stream_id, float stddev) {
    uint32_t key = orc_fill_key(seed, stream_id);
    float scale = (float)((double)stddev * sqrt(3.0) / 65536.0);
    for (size_t i = 0; i < n; i++) {
        uint32_t a = lowbias32(key + 2u * (uint32_t)i);
        uint32_t b = lowbias32(key + 2u * (uint32_t)i + 1u);
        int s = (int)(a & 0xFFFF) + (int)(a >> 16) + (int)(b & 0xFFFF) + (int)(b >> 16);
        out[i] = (float)(s - 131070) * scale;
    }
}

void orc_alibi_slopes(float* slopes, int H) {
    /* flash_attn.c:368-374: base = 2^(-8/H), slope_h = base^(h+1) */
    float base = powf(2.0f, -8.0f / H);
    for (int h = 0; h < H; h++) slopes[h] = powf(base, (float)(h + 1));
}

void orc_alibi_bias(float* bias, int Sq, int Sk, int H, const float* slopes) {
    /* flash_attn.c:376-388: bias[h][q][k] = slope_h * (k - q) */
    for (int h = 0; h < H; h++)
        for (int q = 0; q < Sq; q++)
            for (int k = 0; k < Sk; k++)
                bias[((size_t)h * Sq + q) * Sk + k] = slopes[h] * (k - q);
}

void orc_rmsnorm(const float* x, const float* w, float* y, int rows, int d,
                 float eps) {
    /* tensor_kernels.c:894-907 */
    for (int b = 0; b < rows; b++) {
        const float* xr = x + (size_t)b * d;
        float* yr = y + (size_t)b * d;
        float rms = 0.0f;
        for (int i = 0; i < d; i++) rms += xr[i] * xr[i];
        rms = sqrtf(rms / d + eps);
        for (int i = 0; i < d; i++) yr[i] = w[i] * xr[i] / rms;
    }
}

void orc_swiglu(const float* g, const float* u, float* out, int n) {
    /* transformer.c:122-127 */
    for (int i = 0; i < n; i++) {
        float gv = g[i];
        float sg = gv / (1.0f + expf(-gv));
        out[i] = sg * u[i];
    }
}

void orc_softmax_rows(const float* x, float* y, int rows, int V) {
    /* tensor_kernels.c:716-738 */
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * V;
        float* yr = y + (size_t)r * V;
        float mx = -INFINITY;
        for (int i = 0; i < V; i++) if (xr[i] > mx) mx = xr[i];
        float sum = 0.0f;
        for (int i = 0; i < V; i++) { float e = expf(xr[i] - mx); yr[i] = e; sum += e; }
        for (int i = 0; i < V; i++) yr[i] /= sum;
    }
}

void orc_tree_mask_chain(float* mask, int seqlen, int depth) {
    /* speculative.c:205-235 */
    int size = seqlen + depth;
    for (int i = 0; i < size * size; i++) mask[i] = -1e9f;
    for (int i = 0; i < seqlen; i++)
        for (int j = 0; j <= i; j++) mask[i * size + j] = 0.0f;
    for (int i = 0; i < depth; i++) {
        int r = seqlen + i;
        for (int j = 0; j < seqlen; j++) mask[r * size + j] = 0.0f;
        for (int j = 0; j <= i; j++) mask[r * size + seqlen + j] = 0.0f;
    }
}

/* ------------------------------------------------------------ tree walk */

void orc_topk_lists(const float* z, int V, int k, float top_p, int* lidx, float* lp) {
    /* the list of cg_sample_top_k (speculative.c:122-146) over z = logits / T:
     * entry j = (index, probability), the probabilities the softmax of the
     * list at T = 1 (speculative.c:54-75), then the top-p cutoff of the
     * filtered verify (list_cutoff) renormalised; 0 past the cutoff */
    float* vals = (float*)malloc((size_t)k * sizeof(float));
    float* pr = (float*)malloc((size_t)k * sizeof(float));
    orc_top_k_list(z, V, k, vals, lidx);
    orc_temperature_probs(vals, k, 1.0f, pr);
    int keep = k;
    float mass = 1.0f;
    int up = use_top_p(top_p);
    if (up) keep = list_cutoff(pr, k, top_p, &mass);
    for (int j = 0; j < k; j++) lp[j] = j < keep ? (up ? pr[j] / mass : pr[j]) : 0.0f;
    free(vals);
    free(pr);
}

int orc_tree_accept(const int* parent, int nodes, int K, const int* lidx, const float* lp,
                    const int* tok, const float* u, int* out, int* path) {
    /* No reference counterpart (cogito's EAGLE tree builder is a stub,
     * speculative.c:244-262).  Recursive rejection with point-mass drafts:
     * at the current node (target list lidx/lp [nodes][K]) candidate x of
     * rank r is accepted with probability w[x] / W (u[s][r] < w[x] / W),
     * else its mass is removed; no candidate left: draw from w / W with
     * u[s][4] by the scan of speculative.c:66-72 (r = u * W, first running
     * sum above r); u [depth + 1][5]; returns the accepted count. */
    int depth = 0, dep[64], nk[64], kids[64][4];
    memset(nk, 0, sizeof nk);
    dep[0] = 0;
    for (int i = 1; i < nodes; i++) {
        dep[i] = dep[parent[i]] + 1;
        if (dep[i] > depth) depth = dep[i];
        kids[parent[i]][nk[parent[i]]++] = i;
    }
    float w[64];
    int node = 0, n = 0;
    for (int s = 0; s <= depth; s++) {
        const int* li = lidx + (size_t)node * K;
        const float* pl = lp + (size_t)node * K;
        float W = 0.0f;
        for (int j = 0; j < K; j++) { w[j] = pl[j]; W += w[j]; }
        int next = -1;
        for (int r = 0; r < nk[node]; r++) {
            int c = kids[node][r], x = tok[c], jx = -1;
            for (int j = 0; j < K; j++)
                if (w[j] > 0.0f && li[j] == x) { jx = j; break; }
            float a = jx >= 0 ? w[jx] / W : 0.0f;
            if (u[s * 5 + r] < a) { next = c; break; }
            if (jx >= 0) { W -= w[jx]; w[jx] = 0.0f; }
        }
        if (next >= 0) {
            path[n] = next;
            out[n++] = tok[next];
            node = next;
            continue;
        }
        if (!(W > 0.0f)) {
            W = 0.0f;
            for (int j = 0; j < K; j++) { w[j] = pl[j]; W += w[j]; }
        }
        float rr = u[s * 5 + 4] * W, cum = 0.0f;
        int t = li[0];
        for (int j = 0; j < K; j++) {
            if (!(w[j] > 0.0f)) continue;
            cum += w[j];
            t = li[j];
            if (rr < cum) break;
        }
        out[n] = t;
        break;
    }
    return n;
}
