/*
 * check.c -- drives the CPU checkers (oracle/cg_oracle.c) and the library's
 * host-only modules (tensor.c, speculative.c, serialize.c) through random
 * and edge-case inputs under AddressSanitizer and UndefinedBehaviorSanitizer
 * (tests/sanitize/Makefile).  Exit status 0 and no sanitizer report is a
 * pass.  Test infrastructure only.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cg_oracle.h"
#include "cg_mi355x.h"

static uint64_t g_s = 0x9e3779b97f4a7c15ull;
static double unif(void) {   /* splitmix64 -> [0, 1) */
    uint64_t z = (g_s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return (double)((z ^ (z >> 31)) >> 11) * 0x1p-53;
}
static float gauss(float s) {
    double a = unif() + 1e-12, b = unif();
    return (float)(s * sqrt(-2 * log(a)) * cos(6.283185307179586 * b));
}
static void fill(float* x, int n, float s, int kind) {
    for (int i = 0; i < n; i++)
        x[i] = kind == 0 ? gauss(s) : kind == 1 ? (float)((int)(unif() * 4) - 2)
             : kind == 2 ? 0.0f : (unif() < 0.9 ? -1e30f : gauss(s));
}

static void samplers(int V) {
    float* t = malloc(sizeof(float) * 5 * V);
    float* d = malloc(sizeof(float) * 4 * V);
    float* p = malloc(sizeof(float) * V);
    float* q = malloc(sizeof(float) * V);
    float* sp = malloc(sizeof(float) * V);
    int* si = malloc(sizeof(int) * V);
    int x[4], out[5], lidx[8];
    float u[5], ap[4], lp[8], mass;
    for (int kind = 0; kind < 4; kind++) {
        fill(t, 5 * V, 2.0f, kind);
        fill(d, 4 * V, 2.0f, kind);
        for (int i = 0; i < 5; i++) u[i] = (float)unif();
        for (int i = 0; i < 4; i++) x[i] = (int)(unif() * V);
        orc_temperature_probs(t, V, 0.7f, p);
        orc_temperature_probs(d, V, 1.0f, q);
        orc_sample_temperature(t, V, 1.3f, u[0]);
        orc_sample_corrected(q, p, V, u[1]);
        orc_sample_corrected(p, p, V, u[1]);            /* zero residual: fallback */
        for (int k = 1; k < V; k += V / 3 + 1) orc_sample_top_k(t, V, k, u[2]);
        orc_top_p_sorted(t, V, 0.9f, sp, si, &mass);
        orc_sample_top_p(t, V, 0.0f, u[3]);
        orc_sample_top_p(t, V, 1.0f, u[3]);
        for (int k = 0; k <= V; k += V / 2 + 1)
            for (float tp = 0.3f; tp <= 1.0f; tp += 0.35f) {
                orc_filtered_dist(t, V, 0.8f, k, tp, p);
                orc_sample_filtered(t, V, 0.8f, k, tp, u[4]);
                orc_verify_chain(t, d, x, u, 4, V, 0.8f, k, tp, out, ap);
            }
        orc_typical_dist(t, V, 0.9f, p);
        orc_sample_typical(t, V, 0.5f, u[0]);
        if (V > 8) orc_topk_lists(t, V, 8, 0.9f, lidx, lp);
    }
    int par[7] = {-1, 0, 0, 1, 1, 2, 5}, tok[7], opath[8], o[9];
    int K = 4;
    int* li = malloc(sizeof(int) * 7 * K);
    float* lpv = malloc(sizeof(float) * 7 * K);
    for (int i = 0; i < 7; i++) {
        if (V > K) orc_topk_lists(t + i % 5 * V, V, K, 1.0f, li + i * K, lpv + i * K);
        else for (int j = 0; j < K; j++) { li[i * K + j] = 0; lpv[i * K + j] = 0.25f; }
        tok[i] = li[i * K];
    }
    float tu[4 * 5];
    for (int i = 0; i < 20; i++) tu[i] = (float)unif();
    orc_tree_accept(par, 7, K, li, lpv, tok, tu, o, opath);
    free(li); free(lpv);
    free(t); free(d); free(p); free(q); free(sp); free(si);
}

static void int4_and_attention(void) {
    const int K = 64, N = 48, gs = 16, M = 3;
    float* w = malloc(sizeof(float) * K * N);
    float* x = malloc(sizeof(float) * M * K);
    float* y = malloc(sizeof(float) * M * N);
    uint8_t* data = malloc(K * N / 2);
    float* sc = malloc(sizeof(float) * K * N / gs);
    fill(w, K * N, 0.05f, 0);
    memset(w, 0, sizeof(float) * gs);                   /* an all-zero group */
    fill(x, M * K, 1.0f, 0);
    orc_quantize_int4(w, K * N, gs, data, sc);
    orc_dequantize_int4(data, sc, K * N, gs, w);
    orc_matmul_int4(x, M, K, data, sc, N, gs, y);
    uint8_t odd[3];
    float osc[2], ov[5] = {1, -2, 3, 0.5f, -7};
    orc_quantize_int4(ov, 5, 3, odd, osc);               /* group not dividing n */
    const int H = 4, Hk = 2, D = 16, S = 20, kgs = 8;
    uint8_t* kc = calloc(S * Hk * D / 2, 1);
    uint8_t* vc = calloc(S * Hk * D / 2, 1);
    float* ks = calloc(S * Hk * D / kgs, sizeof(float));
    float* vs = calloc(S * Hk * D / kgs, sizeof(float));
    float kt[Hk * D], vt[Hk * D];
    for (int pos = 0; pos < S; pos++) {
        fill(kt, Hk * D, 1.0f, pos == 3 ? 2 : 0);
        fill(vt, Hk * D, 1.0f, 0);
        orc_kv_append(kc, vc, ks, vs, pos, Hk, D, kgs, kt, vt);
    }
    float* Kf = malloc(sizeof(float) * S * Hk * D);
    float* Vf = malloc(sizeof(float) * S * Hk * D);
    orc_kv_get(kc, vc, ks, vs, S, Hk, D, kgs, Kf, Vf);
    const int Nq = 5;
    float* Q = malloc(sizeof(float) * Nq * H * D);
    float* O = malloc(sizeof(float) * Nq * H * D);
    float* lse = malloc(sizeof(float) * H * Nq);
    float* mask = malloc(sizeof(float) * Nq * S);
    fill(Q, Nq * H * D, 1.0f, 0);
    for (int i = 0; i < Nq * S; i++) mask[i] = unif() < 0.3 ? -INFINITY : 0.0f;
    for (int mt = 0; mt <= 4; mt++)
        orc_flash_fwd(Q, Kf, Vf, O, lse, 1, Nq, S, H, Hk, D, 0.25f, mt, 3, mask);
    orc_apply_rope(Q, Nq, H, D, 7, 10000.0f);
    float cs[S * D / 2], sn[S * D / 2], slopes[8], bias[8 * 3 * 4];
    orc_rope_freqs(cs, sn, S, D, 10000.0f);
    orc_alibi_slopes(slopes, 8);
    orc_alibi_bias(bias, 3, 4, 8, slopes);
    float g[10], uu[10], a[10], nw[16], r[2 * 16];
    fill(g, 10, 3.0f, 0);
    fill(uu, 10, 1.0f, 0);
    orc_swiglu(g, uu, a, 10);
    for (int i = 0; i < 16; i++) nw[i] = 1.0f;
    orc_rmsnorm(Q, nw, r, 2, 16, 1e-5f);
    orc_softmax_rows(Q, r, 2, 16);
    float nrm[37];
    orc_fill_normal(nrm, 37, 12345, 7, 0.02f);
    float chain[(6 + 3) * (6 + 3)];
    orc_tree_mask_chain(chain, 6, 3);
    free(w); free(x); free(y); free(data); free(sc); free(kc); free(vc); free(ks); free(vs);
    free(Kf); free(Vf); free(Q); free(O); free(lse); free(mask);
}

static int host_modules(const char* dir) {
    int fails = 0;
    cg_token_tree* t = cg_token_tree_new(5);
    for (int i = 0; i < 5; i++) t->tokens[i] = 10 + i;
    cg_token_tree_add_token(t, 3, NULL);
    cg_tensor* tt = cg_token_tree_to_tensor(t);
    cg_tensor* m = cg_tree_attention_mask(t, 7);
    int par[6] = {-1, 0, 0, 1, -1, 4};
    cg_tensor* mp = cgx_tree_attention_mask_parents(par, 6, 3);
    fails += !tt || !m || !mp || m->size != 144 || mp->size != 81;
    cg_tensor_free(tt); cg_tensor_free(m); cg_tensor_free(mp);
    cg_token_tree_free(t);
    cg_token_tree_free(cg_token_tree_new(0));
    int shape[3] = {2, 3, 4};
    cg_tensor* a = cg_tensor_full(shape, 3, 1.5f, false);
    cg_tensor* b = cg_tensor_clone(a);
    int ns[2] = {6, 4};
    cg_tensor_reshape(b, ns, 2);
    cg_tensor_retain(a);
    cg_tensor_release(a);
    fails += cg_tensor_shape_equal(a, b);
    char path[512];
    snprintf(path, sizeof(path), "%s/m.cog", dir);
    cg_tensor* arr[2] = {a, b};
    const char* names[2] = {"a", "b"};
    cg_save_model(path, arr, names, 2);
    cg_tensor** lt = NULL;
    char** ln = NULL;
    int lc = 0;
    cg_load_model(path, &lt, &ln, &lc);
    fails += lc != 2;
    for (int i = 0; i < lc; i++) {
        fails += memcmp(lt[i]->data, arr[i]->data, sizeof(float) * 24) != 0;
        cg_tensor_free(lt[i]);
        free(ln[i]);
    }
    free(lt); free(ln);
    /* INT4 entries */
    const int K = 8, N = 6, gs = 4;
    float w[8 * 6];
    fill(w, K * N, 0.1f, 0);
    cg_tensor_quant q;
    memset(&q, 0, sizeof(q));
    int qshape[2] = {K, N};
    uint8_t data[24];
    float sc[12], zs[12] = {0};
    orc_quantize_int4(w, K * N, gs, data, sc);
    q.data = data; q.scales = sc; q.zeros = zs; q.shape = qshape; q.ndim = 2;
    q.size = K * N; q.quant_type = QUANT_INT4; q.group_size = gs; q.num_groups = 12;
    cg_tensor_quant* qa[1] = {&q};
    const char* qn[1] = {"w"};
    snprintf(path, sizeof(path), "%s/q.cog", dir);
    fails += cgx_save_quantized(path, qa, qn, 1) != 0;
    cg_tensor_quant** lq = NULL;
    char** lqn = NULL;
    int lqc = 0;
    fails += cgx_load_quantized(path, &lq, &lqn, &lqc) != 0 || lqc != 1;
    for (int i = 0; i < lqc; i++) {
        fails += memcmp(lq[i]->data, data, 24) != 0 || memcmp(lq[i]->scales, sc, 48) != 0;
        cg_tensor_quant_free(lq[i]);
        free(lqn[i]);
    }
    free(lq); free(lqn);
    cg_tensor_free(a);
    cg_tensor_free(b);
    return fails;
}

int main(int argc, char** argv) {
    const char* dir = argc > 1 ? argv[1] : ".";
    int Vs[] = {1, 2, 3, 17, 300};
    for (int i = 0; i < 5; i++) samplers(Vs[i]);
    int4_and_attention();
    uint32_t st = 42;
    for (int i = 0; i < 100; i++) orc_lcg_uniform(&st);
    const int fails = host_modules(dir);
    printf("sanitize check: %s (%d failed checks)\n", fails ? "FAIL" : "ok", fails);
    return fails ? 1 : 0;
}
