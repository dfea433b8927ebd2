/*
 * cg_oracle.h -- CPU restatement of cogito's verify-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (cogito_amd/) may link,
 * load or call this code; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, as the checker.
 *
 * Every function restates one reference function with the same fp32
 * operation order (compiled with -O2 -ffp-contract=off, glibc libm), over
 * plain arrays instead of cg_tensor.  Citations are to cogito-ml/cogito.
 *
 * Pinning (see tests/): each function is checked against the compiled
 * reference (oracle/_ref, where /root/reference is present), against the
 * committed golden fixtures made from it (tests/golden/), and against closed
 * forms.  Functions that go beyond the reference are pinned by what the
 * mathematics fixes: the verify composition and the filtered distribution by
 * the losslessness of speculative sampling and a float64 recomputation
 * (tests/test_verify_law.py, with planted mistakes that the checks catch),
 * the tree walk likewise (tests/test_tree_oracle.py); the corrected KV cache
 * and the aligned causal mask by closed forms.
 */
#ifndef CG_ORACLE_H
#define CG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A1: global LCG of src/inference/speculative.c:11-12. */
uint32_t orc_lcg_next_state(uint32_t state);
float orc_lcg_uniform(uint32_t* state);

/* A2: src/inference/speculative.c:49-52. */
float orc_acceptance_prob(float draft_prob, float target_prob);

/* A3: src/inference/speculative.c:54-75, with the uniform passed in. */
int orc_sample_temperature(const float* logits, int V, float T, float u);
/* The probability vector A3 builds before its CDF scan (:55-64). */
void orc_temperature_probs(const float* logits, int V, float T, float* probs);

/* A4: src/inference/speculative.c:122-146.  orc_top_k_list returns the
 * insertion-sorted list of :128-139 (vals descending, ties: earlier index
 * first). */
void orc_top_k_list(const float* logits, int V, int k, float* vals, int* idx);
int orc_sample_top_k(const float* logits, int V, int k, float u);

/* A5: src/inference/speculative.c:77-120 including its O(V^2) unstable
 * selection sort (:93-100).  orc_top_p_sorted exposes the sorted
 * probabilities / indices and returns the cutoff count (:102-107). */
int orc_top_p_sorted(const float* logits, int V, float top_p,
                     float* sorted_probs, int* sorted_idx, float* cum_at_cutoff);
int orc_sample_top_p(const float* logits, int V, float top_p, float u);

/* A6: src/inference/speculative.c:148-172 (u is the single draw it makes,
 * in either branch). */
int orc_sample_corrected(const float* draft_probs, const float* target_probs,
                         int V, float u);

/* Filtered distribution used by the verify composition (decision D5 of the
 * build): z = logits / T; top-k (A4 list) -> softmax over the list (A3 with
 * T = 1) -> top-p over that (A5 cutoff rule) -> renormalise by the kept mass.
 * top_k <= 0 or >= V: no top-k.  top_p >= 1: no top-p.  With neither filter
 * this is exactly orc_temperature_probs.  Composed from A3/A4/A5.
 * Returns the number of nonzero entries written into dist[V]. */
int orc_filtered_dist(const float* logits, int V, float T, int top_k,
                      float top_p, float* dist);
/* Draw from that distribution exactly as the reference sampler of the same
 * filter would (A3 / A4 / A5 scans). */
int orc_sample_filtered(const float* logits, int V, float T, int top_k,
                        float top_p, float u);

/* A7: chain verification (decisions D4, D6 of the build; the reference only
 * declares cg_target_verify, include/cg_speculative.h:99-103).
 *   target_logits [gamma+1][V], draft_logits [gamma][V], draft_tokens[gamma]
 *   u: the uniforms in draw order; draw k is u[k].  Accept tests consume
 *   u[0..j]; the final token consumes u[j+1] (u[gamma] if all accepted).
 * Writes out_tokens[0..n] (accepted drafts then correction/bonus), returns n
 * (accepted count).  accept_prob[gamma] (optional) gets the ratios. */
int orc_verify_chain(const float* target_logits, const float* draft_logits,
                     const int* draft_tokens, const float* u, int gamma, int V,
                     float T, int top_k, float top_p,
                     int* out_tokens, float* accept_prob);

/* orc_verify_chain over N draw sets on the same logits (a plain loop, for
 * the law tests): draft_tokens [N][gamma], u [N][gamma+1], out_tokens
 * [N][gamma+1], n_accepted [N]. */
void orc_verify_chain_many(const float* target_logits, const float* draft_logits,
                           const int* draft_tokens, const float* u, int N, int gamma,
                           int V, float T, int top_k, float top_p, int* out_tokens,
                           int* n_accepted);

/* Typical sampling (decision D16 of the build; the reference declares
 * cg_sample_typical, include/cg_speculative.h:186, without a definition).
 * orc_typ_log: log of a positive float in binary64 by a fixed IEEE sequence
 * (shared bit for bit with the device).  orc_typical_sorted: probabilities
 * (probs[V]), the typical order (order[V]) and the kept count; *mass gets
 * the kept mass.  Pinned by closed forms and brute force in
 * tests/test_typical_oracle.py. */
double orc_typ_log(float x);
int orc_typical_sorted(const float* logits, int V, float typical_p, float* probs, int* order,
                       float* mass);
int orc_sample_typical(const float* logits, int V, float typical_p, float u);
void orc_typical_dist(const float* logits, int V, float typical_p, float* dist);

/* A9-A12: include/cg_quantize.h:155-175, src/quantize/int4.c:10-114. */
void orc_quantize_int4(const float* x, int n, int group_size,
                       uint8_t* data, float* scales);
void orc_dequantize_int4(const uint8_t* data, const float* scales, int n,
                         int group_size, float* out);
void orc_matmul_int4(const float* x, int M, int K, const uint8_t* data,
                     const float* scales, int N, int group_size, float* y);

/* A14: src/quantize/int4.c:147-289 for one layer slice.  Cache arrays are
 * [max_seq][H][D/2] bytes and [max_seq][H][D/gs] scales; the token is
 * written at `pos` (the build's per-token position rule, decision D8). */
void orc_kv_append(uint8_t* kc, uint8_t* vc, float* ks, float* vs,
                   int pos, int H, int D, int gs,
                   const float* k_tok, const float* v_tok);
void orc_kv_get(const uint8_t* kc, const uint8_t* vc, const float* ks,
                const float* vs, int len, int H, int D, int gs,
                float* k_out, float* v_out);

/* A17: src/cuda/flash_attn_kernels.c:261-396 (GQA online softmax, Br=Bc=64).
 * mask_type: 0 none, 1 causal, 2 sliding window, 3 custom additive mask
 * [Nq][Nk], 4 causal aligned bottom-right (query i sees [0, Nk-Nq+i]).
 * Types 0-2 are the reference's rules; 3-4 are the build's verify masks
 * (decision D7), applied at the same point of the loop. */
void orc_flash_fwd(const float* Q, const float* K, const float* V, float* O,
                   float* lse, int B, int Nq, int Nk, int H, int Hk, int D,
                   float scale, int mask_type, int window, const float* mask);

/* A18: src/attention/flash_attn.c:330-362 (in place on [S][H][D]). */
void orc_apply_rope(float* x, int S, int H, int D, int pos0, float theta);
/* src/attention/flash_attn.c:318-328. */
void orc_rope_freqs(float* cos_c, float* sin_c, int max_s, int D, float theta);
/* Seeded weights of the synthetic stack (no reference counterpart; the
 * rule the library documents for cgx_fill_normal_dev): lowbias32 counter
 * hash, four 16-bit uniforms per value, centred sum times
 * std * sqrt(3) / 65536. */
uint32_t orc_fill_key(uint64_t seed, uint32_t stream_id);
void orc_fill_normal(float* out, size_t n, uint64_t seed, uint32_t stream_id, float stddev);

/* ALiBi slopes and bias (src/attention/flash_attn.c:368-388). */
void orc_alibi_slopes(float* slopes, int H);
void orc_alibi_bias(float* bias, int Sq, int Sk, int H, const float* slopes);

/* A19: src/cuda/tensor_kernels.c:888-909. */
void orc_rmsnorm(const float* x, const float* w, float* y, int rows, int d,
                 float eps);
/* A20: src/layers/transformer.c:122-127. */
void orc_swiglu(const float* g, const float* u, float* out, int n);
/* A22: src/cuda/tensor_kernels.c:699-740 (last-axis softmax). */
void orc_softmax_rows(const float* x, float* y, int rows, int V);

/* Tree mask of src/inference/speculative.c:197-238 (chain). */
void orc_tree_mask_chain(float* mask, int seqlen, int depth);
void orc_topk_lists(const float* z, int V, int k, float top_p, int* lidx, float* lp);
int orc_tree_accept(const int* parent, int nodes, int K, const int* lidx, const float* lp,
                    const int* tok, const float* u, int* out, int* path);

#ifdef __cplusplus
}
#endif

#endif /* CG_ORACLE_H */
