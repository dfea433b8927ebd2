/*
 * cg_speculative.h -- speculative-decoding sampling and verification
 * (cogito's include/cg_speculative.h, same declarations).
 *
 * Randomness: exactly as in the reference (src/inference/speculative.c:11-12)
 * every sampler draws one uniform from a process-global LCG
 *     s = s * 1103515245 + 12345 (mod 2^32), u = (s % 10000) / 10000.0f,
 * seeded with 42.  cgx_lcg_seed()/cgx_lcg_state() (cg_mi355x.h) expose the
 * state; the cgx_* entry points take pre-drawn uniforms instead.
 *
 * MI355X implementation: the samplers and the verify composition run in HIP
 * kernels (cogito_amd/csrc/accept.hip) that reproduce the reference's fp32
 * arithmetic bit for bit: glibc-identical expf, and exact emulation of the
 * reference's left-to-right fp32 sums.  Token decisions are therefore
 * identical to the reference CPU path on the same logits and uniforms.
 */
#ifndef CG_SPECULATIVE_H
#define CG_SPECULATIVE_H

#include "cg_tensor.h"
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Draft chain under verification (reference :15-25).  tokens[depth],
 * accepted[depth].  In this library draft_probs holds the draft LOGITS
 * [depth][vocab] and target_probs the target LOGITS [depth + 1][vocab] (row
 * depth scores the token after the last draft); both are host buffers owned
 * by the tree (cg_token_tree_free frees them).  branch_points / num_branches
 * are the caller's, as in the reference: the library neither reads nor frees
 * them.  Trees with parent links go through cgx_tree_attention_mask_parents
 * and the cgx_tree_spec_* loop (cg_mi355x.h). */
typedef struct {
    int* tokens;
    float* draft_probs;
    float* target_probs;
    bool* accepted;
    cg_tensor* hidden_states;
    int depth;
    int* branch_points;
    int num_branches;
} cg_token_tree;

/* Decoder state (reference :31-55). */
typedef struct {
    void* draft_model;
    void* target_model;
    int gamma;
    float temperature;
    float top_p;
    int top_k;
    float accept_threshold;
    bool use_typical_sampling;
    int total_draft_tokens;
    int accepted_draft_tokens;
    float avg_acceptance_rate;
    int num_steps;
    void* draft_kv_cache;
    void* target_kv_cache;
} cg_speculative_decoder;

cg_speculative_decoder* cg_speculative_decoder_new(
    void* draft_model, void* target_model, int gamma
);

/* Generation driver (declared only in the reference).  draft_model and
 * target_model must be cgx_model handles (cg_mi355x.h); otherwise the calls
 * set the last error and return NULL / -1.
 *
 * input_ids holds the sequence so far as float token ids ([1, n] or [n],
 * host or device).  Each model's KV cache is cut to the longest prefix it
 * shares with input_ids and the rest is run, so any input_ids is served and
 * a growing sequence reuses the cache.  Draws come from the global LCG in the
 * order of a sequential implementation: one per drafted token (the
 * decoder's temperature / top_k / top_p filter, as cg_sample_temperature /
 * cg_sample_top_k / cg_sample_top_p draw), then one per accept test and one
 * for the token after the accepted drafts.
 *
 * cg_speculative_generate sets decoder->temperature / top_p from its
 * arguments and steps until max_new_tokens are out (or a cache is full);
 * returns a new host tensor [1, n + generated] of float token ids. */
cg_tensor* cg_speculative_generate(
    cg_speculative_decoder* decoder,
    cg_tensor* input_ids,
    int max_new_tokens,
    float temperature,
    float top_p
);

/* One step with a chain of tree->depth drafts: fills tree->tokens and the
 * tree's draft / target logits, then verifies as cg_target_verify. */
int cg_speculative_step(
    cg_speculative_decoder* decoder,
    cg_tensor* input_ids,
    cg_token_tree* tree
);

/* A new tree of decoder->gamma drafted tokens after input_ids, with their
 * draft logits in draft_probs. */
cg_token_tree* cg_draft_generate(
    cg_speculative_decoder* decoder,
    cg_tensor* input_ids
);

/* Verification of the chain tree->tokens[0..depth) against the draft
 * logits in tree->draft_probs [depth][vocab] (host or device).  The target
 * logits [depth + 1][vocab] are tree->target_probs when set (host or
 * device); when NULL the target model scores [last input token, drafts] and
 * target_probs receives them, and its cache keeps the accepted drafts.  The
 * verify kernels run with the decoder's temperature / top_k / top_p and LCG
 * draws; the call writes tree->accepted[], updates total_draft_tokens,
 * accepted_draft_tokens, avg_acceptance_rate and num_steps, and returns the
 * number n of accepted drafts (0..depth).  The token that follows them (the
 * correction, or the bonus when all are accepted) is written to
 * tree->tokens[n] when n < depth and is always returned by
 * cgx_last_verify_token() (cg_mi355x.h).  vocab is the target model's. */
int cg_target_verify(
    cg_speculative_decoder* decoder,
    cg_tensor* input_ids,
    cg_token_tree* tree
);

void cg_speculative_decoder_free(cg_speculative_decoder* decoder);

/* Token tree API (reference :111-114). */
cg_token_tree* cg_token_tree_new(int depth);
void cg_token_tree_add_token(cg_token_tree* tree, int token, float* probs);
cg_tensor* cg_token_tree_to_tensor(cg_token_tree* tree);
void cg_token_tree_free(cg_token_tree* tree);

/* Tree attention (reference :123-130).  cg_tree_attention_mask returns the
 * additive [1,1,S,S] mask (0 / -1e9) with S = seqlen + depth: causal prefix,
 * every node sees the prefix and the nodes up to itself (the reference's
 * chain; cgx_tree_attention_mask_parents builds it for a tree).
 * cg_forward_tree_attention runs a cgx_model over input (float token ids,
 * [S]) under such a mask: a causal prefix followed by at most 64 tree rows,
 * each seeing the whole prefix, itself and any of the other tree rows, at
 * rotary position prefix + (visible tree rows - 1).  Mask entries must be 0
 * (visible) or <= -1e4 (hidden).  Returns the logits of every row as a new
 * host tensor [1, S, vocab]; the model's cache is the workspace and keeps the
 * causal prefix. */
cg_tensor* cg_tree_attention_mask(cg_token_tree* tree, int seqlen);
cg_tensor* cg_forward_tree_attention(
    void* model, cg_tensor* input, cg_tensor* tree_mask
);

/* EAGLE draft (reference :136-162).  cg_eagle_generate_tree with a
 * cgx_model as base_draft drafts the most likely token at each depth (ties:
 * the lower id) after input (float token ids), with the draft logits in
 * draft_probs; with any other base_draft it returns the reference's
 * placeholder tree (every token 1, src/inference/speculative.c:244-262).
 * cg_eagle_compute_branching takes draft logits [rows][vocab] (host or
 * device) and returns a malloc'd int[rows] (free with free()): per row the
 * number of most likely tokens (1..4, top-k order) whose softmax
 * probabilities, summed in that order, first reach 0.8. */
typedef struct {
    void* base_draft;
    void* feature_proj;
    void* uncertainty_head;
    float* feature_cache;
} cg_eagle_draft;

cg_eagle_draft* cg_eagle_draft_new(void* base_draft);
cg_token_tree* cg_eagle_generate_tree(
    cg_eagle_draft* eagle,
    cg_tensor* input,
    int max_depth
);
int* cg_eagle_compute_branching(cg_eagle_draft* eagle, cg_tensor* features);
void cg_eagle_draft_free(cg_eagle_draft* eagle);

/* Samplers (reference :171-196).  `logits` may be host or device memory.
 * Each draws one uniform from the global LCG.  cg_sample_typical, declared
 * only in the reference, is locally typical sampling in the style of
 * cg_sample_top_p: probabilities p (softmax at T = 1), L_i = log p_i (a
 * binary64 log rounded to float), entropy H = sum fl(p_i * -L_i) left to
 * right in fp32, tokens ordered by (|-L_i - H| ascending, index ascending),
 * kept up to the first cumsum >= typical_p, drawn by r = u * kept mass. */
int cg_sample_temperature(float* logits, int vocab_size, float temperature);
int cg_sample_top_p(float* logits, int vocab_size, float top_p);
int cg_sample_top_k(float* logits, int vocab_size, int top_k);
int cg_sample_typical(float* logits, int vocab_size, float typical_p);
float cg_acceptance_prob(float draft_prob, float target_prob);
int cg_sample_corrected(float* draft_probs, float* target_probs, int vocab_size);

#ifdef __cplusplus
}
#endif

#endif /* CG_SPECULATIVE_H */
