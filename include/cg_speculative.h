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

/* Draft chain / tree under verification (reference :15-25).
 * tokens[depth]; draft_probs/target_probs [depth, vocab] when filled;
 * accepted[depth].  In this library `branch_points`, when non-NULL, holds a
 * parent index per node (-1 = child of the verified prefix), which turns the
 * chain into a tree for cg_tree_attention_mask / tree verification. */
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

/* Generation driver.  draft_model/target_model must be cgx_model handles
 * (cg_mi355x.h) for these to run; otherwise they set the last error and
 * return NULL / -1. */
cg_tensor* cg_speculative_generate(
    cg_speculative_decoder* decoder,
    cg_tensor* input_ids,
    int max_new_tokens,
    float temperature,
    float top_p
);

int cg_speculative_step(
    cg_speculative_decoder* decoder,
    cg_tensor* input_ids,
    cg_token_tree* tree
);

cg_token_tree* cg_draft_generate(
    cg_speculative_decoder* decoder,
    cg_tensor* input_ids
);

/* Verification of a filled token tree (chain when branch_points == NULL).
 * With tree->target_probs [depth+1, vocab] holding TARGET LOGITS and
 * tree->draft_probs [depth, vocab] holding DRAFT LOGITS (either host or
 * device memory), runs the acceptance kernel with the decoder's temperature /
 * top_k / top_p, writes tree->accepted[], updates the decoder statistics, and
 * returns the number of accepted draft tokens n (0..depth).  The token that
 * follows them (correction or bonus) is written to tree->tokens[n] when
 * n < depth, and is otherwise available from cgx_last_verify_token(). */
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
 * every node sees the prefix, itself and its ancestors. */
cg_tensor* cg_tree_attention_mask(cg_token_tree* tree, int seqlen);
cg_tensor* cg_forward_tree_attention(
    void* model, cg_tensor* input, cg_tensor* tree_mask
);

/* EAGLE draft (reference :136-162). */
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
 * Each draws one uniform from the global LCG. */
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
