/*
 * pending.c -- entry points whose GPU kernels are not wired yet.  Each one
 * records "not implemented yet" in the last error and returns an error
 * value; none computes anything on the CPU.  Entries move out of this file
 * as their kernels land.
 */
#include <stddef.h>

#include "cg_mi355x.h"
#include "cgx_internal.h"

#define PENDING(name) cgx_set_error("%s: not implemented yet", name)

/* cg_speculative.h: sampling and verification */
int cg_sample_typical(float* l, int V, float p) { (void)l; (void)V; (void)p; PENDING("cg_sample_typical"); return -1; }
int cg_target_verify(cg_speculative_decoder* d, cg_tensor* ids, cg_token_tree* t) {
    (void)d; (void)ids; (void)t; PENDING("cg_target_verify"); return -1;
}
int cg_speculative_step(cg_speculative_decoder* d, cg_tensor* ids, cg_token_tree* t) {
    (void)d; (void)ids; (void)t; PENDING("cg_speculative_step"); return -1;
}
cg_tensor* cg_speculative_generate(cg_speculative_decoder* d, cg_tensor* ids, int n, float T, float p) {
    (void)d; (void)ids; (void)n; (void)T; (void)p; PENDING("cg_speculative_generate"); return NULL;
}
cg_token_tree* cg_draft_generate(cg_speculative_decoder* d, cg_tensor* ids) {
    (void)d; (void)ids; PENDING("cg_draft_generate"); return NULL;
}
cg_tensor* cg_forward_tree_attention(void* m, cg_tensor* in, cg_tensor* mask) {
    (void)m; (void)in; (void)mask; PENDING("cg_forward_tree_attention"); return NULL;
}
cg_token_tree* cg_eagle_generate_tree(cg_eagle_draft* e, cg_tensor* in, int d) {
    (void)e; (void)in; (void)d; PENDING("cg_eagle_generate_tree"); return NULL;
}
int* cg_eagle_compute_branching(cg_eagle_draft* e, cg_tensor* f) {
    (void)e; (void)f; PENDING("cg_eagle_compute_branching"); return NULL;
}
