/*
 * pending.c -- entry points declared by cogito with no GPU implementation
 * here yet.  Each records "not implemented yet" in the last error and
 * returns an error value; none computes anything on the CPU.
 */
#include <stddef.h>

#include "cg_mi355x.h"
#include "cgx_internal.h"

#define PENDING(name) cgx_set_error("%s: not implemented yet", name)

/* cg_speculative.h: EAGLE branching (declared only in the reference,
 * include/cg_speculative.h:160) */
int* cg_eagle_compute_branching(cg_eagle_draft* e, cg_tensor* f) {
    (void)e; (void)f; PENDING("cg_eagle_compute_branching"); return NULL;
}
