/*
 * host_runtime.c -- the few runtime entry points of the library that its
 * host-only modules (tensor.c, speculative.c, serialize.c) call, for the
 * sanitizer build, which has no HIP runtime: last-error recording, and
 * device-memory calls that report "no device" (every pointer is host memory
 * there).  Test infrastructure only.
 */
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>

#include "cgx_internal.h"

static char g_err[1024];

void cgx_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}
const char* cgx_last_error(void) { return g_err; }
void cgx_clear_error(void) { g_err[0] = 0; }
int cgx_ensure_init(void) {
    cgx_set_error("no device in the sanitizer build");
    return -1;
}
int cgx_is_device_ptr(const void* p) { (void)p; return 0; }
void* cgx_malloc(size_t b) { (void)b; cgx_ensure_init(); return NULL; }
int cgx_free(void* p) { return p ? cgx_ensure_init() : 0; }
int cgx_memcpy_h2d(void* d, const void* s, size_t b) { (void)d; (void)s; (void)b; return cgx_ensure_init(); }
int cgx_memcpy_d2h(void* d, const void* s, size_t b) { (void)d; (void)s; (void)b; return cgx_ensure_init(); }
int cgx_memcpy_d2d(void* d, const void* s, size_t b) { (void)d; (void)s; (void)b; return cgx_ensure_init(); }
int cgx_memset(void* d, int v, size_t b) { (void)d; (void)v; (void)b; return cgx_ensure_init(); }
int cgx_quant_lookup(const cg_tensor_quant* q, cgx_qinfo* info) { (void)q; (void)info; return 0; }
cg_tensor_quant* cgx_quant_to_device_flat(cg_tensor_quant* q) { (void)q; cgx_ensure_init(); return NULL; }

/* The host-memory branch of cg_tensor_quant_free (host/quantize.c, which
 * also holds the GPU launchers this build leaves out). */
void cg_tensor_quant_free(cg_tensor_quant* q) {
    if (!q) return;
    free(q->data);
    free(q->scales);
    free(q->zeros);
    free(q->shape);
    free(q);
}
