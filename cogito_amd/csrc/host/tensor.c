/*
 * tensor.c -- the cg_tensor container (reference src/core/tensor.c:40-158,
 * 316-341 for the functions kept).  Host tensors are calloc'd like the
 * reference's; device tensors (data in HBM) come from
 * cgx_tensor_device_new and are released by cg_tensor_free through the
 * registry of library-owned device buffers below.
 */
#include <stdlib.h>
#include <string.h>

#include "cg_tensor.h"
#include "cgx_internal.h"

/* ----------------------------------------- library-owned device buffers */

static void** g_owned = NULL;
static size_t g_owned_n = 0, g_owned_cap = 0;

static void owned_add(void* p) {
    if (g_owned_n == g_owned_cap) {
        size_t cap = g_owned_cap ? 2 * g_owned_cap : 64;
        void** n = (void**)realloc(g_owned, cap * sizeof(void*));
        if (!n) return;
        g_owned = n;
        g_owned_cap = cap;
    }
    g_owned[g_owned_n++] = p;
}

static int owned_contains(const void* p) {
    for (size_t i = 0; i < g_owned_n; i++)
        if (g_owned[i] == p) return 1;
    return 0;
}

static int owned_remove(void* p) {
    for (size_t i = 0; i < g_owned_n; i++) {
        if (g_owned[i] == p) {
            g_owned[i] = g_owned[--g_owned_n];
            return 1;
        }
    }
    return 0;
}

/* ----------------------------------------------------------- helpers */

static int shape_ok(const int* shape, int ndim) {
    if (!shape || ndim <= 0 || ndim > CG_MAX_DIMS) return 0;
    long long n = 1;
    for (int i = 0; i < ndim; i++) {
        if (shape[i] <= 0) return 0;
        n *= shape[i];
        if (n > 0x7fffffffLL) return 0;
    }
    return 1;
}

static void init_fields(cg_tensor* t, const int* shape, int ndim, bool rg) {
    t->ndim = ndim;
    int stride = 1;
    for (int i = ndim - 1; i >= 0; i--) {
        t->shape[i] = shape[i];
        t->strides[i] = stride;
        stride *= shape[i];
    }
    t->size = stride;
    t->requires_grad = rg;
    t->ref_count = 1;
}

/* ---------------------------------------------------------- creation */

cg_tensor* cg_tensor_new(int* shape, int ndim, bool requires_grad) {
    if (!shape_ok(shape, ndim)) {
        cgx_set_error("cg_tensor_new: invalid shape");
        return NULL;
    }
    cg_tensor* t = (cg_tensor*)calloc(1, sizeof(cg_tensor));
    if (!t) return NULL;
    init_fields(t, shape, ndim, requires_grad);
    t->data = (float*)calloc((size_t)t->size, sizeof(float));
    if (!t->data) {
        free(t);
        return NULL;
    }
    if (requires_grad) {
        t->grad = (float*)calloc((size_t)t->size, sizeof(float));
        if (!t->grad) {
            free(t->data);
            free(t);
            return NULL;
        }
    }
    return t;
}

cg_tensor* cg_tensor_zeros(int* shape, int ndim, bool requires_grad) {
    return cg_tensor_new(shape, ndim, requires_grad);
}

cg_tensor* cg_tensor_full(int* shape, int ndim, float value, bool requires_grad) {
    cg_tensor* t = cg_tensor_new(shape, ndim, requires_grad);
    if (!t) return NULL;
    for (int i = 0; i < t->size; i++) t->data[i] = value;
    return t;
}

cg_tensor* cg_tensor_ones(int* shape, int ndim, bool requires_grad) {
    return cg_tensor_full(shape, ndim, 1.0f, requires_grad);
}

cg_tensor* cg_tensor_from_data(float* data, int* shape, int ndim, bool requires_grad) {
    if (!data) {
        cgx_set_error("cg_tensor_from_data: null data");
        return NULL;
    }
    cg_tensor* t = cg_tensor_new(shape, ndim, requires_grad);
    if (!t) return NULL;
    memcpy(t->data, data, (size_t)t->size * sizeof(float));
    return t;
}

cg_tensor* cg_tensor_clone(cg_tensor* src) {
    if (!src) return NULL;
    if (owned_contains(src->data)) {     /* device tensor: clone in HBM */
        cg_tensor* t = cgx_tensor_device_new(src->shape, src->ndim);
        if (t && cgx_memcpy_d2d(t->data, src->data, (size_t)src->size * 4)) {
            cg_tensor_free(t);
            return NULL;
        }
        return t;
    }
    cg_tensor* t = cg_tensor_new(src->shape, src->ndim, src->requires_grad);
    if (!t) return NULL;
    memcpy(t->data, src->data, (size_t)t->size * sizeof(float));
    if (src->grad && t->grad) memcpy(t->grad, src->grad, (size_t)t->size * sizeof(float));
    return t;
}

/* ------------------------------------------------------- device tensors */

cg_tensor* cgx_tensor_device_new(int* shape, int ndim) {
    if (!shape_ok(shape, ndim)) {
        cgx_set_error("cgx_tensor_device_new: invalid shape");
        return NULL;
    }
    cg_tensor* t = (cg_tensor*)calloc(1, sizeof(cg_tensor));
    if (!t) return NULL;
    init_fields(t, shape, ndim, false);
    t->data = (float*)cgx_malloc((size_t)t->size * sizeof(float));
    if (!t->data || cgx_memset(t->data, 0, (size_t)t->size * sizeof(float))) {
        cgx_free(t->data);
        free(t);
        return NULL;
    }
    owned_add(t->data);
    return t;
}

cg_tensor* cgx_tensor_to_device(cg_tensor* host) {
    if (!host || !host->data) {
        cgx_set_error("cgx_tensor_to_device: null tensor");
        return NULL;
    }
    cg_tensor* t = cgx_tensor_device_new(host->shape, host->ndim);
    if (!t) return NULL;
    int rc = cgx_is_device_ptr(host->data)
                 ? cgx_memcpy_d2d(t->data, host->data, (size_t)host->size * 4)
                 : cgx_memcpy_h2d(t->data, host->data, (size_t)host->size * 4);
    if (rc) {
        cg_tensor_free(t);
        return NULL;
    }
    return t;
}

int cgx_tensor_to_host(cg_tensor* t, float* out) {
    if (!t || !t->data || !out) {
        cgx_set_error("cgx_tensor_to_host: null argument");
        return -1;
    }
    if (!cgx_is_device_ptr(t->data)) {
        memcpy(out, t->data, (size_t)t->size * sizeof(float));
        return 0;
    }
    return cgx_memcpy_d2h(out, t->data, (size_t)t->size * sizeof(float));
}

/* ----------------------------------------------------------- lifetime */

void cg_tensor_retain(cg_tensor* t) {
    if (t) t->ref_count++;
}

void cg_tensor_release(cg_tensor* t) {
    if (!t) return;
    if (--t->ref_count <= 0) cg_tensor_free(t);
}

void cg_tensor_free(cg_tensor* t) {
    if (!t) return;
    if (t->arena) return;                /* arena-owned, as the reference */
    for (int i = 0; i < t->num_parents; i++)
        if (t->parents[i]) cg_tensor_release(t->parents[i]);
    free(t->backward_ctx);
    if (!t->is_view) {
        if (owned_remove(t->data)) cgx_free(t->data);
        else free(t->data);
    }
    free(t->grad);
    free(t);
}

void cg_tensor_reshape(cg_tensor* t, int* new_shape, int new_ndim) {
    if (!t || !shape_ok(new_shape, new_ndim)) {
        cgx_set_error("cg_tensor_reshape: invalid shape");
        return;
    }
    long long n = 1;
    for (int i = 0; i < new_ndim; i++) n *= new_shape[i];
    if (n != t->size) {
        cgx_set_error("cg_tensor_reshape: size %lld != %d", n, t->size);
        return;
    }
    int rc = t->ref_count;
    init_fields(t, new_shape, new_ndim, t->requires_grad);
    t->ref_count = rc;
}

bool cg_tensor_shape_equal(cg_tensor* a, cg_tensor* b) {
    if (!a || !b || a->ndim != b->ndim) return false;
    for (int i = 0; i < a->ndim; i++)
        if (a->shape[i] != b->shape[i]) return false;
    return true;
}
