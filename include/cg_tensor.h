/*
 * cg_tensor.h -- the fp32 tensor container that the verify-path API passes
 * around (cogito's `cg_tensor`).
 *
 * ABI-identical to the reference struct (include/cg_tensor.h:33-55 of
 * cogito-ml/cogito) so that a program compiled against cogito's header links
 * against this library unchanged.  Only the container functions are
 * provided (creation, free, refcount, reshape, shape compare): cogito's dense
 * fp32 ops and autograd are not part of the verify path.
 *
 * Device residency: `data` may hold a device pointer (HBM) instead of a host
 * pointer.  Tensors made by cgx_tensor_device_new() (cg_mi355x.h) are such
 * tensors; every API entry in this library accepts either kind and detects
 * which it got.  The same convention exists in the reference
 * (src/cuda/cg_cuda.c:380-415, cg_tensor_cuda_new).
 */
#ifndef CG_TENSOR_H
#define CG_TENSOR_H

#include <stddef.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cg_tensor cg_tensor;
typedef struct cg_arena cg_arena;

#define CG_MAX_DIMS 8
#define CG_MAX_PARENTS 4

typedef void (*cg_backward_fn)(cg_tensor* self);

/* Row-major fp32 tensor.  Field order and types match the reference. */
struct cg_tensor {
    float* data;                         /* host or device pointer           */
    float* grad;                         /* unused on the verify path        */
    int shape[CG_MAX_DIMS];
    int strides[CG_MAX_DIMS];
    int ndim;
    int size;                            /* element count (< 2^31)           */
    bool requires_grad;
    cg_backward_fn backward_fn;
    cg_tensor* parents[CG_MAX_PARENTS];
    int num_parents;
    void* backward_ctx;
    int ref_count;
    bool is_view;                        /* true: data is not owned          */
    cg_arena* arena;
};

/* Creation (reference include/cg_tensor.h:69-105). Host memory, zero-filled. */
cg_tensor* cg_tensor_new(int* shape, int ndim, bool requires_grad);
cg_tensor* cg_tensor_zeros(int* shape, int ndim, bool requires_grad);
cg_tensor* cg_tensor_ones(int* shape, int ndim, bool requires_grad);
cg_tensor* cg_tensor_full(int* shape, int ndim, float value, bool requires_grad);
cg_tensor* cg_tensor_from_data(float* data, int* shape, int ndim, bool requires_grad);
cg_tensor* cg_tensor_clone(cg_tensor* t);

/* Memory management (reference include/cg_tensor.h:120-134).  cg_tensor_free
 * also releases device memory when `data` is a device allocation owned by
 * this library. */
void cg_tensor_retain(cg_tensor* t);
void cg_tensor_release(cg_tensor* t);
void cg_tensor_free(cg_tensor* t);

/* Utilities (reference include/cg_tensor.h:230-253). */
void cg_tensor_reshape(cg_tensor* t, int* new_shape, int new_ndim);
bool cg_tensor_shape_equal(cg_tensor* a, cg_tensor* b);

#ifdef __cplusplus
}
#endif

#endif /* CG_TENSOR_H */
