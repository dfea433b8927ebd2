/*
 * quantize.c -- cogito's quantization API (include/cg_quantize.h:73-117,
 * 184-196) on top of the INT4 HIP kernels.
 *
 *   cg_quantize_int4   reference src/quantize/int4.c:10-59   (GPU kernels)
 *   cg_dequantize      reference src/quantize/int4.c:61-79   (GPU kernel)
 *   cg_matmul_int4     reference src/quantize/int4.c:90-114  (GPU GEMV)
 *   cg_gemv_int4       declared only in the reference (:111) (GPU GEMV)
 *
 * Ownership follows the reference: constructors return calloc'd structs,
 * *_free is NULL-safe, outputs are caller-allocated.  A quantized tensor
 * returned by cg_quantize_int4 is host-resident (drop-in); one returned by
 * cgx_quant_to_device lives in HBM and is the fast path.
 */
#include <stdlib.h>
#include <string.h>

#include "cg_mi355x.h"
#include "cg_quantize.h"
#include "cgx_internal.h"

/* --------------------------------------------------------- quantization */

cg_tensor_quant* cg_quantize_int4(cg_tensor* tensor, int group_size) {
    if (!tensor || !tensor->data || tensor->size <= 0 || group_size <= 0) {
        cgx_set_error("cg_quantize_int4: invalid tensor or group size");
        return NULL;
    }
    if (cgx_ensure_init()) return NULL;
    int n = tensor->size;
    int ng = (n + group_size - 1) / group_size;
    size_t nb = ((size_t)n + 1) / 2;
    const float* dx = (const float*)cgx_dev_in(tensor->data, (size_t)n * 4, CGX_SLOT_IN0);
    uint8_t* dd = (uint8_t*)cgx_scratch(CGX_SLOT_OUT0, nb);
    float* ds = (float*)cgx_scratch(CGX_SLOT_OUT1, (size_t)ng * 4);
    if (!dx || !dd || !ds) return NULL;
    if (cgk_int4_quantize(dx, n, group_size, dd, ds)) return NULL;

    cg_tensor_quant* q = (cg_tensor_quant*)calloc(1, sizeof(cg_tensor_quant));
    if (!q) return NULL;
    q->quant_type = QUANT_INT4;
    q->group_size = group_size;
    q->size = n;
    q->ndim = tensor->ndim;
    q->shape = (int*)malloc((size_t)tensor->ndim * sizeof(int));
    q->num_groups = ng;
    q->scales = (float*)malloc((size_t)ng * sizeof(float));
    q->zeros = (float*)calloc((size_t)ng, sizeof(float));
    q->data = (uint8_t*)malloc(nb);
    q->symmetric = true;
    if (!q->shape || !q->scales || !q->zeros || !q->data) {
        cg_tensor_quant_free(q);
        cgx_set_error("cg_quantize_int4: out of host memory");
        return NULL;
    }
    memcpy(q->shape, tensor->shape, (size_t)tensor->ndim * sizeof(int));
    if (cgx_memcpy_d2h(q->data, dd, nb) ||
        cgx_memcpy_d2h(q->scales, ds, (size_t)ng * 4)) {
        cg_tensor_quant_free(q);
        return NULL;
    }
    return q;
}

cg_tensor_quant* cg_quantize_gptq(cg_tensor* tensor, cg_tensor* hessian,
                                   int group_size, int bits) {
    (void)tensor; (void)hessian; (void)group_size; (void)bits;
    cgx_set_error("cg_quantize_gptq: not implemented (declared only in cogito)");
    return NULL;
}

cg_tensor_quant* cg_quantize_awq(cg_tensor* tensor, cg_tensor* activations,
                                  int group_size) {
    (void)tensor; (void)activations; (void)group_size;
    cgx_set_error("cg_quantize_awq: not implemented (declared only in cogito)");
    return NULL;
}

cg_tensor_quant* cg_quantize_nf4(cg_tensor* tensor, int group_size) {
    (void)tensor; (void)group_size;
    cgx_set_error("cg_quantize_nf4: not implemented (declared only in cogito)");
    return NULL;
}

/* -------------------------------------------------- device residency */

static int quant_dims(const cg_tensor_quant* q, int* K, int* N) {
    if (q->ndim >= 2) {
        *N = q->shape[q->ndim - 1];
        *K = q->size / *N;
    } else {
        *K = 1;
        *N = q->size;
    }
    return (*K) * (*N) == q->size ? 0 : -1;
}

static cg_tensor_quant* quant_to_device_layout(cg_tensor_quant* q, int want) {
    if (!q || !q->data || !q->scales || q->size <= 0 || q->group_size <= 0) {
        cgx_set_error("cgx_quant_to_device: invalid quantized tensor");
        return NULL;
    }
    if (cgx_quant_lookup(q, NULL)) {
        cgx_set_error("cgx_quant_to_device: tensor is already device-resident");
        return NULL;
    }
    if (cgx_ensure_init()) return NULL;
    int K, N;
    if (quant_dims(q, &K, &N)) {
        cgx_set_error("cgx_quant_to_device: inconsistent shape");
        return NULL;
    }
    int gs = q->group_size;
    int ng = (q->size + gs - 1) / gs;
    size_t nb = ((size_t)q->size + 1) / 2;
    /* tiled layouts (2: VALU GEMV strips, 3: MFMA GEMV tiles) need K % 256,
     * N % 16, group % 16 and N % group; otherwise the reference layout */
    int fits = q->ndim == 2 && K % 256 == 0 && N % 16 == 0 && gs % 16 == 0 && N % gs == 0;
    int layout = (want != CGX_LAYOUT_FLAT && fits) ? want : CGX_LAYOUT_FLAT;
    int tiled = layout != CGX_LAYOUT_FLAT;

    cg_tensor_quant* d = (cg_tensor_quant*)calloc(1, sizeof(cg_tensor_quant));
    if (!d) return NULL;
    *d = *q;
    d->zeros = NULL;
    d->shape = (int*)malloc((size_t)q->ndim * sizeof(int));
    if (!d->shape) {
        free(d);
        return NULL;
    }
    memcpy(d->shape, q->shape, (size_t)q->ndim * sizeof(int));
    d->data = (uint8_t*)cgx_malloc(nb);
    d->scales = (float*)cgx_malloc((size_t)ng * 4);
    if (!d->data || !d->scales) goto fail;
    if (tiled) {
        const uint8_t* fd = (const uint8_t*)cgx_dev_in(q->data, nb, CGX_SLOT_IN0);
        const float* fs = (const float*)cgx_dev_in(q->scales, (size_t)ng * 4, CGX_SLOT_IN1);
        if (!fd || !fs) goto fail;
        if (layout == CGX_LAYOUT_MFMA
                ? cgk_int4_repack_mfma(fd, fs, K, N, gs, 0, d->data, d->scales)
                : cgk_int4_repack_tiled(fd, fs, K, N, gs, d->data, d->scales))
            goto fail;
        if (cgx_synchronize()) goto fail;
    } else {
        int dev = cgx_is_device_ptr(q->data);
        if ((dev ? cgx_memcpy_d2d(d->data, q->data, nb)
                 : cgx_memcpy_h2d(d->data, q->data, nb)) ||
            (dev ? cgx_memcpy_d2d(d->scales, q->scales, (size_t)ng * 4)
                 : cgx_memcpy_h2d(d->scales, q->scales, (size_t)ng * 4)) ||
            cgx_synchronize())
            goto fail;
    }
    {
        cgx_qinfo info = {layout, K, N, gs, 0, 0.0f};
        if (layout == CGX_LAYOUT_MFMA && cgk_absmax(d->scales, (size_t)ng, &info.smax)) goto fail;
        cgx_quant_register(d, &info);
    }
    return d;
fail:
    cgx_free(d->data);
    cgx_free(d->scales);
    free(d->shape);
    free(d);
    return NULL;
}

cg_tensor_quant* cgx_quant_to_device(cg_tensor_quant* q) {
    return quant_to_device_layout(q, CGX_LAYOUT_MFMA);
}

cg_tensor_quant* cgx_quant_to_device_flat(cg_tensor_quant* q) {
    return quant_to_device_layout(q, CGX_LAYOUT_FLAT);
}

cg_tensor_quant* cgx_quant_to_device_layout(cg_tensor_quant* q, int layout) {
    if (layout < CGX_LAYOUT_FLAT || layout > CGX_LAYOUT_MFMA) {
        cgx_set_error("cgx_quant_to_device_layout: layout must be 1, 2 or 3");
        return NULL;
    }
    return quant_to_device_layout(q, layout);
}

int cgx_quant_layout(cg_tensor_quant* q) {
    cgx_qinfo info;
    if (!q) return -1;
    return cgx_quant_lookup(q, &info) ? info.layout : CGX_LAYOUT_HOST;
}

void cg_tensor_quant_free(cg_tensor_quant* q) {
    if (!q) return;
    if (cgx_quant_lookup(q, NULL)) {
        cgx_quant_unregister(q);
        cgx_free(q->data);
        cgx_free(q->scales);
        free(q->shape);
        free(q);
        return;
    }
    free(q->data);
    free(q->scales);
    free(q->zeros);
    free(q->shape);
    free(q);
}

/* ---------------------------------------------------------- dequantize */

cg_tensor* cg_dequantize(cg_tensor_quant* q) {
    if (!q || !q->data || !q->scales || q->size <= 0) {
        cgx_set_error("cg_dequantize: invalid quantized tensor");
        return NULL;
    }
    if (cgx_ensure_init()) return NULL;
    cgx_qinfo info;
    if (cgx_quant_lookup(q, &info)) {
        cg_tensor* out = cgx_tensor_device_new(q->shape, q->ndim);
        if (!out) return NULL;
        int rc = info.layout == CGX_LAYOUT_TILED
                     ? cgk_int4_dequantize_tiled(q->data, q->scales, info.K, info.N,
                                                 info.group_size, out->data)
                 : info.layout == CGX_LAYOUT_MFMA
                     ? cgk_int4_dequantize_mfma(q->data, q->scales, info.K, info.N,
                                                info.group_size, info.paired, out->data)
                     : cgk_int4_dequantize_flat(q->data, q->scales, q->size,
                                                q->group_size, out->data);
        if (rc || cgx_synchronize()) {
            cg_tensor_free(out);
            return NULL;
        }
        return out;
    }
    int n = q->size, ng = (n + q->group_size - 1) / q->group_size;
    size_t nb = ((size_t)n + 1) / 2;
    const uint8_t* dd = (const uint8_t*)cgx_dev_in(q->data, nb, CGX_SLOT_IN0);
    const float* ds = (const float*)cgx_dev_in(q->scales, (size_t)ng * 4, CGX_SLOT_IN1);
    float* dout = (float*)cgx_scratch(CGX_SLOT_OUT0, (size_t)n * 4);
    if (!dd || !ds || !dout) return NULL;
    if (cgk_int4_dequantize_flat(dd, ds, n, q->group_size, dout)) return NULL;
    cg_tensor* out = cg_tensor_new(q->shape, q->ndim, false);
    if (!out) return NULL;
    if (cgx_memcpy_d2h(out->data, dout, (size_t)n * 4)) {
        cg_tensor_free(out);
        return NULL;
    }
    return out;
}

/* -------------------------------------------------------------- matmul */

int cgx_matmul_int4_dev_kernel(const float* x, int M, cg_tensor_quant* w,
                               float* y, int kernel) {
    cgx_qinfo info;
    if (!x || !y || !w || M <= 0) {
        cgx_set_error("cgx_matmul_int4: invalid argument");
        return -1;
    }
    if (!cgx_quant_lookup(w, &info)) {
        cgx_set_error("cgx_matmul_int4: weight is not device-resident "
                      "(use cgx_quant_to_device)");
        return -1;
    }
    if (kernel == 0)
        kernel = info.layout == CGX_LAYOUT_TILED ? 1 : info.layout == CGX_LAYOUT_MFMA ? 3 : 2;
    if (kernel == 3 || kernel == 4) {
        if (info.layout != CGX_LAYOUT_MFMA) {
            cgx_set_error("cgx_matmul_int4: MFMA kernels need a layout-3 weight");
            return -1;
        }
        if (kernel == 4)      /* the GEMM of the batched / tree verify (M >= 16) */
            return cgk_gemm_int4(x, info.K, M, info.K, info.N, info.group_size, w->data,
                                 w->scales, info.smax, y, info.N, 0, NULL, 0.0f, 0, NULL, 0,
                                 NULL, NULL);
        return cgk_gemv_mfma(x, info.K, M, info.K, info.N, info.group_size, w->data,
                             w->scales, y, info.N, 0, NULL, 0.0f, 0);
    }
    if (kernel == 1) {
        if (info.layout != CGX_LAYOUT_TILED) {
            cgx_set_error("cgx_matmul_int4: tiled kernel needs a tiled weight");
            return -1;
        }
        return cgk_int4_gemv_tiled(x, M, info.K, info.N, info.group_size, w->data,
                                   w->scales, y);
    }
    if (kernel == 2) {
        if (info.layout != CGX_LAYOUT_FLAT) {
            cgx_set_error("cgx_matmul_int4: generic kernel needs a flat weight");
            return -1;
        }
        return cgk_int4_matmul_generic(x, M, info.K, info.N, info.group_size,
                                       w->data, w->scales, y);
    }
    cgx_set_error("cgx_matmul_int4: unknown kernel %d", kernel);
    return -1;
}

int cgx_matmul_int4_dev(const float* x, int M, cg_tensor_quant* w, float* y) {
    return cgx_matmul_int4_dev_kernel(x, M, w, y, 0);
}

static void matmul_api(const char* fn, cg_tensor* input, cg_tensor_quant* weight,
                       cg_tensor* output) {
    if (!input || !weight || !output || !input->data || !output->data ||
        !weight->data || !weight->scales) {
        cgx_set_error("%s: null argument", fn);
        return;
    }
    if (cgx_ensure_init()) return;
    /* reference int4.c:91-93: M = input rows, K = input cols, N = W cols */
    int M = input->ndim >= 2 ? input->size / input->shape[input->ndim - 1] : 1;
    int K = input->shape[input->ndim - 1];
    int N = weight->ndim >= 2 ? weight->shape[weight->ndim - 1] : weight->size;
    if ((long long)K * N != weight->size || output->size < M * N) {
        cgx_set_error("%s: shape mismatch (M=%d K=%d N=%d, weight %d, output %d)",
                      fn, M, K, N, weight->size, output->size);
        return;
    }
    const float* dx = (const float*)cgx_dev_in(input->data, (size_t)M * K * 4, CGX_SLOT_IN2);
    if (!dx) return;
    int out_dev = cgx_is_device_ptr(output->data);
    float* dy = out_dev ? output->data
                        : (float*)cgx_scratch(CGX_SLOT_OUT0, (size_t)M * N * 4);
    if (!dy) return;
    int rc;
    cgx_qinfo info;
    if (cgx_quant_lookup(weight, &info)) {
        rc = cgx_matmul_int4_dev(dx, M, weight, dy);
    } else {
        /* host weight in the reference layout: stage and run the
         * reference-order kernel */
        int ng = (weight->size + weight->group_size - 1) / weight->group_size;
        size_t nb = ((size_t)weight->size + 1) / 2;
        const uint8_t* dd = (const uint8_t*)cgx_dev_in(weight->data, nb, CGX_SLOT_IN0);
        const float* ds = (const float*)cgx_dev_in(weight->scales, (size_t)ng * 4,
                                                   CGX_SLOT_IN1);
        if (!dd || !ds) return;
        rc = cgk_int4_matmul_generic(dx, M, K, N, weight->group_size, dd, ds, dy);
    }
    if (rc) return;
    if (!out_dev) {
        if (output->size > M * N)
            memset(output->data + (size_t)M * N, 0,
                   (size_t)(output->size - M * N) * sizeof(float));
        cgx_memcpy_d2h(output->data, dy, (size_t)M * N * 4);
    } else if (output->size > M * N) {
        cgx_memset(output->data + (size_t)M * N, 0,
                   (size_t)(output->size - M * N) * sizeof(float));
    }
}

void cg_matmul_int4(cg_tensor* input, cg_tensor_quant* weight, cg_tensor* output) {
    matmul_api("cg_matmul_int4", input, weight, output);
}

void cg_gemv_int4(cg_tensor* input, cg_tensor_quant* weight, cg_tensor* output) {
    matmul_api("cg_gemv_int4", input, weight, output);
}

/* --------------------------------------------------------- calibration */

cg_quant_calibration* cg_calibration_new(int channels) {
    if (channels <= 0) {
        cgx_set_error("cg_calibration_new: channels must be positive");
        return NULL;
    }
    cg_quant_calibration* c = (cg_quant_calibration*)calloc(1, sizeof(*c));
    if (!c) return NULL;
    c->channels = channels;
    c->min_vals = (float*)malloc((size_t)channels * sizeof(float));
    c->max_vals = (float*)malloc((size_t)channels * sizeof(float));
    c->absmax = (float*)calloc((size_t)channels, sizeof(float));
    if (!c->min_vals || !c->max_vals || !c->absmax) {
        cg_calibration_free(c);
        return NULL;
    }
    for (int i = 0; i < channels; i++) {
        c->min_vals[i] = 1e9f;
        c->max_vals[i] = -1e9f;
    }
    return c;
}

void cg_calibration_update(cg_quant_calibration* c, cg_tensor* act) {
    /* reference int4.c:304-317: per-channel running min / max / absmax over
     * the rows of a [batch, features] activation tensor (host statistics) */
    if (!c || !act || !act->data || act->ndim < 2) {
        cgx_set_error("cg_calibration_update: invalid argument");
        return;
    }
    int batch = act->shape[0], features = act->shape[1];
    float* host = act->data;
    float* tmp = NULL;
    if (cgx_is_device_ptr(act->data)) {
        tmp = (float*)malloc((size_t)act->size * sizeof(float));
        if (!tmp || cgx_memcpy_d2h(tmp, act->data, (size_t)act->size * 4)) {
            free(tmp);
            return;
        }
        host = tmp;
    }
    for (int b = 0; b < batch; b++) {
        for (int f = 0; f < features && f < c->channels; f++) {
            float v = host[b * features + f];
            if (v < c->min_vals[f]) c->min_vals[f] = v;
            if (v > c->max_vals[f]) c->max_vals[f] = v;
            float a = v < 0 ? -v : v;
            if (a > c->absmax[f]) c->absmax[f] = a;
        }
    }
    c->num_samples++;
    free(tmp);
}

void cg_calibration_compute_scales(cg_quant_calibration* c, float* scales,
                                   float* zeros, int group_size) {
    /* declared only in the reference (cg_quantize.h:194): symmetric INT4
     * scales from the per-channel absmax, grouped like cg_quantize_int4
     * (absmax / 7 with the 1e-10 floor), zero points 0 */
    if (!c || !scales || group_size <= 0) {
        cgx_set_error("cg_calibration_compute_scales: invalid argument");
        return;
    }
    int ng = (c->channels + group_size - 1) / group_size;
    for (int g = 0; g < ng; g++) {
        float m = 0.0f;
        for (int i = g * group_size; i < (g + 1) * group_size && i < c->channels; i++)
            if (c->absmax[i] > m) m = c->absmax[i];
        float s = m / 7.0f;
        scales[g] = s < 1e-10f ? 1.0f : s;
        if (zeros) zeros[g] = 0.0f;
    }
}

void cg_calibration_free(cg_quant_calibration* c) {
    if (!c) return;
    free(c->min_vals);
    free(c->max_vals);
    free(c->absmax);
    free(c);
}
