/*
 * cg_quantize.h -- INT4 weights, the INT4 KV cache and the quantized ops of
 * the verify path (cogito's include/cg_quantize.h, same declarations).
 *
 * Value format (identical to the reference, include/cg_quantize.h:155-175 and
 * src/quantize/int4.c:10-114):
 *   - element i of a tensor lives in byte i/2; even i in the low nibble;
 *   - a nibble is a two's-complement value in [-8, 7];
 *   - groups of `group_size` elements run over the flattened row-major index,
 *     so for a weight W[K,N] (y = x @ W) the groups run along N;
 *   - scales are fp32; zeros are all 0 and the matmul ignores them.
 *
 * MI355X implementation: every function below runs its arithmetic in HIP
 * kernels on the GPU (the .hip sources under cogito_amd/csrc).  A cg_tensor_quant returned by
 * cgx_quant_to_device() (cg_mi355x.h) keeps its data in HBM in a tiled layout
 * and is the fast path; a host-resident one is uploaded per call.
 */
#ifndef CG_QUANTIZE_H
#define CG_QUANTIZE_H

#include "cg_tensor.h"
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    QUANT_NONE = 0,
    QUANT_INT8,
    QUANT_INT4,
    QUANT_NF4,
    QUANT_FP8_E4M3,
    QUANT_FP8_E5M2,
    QUANT_GPTQ,
    QUANT_AWQ,
    QUANT_GGML
} cg_quant_type;

/* Quantized tensor (reference include/cg_quantize.h:32-46). */
typedef struct {
    uint8_t* data;              /* packed nibbles, (size+1)/2 bytes            */
    float* scales;              /* one per group                               */
    float* zeros;               /* one per group, all zero                     */
    int* shape;
    int ndim;
    int size;                   /* element count                               */
    cg_quant_type quant_type;
    int group_size;
    int num_groups;
    bool symmetric;
} cg_tensor_quant;

/* INT4 KV cache (reference include/cg_quantize.h:52-64).
 * k_cache/v_cache: [layers, max_seq, n_heads, head_dim/2] bytes;
 * k_scales/v_scales: [layers, max_seq, n_heads, head_dim/group_size] fp32.
 * In this library all four arrays live in HBM. */
typedef struct {
    uint8_t* k_cache;
    uint8_t* v_cache;
    float* k_scales;
    float* v_scales;
    int current_len;
    int max_seq_len;
    int num_layers;
    int n_heads;
    int head_dim;
    int group_size;
} cg_kv_cache_int4;

/* Quantization (reference include/cg_quantize.h:73-97). */
cg_tensor_quant* cg_quantize_int4(cg_tensor* tensor, int group_size);
/* GPTQ / AWQ / NF4: declared by cogito but never defined there; here they set
 * the last error ("not implemented") and return NULL. */
cg_tensor_quant* cg_quantize_gptq(cg_tensor* tensor, cg_tensor* hessian,
                                   int group_size, int bits);
cg_tensor_quant* cg_quantize_awq(cg_tensor* tensor, cg_tensor* activations,
                                  int group_size);
cg_tensor_quant* cg_quantize_nf4(cg_tensor* tensor, int group_size);
cg_tensor* cg_dequantize(cg_tensor_quant* quant);
void cg_tensor_quant_free(cg_tensor_quant* quant);

/* Quantized ops (reference include/cg_quantize.h:106-117).
 * cg_matmul_int4: output[M,N] = input[M,K] @ W[K,N].
 * cg_gemv_int4:   the same with M = 1 (any M <= 8 takes the GEMV kernel).
 * cg_attention_int4_kv: Q [Nq, H, D] (or [1, Nq, H, D]) attends to the
 *   cache of `layer_idx` over [0, current_len) with GQA (cache n_heads are the
 *   KV heads) and the chain-verify mask: the Nq queries are the last Nq
 *   tokens of the cache, query i sees keys [0, current_len - Nq + i].
 *   Output has Q's shape. */
void cg_matmul_int4(cg_tensor* input, cg_tensor_quant* weight, cg_tensor* output);
void cg_gemv_int4(cg_tensor* input, cg_tensor_quant* weight, cg_tensor* output);
void cg_attention_int4_kv(cg_tensor* Q, cg_kv_cache_int4* kv_cache,
                          int layer_idx, cg_tensor* output);

/* KV cache (reference include/cg_quantize.h:126-146).
 * append: new_k/new_v hold T tokens as [T, n_heads, head_dim] (any leading
 * shape with that trailing size); current_len advances by T once all layers'
 * rows for those positions are written -- i.e. by the append of the last
 * layer (num_layers - 1).  The reference advances once per call
 * (src/quantize/int4.c:233), which breaks multi-layer caches. */
cg_kv_cache_int4* cg_kv_cache_int4_new(int num_layers, int max_seq_len,
                                        int n_heads, int head_dim, int group_size);
void cg_kv_cache_int4_append(cg_kv_cache_int4* cache, int layer_idx,
                             cg_tensor* new_k, cg_tensor* new_v);
void cg_kv_cache_int4_get(cg_kv_cache_int4* cache, int layer_idx,
                          cg_tensor* k_out, cg_tensor* v_out);
void cg_kv_cache_int4_reset(cg_kv_cache_int4* cache);
void cg_kv_cache_int4_free(cg_kv_cache_int4* cache);

/* Packing helpers: byte-identical behaviour to the reference inline helpers
 * (include/cg_quantize.h:155-175). */
static inline uint8_t pack_int4(int8_t a, int8_t b) {
    return (uint8_t)((a & 0x0F) | ((b & 0x0F) << 4));
}

static inline void unpack_int4(uint8_t packed, int8_t* a, int8_t* b) {
    int lo = packed & 0x0F, hi = (packed >> 4) & 0x0F;
    *a = (int8_t)(lo >= 8 ? lo - 16 : lo);
    *b = (int8_t)(hi >= 8 ? hi - 16 : hi);
}

static inline float dequant_int4(int8_t val, float scale, float zero) {
    return ((float)val - zero) * scale;
}

/* Calibration (reference include/cg_quantize.h:184-196).  Host-side
 * statistics; cg_calibration_compute_scales (declared only in the reference)
 * writes absmax/7 per group of channels and zero zero-points. */
typedef struct {
    float* min_vals;
    float* max_vals;
    float* absmax;
    int num_samples;
    int channels;
} cg_quant_calibration;

cg_quant_calibration* cg_calibration_new(int channels);
void cg_calibration_update(cg_quant_calibration* calib, cg_tensor* activations);
void cg_calibration_compute_scales(cg_quant_calibration* calib,
                                   float* scales, float* zeros, int group_size);
void cg_calibration_free(cg_quant_calibration* calib);

#ifdef __cplusplus
}
#endif

#endif /* CG_QUANTIZE_H */
