/*
 * cg_serialization.h -- "COG1" tensor files (cogito's include/cg_serialization.h,
 * same declarations and struct layouts).
 *
 * cg_save_model / cg_load_model keep the reference's format and semantics
 * (src/core/serialization.c:9-77): a header, a directory of entries, then the
 * data, FP32 tensors.  This library also writes and reads INT4 tensors in the
 * same files through cgx_save_quantized / cgx_load_quantized (cg_mi355x.h),
 * using the directory's INT4 dtype (2), which the reference declares and
 * never writes.
 */
#ifndef CG_SERIALIZATION_H
#define CG_SERIALIZATION_H

#include <stdint.h>
#include <stdio.h>

#include "cg_tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CG_MODEL_MAGIC 0x434F4731  /* "COG1" */

typedef struct {
    uint32_t magic;
    uint32_t version;
    uint32_t num_tensors;
    uint64_t total_size;
} cg_model_header;

typedef struct {
    char name[64];
    int ndim;
    int shape[8];
    int dtype; /* 0=FP32, 1=BF16, 2=INT4 */
    uint64_t offset;
    uint64_t size_bytes;
} cg_tensor_entry;

void cg_save_model(const char* filename, cg_tensor** tensors, const char** names, int count);
void cg_load_model(const char* filename, cg_tensor*** out_tensors, char*** out_names,
                   int* out_count);

#ifdef __cplusplus
}
#endif

#endif /* CG_SERIALIZATION_H */
