/*
 * serialize.c -- "COG1" tensor files.
 *
 *   cg_save_model / cg_load_model   reference src/core/serialization.c:9-77
 *                                   (FP32 tensors; device-resident tensors are
 *                                   copied to the host on save)
 *   cgx_save_quantized / _load_     INT4 tensors in the same format
 *
 * INT4 entries.  The reference's directory has an INT4 dtype (2) it never
 * writes.  Here an INT4 tensor is two entries:
 *   "<name>"         dtype 2; shape[0..ndim) the logical shape and shape[7]
 *                    the quantization group size (ndim <= 7); data: the
 *                    reference's packed nibbles ((size + 1) / 2 bytes, low
 *                    nibble = even element, two's complement, flat groups);
 *   "<name>.scales"  dtype 0, shape {num_groups}: the fp32 scales.
 * Zero points are 0 in the reference's INT4 format (src/quantize/int4.c:21)
 * and are not stored.  A reference reader sees two ordinary entries.
 */
#include <stdlib.h>
#include <string.h>

#include "cg_mi355x.h"
#include "cg_serialization.h"
#include "cgx_internal.h"

/* malloc'd copy of a string (strdup is POSIX, outside C11). */
static char* copy_name(const char* s) {
    const size_t n = strlen(s) + 1;
    char* d = (char*)malloc(n);
    if (d) memcpy(d, s, n);
    return d;
}

/* A host copy of n bytes at p (host or device); *owned set when allocated. */
static const void* host_view(const void* p, size_t n, void** owned) {
    *owned = NULL;
    if (!cgx_is_device_ptr(p)) return p;
    void* h = malloc(n ? n : 1);
    if (!h || cgx_memcpy_d2h(h, p, n)) {
        free(h);
        return NULL;
    }
    *owned = h;
    return h;
}

void cg_save_model(const char* filename, cg_tensor** tensors, const char** names, int count) {
    /* reference src/core/serialization.c:9-43: header, directory
     * with offsets, then the data of each tensor */
    if (!filename || (count > 0 && (!tensors || !names)) || count < 0) {
        cgx_set_error("cg_save_model: invalid argument");
        return;
    }
    FILE* f = fopen(filename, "wb");
    if (!f) {
        cgx_set_error("cg_save_model: cannot open %s", filename);
        return;
    }
    cg_model_header h;
    memset(&h, 0, sizeof(h));
    h.magic = CG_MODEL_MAGIC;
    h.version = 1;
    h.num_tensors = (uint32_t)count;
    fwrite(&h, sizeof(h), 1, f);
    uint64_t off = sizeof(h) + (uint64_t)count * sizeof(cg_tensor_entry);
    for (int i = 0; i < count; i++) {
        cg_tensor_entry e;
        memset(&e, 0, sizeof(e));
        strncpy(e.name, names[i], 63);
        e.ndim = tensors[i]->ndim;
        memcpy(e.shape, tensors[i]->shape, (size_t)e.ndim * sizeof(int));
        e.dtype = 0;
        e.offset = off;
        e.size_bytes = (uint64_t)tensors[i]->size * sizeof(float);
        fwrite(&e, sizeof(e), 1, f);
        off += e.size_bytes;
    }
    for (int i = 0; i < count; i++) {
        void* owned;
        const void* d = host_view(tensors[i]->data, (size_t)tensors[i]->size * sizeof(float),
                                  &owned);
        if (d) fwrite(d, sizeof(float), (size_t)tensors[i]->size, f);
        free(owned);
    }
    fclose(f);
}

static cg_tensor_entry* read_directory(FILE* f, cg_model_header* h, const char* who) {
    if (fread(h, sizeof(*h), 1, f) != 1 || h->magic != CG_MODEL_MAGIC) {
        cgx_set_error("%s: not a COG1 file", who);
        return NULL;
    }
    cg_tensor_entry* e = (cg_tensor_entry*)malloc((h->num_tensors ? h->num_tensors : 1) *
                                                  sizeof(cg_tensor_entry));
    if (!e || fread(e, sizeof(cg_tensor_entry), h->num_tensors, f) != h->num_tensors) {
        free(e);
        cgx_set_error("%s: truncated directory", who);
        return NULL;
    }
    return e;
}

void cg_load_model(const char* filename, cg_tensor*** out_tensors, char*** out_names,
                   int* out_count) {
    /* reference src/core/serialization.c:45-77 */
    if (!filename || !out_tensors || !out_names || !out_count) {
        cgx_set_error("cg_load_model: invalid argument");
        return;
    }
    FILE* f = fopen(filename, "rb");
    if (!f) {
        cgx_set_error("cg_load_model: cannot open %s", filename);
        return;
    }
    cg_model_header h;
    cg_tensor_entry* e = read_directory(f, &h, "cg_load_model");
    if (!e) {
        fclose(f);
        return;
    }
    /* Only fp32 entries (dtype 0) become tensors.  Entries of other dtypes
     * (this library's INT4 entries, dtype 2) are skipped and counted in the
     * last-error string; cgx_load_quantized reads them.  An fp32 entry must
     * hold exactly the elements its shape names. */
    int count = 0, skipped = 0;
    for (uint32_t i = 0; i < h.num_tensors; i++) {
        if (e[i].dtype == 0)
            count++;
        else
            skipped++;
    }
    cg_tensor** ts = (cg_tensor**)calloc((size_t)(count ? count : 1), sizeof(cg_tensor*));
    char** ns = (char**)calloc((size_t)(count ? count : 1), sizeof(char*));
    int ok = ts && ns, k = 0;
    for (uint32_t i = 0; ok && i < h.num_tensors; i++) {
        if (e[i].dtype != 0) continue;
        e[i].name[63] = 0;
        uint64_t n = 1;
        for (int d = 0; ok && e[i].ndim >= 1 && e[i].ndim <= 8 && d < e[i].ndim; d++) {
            n *= e[i].shape[d] > 0 ? (uint64_t)e[i].shape[d] : 0;
            ok = n < (1ull << 31);
        }
        ok = ok && e[i].ndim >= 1 && e[i].ndim <= 8 && n > 0 && e[i].size_bytes == n * 4;
        ns[k] = ok ? copy_name(e[i].name) : NULL;
        ts[k] = ok ? cg_tensor_new(e[i].shape, e[i].ndim, false) : NULL;
        k++;
        ok = ok && ns[k - 1] && ts[k - 1] && fseek(f, (long)e[i].offset, SEEK_SET) == 0 &&
             fread(ts[k - 1]->data, 1, (size_t)e[i].size_bytes, f) == e[i].size_bytes;
    }
    free(e);
    fclose(f);
    if (!ok) {
        for (int i = 0; ts && ns && i < k; i++) {
            cg_tensor_free(ts[i]);
            free(ns[i]);
        }
        free(ts);
        free(ns);
        cgx_set_error("cg_load_model: malformed entry in %s", filename);
        return;
    }
    if (skipped)
        cgx_set_error("cg_load_model: skipped %d entries of dtype other than fp32 in %s "
                      "(INT4 entries: cgx_load_quantized)", skipped, filename);
    *out_tensors = ts;
    *out_names = ns;
    *out_count = count;
}

/* ------------------------------------------------------------- INT4 */

int cgx_save_quantized(const char* filename, cg_tensor_quant* const* tensors,
                       const char* const* names, int count) {
    if (!filename || count < 0 || (count > 0 && (!tensors || !names))) {
        cgx_set_error("cgx_save_quantized: invalid argument");
        return -1;
    }
    for (int i = 0; i < count; i++) {
        const cg_tensor_quant* q = tensors[i];
        cgx_qinfo info;
        if (!q || !q->data || !q->scales || q->ndim < 1 || q->ndim > 7 || q->size <= 0 ||
            q->group_size <= 0 || !names[i] || strlen(names[i]) > 63 - 7) {
            cgx_set_error("cgx_save_quantized: tensor %d: invalid tensor or name longer than "
                          "56 characters", i);
            return -1;
        }
        if (cgx_quant_lookup(q, &info) && info.layout != CGX_LAYOUT_FLAT) {
            cgx_set_error("cgx_save_quantized: tensor %d is in a tiled device layout; save the "
                          "host tensor or a flat device copy (cgx_quant_to_device_flat)", i);
            return -1;
        }
    }
    FILE* f = fopen(filename, "wb");
    if (!f) {
        cgx_set_error("cgx_save_quantized: cannot open %s", filename);
        return -1;
    }
    cg_model_header h;
    memset(&h, 0, sizeof(h));
    h.magic = CG_MODEL_MAGIC;
    h.version = 1;
    h.num_tensors = (uint32_t)(2 * count);
    int rc = fwrite(&h, sizeof(h), 1, f) == 1 ? 0 : -1;
    uint64_t off = sizeof(h) + (uint64_t)h.num_tensors * sizeof(cg_tensor_entry);
    for (int i = 0; !rc && i < count; i++) {
        const cg_tensor_quant* q = tensors[i];
        cg_tensor_entry e;
        memset(&e, 0, sizeof(e));
        strncpy(e.name, names[i], 63);
        e.ndim = q->ndim;
        memcpy(e.shape, q->shape, (size_t)q->ndim * sizeof(int));
        e.shape[7] = q->group_size;
        e.dtype = 2;
        e.offset = off;
        e.size_bytes = ((uint64_t)q->size + 1) / 2;
        off += e.size_bytes;
        cg_tensor_entry s;
        memset(&s, 0, sizeof(s));
        snprintf(s.name, sizeof(s.name), "%s.scales", names[i]);
        s.ndim = 1;
        s.shape[0] = q->num_groups;
        s.dtype = 0;
        s.offset = off;
        s.size_bytes = (uint64_t)q->num_groups * sizeof(float);
        off += s.size_bytes;
        rc = (fwrite(&e, sizeof(e), 1, f) == 1 && fwrite(&s, sizeof(s), 1, f) == 1) ? 0 : -1;
    }
    for (int i = 0; !rc && i < count; i++) {
        const cg_tensor_quant* q = tensors[i];
        const size_t nb = ((size_t)q->size + 1) / 2, ns = (size_t)q->num_groups * sizeof(float);
        void *od, *os;
        const void* d = host_view(q->data, nb, &od);
        const void* s = host_view(q->scales, ns, &os);
        rc = (d && s && fwrite(d, 1, nb, f) == nb && fwrite(s, 1, ns, f) == ns) ? 0 : -1;
        free(od);
        free(os);
    }
    if (fclose(f) || rc) {
        cgx_set_error("cgx_save_quantized: write to %s failed", filename);
        return -1;
    }
    return 0;
}

int cgx_load_quantized(const char* filename, cg_tensor_quant*** out_tensors, char*** out_names,
                       int* out_count) {
    if (!filename || !out_tensors || !out_names || !out_count) {
        cgx_set_error("cgx_load_quantized: invalid argument");
        return -1;
    }
    FILE* f = fopen(filename, "rb");
    if (!f) {
        cgx_set_error("cgx_load_quantized: cannot open %s", filename);
        return -1;
    }
    cg_model_header h;
    cg_tensor_entry* e = read_directory(f, &h, "cgx_load_quantized");
    if (!e) {
        fclose(f);
        return -1;
    }
    int nq = 0;
    for (uint32_t i = 0; i < h.num_tensors; i++) nq += e[i].dtype == 2;
    cg_tensor_quant** qs = (cg_tensor_quant**)calloc((size_t)(nq ? nq : 1), sizeof(*qs));
    char** ns = (char**)calloc((size_t)(nq ? nq : 1), sizeof(char*));
    int ok = qs && ns, k = 0;
    for (uint32_t i = 0; ok && i < h.num_tensors; i++) {
        if (e[i].dtype != 2) continue;
        e[i].name[63] = 0;
        /* the scales entry: "<name>.scales" */
        char want[80];
        snprintf(want, sizeof(want), "%s.scales", e[i].name);
        int si = -1;
        for (uint32_t j = 0; j < h.num_tensors; j++)
            if (e[j].dtype == 0 && strncmp(e[j].name, want, 64) == 0) si = (int)j;
        const int nd = e[i].ndim, gs = e[i].shape[7];
        size_t n = 1;
        int fits = 1;   /* the product stays below 2^31 at every step */
        for (int d = 0; fits && nd >= 1 && nd <= 7 && d < nd; d++) {
            n *= (size_t)(e[i].shape[d] > 0 ? e[i].shape[d] : 0);
            fits = n < (1u << 31);
        }
        const size_t ng = gs > 0 ? (n + (size_t)gs - 1) / (size_t)gs : 0;
        ok = fits && si >= 0 && nd >= 1 && nd <= 7 && gs > 0 && n > 0 && n < (1u << 31) &&
             e[i].size_bytes == (n + 1) / 2 && e[si].size_bytes == ng * sizeof(float);
        cg_tensor_quant* q = ok ? (cg_tensor_quant*)calloc(1, sizeof(*q)) : NULL;
        ok = ok && q;
        if (ok) {
            q->shape = (int*)malloc((size_t)nd * sizeof(int));
            q->data = (uint8_t*)malloc((n + 1) / 2);
            q->scales = (float*)malloc(ng * sizeof(float));
            q->zeros = (float*)calloc(ng, sizeof(float));
            qs[k] = q;
            ns[k] = copy_name(e[i].name);
            k++;
            ok = q->shape && q->data && q->scales && q->zeros && ns[k - 1];
        }
        if (ok) {
            memcpy(q->shape, e[i].shape, (size_t)nd * sizeof(int));
            q->ndim = nd;
            q->size = (int)n;
            q->quant_type = QUANT_INT4;
            q->group_size = gs;
            q->num_groups = (int)ng;
            q->symmetric = true;
            ok = fseek(f, (long)e[i].offset, SEEK_SET) == 0 &&
                 fread(q->data, 1, (n + 1) / 2, f) == (n + 1) / 2 &&
                 fseek(f, (long)e[si].offset, SEEK_SET) == 0 &&
                 fread(q->scales, sizeof(float), ng, f) == ng;
        }
    }
    free(e);
    fclose(f);
    if (!ok) {
        for (int i = 0; i < k; i++) {
            cg_tensor_quant_free(qs[i]);
            free(ns[i]);
        }
        free(qs);
        free(ns);
        cgx_set_error("cgx_load_quantized: malformed INT4 entry in %s", filename);
        return -1;
    }
    *out_tensors = qs;
    *out_names = ns;
    *out_count = nq;
    return 0;
}
