/*
 * model_file.c -- reading a decoder's weights from a "COG1" file
 * (reference src/core/serialization.c:46-77 reads the same layout).
 *
 * A matrix of the decoder may be stored whole or as column blocks (the
 * reference's transformer keeps q, k, v and gate, up as separate projections,
 * include/cg_transformer.h:41-50), each block either
 *   fp32   dtype 0, shape [K, Nb], K * Nb * 4 bytes, or
 *   INT4   dtype 2, shape [K, Nb], group size in shape[7], (K Nb + 1) / 2
 *          bytes of the reference's packed nibbles, plus an fp32 entry
 *          "<name>.scales" of K Nb / group floats (this library's INT4
 *          entries, written by cgx_save_quantized).
 * Blocks of one matrix share a dtype.  INT4 blocks are concatenated by rows
 * (row k of the matrix is row k of every block in turn), which keeps the
 * reference's flat groups when every block width is a multiple of the group
 * size; fp32 blocks are concatenated the same way and quantized as one matrix.
 * Every check happens on the directory before any data is read.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cg_serialization.h"
#include "cgx_internal.h"

struct cgx_wfile {
    FILE* f;
    cg_tensor_entry* e;
    uint32_t n;
    uint64_t file_bytes;
};

cgx_wfile* cgx_wfile_open(const char* path, const char* who) {
    FILE* f = path ? fopen(path, "rb") : NULL;
    if (!f) {
        cgx_set_error("%s: cannot open %s", who, path ? path : "(null)");
        return NULL;
    }
    cgx_wfile* w = (cgx_wfile*)calloc(1, sizeof(*w));
    cg_model_header h;
    if (!w || fread(&h, sizeof(h), 1, f) != 1 || h.magic != CG_MODEL_MAGIC ||
        h.num_tensors > (1u << 20)) {
        cgx_set_error("%s: %s is not a COG1 file", who, path);
        free(w);
        fclose(f);
        return NULL;
    }
    w->f = f;
    w->n = h.num_tensors;
    w->e = (cg_tensor_entry*)malloc((size_t)(w->n ? w->n : 1) * sizeof(cg_tensor_entry));
    if (!w->e || fread(w->e, sizeof(cg_tensor_entry), w->n, f) != w->n ||
        fseek(f, 0, SEEK_END) != 0) {
        cgx_set_error("%s: %s: truncated directory", who, path);
        cgx_wfile_close(w);
        return NULL;
    }
    const long end = ftell(f);
    w->file_bytes = end > 0 ? (uint64_t)end : 0;
    for (uint32_t i = 0; i < w->n; i++) w->e[i].name[63] = 0;
    return w;
}

void cgx_wfile_close(cgx_wfile* w) {
    if (!w) return;
    if (w->f) fclose(w->f);
    free(w->e);
    free(w);
}

int cgx_wfile_find(const cgx_wfile* w, const char* name) {
    for (uint32_t i = 0; w && i < w->n; i++)
        if (strncmp(w->e[i].name, name, 64) == 0) return (int)i;
    return -1;
}

/* Entry i holds `bytes` bytes inside the file. */
static int entry_in_file(const cgx_wfile* w, int i, uint64_t bytes) {
    const cg_tensor_entry* e = &w->e[i];
    return e->size_bytes == bytes && e->offset <= w->file_bytes &&
           bytes <= w->file_bytes - e->offset;
}

static int is_shape2(const cg_tensor_entry* e, int K, int N) {
    return e->ndim == 2 && e->shape[0] == K && e->shape[1] == N;
}

int cgx_wfile_vector(const cgx_wfile* w, const char* name, int n, const char* who) {
    const int i = cgx_wfile_find(w, name);
    if (i < 0) return -1;
    const cg_tensor_entry* e = &w->e[i];
    const int shape_ok = (e->ndim == 1 && e->shape[0] == n) || is_shape2(e, 1, n);
    if (e->dtype != 0 || !shape_ok || !entry_in_file(w, i, (uint64_t)n * 4)) {
        cgx_set_error("%s: entry %s must be fp32 of shape [%d]", who, name, n);
        return -2;
    }
    return i;
}

int cgx_wfile_matrix_kind(const cgx_wfile* w, const int* idx, const int* widths, int nb, int K,
                          int gs, const char* who) {
    if (!w || nb < 1) return -1;
    const int kind = w->e[idx[0]].dtype;
    for (int b = 0; b < nb; b++) {
        const cg_tensor_entry* e = &w->e[idx[b]];
        const uint64_t n = (uint64_t)K * (uint64_t)widths[b];
        if (e->dtype != kind || (kind != 0 && kind != 2)) {
            cgx_set_error("%s: entry %s: dtype %d (the blocks of one matrix are all fp32 (0) "
                          "or all INT4 (2))", who, e->name, e->dtype);
            return -1;
        }
        if (!is_shape2(e, K, widths[b])) {
            cgx_set_error("%s: entry %s has shape [%d, %d], expected [%d, %d]", who, e->name,
                          e->ndim >= 1 ? e->shape[0] : 0, e->ndim >= 2 ? e->shape[1] : 0, K,
                          widths[b]);
            return -1;
        }
        if (kind == 0) {
            if (!entry_in_file(w, idx[b], n * 4)) {
                cgx_set_error("%s: entry %s: %llu bytes at offset %llu, expected %llu inside "
                              "the file", who, e->name, (unsigned long long)e->size_bytes,
                              (unsigned long long)e->offset, (unsigned long long)(n * 4));
                return -1;
            }
            continue;
        }
        char sname[80];
        snprintf(sname, sizeof(sname), "%s.scales", e->name);
        const int si = cgx_wfile_find(w, sname);
        if (e->shape[7] != gs || (nb > 1 && widths[b] % gs) || n % (uint64_t)gs) {
            cgx_set_error("%s: INT4 entry %s: group size %d (the model's is %d, and a block of "
                          "a split matrix must hold whole groups of its rows)", who, e->name,
                          e->shape[7], gs);
            return -1;
        }
        if (!entry_in_file(w, idx[b], (n + 1) / 2) || si < 0 || w->e[si].dtype != 0 ||
            !entry_in_file(w, si, n / (uint64_t)gs * 4)) {
            cgx_set_error("%s: INT4 entry %s: data or %s missing or of the wrong size", who,
                          e->name, sname);
            return -1;
        }
    }
    return kind;
}

static int read_at(const cgx_wfile* w, uint64_t off, void* dst, size_t bytes) {
    return fseek(w->f, (long)off, SEEK_SET) == 0 && fread(dst, 1, bytes, w->f) == bytes ? 0 : -1;
}

int cgx_wfile_read_vector(const cgx_wfile* w, int i, float* out, int n) {
    if (read_at(w, w->e[i].offset, out, (size_t)n * 4)) {
        cgx_set_error("read of entry %s failed", w->e[i].name);
        return -1;
    }
    return 0;
}

/* Rows of `nb` blocks into one [K][row] matrix: block b's rows of rb[b]
 * units land at column unit offset sum(rb[0..b)).  unit: bytes per unit. */
static int read_blocks(const cgx_wfile* w, const uint64_t* offs, const size_t* rb, int nb,
                       int K, size_t unit, uint8_t* out) {
    size_t row = 0, col = 0;
    for (int b = 0; b < nb; b++) row += rb[b];
    if (nb == 1) return read_at(w, offs[0], out, (size_t)K * row * unit);
    for (int b = 0; b < nb; b++) {
        const size_t bytes = (size_t)K * rb[b] * unit;
        uint8_t* tmp = (uint8_t*)malloc(bytes ? bytes : 1);
        if (!tmp || read_at(w, offs[b], tmp, bytes)) {
            free(tmp);
            return -1;
        }
        for (int k = 0; k < K; k++)
            memcpy(out + ((size_t)k * row + col) * unit, tmp + (size_t)k * rb[b] * unit,
                   rb[b] * unit);
        free(tmp);
        col += rb[b];
    }
    return 0;
}

int cgx_wfile_read_f32(const cgx_wfile* w, const int* idx, const int* widths, int nb, int K,
                       float* out) {
    uint64_t offs[8];
    size_t rb[8];
    if (nb > 8) return -1;
    for (int b = 0; b < nb; b++) {
        offs[b] = w->e[idx[b]].offset;
        rb[b] = (size_t)widths[b];
    }
    if (read_blocks(w, offs, rb, nb, K, 4, (uint8_t*)out)) {
        cgx_set_error("read of entry %s failed", w->e[idx[0]].name);
        return -1;
    }
    return 0;
}

int cgx_wfile_read_int4(const cgx_wfile* w, const int* idx, const int* widths, int nb, int K,
                        int gs, uint8_t* data, float* scales) {
    uint64_t offs[8], soffs[8];
    size_t rb[8], rs[8];
    if (nb > 8) return -1;
    for (int b = 0; b < nb; b++) {
        char sname[80];
        snprintf(sname, sizeof(sname), "%s.scales", w->e[idx[b]].name);
        const int si = cgx_wfile_find(w, sname);
        if (si < 0) return -1;
        offs[b] = w->e[idx[b]].offset;
        soffs[b] = w->e[si].offset;
        rb[b] = (size_t)widths[b] / 2;        /* bytes of a row */
        rs[b] = (size_t)widths[b] / (size_t)gs;
    }
    if (nb == 1) {
        /* one block: the flat nibbles and scales as stored (any width) */
        const size_t n = (size_t)K * (size_t)widths[0];
        if (read_at(w, offs[0], data, (n + 1) / 2) ||
            read_at(w, soffs[0], scales, n / (size_t)gs * 4)) {
            cgx_set_error("read of entry %s failed", w->e[idx[0]].name);
            return -1;
        }
        return 0;
    }
    if (read_blocks(w, offs, rb, nb, K, 1, data) ||
        read_blocks(w, soffs, rs, nb, K, 4, (uint8_t*)scales)) {
        cgx_set_error("read of entry %s failed", w->e[idx[0]].name);
        return -1;
    }
    return 0;
}
