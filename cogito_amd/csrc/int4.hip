// int4.hip -- INT4 weight kernels for gfx950: quantize / dequantize, the
// re-tiling of cogito's row-major nibble layout into the GEMV layout, the
// HBM-streaming GEMV for skinny activations (M <= 8) and a generic kernel
// with the reference's exact flat-index semantics for any shape.
//
// Reference semantics (cogito-ml/cogito):
//   quantize   src/quantize/int4.c:10-59   (absmax/7 per flat group, roundf,
//                                           clamp [-8,7], low nibble = even)
//   dequantize src/quantize/int4.c:61-79   ((float)v - 0) * scale
//   matmul     src/quantize/int4.c:90-114  (y = x @ W, W[K,N], group of
//                                           element (k,j) = (k*N+j)/gs)
//
// Tiled layout (layout 2).  W[K,N] is cut into 64x64 tiles; tiles are stored
// column-strip major (strip = 64 output columns, all K/64 tiles of a strip
// contiguous, 2 KiB each).  Inside a tile, lane L of a wave (rb = L/8,
// cb = L%8) owns rows 8rb..8rb+7 and columns 8cb..8cb+7: 8 little-endian
// u32 words, one per row, nibble j = column 8cb+j, stored offset-binary
// (n = v + 8).  One wave-wide pair of 16-byte loads therefore reads a whole
// 2 KiB tile, fully coalesced.  Scales are transposed to [N/gs][K] so a lane
// reads the 8 scales of its rows with two 16-byte loads.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cgx_internal.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 64;                  // rows == cols per tile
constexpr int kTileBytes = kTile * kTile / 2;

inline hipStream_t stream() { return (hipStream_t)cgx_stream(); }

int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        cgx_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

// ------------------------------------------------------------- quantize

__global__ void k_quant_scales(const float* __restrict__ x, int n, int gs,
                               float* __restrict__ scales, int ng) {
    int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ng) return;
    int start = g * gs, end = min(start + gs, n);
    float absmax = 0.0f;
    for (int i = start; i < end; i++) absmax = fmaxf(absmax, fabsf(x[i]));
    float s = __fdiv_rn(absmax, 7.0f);
    if (s < 1e-10f) s = 1.0f;
    scales[g] = s;
}

__device__ inline int q4(float v, float s) {
    int q = (int)roundf(__fdiv_rn(v, s));
    return q > 7 ? 7 : (q < -8 ? -8 : q);
}

__global__ void k_quant_pack(const float* __restrict__ x, int n, int gs,
                             const float* __restrict__ scales,
                             uint8_t* __restrict__ data) {
    int b = blockIdx.x * blockDim.x + threadIdx.x;
    int i = 2 * b;
    if (i >= n) return;
    float s = scales[i / gs];
    int v0 = q4(x[i], s);
    int v1 = (i + 1 < n) ? q4(x[i + 1], s) : 0;
    data[b] = (uint8_t)((v0 & 0xF) | ((v1 & 0xF) << 4));
}

// ----------------------------------------------------------- dequantize

__device__ inline int sext4(unsigned v) { return (int)(v & 0xF) - (int)((v & 0x8) << 1); }

__global__ void k_dequant_flat(const uint8_t* __restrict__ data,
                               const float* __restrict__ scales, int n, int gs,
                               float* __restrict__ out) {
    int b = blockIdx.x * blockDim.x + threadIdx.x;
    int i = 2 * b;
    if (i >= n) return;
    unsigned byte = data[b];
    float s = scales[i / gs];
    out[i] = (float)sext4(byte) * s;
    if (i + 1 < n) out[i + 1] = (float)sext4(byte >> 4) * s;
}

// ---------------------------------------------------------------- tiling

// One thread per output word: row k, columns c..c+7 (c % 8 == 0).
__global__ void k_repack_tiled(const uint32_t* __restrict__ flat, int K, int N,
                               uint32_t* __restrict__ tiled) {
    size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t words_per_row = (size_t)N / 8;
    if (w >= (size_t)K * words_per_row) return;
    int k = (int)(w / words_per_row);
    int c = (int)(w % words_per_row) * 8;
    uint32_t v = flat[w] ^ 0x88888888u;      // two's complement -> offset binary
    int strip = c / kTile, tr = k / kTile;
    int lane = ((k % kTile) / 8) * 8 + (c % kTile) / 8;
    size_t tile = (size_t)strip * (K / kTile) + tr;
    tiled[tile * (kTileBytes / 4) + lane * 8 + (k % 8)] = v;
}

__global__ void k_transpose_scales(const float* __restrict__ scales, int K,
                                   int G, float* __restrict__ scales_t) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)K * G) return;
    int k = (int)(i / G), g = (int)(i % G);
    scales_t[(size_t)g * K + k] = scales[i];
}

__global__ void k_dequant_tiled(const uint32_t* __restrict__ tiled,
                                const float* __restrict__ scales_t, int K,
                                int N, int gs, float* __restrict__ out) {
    size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t words_per_row = (size_t)N / 8;
    if (w >= (size_t)K * words_per_row) return;
    int k = (int)(w / words_per_row);
    int c = (int)(w % words_per_row) * 8;
    int strip = c / kTile, tr = k / kTile;
    int lane = ((k % kTile) / 8) * 8 + (c % kTile) / 8;
    size_t tile = (size_t)strip * (K / kTile) + tr;
    uint32_t v = tiled[tile * (kTileBytes / 4) + lane * 8 + (k % 8)];
    float s = scales_t[(size_t)(c / gs) * K + k];
    for (int j = 0; j < 8; j++)
        out[(size_t)k * N + c + j] = (float)((int)((v >> (4 * j)) & 0xF) - 8) * s;
}

// ------------------------------------------------------------------ GEMV

// y[M,N] = x[M,K] @ W for M <= 8.  Grid: (N/64 strips) x ksplit blocks of
// 256 threads; block (strip, ks) covers tiles [ks*tpb, ks*tpb + tpb) of the
// strip and wave w takes tiles w, w+4, ... of that range (TPW of them, all
// loads issued before any arithmetic).  Per lane: 8 columns x M partial
// sums over its 8 rows of each tile; the offset-binary bias is removed once
// at the end (sum x*s*(n-8) = sum x*s*n - 8 sum x*s).  Reduction: across the
// 8 row-blocks of a wave by xor-shuffles, across the 4 waves in LDS, and
// across the ksplit blocks of a strip through a partial-sum workspace that
// the last-arriving block sums in fixed order (deterministic, one launch).
template <int M, int TPW>
__global__ __launch_bounds__(256) void k_gemv_tiled(
    const float* __restrict__ x, int K, int N, int gs,
    const u32x4* __restrict__ tiled, const float* __restrict__ scales_t,
    float* __restrict__ y, float* __restrict__ partial,
    unsigned* __restrict__ counters, int ksplit, int tiles_per_block) {
    const int strip = blockIdx.x / ksplit;
    const int ks = blockIdx.x % ksplit;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rb = lane >> 3, cb = lane & 7;
    const int ktiles = K / kTile;
    const int t_begin = ks * tiles_per_block;
    const int t_end = min(t_begin + tiles_per_block, ktiles);
    const float* srow = scales_t + (size_t)((strip * kTile) / gs) * K;
    const u32x4* wbase = tiled + (size_t)strip * ktiles * (kTileBytes / 16) + lane * 2;

    u32x4 wv[TPW][2];
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        int t = t_begin + wave + 4 * j;
        if (t < t_end) {
            wv[j][0] = __builtin_nontemporal_load(wbase + (size_t)t * (kTileBytes / 16));
            wv[j][1] = __builtin_nontemporal_load(wbase + (size_t)t * (kTileBytes / 16) + 1);
        } else {
            wv[j][0] = (u32x4)(0x88888888u);
            wv[j][1] = wv[j][0];
        }
    }

    float acc[M][8];
    float xsum[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        xsum[m] = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) acc[m][c] = 0.0f;
    }

#pragma unroll
    for (int j = 0; j < TPW; j++) {
        int t = t_begin + wave + 4 * j;
        if (t >= t_end) break;
        int k0 = t * kTile + rb * 8;
        float4 sa = *(const float4*)(srow + k0);
        float4 sb = *(const float4*)(srow + k0 + 4);
        float sc[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
        float xv[M][8];
#pragma unroll
        for (int m = 0; m < M; m++) {
            float4 xa = *(const float4*)(x + (size_t)m * K + k0);
            float4 xb = *(const float4*)(x + (size_t)m * K + k0 + 4);
            xv[m][0] = xa.x; xv[m][1] = xa.y; xv[m][2] = xa.z; xv[m][3] = xa.w;
            xv[m][4] = xb.x; xv[m][5] = xb.y; xv[m][6] = xb.z; xv[m][7] = xb.w;
        }
        uint32_t wr[8] = {wv[j][0].x, wv[j][0].y, wv[j][0].z, wv[j][0].w,
                          wv[j][1].x, wv[j][1].y, wv[j][1].z, wv[j][1].w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t lo = wr[i] & 0x0F0F0F0Fu;
            uint32_t hi = (wr[i] >> 4) & 0x0F0F0F0Fu;
            float f[8];
            f[0] = (float)(lo & 0xFF);         f[1] = (float)(hi & 0xFF);
            f[2] = (float)((lo >> 8) & 0xFF);  f[3] = (float)((hi >> 8) & 0xFF);
            f[4] = (float)((lo >> 16) & 0xFF); f[5] = (float)((hi >> 16) & 0xFF);
            f[6] = (float)(lo >> 24);          f[7] = (float)(hi >> 24);
#pragma unroll
            for (int m = 0; m < M; m++) {
                float xs = xv[m][i] * sc[i];
                xsum[m] += xs;
#pragma unroll
                for (int c = 0; c < 8; c++) acc[m][c] = fmaf(xs, f[c], acc[m][c]);
            }
        }
    }

#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int c = 0; c < 8; c++) acc[m][c] = fmaf(-8.0f, xsum[m], acc[m][c]);

    // Sum the 8 row-blocks of the wave (lanes differing in bits 3..5).
#pragma unroll
    for (int off = 8; off < 64; off <<= 1)
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int c = 0; c < 8; c++) acc[m][c] += __shfl_xor(acc[m][c], off);

    __shared__ float red[4][M][kTile];
    __shared__ int s_last;
    if (lane < 8) {
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int c = 0; c < 8; c++) red[wave][m][cb * 8 + c] = acc[m][c];
    }
    __syncthreads();

    const int col0 = strip * kTile;
    if (ksplit == 1) {
        for (int i = threadIdx.x; i < M * kTile; i += 256) {
            int m = i / kTile, col = i % kTile;
            y[(size_t)m * N + col0 + col] =
                (red[0][m][col] + red[1][m][col]) + (red[2][m][col] + red[3][m][col]);
        }
        return;
    }
    for (int i = threadIdx.x; i < M * kTile; i += 256) {
        int m = i / kTile, col = i % kTile;
        partial[((size_t)ks * M + m) * N + col0 + col] =
            (red[0][m][col] + red[1][m][col]) + (red[2][m][col] + red[3][m][col]);
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned prev = atomicAdd(&counters[strip], 1u);
        s_last = (prev == (unsigned)(ksplit - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int i = threadIdx.x; i < M * kTile; i += 256) {
        int m = i / kTile, col = i % kTile;
        float v = 0.0f;
        for (int s = 0; s < ksplit; s++)
            v += __builtin_nontemporal_load(&partial[((size_t)s * M + m) * N + col0 + col]);
        y[(size_t)m * N + col0 + col] = v;
    }
    if (threadIdx.x == 0) counters[strip] = 0u;
}

// Reference-order matmul for any K, N, group size: one thread per output,
// sequential k, products rounded exactly as (x * w) * scale and added in
// order, so the result equals the reference bit for bit.
__global__ void k_matmul_generic(const float* __restrict__ x, int M, int K,
                                 int N, int gs, const uint8_t* __restrict__ data,
                                 const float* __restrict__ scales,
                                 float* __restrict__ y) {
    size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= (size_t)M * N) return;
    int i = (int)(o / N), j = (int)(o % N);
    float sum = 0.0f;
    for (int k = 0; k < K; k++) {
        size_t w_idx = (size_t)k * N + j;
        float scale = scales[w_idx / gs];
        unsigned byte = data[w_idx / 2];
        int w = (w_idx & 1) ? sext4(byte >> 4) : sext4(byte);
        sum = __fadd_rn(sum, __fmul_rn(__fmul_rn(x[(size_t)i * K + k], (float)w), scale));
    }
    y[o] = sum;
}

template <int M>
int launch_gemv_m(const float* x, int K, int N, int gs, const uint8_t* tiled,
                  const float* scales_t, float* y) {
    const int strips = N / kTile, ktiles = K / kTile;
    // Aim for ~2 blocks (8 waves) per CU on 256 CUs, at least 4 tiles
    // (8 KiB) per block so the per-block reduction stays amortised.
    int ksplit = (512 + strips - 1) / strips;
    int max_split = ktiles / 4 > 0 ? ktiles / 4 : 1;
    if (ksplit > max_split) ksplit = max_split;
    if (ksplit < 1) ksplit = 1;
    int tpb = (ktiles + ksplit - 1) / ksplit;
    ksplit = (ktiles + tpb - 1) / tpb;
    int tpw = (tpb + 3) / 4;
    float* partial = nullptr;
    unsigned* counters = nullptr;
    if (ksplit > 1) {
        partial = (float*)cgx_scratch(CGX_SLOT_WS0, (size_t)ksplit * M * N * sizeof(float));
        counters = cgx_counters((size_t)strips);
        if (!partial || !counters) return -1;
    }
    dim3 grid(strips * ksplit), block(256);
    const u32x4* t = (const u32x4*)tiled;
#define CGX_GEMV_CASE(TPW)                                                         \
    hipLaunchKernelGGL((k_gemv_tiled<M, TPW>), grid, block, 0, stream(), x, K, N, \
                       gs, t, scales_t, y, partial, counters, ksplit, tpb)
    if (tpw <= 1) CGX_GEMV_CASE(1);
    else if (tpw <= 2) CGX_GEMV_CASE(2);
    else if (tpw <= 4) CGX_GEMV_CASE(4);
    else if (tpw <= 8) CGX_GEMV_CASE(8);
    else if (tpw <= 16) CGX_GEMV_CASE(16);
    else {
        cgx_set_error("gemv: K=%d too deep for one launch (tpw %d)", K, tpw);
        return -1;
    }
#undef CGX_GEMV_CASE
    return launch_check("k_gemv_tiled");
}

}  // namespace

extern "C" int cgk_int4_quantize(const float* x, int n, int gs, uint8_t* data,
                                 float* scales) {
    int ng = (n + gs - 1) / gs;
    hipLaunchKernelGGL(k_quant_scales, dim3((ng + 255) / 256), dim3(256), 0,
                       stream(), x, n, gs, scales, ng);
    if (launch_check("k_quant_scales")) return -1;
    int nb = (n + 1) / 2;
    hipLaunchKernelGGL(k_quant_pack, dim3((nb + 255) / 256), dim3(256), 0,
                       stream(), x, n, gs, scales, data);
    return launch_check("k_quant_pack");
}

extern "C" int cgk_int4_dequantize_flat(const uint8_t* data, const float* scales,
                                        int n, int gs, float* out) {
    int nb = (n + 1) / 2;
    hipLaunchKernelGGL(k_dequant_flat, dim3((nb + 255) / 256), dim3(256), 0,
                       stream(), data, scales, n, gs, out);
    return launch_check("k_dequant_flat");
}

extern "C" int cgk_int4_repack_tiled(const uint8_t* flat, const float* scales,
                                     int K, int N, int gs, uint8_t* tiled,
                                     float* scales_t) {
    size_t words = (size_t)K * N / 8;
    hipLaunchKernelGGL(k_repack_tiled, dim3((unsigned)((words + 255) / 256)),
                       dim3(256), 0, stream(), (const uint32_t*)flat, K, N,
                       (uint32_t*)tiled);
    if (launch_check("k_repack_tiled")) return -1;
    int G = N / gs;
    size_t ns = (size_t)K * G;
    hipLaunchKernelGGL(k_transpose_scales, dim3((unsigned)((ns + 255) / 256)),
                       dim3(256), 0, stream(), scales, K, G, scales_t);
    return launch_check("k_transpose_scales");
}

extern "C" int cgk_int4_dequantize_tiled(const uint8_t* tiled,
                                         const float* scales_t, int K, int N,
                                         int gs, float* out) {
    size_t words = (size_t)K * N / 8;
    hipLaunchKernelGGL(k_dequant_tiled, dim3((unsigned)((words + 255) / 256)),
                       dim3(256), 0, stream(), (const uint32_t*)tiled, scales_t,
                       K, N, gs, out);
    return launch_check("k_dequant_tiled");
}

extern "C" int cgk_int4_gemv_tiled(const float* x, int M, int K, int N, int gs,
                                   const uint8_t* tiled, const float* scales_t,
                                   float* y) {
    if (M < 1 || K % kTile || N % kTile || gs % kTile || N % gs) {
        cgx_set_error("gemv_tiled: unsupported shape M=%d K=%d N=%d gs=%d", M, K,
                      N, gs);
        return -1;
    }
    // M > 8: process rows in chunks of 8 (each chunk streams W once).
    for (int m0 = 0; m0 < M; m0 += 8) {
        int mc = M - m0 < 8 ? M - m0 : 8;
        const float* xc = x + (size_t)m0 * K;
        float* yc = y + (size_t)m0 * N;
        int rc;
        switch (mc) {
            case 1: rc = launch_gemv_m<1>(xc, K, N, gs, tiled, scales_t, yc); break;
            case 2: rc = launch_gemv_m<2>(xc, K, N, gs, tiled, scales_t, yc); break;
            case 3: rc = launch_gemv_m<3>(xc, K, N, gs, tiled, scales_t, yc); break;
            case 4: rc = launch_gemv_m<4>(xc, K, N, gs, tiled, scales_t, yc); break;
            case 5: rc = launch_gemv_m<5>(xc, K, N, gs, tiled, scales_t, yc); break;
            case 6: rc = launch_gemv_m<6>(xc, K, N, gs, tiled, scales_t, yc); break;
            case 7: rc = launch_gemv_m<7>(xc, K, N, gs, tiled, scales_t, yc); break;
            default: rc = launch_gemv_m<8>(xc, K, N, gs, tiled, scales_t, yc); break;
        }
        if (rc) return rc;
    }
    return 0;
}

extern "C" int cgk_int4_matmul_generic(const float* x, int M, int K, int N,
                                       int gs, const uint8_t* flat,
                                       const float* scales, float* y) {
    size_t outs = (size_t)M * N;
    hipLaunchKernelGGL(k_matmul_generic, dim3((unsigned)((outs + 255) / 256)),
                       dim3(256), 0, stream(), x, M, K, N, gs, flat, scales, y);
    return launch_check("k_matmul_generic");
}
