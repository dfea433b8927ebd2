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
// Tiled layout (layout 2).  W[K,N] is cut into column strips of 16 output
// columns; a strip is stored contiguously as K/256 tiles of 256 rows x 16
// columns (2 KiB each).  Inside a tile, lane L of a wave (cb = L/32,
// rb = L%32) owns rows 8rb..8rb+7 and columns 8cb..8cb+7 of the strip: 8
// little-endian
// u32 words, one per row, nibble j = column 8cb+j, stored offset-binary
// (n = v + 8).  One wave-wide pair of 16-byte loads reads a whole 2 KiB
// tile, fully coalesced.  Scales are transposed to [N/gs][K] so a lane reads
// the 8 scales of its rows with two 16-byte loads.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cgx_internal.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kStripCols = 16;             // output columns per strip
constexpr int kTileRows = 256;             // rows per tile
constexpr int kTileBytes = kTileRows * kStripCols / 2;   // 2 KiB
constexpr int kTileWords = kTileBytes / 4;

// Word index (u32) of row k, columns c..c+7 (c % 8 == 0) in the tiled layout.
__device__ __forceinline__ size_t tiled_word(int k, int c, int K) {
    int strip = c / kStripCols, tr = k / kTileRows;
    int r = k % kTileRows;
    int lane = ((c % kStripCols) / 8) * 32 + r / 8;
    size_t tile = (size_t)strip * (K / kTileRows) + tr;
    return tile * kTileWords + (size_t)lane * 8 + (r % 8);
}

// v + (v of the lane selected by the DPP control); lanes whose source falls
// outside the row read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float add_dpp(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL,
                                                          ROW_MASK, 0xF, true));
}

// Sum over each 32-lane half of the wave; the totals land in lanes 31 and 63.
__device__ __forceinline__ float half_wave_sum(float v) {
    v = add_dpp<0x111>(v);         // row_shr:1
    v = add_dpp<0x112>(v);         // row_shr:2
    v = add_dpp<0x114>(v);         // row_shr:4
    v = add_dpp<0x118>(v);         // row_shr:8  -> lane 15 of each row: row sum
    v = add_dpp<0x142, 0xA>(v);    // row_bcast:15 into rows 1 and 3
    return v;
}

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
    tiled[tiled_word(k, c, K)] = v;
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
    uint32_t v = tiled[tiled_word(k, c, K)];
    float s = scales_t[(size_t)(c / gs) * K + k];
    for (int j = 0; j < 8; j++)
        out[(size_t)k * N + c + j] = (float)((int)((v >> (4 * j)) & 0xF) - 8) * s;
}

// ------------------------------------------------------------------ GEMV

// y[M,N] = x[M,K] @ W for M <= 8.  One block per 16-column strip, W waves;
// wave w takes tiles w, w+W, ... of the strip (TPW of them; all weight loads
// are issued before any arithmetic, activations/scales one tile ahead).
//
// Nibble -> float conversion is folded into the FMA: the two nibbles of a
// 16-bit half, masked to 4 bits, are the binary16 subnormals n * 2^-24, and
// v_fma_mix_f32 multiplies a binary32 by either half of a packed pair.  The
// activation carries the 2^24 (x * s * 2^24, exact), so each product is
// exactly x * s * n, rounded once in the FMA.  Per lane: 8 columns x M
// partial sums over its 8 rows of each tile; the offset-binary bias is
// removed at the end (sum x*s*(n-8) = sum x*s*n - 8 sum x*s).  Reduction:
// lane partials through LDS, 4 threads per output, a quad DPP sum, fixed
// order (one launch, no inter-block traffic, deterministic).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Fusions around the GEMV (the decoder's linear layers):
//   PRO = kProNone:    activations x[m][k] as given (row stride ldx);
//   PRO = kProRmsNorm: RMSNorm of the rows first: x * nw[k], and the output
//                      is scaled by 1/sqrt(mean(x^2) + eps) of its row (the
//                      block computes the row sums of squares itself);
//   PRO = kProSwiGlu:  activations silu(g) * u with g = x[m][k] and
//                      u = x[m][K + k] (the fused gate|up output).
//   accumulate:        y += result (residual connection) instead of y =.
enum { kProNone = 0, kProRmsNorm = 1, kProSwiGlu = 2 };

struct GemvEpi {
    int ldx;                     // row stride of x in floats
    const float* nw;             // RMSNorm weights [K]
    float eps;
    int accumulate;
};

template <int M, int TPW, int W, int PRO>
__global__ __launch_bounds__(64 * W) void k_gemv_strip(
    const float* __restrict__ x, int K, int N, int gs,
    const u32x4* __restrict__ tiled, const float* __restrict__ scales_t,
    float* __restrict__ y, GemvEpi ep) {
    // Workgroups are dispatched round-robin over the 8 XCDs (block b runs on
    // XCD b % 8).  Give each XCD a contiguous run of strips so the strips
    // that share a scale group (and its scale row) hit the same L2.
    const int per_xcd = gridDim.x / 8;
    const int strip = (int)blockIdx.x < per_xcd * 8
                          ? (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8)
                          : (int)blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rb = lane & 31;
    const int ktiles = K / kTileRows;
    const float* srow = scales_t + (size_t)((strip * kStripCols) / gs) * K;
    const u32x4* wbase = tiled + (size_t)strip * ktiles * (kTileBytes / 16) + lane * 2;

    u32x4 wv[TPW][2];
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        int t = wave + W * j;
        int tc = t < ktiles ? t : 0;          // clamped: an invalid tile adds 0
        wv[j][0] = __builtin_nontemporal_load(wbase + (size_t)tc * (kTileBytes / 16));
        wv[j][1] = __builtin_nontemporal_load(wbase + (size_t)tc * (kTileBytes / 16) + 1);
    }

    float acc[M][8];
    float xsum[M];
    float ssq[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        xsum[m] = 0.0f;
        ssq[m] = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) acc[m][c] = 0.0f;
    }

    float sc[2][8];
    float xv[2][M][8];
    auto load_tile = [&](int j, int b) {
        int t = wave + W * j;
        bool valid = t < ktiles;
        int k0 = (valid ? t : 0) * kTileRows + rb * 8;
        float4 sa = *(const float4*)(srow + k0);
        float4 sb = *(const float4*)(srow + k0 + 4);
        float z = valid ? 0x1p24f : 0.0f;
        sc[b][0] = sa.x * z; sc[b][1] = sa.y * z; sc[b][2] = sa.z * z; sc[b][3] = sa.w * z;
        sc[b][4] = sb.x * z; sc[b][5] = sb.y * z; sc[b][6] = sb.z * z; sc[b][7] = sb.w * z;
        float nw[8];
        if (PRO == kProRmsNorm) {
            float4 na = *(const float4*)(ep.nw + k0);
            float4 nb = *(const float4*)(ep.nw + k0 + 4);
            nw[0] = na.x; nw[1] = na.y; nw[2] = na.z; nw[3] = na.w;
            nw[4] = nb.x; nw[5] = nb.y; nw[6] = nb.z; nw[7] = nb.w;
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float* xr = x + (size_t)m * ep.ldx + k0;
            float4 xa = *(const float4*)(xr);
            float4 xb = *(const float4*)(xr + 4);
            float v[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            if (PRO == kProSwiGlu) {
                float4 ua = *(const float4*)(xr + K);
                float4 ub = *(const float4*)(xr + K + 4);
                float u[8] = {ua.x, ua.y, ua.z, ua.w, ub.x, ub.y, ub.z, ub.w};
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = v[i] / (1.0f + __expf(-v[i])) * u[i];
            }
            if (PRO == kProRmsNorm) {
                if (valid && lane < 32) {
#pragma unroll
                    for (int i = 0; i < 8; i++) ssq[m] = fmaf(v[i], v[i], ssq[m]);
                }
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] *= nw[i];
            }
#pragma unroll
            for (int i = 0; i < 8; i++) xv[b][m][i] = v[i];
        }
    };
    load_tile(0, 0);
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int b = j & 1;
        if (j + 1 < TPW) load_tile(j + 1, b ^ 1);
        uint32_t wr[8] = {wv[j][0].x, wv[j][0].y, wv[j][0].z, wv[j][0].w,
                          wv[j][1].x, wv[j][1].y, wv[j][1].z, wv[j][1].w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t w = wr[i];
            f16x2 h[4] = {__builtin_bit_cast(f16x2, w & 0x000F000Fu),
                          __builtin_bit_cast(f16x2, (w >> 4) & 0x000F000Fu),
                          __builtin_bit_cast(f16x2, (w >> 8) & 0x000F000Fu),
                          __builtin_bit_cast(f16x2, (w >> 12) & 0x000F000Fu)};
#pragma unroll
            for (int m = 0; m < M; m++) {
                float xs = xv[b][m][i] * sc[b][i];
                xsum[m] += xs;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    acc[m][c] = fmaf(xs, (float)h[c].x, acc[m][c]);
                    acc[m][c + 4] = fmaf(xs, (float)h[c].y, acc[m][c + 4]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // lane partials -> LDS, row of 8*M (+4 pad) floats per lane
    constexpr int kStride = 8 * M + 4;
    __shared__ float red[64 * W * kStride];
    __shared__ float s_ssq[PRO == kProRmsNorm ? W * M : 1];
#pragma unroll
    for (int m = 0; m < M; m++) {
        float corr = -8.0f * 0x1p-24f * xsum[m];
#pragma unroll
        for (int c = 0; c < 8; c++) red[threadIdx.x * kStride + m * 8 + c] = acc[m][c] + corr;
    }
    if (PRO == kProRmsNorm) {
#pragma unroll
        for (int m = 0; m < M; m++) {
            float v = ssq[m];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
            if (lane == 0) s_ssq[wave * M + m] = v;
        }
    }
    __syncthreads();
    // 4 threads per output (m, col): part p sums row blocks p, p+4, ... of
    // every wave; a quad DPP sum combines the parts.
    const int o = threadIdx.x >> 2, part = threadIdx.x & 3;
    float v = 0.0f;
    if (o < kStripCols * M) {
        int m = o / kStripCols, col = o % kStripCols;
        int cbo = col / 8, c = col % 8;
#pragma unroll
        for (int w = 0; w < W; w++)
#pragma unroll
            for (int r = part; r < 32; r += 4)
                v += red[(w * 64 + cbo * 32 + r) * kStride + m * 8 + c];
    }
    v = add_dpp<0xB1>(v);            // quad_perm [1,0,3,2]
    v = add_dpp<0x4E>(v);            // quad_perm [2,3,0,1]
    if (o < kStripCols * M && part == 0) {
        int m = o / kStripCols, col = o % kStripCols;
        if (PRO == kProRmsNorm) {
            float ss = 0.0f;
            for (int w = 0; w < W; w++) ss += s_ssq[w * M + m];
            v *= 1.0f / sqrtf(ss / (float)K + ep.eps);
        }
        float* yp = y + (size_t)m * N + strip * kStripCols + col;
        *yp = ep.accumulate ? *yp + v : v;
    }
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

template <int M, int PRO>
int launch_gemv_m(const float* x, int K, int N, int gs, const uint8_t* tiled,
                  const float* scales_t, float* y, const GemvEpi& ep) {
    const int strips = N / kStripCols, ktiles = K / kTileRows;
    constexpr int W = 8;
    int tpw = (ktiles + W - 1) / W;
    dim3 grid(strips), block(64 * W);
    const u32x4* t = (const u32x4*)tiled;
#define CGX_GEMV_CASE(TPW)                                                               \
    hipLaunchKernelGGL((k_gemv_strip<M, TPW, W, PRO>), grid, block, 0, stream(), x, K, N, \
                       gs, t, scales_t, y, ep)
    if (tpw <= 1) CGX_GEMV_CASE(1);
    else if (tpw <= 2) CGX_GEMV_CASE(2);
    else if (tpw <= 3) CGX_GEMV_CASE(3);
    else if (tpw <= 4) CGX_GEMV_CASE(4);
    else if (tpw <= 6) CGX_GEMV_CASE(6);
    else if (tpw <= 8) CGX_GEMV_CASE(8);
    else {
        cgx_set_error("gemv: K=%d too deep for one launch (%d tiles per wave)", K, tpw);
        return -1;
    }
#undef CGX_GEMV_CASE
    return launch_check("k_gemv_strip");
}

template <int PRO>
int launch_gemv_pro(int mc, const float* x, int K, int N, int gs, const uint8_t* tiled,
                    const float* scales_t, float* y, const GemvEpi& ep) {
    switch (mc) {
        case 1: return launch_gemv_m<1, PRO>(x, K, N, gs, tiled, scales_t, y, ep);
        case 2: return launch_gemv_m<2, PRO>(x, K, N, gs, tiled, scales_t, y, ep);
        case 3: return launch_gemv_m<3, PRO>(x, K, N, gs, tiled, scales_t, y, ep);
        case 4: return launch_gemv_m<4, PRO>(x, K, N, gs, tiled, scales_t, y, ep);
        case 5: return launch_gemv_m<5, PRO>(x, K, N, gs, tiled, scales_t, y, ep);
        case 6: return launch_gemv_m<6, PRO>(x, K, N, gs, tiled, scales_t, y, ep);
        case 7: return launch_gemv_m<7, PRO>(x, K, N, gs, tiled, scales_t, y, ep);
        default: return launch_gemv_m<8, PRO>(x, K, N, gs, tiled, scales_t, y, ep);
    }
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

extern "C" int cgk_int4_transpose_scales(const float* scales, int K, int G, float* scales_t) {
    size_t ns = (size_t)K * G;
    hipLaunchKernelGGL(k_transpose_scales, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0,
                       stream(), scales, K, G, scales_t);
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

extern "C" int cgk_int4_gemv_fused(const float* x, int ldx, int M, int K, int N, int gs,
                                   const uint8_t* tiled, const float* scales_t, float* y,
                                   int pro, const float* norm_w, float eps, int accumulate) {
    if (M < 1 || K % kTileRows || N % kStripCols || gs % kStripCols || N % gs ||
        ldx < (pro == kProSwiGlu ? 2 * K : K) || (pro == kProRmsNorm && !norm_w) ||
        pro < kProNone || pro > kProSwiGlu) {
        cgx_set_error("gemv_tiled: unsupported shape M=%d K=%d N=%d gs=%d ldx=%d", M, K, N, gs,
                      ldx);
        return -1;
    }
    GemvEpi ep{ldx, norm_w, eps, accumulate};
    // M > 8: process rows in chunks of 8 (each chunk streams W once).
    for (int m0 = 0; m0 < M; m0 += 8) {
        int mc = M - m0 < 8 ? M - m0 : 8;
        const float* xc = x + (size_t)m0 * ldx;
        float* yc = y + (size_t)m0 * N;
        int rc;
        if (pro == kProRmsNorm)
            rc = launch_gemv_pro<kProRmsNorm>(mc, xc, K, N, gs, tiled, scales_t, yc, ep);
        else if (pro == kProSwiGlu)
            rc = launch_gemv_pro<kProSwiGlu>(mc, xc, K, N, gs, tiled, scales_t, yc, ep);
        else
            rc = launch_gemv_pro<kProNone>(mc, xc, K, N, gs, tiled, scales_t, yc, ep);
        if (rc) return rc;
    }
    return 0;
}

extern "C" int cgk_int4_gemv_tiled(const float* x, int M, int K, int N, int gs,
                                   const uint8_t* tiled, const float* scales_t,
                                   float* y) {
    return cgk_int4_gemv_fused(x, K, M, K, N, gs, tiled, scales_t, y, kProNone, nullptr, 0.0f,
                               0);
}

extern "C" int cgk_int4_matmul_generic(const float* x, int M, int K, int N,
                                       int gs, const uint8_t* flat,
                                       const float* scales, float* y) {
    size_t outs = (size_t)M * N;
    hipLaunchKernelGGL(k_matmul_generic, dim3((unsigned)((outs + 255) / 256)),
                       dim3(256), 0, stream(), x, M, K, N, gs, flat, scales, y);
    return launch_check("k_matmul_generic");
}
