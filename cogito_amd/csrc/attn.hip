// attn.hip -- INT4 KV cache and flash attention (decode / verify / prefill)
// for gfx950.
//
// Reference (cogito-ml/cogito):
//   KV append / get      src/quantize/int4.c:147-289  (absmax/7 per group of
//                        `group_size` in head_dim, floor 1e-8, roundf, clamp)
//   flash forward (GQA)  src/cuda/flash_attn_kernels.c:261-396 (online
//                        softmax; KV head of query head h = h * H_k / H)
//   RoPE                 src/attention/flash_attn.c:318-362
//
// Attention kernel: split-KV flash decoding on fp32 matrix cores.  A block
// is (key split, KV head [x batch], chunk of 32 query rows); the query rows of
// a KV head are every (query head h mapped to it, query position).  Each of
// the 4 waves is an independent online-softmax worker over its own 32-key
// tiles: S = Q K^T with v_mfma_f32_32x32x2f32 (K read and dequantised straight
// into the B operand), mask, running max / sum, P staged through LDS into the
// A layout, O += P V with V tiles dequantised into LDS.  The 4 waves merge in
// LDS; splits merge in a second kernel.  fp32 products throughout (the
// reference's arithmetic type), accumulation order differs (within 1e-3).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>

#include "cgx_internal.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

inline hipStream_t stream() { return (hipStream_t)cgx_stream(); }

int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        cgx_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

__device__ __forceinline__ int sext4(unsigned v) { return (int)(v & 0xF) - (int)((v & 0x8) << 1); }

// ------------------------------------------------------------- KV cache

// One thread per (token, head, group): quantise K and V of that group.
__global__ void k_kv_append(const float* __restrict__ k, const float* __restrict__ v,
                            int T, int H, int D, int gs, int pos,
                            uint8_t* __restrict__ kc, uint8_t* __restrict__ vc,
                            float* __restrict__ ks, float* __restrict__ vs) {
    int ngh = D / gs;
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= T * H * ngh) return;
    int g = idx % ngh, h = (idx / ngh) % H, t = idx / (ngh * H);
    const float* kr = k + ((size_t)t * H + h) * D + g * gs;
    const float* vr = v + ((size_t)t * H + h) * D + g * gs;
    float mk = 0.0f, mv = 0.0f;
    for (int i = 0; i < gs; i++) {
        float ak = fabsf(kr[i]), av = fabsf(vr[i]);
        if (ak > mk) mk = ak;
        if (av > mv) mv = av;
    }
    float sk = __fdiv_rn(mk, 7.0f), sv = __fdiv_rn(mv, 7.0f);
    if (sk < 1e-8f) sk = 1.0f;
    if (sv < 1e-8f) sv = 1.0f;
    size_t tok = (size_t)pos + t;
    ks[(tok * H + h) * ngh + g] = sk;
    vs[(tok * H + h) * ngh + g] = sv;
    uint8_t* kp = kc + (tok * H + h) * (D / 2) + g * gs / 2;
    uint8_t* vp = vc + (tok * H + h) * (D / 2) + g * gs / 2;
    for (int i = 0; i < gs; i += 2) {
        int k0 = (int)roundf(__fdiv_rn(kr[i], sk)), k1 = (int)roundf(__fdiv_rn(kr[i + 1], sk));
        int v0 = (int)roundf(__fdiv_rn(vr[i], sv)), v1 = (int)roundf(__fdiv_rn(vr[i + 1], sv));
        k0 = k0 > 7 ? 7 : (k0 < -8 ? -8 : k0);
        k1 = k1 > 7 ? 7 : (k1 < -8 ? -8 : k1);
        v0 = v0 > 7 ? 7 : (v0 < -8 ? -8 : v0);
        v1 = v1 > 7 ? 7 : (v1 < -8 ? -8 : v1);
        kp[i / 2] = (uint8_t)((k0 & 0xF) | ((k1 & 0xF) << 4));
        vp[i / 2] = (uint8_t)((v0 & 0xF) | ((v1 & 0xF) << 4));
    }
}

// One thread per packed byte of [len][H][D/2]: (float)v * scale.
__global__ void k_kv_get(const uint8_t* __restrict__ kc, const uint8_t* __restrict__ vc,
                         const float* __restrict__ ks, const float* __restrict__ vs,
                         int len, int H, int D, int gs, float* __restrict__ ko,
                         float* __restrict__ vo) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t nb = (size_t)len * H * (D / 2);
    if (b >= nb) return;
    size_t th = b / (D / 2);                 // token * H + head
    int d = (int)(b % (D / 2)) * 2;
    int ngh = D / gs;
    float sk = ks[th * ngh + d / gs], sv = vs[th * ngh + d / gs];
    unsigned kb = kc[b], vb = vc[b];
    ko[th * D + d] = (float)sext4(kb) * sk;
    ko[th * D + d + 1] = (float)sext4(kb >> 4) * sk;
    vo[th * D + d] = (float)sext4(vb) * sv;
    vo[th * D + d + 1] = (float)sext4(vb >> 4) * sv;
}

// ------------------------------------------------------------ attention

// kMaskCausal: bottom-right aligned (query q sees keys <= Nk - Nq + q), the
// verify rule; kMaskCausalTL: the reference's rule (keys <= q); kMaskTree:
// every key before the last Nq, plus the query's ancestors among the last Nq.
enum MaskKind {
    kMaskNone = 0, kMaskCausal = 1, kMaskWindow = 2, kMaskCustom = 3, kMaskTree = 4,
    kMaskCausalTL = 5
};

struct AttnArgs {
    const float* Q;              // [B][Nq][H][D]
    // INT4 cache slice of one layer (int4 = 1) or fp32 K/V [B][Nk][Hk][D]
    int int4;
    const uint8_t* kc;
    const uint8_t* vc;
    const float* ks;
    const float* vs;
    int gs;
    const float* K;
    const float* V;
    int B, Nq, Nk, H, Hk, D;
    float scale;
    int mask_kind, window;
    const float* mask;           // custom additive [Nq][Nk]
    unsigned long long anc[64];  // tree: ancestor bits per query over the last Nq keys
    int splits, keys_per_split;
    float* O;                    // [B][Nq][H][D] (splits == 1)
    float* part_o;               // [splits][B][Nq][H][D]
    float* part_ml;              // [splits][B][Nq][H][2]
    float* lse;                  // optional [B][H][Nq] (splits == 1)
};

__device__ __forceinline__ int head_begin(int hk, int H, int Hk) { return (hk * H + Hk - 1) / Hk; }

// KV source of the attention kernel: INT4 cache with D == DP (16-byte rows,
// vector loads), INT4 cache of any even D, or fp32 K/V.
enum KvMode { kKvInt4Vec = 0, kKvInt4 = 1, kKvF32 = 2 };

template <int DP, int MODE>   // DP: head_dim padded to a multiple of 32 (32, 64, 128)
__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
    constexpr int CB = DP / 32;         // 32-wide column blocks of O (and K chunks)
    __shared__ float sQ[32][DP + 1];    // scaled Q rows of this block
    __shared__ float sV[4][32][DP + 1]; // per-wave V tile (reused for the merge)
    __shared__ float sP[4][32][33];     // per-wave S, then P, tile
    __shared__ float sM[4][32], sL[4][32], sAlpha[4][32];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int split = blockIdx.x;
    const int hk = blockIdx.y % a.Hk, b = blockIdx.y / a.Hk;
    const int h0 = head_begin(hk, a.H, a.Hk), h1 = head_begin(hk + 1, a.H, a.Hk);
    const int R = (h1 - h0) * a.Nq;
    const int row0 = blockIdx.z * 32;
    if (row0 >= R) return;                       // uniform over the block
    const int par = lane >> 5;                   // k-parity of this lane's operands

    // scaled Q rows -> LDS (rows past R and columns past D are zero)
    for (int e = threadIdx.x; e < 32 * DP; e += 256) {
        int i = e / DP, d = e % DP, rr = row0 + i;
        float v = 0.0f;
        if (rr < R && d < a.D) {
            int h = h0 + rr / a.Nq, q = rr % a.Nq;
            v = a.Q[(((size_t)b * a.Nq + q) * a.H + h) * a.D + d] * a.scale;
        }
        sQ[i][d] = v;
    }
    __syncthreads();

    // softmax state: lane owns row (lane & 31) and key half (lane >> 5)
    const int srow = lane & 31, khalf = lane >> 5;
    const int s_rr = row0 + srow;
    const bool s_rok = s_rr < R;
    const int s_q = s_rok ? s_rr % a.Nq : 0;
    const unsigned long long s_anc = (a.mask_kind == kMaskTree && s_rok) ? a.anc[s_q] : 0ull;
    float m_run = -INFINITY, l_run = 0.0f;
    f32x16 o[CB];
#pragma unroll
    for (int c = 0; c < CB; c++) o[c] = (f32x16)(0.0f);

    const int k_begin = split * a.keys_per_split;
    const int k_end = min(a.Nk, k_begin + a.keys_per_split);
    const int ntiles = (k_end - k_begin + 31) / 32;
    const int rounds = (ntiles + 3) / 4;       // every wave runs the same count
    const int ngh = MODE != kKvF32 ? a.D / a.gs : 1;

    for (int rd = 0; rd < rounds; rd++) {
        const int tile = rd * 4 + wave;
        const int kt = k_begin + tile * 32;     // first key of this wave's tile
        const int kk_b = kt + (lane & 31);      // key of this lane's B operand / S column
        const bool key_ok = tile < ntiles && kk_b < k_end;
        const size_t th = (size_t)(key_ok ? kk_b : 0) * a.Hk + hk;

        // ---- S = Q K^T, head_dim in chunks of 32 (16 MFMA k-steps each)
        f32x16 sacc = (f32x16)(0.0f);
#pragma unroll
        for (int c = 0; c < CB; c++) {
            float kb[16];
            if (MODE == kKvInt4Vec) {
                u32x4 w4 = ((const u32x4*)(a.kc + th * (a.D / 2)))[c];
                uint32_t words[4] = {w4.x, w4.y, w4.z, w4.w};
                const float* srow = a.ks + th * ngh;
#pragma unroll
                for (int s = 0; s < 16; s++) {
                    unsigned byte = (words[s / 4] >> (8 * (s % 4))) & 0xFF;
                    int d = 32 * c + 2 * s + par;
                    kb[s] = key_ok ? (float)sext4(par ? byte >> 4 : byte) * srow[d / a.gs] : 0.0f;
                }
            } else {
#pragma unroll
                for (int s = 0; s < 16; s++) {
                    int d = 32 * c + 2 * s + par;
                    float val = 0.0f;
                    if (key_ok && d < a.D) {
                        if (MODE == kKvInt4) {
                            unsigned byte = a.kc[th * (a.D / 2) + d / 2];
                            val = (float)sext4(par ? byte >> 4 : byte) * a.ks[th * ngh + d / a.gs];
                        } else {
                            val = a.K[(((size_t)b * a.Nk + kk_b) * a.Hk + hk) * a.D + d];
                        }
                    }
                    kb[s] = val;
                }
            }
#pragma unroll
            for (int s = 0; s < 16; s++)
                sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(sQ[lane & 31][32 * c + 2 * s + par],
                                                              kb[s], sacc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);     // bound the live operands to one chunk
        }
        // ---- V tile into LDS (dequantised): lane -> key lane/2, half lane%2
        {
            const int vj = lane >> 1, half = lane & 1;
            const int kk = kt + vj;
            const bool ok = tile < ntiles && kk < k_end;
            const size_t tv = (size_t)(ok ? kk : 0) * a.Hk + hk;
            if (MODE == kKvInt4Vec) {
                // DP/4 bytes of this half of the row, up to 16 bytes at a time
                constexpr int QB = DP / 4 < 16 ? DP / 4 : 16;   // bytes per load
                const uint8_t* vrow = a.vc + tv * (a.D / 2) + half * (DP / 4);
                const float* srow = a.vs + tv * ngh;
#pragma unroll
                for (int q = 0; q < DP / 4 / QB; q++) {
                    uint32_t words[4] = {0u, 0u, 0u, 0u};
                    if (QB == 16) {
                        u32x4 w4 = ok ? ((const u32x4*)vrow)[q] : (u32x4)(0u);
                        words[0] = w4.x; words[1] = w4.y; words[2] = w4.z; words[3] = w4.w;
                    } else if (ok) {
                        uint2 w2 = ((const uint2*)vrow)[q];
                        words[0] = w2.x; words[1] = w2.y;
                    }
#pragma unroll
                    for (int e = 0; e < QB; e++) {
                        int dd = half * (DP / 2) + q * 2 * QB + 2 * e;
                        unsigned byte = (words[e / 4] >> (8 * (e % 4))) & 0xFF;
                        float sc = ok ? srow[dd / a.gs] : 0.0f;
                        sV[wave][vj][dd] = (float)sext4(byte) * sc;
                        sV[wave][vj][dd + 1] = (float)sext4(byte >> 4) * sc;
                    }
                }
            } else {
                for (int dd = half * (DP / 2); dd < (half + 1) * (DP / 2); dd += 2) {
                    float v0 = 0.0f, v1 = 0.0f;
                    if (ok && dd < a.D) {
                        if (MODE == kKvInt4) {
                            unsigned byte = a.vc[tv * (a.D / 2) + dd / 2];
                            float sc = a.vs[tv * ngh + dd / a.gs];
                            v0 = (float)sext4(byte) * sc;
                            v1 = (float)sext4(byte >> 4) * sc;
                        } else {
                            const float* vr = a.V + (((size_t)b * a.Nk + kk) * a.Hk + hk) * a.D;
                            v0 = vr[dd];
                            v1 = dd + 1 < a.D ? vr[dd + 1] : 0.0f;
                        }
                    }
                    sV[wave][vj][dd] = v0;
                    sV[wave][vj][dd + 1] = v1;
                }
            }
        }
        // ---- S -> LDS; online softmax with one row per lane (16 keys each)
#pragma unroll
        for (int v = 0; v < 16; v++) sP[wave][(v / 4) * 8 + par * 4 + (v % 4)][lane & 31] = sacc[v];
        __syncthreads();
        {
            float sv[16];
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                int jj = khalf * 16 + j, kk = kt + jj;
                // keys past the split do not exist (-inf, weight 0); keys a mask
                // hides score -FLT_MAX as in the reference, so a row that sees
                // no key at all averages V uniformly, as the reference does
                const bool exists = s_rok && tile < ntiles && kk < k_end;
                bool vis = exists;
                switch (a.mask_kind) {
                    case kMaskCausal: vis = vis && kk <= a.Nk - a.Nq + s_q; break;
                    case kMaskCausalTL: vis = vis && kk <= s_q; break;
                    case kMaskWindow: vis = vis && abs(kk - s_q) <= a.window; break;
                    case kMaskTree: {
                        int base = a.Nk - a.Nq;
                        vis = vis && (kk < base || ((s_anc >> (kk - base)) & 1ull));
                        break;
                    }
                    default: break;
                }
                float x = sP[wave][srow][jj];
                if (exists && a.mask_kind == kMaskCustom) x += a.mask[(size_t)s_q * a.Nk + kk];
                sv[j] = !exists ? -INFINITY : (vis ? x : -FLT_MAX);
                mx = fmaxf(mx, sv[j]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            float m_new = fmaxf(m_run, mx);
            float alpha = (m_new == -INFINITY) ? 1.0f : __expf(m_run - m_new);
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                float pv = (m_new == -INFINITY) ? 0.0f : __expf(sv[j] - m_new);
                sP[wave][srow][khalf * 16 + j] = pv;
                sum += pv;
            }
            sum += __shfl_xor(sum, 32);
            l_run = l_run * alpha + sum;
            m_run = m_new;
            if (khalf == 0) sAlpha[wave][srow] = alpha;
        }
        __syncthreads();
#pragma unroll
        for (int v = 0; v < 16; v++) {
            float al = sAlpha[wave][(v / 4) * 8 + par * 4 + (v % 4)];
#pragma unroll
            for (int c = 0; c < CB; c++) o[c][v] *= al;
        }
        // ---- O += P V
#pragma unroll
        for (int s = 0; s < 16; s++) {
            float pa = sP[wave][lane & 31][2 * s + par];
#pragma unroll
            for (int c = 0; c < CB; c++) {
                float vb = sV[wave][2 * s + par][c * 32 + (lane & 31)];
                o[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(pa, vb, o[c], 0, 0, 0);
            }
            if ((s & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
    }

    // ---- merge the 4 waves: per row (m, l), then O
    if (khalf == 0) {
        sM[wave][srow] = m_run;
        sL[wave][srow] = l_run;
    }
#pragma unroll
    for (int c = 0; c < CB; c++)
#pragma unroll
        for (int v = 0; v < 16; v++)
            sV[wave][(v / 4) * 8 + par * 4 + (v % 4)][c * 32 + (lane & 31)] = o[c][v];
    __syncthreads();
    for (int e = threadIdx.x; e < 32 * DP; e += 256) {
        int i = e / DP, d = e % DP;
        int rr = row0 + i;
        if (rr >= R || d >= a.D) continue;
        float M = fmaxf(fmaxf(sM[0][i], sM[1][i]), fmaxf(sM[2][i], sM[3][i]));
        float L = 0.0f, acc = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            float wgt = (sM[w][i] == -INFINITY) ? 0.0f : __expf(sM[w][i] - M);
            L += sL[w][i] * wgt;
            acc += sV[w][i][d] * wgt;
        }
        int h = h0 + rr / a.Nq, q = rr % a.Nq;
        size_t orow = ((size_t)b * a.Nq + q) * a.H + h;
        if (a.splits == 1) {
            a.O[orow * a.D + d] = L > 0.0f ? acc / L : 0.0f;
            if (a.lse && d == 0)
                a.lse[((size_t)b * a.H + h) * a.Nq + q] = L > 0.0f ? M + logf(L) : -INFINITY;
        } else {
            size_t nrow = (size_t)a.B * a.Nq * a.H;
            a.part_o[((size_t)split * nrow + orow) * a.D + d] = acc;
            if (d == 0) {
                a.part_ml[((size_t)split * nrow + orow) * 2] = M;
                a.part_ml[((size_t)split * nrow + orow) * 2 + 1] = L;
            }
        }
    }
}

// Merge the per-split partials: one thread per (row, d).
__global__ void k_attn_combine(const float* __restrict__ part_o,
                               const float* __restrict__ part_ml, int splits, int nrow,
                               int D, int Nq, int H, float* __restrict__ O,
                               float* __restrict__ lse) {
    size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (size_t)nrow * D) return;
    size_t row = e / D;
    int d = (int)(e % D);
    float M = -INFINITY;
    for (int s = 0; s < splits; s++) M = fmaxf(M, part_ml[((size_t)s * nrow + row) * 2]);
    float L = 0.0f, acc = 0.0f;
    for (int s = 0; s < splits; s++) {
        float m = part_ml[((size_t)s * nrow + row) * 2];
        float w = (m == -INFINITY) ? 0.0f : __expf(m - M);
        L += part_ml[((size_t)s * nrow + row) * 2 + 1] * w;
        acc += part_o[((size_t)s * nrow + row) * D + d] * w;
    }
    O[row * D + d] = L > 0.0f ? acc / L : 0.0f;
    if (lse && d == 0) {
        // row = (b * Nq + q) * H + h  ->  lse[(b * H + h) * Nq + q]
        size_t h = row % H, bq = row / H, q = bq % Nq, b = bq / Nq;
        lse[(b * H + h) * Nq + q] = L > 0.0f ? M + logf(L) : -INFINITY;
    }
}

// --------------------------------------------------------------- RoPE

// cg_apply_rope arithmetic (flash_attn.c:342-358), one thread per pair.
__global__ void k_rope(float* __restrict__ x, int S, int H, int D, int pos0, float theta) {
    int half = D / 2;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)S * H * half) return;
    int i = (int)(idx % half);
    size_t sh = idx / half;                 // pos * H + h
    int pos = (int)(sh / H);
    float freq = __fdiv_rn(1.0f, powf(theta, __fdiv_rn((float)(2 * i), (float)D)));
    float angle = __fmul_rn((float)(pos0 + pos), freq);
    float c = cosf(angle), s = sinf(angle);
    float* v = x + sh * D;
    float x0 = v[i], x1 = v[i + half];
    v[i] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
    v[i + half] = __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
}

__global__ void k_rope_freqs(float* __restrict__ cs, float* __restrict__ sn, int S, int D,
                             float theta) {
    int half = D / 2;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)S * half) return;
    int i = (int)(idx % half), pos = (int)(idx / half);
    float freq = __fdiv_rn(1.0f, powf(theta, __fdiv_rn((float)(2 * i), (float)D)));
    float angle = __fmul_rn((float)pos, freq);
    cs[idx] = cosf(angle);
    sn[idx] = sinf(angle);
}

// ALiBi (flash_attn.c:368-388).
__global__ void k_alibi_slopes(float* slopes, int H) {
    int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= H) return;
    float base = powf(2.0f, __fdiv_rn(-8.0f, (float)H));
    slopes[h] = powf(base, (float)(h + 1));
}

__global__ void k_alibi_bias(float* bias, int Sq, int Sk, int H, const float* slopes) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)H * Sq * Sk) return;
    int ki = (int)(idx % Sk);
    size_t hq = idx / Sk;
    int qi = (int)(hq % Sq), h = (int)(hq / Sq);
    bias[idx] = __fmul_rn(slopes[h], (float)(ki - qi));
}

}  // namespace

// -------------------------------------------------------------- launchers

extern "C" int cgk_kv_append(const float* k, const float* v, int T, int H, int D, int gs,
                             int pos, uint8_t* kc, uint8_t* vc, float* ks, float* vs) {
    int n = T * H * (D / gs);
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_kv_append, dim3((n + 127) / 128), dim3(128), 0, stream(), k, v, T, H,
                       D, gs, pos, kc, vc, ks, vs);
    return launch_check("k_kv_append");
}

extern "C" int cgk_kv_get(const uint8_t* kc, const uint8_t* vc, const float* ks,
                          const float* vs, int len, int H, int D, int gs, float* ko,
                          float* vo) {
    size_t nb = (size_t)len * H * (D / 2);
    if (!nb) return 0;
    hipLaunchKernelGGL(k_kv_get, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, stream(),
                       kc, vc, ks, vs, len, H, D, gs, ko, vo);
    return launch_check("k_kv_get");
}

// Attention launcher shared by the INT4-cache and fp32 entry points.
extern "C" int cgk_attention(const float* Q, int int4, const uint8_t* kc, const uint8_t* vc,
                             const float* ks, const float* vs, int gs, const float* K,
                             const float* V, int B, int Nq, int Nk, int H, int Hk, int D,
                             float scale, int mask_kind, int window, const float* mask,
                             const unsigned long long* anc, float* O, float* lse) {
    if (D <= 0 || D > 128 || (int4 && ((D & 1) || gs <= 0 || D % gs || B != 1)) || H <= 0 ||
        Hk <= 0 || Nq <= 0 || Nk <= 0 || B <= 0) {
        cgx_set_error("attention: unsupported shape B=%d Nq=%d Nk=%d H=%d Hk=%d D=%d", B, Nq,
                      Nk, H, Hk, D);
        return -1;
    }
    if (mask_kind == kMaskTree && (Nq > 64 || !anc)) {
        cgx_set_error("attention: tree mask needs ancestor bits for at most 64 new tokens");
        return -1;
    }
    // the decode kernel reads Q and the K cache and writes O in 16-byte units
    const int aligned = !(((uintptr_t)Q | (uintptr_t)O | (uintptr_t)kc) & 15);
    if (int4 && !lse && aligned && cgk_attn_dec_supported(D, gs, B, mask_kind))
        return cgk_attn_dec(Q, kc, vc, ks, vs, Nq, Nk, H, Hk, D, scale, mask_kind, anc, O);
    AttnArgs a;
    a.Q = Q; a.int4 = int4; a.kc = kc; a.vc = vc; a.ks = ks; a.vs = vs; a.gs = gs;
    a.K = K; a.V = V; a.B = B; a.Nq = Nq; a.Nk = Nk; a.H = H; a.Hk = Hk; a.D = D;
    a.scale = scale; a.mask_kind = mask_kind; a.window = window; a.mask = mask;
    for (int i = 0; i < 64; i++) a.anc[i] = (mask_kind == kMaskTree && i < Nq) ? anc[i] : 0ull;
    a.O = O; a.lse = lse;
    int max_g = 0;
    for (int hk = 0; hk < Hk; hk++) {
        int g = ((hk + 1) * H + Hk - 1) / Hk - (hk * H + Hk - 1) / Hk;
        max_g = g > max_g ? g : max_g;
    }
    int chunks = (max_g * Nq + 31) / 32;
    // enough blocks to fill 256 CUs twice, at least 128 keys (4 tiles) per split
    long long base_blocks = (long long)Hk * B * chunks;
    int splits = (int)((512 + base_blocks - 1) / base_blocks);
    int max_splits = (Nk + 127) / 128;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    int kps = (Nk + splits - 1) / splits;
    kps = (kps + 31) / 32 * 32;
    splits = (Nk + kps - 1) / kps;
    a.splits = splits;
    a.keys_per_split = kps;
    size_t nrow = (size_t)B * Nq * H;
    if (splits > 1) {
        a.part_o = (float*)cgx_scratch(CGX_SLOT_WS2, (size_t)splits * nrow * D * 4);
        a.part_ml = (float*)cgx_scratch(CGX_SLOT_WS3, (size_t)splits * nrow * 2 * 4);
        if (!a.part_o || !a.part_ml) return -1;
    } else {
        a.part_o = a.part_ml = nullptr;
    }
    if ((long long)Hk * B > 65535 || chunks > 65535) {
        cgx_set_error("attention: grid too large");
        return -1;
    }
    dim3 grid(splits, Hk * B, chunks), block(256);
    int dp = D <= 32 ? 32 : (D <= 64 ? 64 : 128);
    int mode = !int4 ? kKvF32 : (D == dp ? kKvInt4Vec : kKvInt4);
#define CGX_ATTN(DPV, MV) hipLaunchKernelGGL((k_attn<DPV, MV>), grid, block, 0, stream(), a)
#define CGX_ATTN_DP(DPV)                                   \
    do {                                                   \
        if (mode == kKvInt4Vec) CGX_ATTN(DPV, kKvInt4Vec); \
        else if (mode == kKvInt4) CGX_ATTN(DPV, kKvInt4);  \
        else CGX_ATTN(DPV, kKvF32);                        \
    } while (0)
    if (dp == 32) CGX_ATTN_DP(32);
    else if (dp == 64) CGX_ATTN_DP(64);
    else CGX_ATTN_DP(128);
#undef CGX_ATTN_DP
#undef CGX_ATTN
    if (launch_check("k_attn")) return -1;
    if (splits > 1) {
        size_t n = nrow * D;
        hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           stream(), a.part_o, a.part_ml, splits, (int)nrow, D, Nq, H, O, lse);
        if (launch_check("k_attn_combine")) return -1;
    }
    return 0;
}

extern "C" int cgk_rope(float* x, int S, int H, int D, int pos0, float theta) {
    size_t n = (size_t)S * H * (D / 2);
    if (!n) return 0;
    hipLaunchKernelGGL(k_rope, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream(), x, S,
                       H, D, pos0, theta);
    return launch_check("k_rope");
}

extern "C" int cgk_rope_freqs(float* cs, float* sn, int S, int D, float theta) {
    size_t n = (size_t)S * (D / 2);
    if (!n) return 0;
    hipLaunchKernelGGL(k_rope_freqs, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream(),
                       cs, sn, S, D, theta);
    return launch_check("k_rope_freqs");
}

extern "C" int cgk_alibi_slopes(float* slopes, int H) {
    if (H <= 0) return 0;
    hipLaunchKernelGGL(k_alibi_slopes, dim3((H + 63) / 64), dim3(64), 0, stream(), slopes, H);
    return launch_check("k_alibi_slopes");
}

extern "C" int cgk_alibi_bias(float* bias, int Sq, int Sk, int H, const float* slopes) {
    size_t n = (size_t)H * Sq * Sk;
    if (!n) return 0;
    hipLaunchKernelGGL(k_alibi_bias, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream(),
                       bias, Sq, Sk, H, slopes);
    return launch_check("k_alibi_bias");
}
