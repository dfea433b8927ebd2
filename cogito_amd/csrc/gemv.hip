// gemv.hip -- INT4 dequant GEMV / skinny GEMM on the gfx950 matrix cores.
//
// y[M,N] = x[M,K] @ W, W[K,N] INT4 with one scale per (row k, group of gs
// columns) -- cogito's flat-index groups (src/quantize/int4.c:90-114: element
// (k, j) uses scales[(k*N + j) / gs]; N % gs == 0 here, so the group of
// column j in row k is k*(N/gs) + j/gs).  M <= 16 rows per launch.
//
// Arithmetic.  The scale varies along the reduction index k, so it is folded
// into the activation: a[m][k] = x[m][k] * s[k][g].  The nibble side is exact
// in fp16 (integers -8..7); the activation side is carried as hi + lo, two
// fp16 numbers with 22 significant bits (relative error <= 2^-22 per
// element), after scaling by a power of two 2^E chosen per (wave, round) so
// that |a * 2^E| < 2^15.  v_mfma_f32_16x16x32_f16 forms the exact products and
// accumulates in fp32; the 2^-E is undone in fp32 at the end of each round.
//
// Layout 3 (HBM).  Column tiles of 16 columns; a tile is K/128 chunks of 1
// KiB; in chunk c, lane l (0..63) owns bytes 16l..16l+15: u32 word j (0..3)
// holds rows 32(4c+j) + 8(l/16) + p, p = 0..7, of column 16*tile + l%16, the
// row of position p in nibble slot {0,4,1,5,2,6,3,7}[p], offset-binary
// (v + 8).  So one dwordx4 per lane reads four MFMA B operands of a tile and
// a wave reads 1 KiB contiguous.  Optional pairing (SwiGLU): layout tile 2t is
// column tile t (gate), 2t+1 is column tile ff/16 + t (up).  Scales: fp32
// [N/gs][K] (transposed), shared with layout 2.
//
// Block = 8 waves, T column tiles (T*16 columns), the full K: waves take
// rounds of 256 rows round-robin, each wave its own accumulators; the waves
// are summed in a fixed order at the end (deterministic, no atomics).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "cgx_internal.h"

namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kRoundK = 256;            // rows per wave round
constexpr int kChunkK = 128;            // rows per 1 KiB chunk
constexpr int kChunkBytes = 1024;
// A-operand rows in LDS: 256 halfs + 16 bytes of padding, so the 16 rows a
// ds_read_b128 touches start in different bank quads
constexpr int kRowH = kRoundK + 8;
constexpr int kBufWord3 = 0x00020000;    // buffer resource word 3 (raw dword access)

inline hipStream_t stream() { return (hipStream_t)cgx_stream(); }

int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        cgx_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

enum { kProNone = 0, kProRmsNorm = 1 };
enum { kEpiStore = 0, kEpiAccumulate = 1, kEpiSwiGlu = 2 };

struct MfmaArgs {
    const float* x;          // [M][ldx]
    int ldx, M, K, N, gs;
    const uint8_t* w;        // layout 3
    const float* scales_t;   // [N/gs][K]
    float* y;                // [M][ldy]
    int ldy;
    const float* nw;         // RMSNorm weights [K]
    float eps;
    int ff;                  // SwiGLU: columns of the gate half (N / 2)
};

// Logical column tile of layout tile L.
__device__ __forceinline__ int logical_tile(int L, int paired, int ff_tiles) {
    return paired ? ((L & 1) ? ff_tiles + (L >> 1) : (L >> 1)) : L;
}

// Nibble-decode constants: the masks in SGPRs and the fp16 exponent bits in
// a VGPR, produced where the compiler does not see them as constants.  It
// then forms (w & m) | c as one v_and_or_b32; with literal masks it emits a
// separate AND and OR, because VOP3 takes no literal operand on this target.
struct NibConst {
    uint32_t mlo, mhi, mag;
};

__device__ __forceinline__ NibConst nib_consts() {
    NibConst k;
    asm volatile("s_mov_b32 %0, 0x000f000f" : "=s"(k.mlo));
    asm volatile("s_mov_b32 %0, 0x00f000f0" : "=s"(k.mhi));
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(k.mag));
    return k;
}

// Four MFMA B operands (one per k-block of a chunk) from the lane's 16 bytes.
__device__ __forceinline__ f16x8 nib_to_f16(uint32_t w, const NibConst& nk) {
    const uint32_t w8 = w >> 8;
    const f16x2 m1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const f16x2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const f16x2 m72 = {(_Float16)-72.0f, (_Float16)-72.0f};
    f16x2 p0 = __builtin_bit_cast(f16x2, (w & nk.mlo) | nk.mag) + m1032;
    f16x2 p1 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (w & nk.mhi) | nk.mag), s16, m72);
    f16x2 p2 = __builtin_bit_cast(f16x2, (w8 & nk.mlo) | nk.mag) + m1032;
    f16x2 p3 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (w8 & nk.mhi) | nk.mag), s16, m72);
    f16x8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// Maximum over the wave of non-negative values (DPP within rows of 16, row
// broadcasts, then lane 63); every lane gets the result.
__device__ __forceinline__ float wave_max_nonneg(float v) {
#define CGX_DPP_MAX(CTRL, RMASK)                                                           \
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL,    \
                                                            RMASK, 0xF, true)))
    CGX_DPP_MAX(0x111, 0xF);      // row_shr:1
    CGX_DPP_MAX(0x112, 0xF);      // row_shr:2
    CGX_DPP_MAX(0x114, 0xF);      // row_shr:4
    CGX_DPP_MAX(0x118, 0xF);      // row_shr:8   -> lane 15 of each row: row max
    CGX_DPP_MAX(0x142, 0xA);      // row_bcast:15 into rows 1 and 3
    CGX_DPP_MAX(0x143, 0xC);      // row_bcast:31 into rows 2 and 3
#undef CGX_DPP_MAX
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over the wave with the same DPP pattern (no LDS round trips: a chain of
// ds_bpermute exchanges at the end of every wave cost ~1.5 us on the 7B
// gate|up launch); fixed order, so the result is deterministic.
__device__ __forceinline__ float wave_sum(float v) {
#define CGX_DPP_ADD(CTRL, RMASK)                                                           \
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, RMASK, 0xF, true))
    CGX_DPP_ADD(0x111, 0xF);      // row_shr:1
    CGX_DPP_ADD(0x112, 0xF);      // row_shr:2
    CGX_DPP_ADD(0x114, 0xF);      // row_shr:4
    CGX_DPP_ADD(0x118, 0xF);      // row_shr:8   -> lane 15 of each row: row sum
    CGX_DPP_ADD(0x142, 0xA);      // row_bcast:15 into rows 1 and 3
    CGX_DPP_ADD(0x143, 0xC);      // row_bcast:31 into rows 2 and 3
#undef CGX_DPP_ADD
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Inclusive scans over the 16 lanes of each DPP row (row_shr 1, 2, 4, 8):
// lane 15 of a row holds the row's sum / maximum (non-negative values).
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xF, 0xF, true));
    return v;
}
__device__ __forceinline__ float row16_max_nonneg(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xF, 0xF, true)));
    return v;
}
// The same over each 32-lane half (row_bcast:15 adds row 0's total into row
// 1 and row 2's into row 3): lanes 31 and 63 hold the halves' results.
__device__ __forceinline__ float half_sum(float v) {
    v = row16_sum(v);
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, true));
}
__device__ __forceinline__ float half_max_nonneg(float v) {
    v = row16_max_nonneg(v);
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, true)));
}

// MP: rows padded (1, 2, 4, 5, 8 or 16); T: column tiles per block; NG: scale groups
// per block (1, or 2 for a gate|up pair).
// W: waves per block (8; 16 for deep K, each wave then has fewer rounds).
// The gate|up pair at up to 5 rows asks for 4 waves per SIMD (at most 128
// VGPRs), so that two 8-wave blocks share a CU; unconstrained it takes 138.
template <int MP, int T, int NG, int PRO, int EPI, int W>
__global__ __launch_bounds__(64 * W, (NG == 2 && T == 2 && MP <= 5) ? 4 : 1) void k_gemv_mfma(MfmaArgs a) {
    // per wave: A operands of one round and scale group, [hi|lo][MP][256] halfs
    constexpr int kAHalfs = 2 * MP * kRowH;
    constexpr int kRedFloats = W * T * MP * 16;
    constexpr int kLdsFloats =
        (W * kAHalfs / 2) > kRedFloats ? (W * kAHalfs / 2) : kRedFloats;
    __shared__ float lds[kLdsFloats];
    __shared__ float s_ssq[W][MP];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const NibConst nk = nib_consts();
    const int M = a.M;
    const int paired = EPI == kEpiSwiGlu;
    const int ff_tiles = a.ff / 16;
    // XCD-aware order: consecutive blocks share scale rows; give each XCD a
    // contiguous run (block b runs on XCD b % 8).
    const int nblk = gridDim.x;
    const int per_xcd = nblk / 8;
    const int sb = (int)blockIdx.x < per_xcd * 8
                       ? (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8)
                       : (int)blockIdx.x;
    const int L0 = sb * T;                         // first layout tile

    // scale rows of the block's groups: one, or for a gate|up pair (layout
    // tiles alternate gate / up, and T and L0 are even) the gate group in
    // slot 0 for the even tiles and the up group in slot 1 for the odd ones
    static_assert(NG == 1 || T % 2 == 0, "a gate|up block holds whole pairs");
    int grp[NG];
#pragma unroll
    for (int j = 0; j < T; j++) {
        int lt = logical_tile(L0 + j, paired, ff_tiles);
        grp[NG == 1 ? 0 : (j & 1)] = lt * 16 / a.gs;
    }

    const int K = a.K;
    const int rounds = K / kRoundK;
    const int nchunks = K / kChunkK;
    const int my_rounds = (rounds - wave + W - 1) / W;   // may be 0

    _Float16* abuf = (_Float16*)lds + (size_t)wave * kAHalfs;
    const int mrow = (lane & 15) < M ? (lane & 15) : M - 1;    // A row this lane feeds
    const int g4 = lane >> 4;
    // with 8 or fewer rows one MFMA takes both parts: A rows 0-7 are the hi
    // parts of rows 0-7, A rows 8-15 their lo parts; the two halves of D are
    // summed at the end
    const int hl8 = (lane >> 3) & 1;
    const int mrow8 = (lane & 7) < M ? (lane & 7) : M - 1;

    f32x4 tot[T];
#pragma unroll
    for (int j = 0; j < T; j++) tot[j] = (f32x4)(0.0f);
    float ssq[MP];
#pragma unroll
    for (int m = 0; m < MP; m++) ssq[m] = 0.0f;

    // weights of one round: T tiles x 2 chunks x 16 bytes per lane
    u32x4 wcur[T][2], wnxt[T][2];
    auto load_w = [&](int r, u32x4 (&dst)[T][2]) {
#pragma unroll
        for (int j = 0; j < T; j++)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                size_t off = ((size_t)(L0 + j) * nchunks + 2 * r + c) * kChunkBytes + 16 * lane;
                dst[j][c] = __builtin_nontemporal_load((const u32x4*)(a.w + off));
            }
    };
    // activations / scales / norm weights of one round (lane -> rows k0..k0+3),
    // fetched one round ahead like the weights
    struct ARaw {
        float4 x[MP];
        float4 s[NG];
        float4 nw;
    };
    auto load_a = [&](int r, ARaw& d) {
        const int k0 = r * kRoundK + 4 * lane;
#pragma unroll
        for (int q = 0; q < NG; q++) d.s[q] = *(const float4*)(a.scales_t + (size_t)grp[q] * K + k0);
        d.nw = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        if (PRO == kProRmsNorm) d.nw = *(const float4*)(a.nw + k0);
#pragma unroll
        for (int m = 0; m < MP; m++)
            d.x[m] = m < M ? *(const float4*)(a.x + (size_t)m * a.ldx + k0)
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    auto round_body = [&](ARaw& acur, u32x4 (&wcur)[T][2]) {
        // ---- A operands of this round
        float4 xv[MP];
        float amax = 0.0f;
#pragma unroll
        for (int m = 0; m < MP; m++) {
            float4 t = acur.x[m];
            if (PRO == kProRmsNorm) {
                ssq[m] = fmaf(t.x, t.x, ssq[m]);
                ssq[m] = fmaf(t.y, t.y, ssq[m]);
                ssq[m] = fmaf(t.z, t.z, ssq[m]);
                ssq[m] = fmaf(t.w, t.w, ssq[m]);
            }
            xv[m] = t;
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w))));
        }
        // the RMSNorm weight multiplies the scale of each k (x * nw * s =
        // x * (nw * s)): 4 products per group and round instead of one per
        // row and k, and no second copy of the rows (the 7B gate|up instance
        // spilled with one: 20.6 -> 17.4 us)
        float smax = 0.0f;
#pragma unroll
        for (int q = 0; q < NG; q++) {
            if (PRO == kProRmsNorm) {
                acur.s[q].x *= acur.nw.x; acur.s[q].y *= acur.nw.y;
                acur.s[q].z *= acur.nw.z; acur.s[q].w *= acur.nw.w;
            }
            smax = fmaxf(smax, fmaxf(fmaxf(fabsf(acur.s[q].x), fabsf(acur.s[q].y)),
                                     fmaxf(fabsf(acur.s[q].z), fabsf(acur.s[q].w))));
        }
        // |x * s| <= amax * smax over the round; scale so that it is < 2^15
        float bound = wave_max_nonneg(amax) * wave_max_nonneg(smax);
        int E = 0;
        if (bound > 0.0f && bound < __builtin_inff()) E = 14 - ilogbf(bound);
        E = E > 100 ? 100 : (E < -100 ? -100 : E);
        const float up = ldexpf(1.0f, E);
        const float down = ldexpf(1.0f, -E);
        f32x4 acc[T];
#pragma unroll
        for (int j = 0; j < T; j++) acc[j] = (f32x4)(0.0f);
        // one scale group at a time through the wave's A buffer (a gate|up
        // pair: the gate group for the even tiles, then the up group for the
        // odd ones)
#pragma unroll
        for (int q = 0; q < NG; q++) {
            if (q > 0) __builtin_amdgcn_wave_barrier();   // group q-1's reads came first
            const float s0 = acur.s[q].x * up, s1 = acur.s[q].y * up, s2 = acur.s[q].z * up,
                        s3 = acur.s[q].w * up;
#pragma unroll
            for (int m = 0; m < MP; m++) {
                if (m < M) {
                    // hi = v rounded toward zero to fp16 (packed conversion),
                    // lo = the exact remainder rounded to fp16
                    float v0 = xv[m].x * s0, v1 = xv[m].y * s1, v2 = xv[m].z * s2,
                          v3 = xv[m].w * s3;
                    const f16x2 h01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(v0, v1));
                    const f16x2 h23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(v2, v3));
                    const f16x2 l01 = __builtin_bit_cast(
                        f16x2, __builtin_amdgcn_cvt_pkrtz(v0 - (float)h01[0], v1 - (float)h01[1]));
                    const f16x2 l23 = __builtin_bit_cast(
                        f16x2, __builtin_amdgcn_cvt_pkrtz(v2 - (float)h23[0], v3 - (float)h23[1]));
                    *(uint2*)(abuf + (0 * MP + m) * kRowH + 4 * lane) =
                        make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
                    *(uint2*)(abuf + (1 * MP + m) * kRowH + 4 * lane) =
                        make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
                }
            }
            // the A buffer is private to this wave: its own LDS writes must
            // land before its lanes read each other's rows
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int kb = 0; kb < 8; kb++) {
                f16x8 ah, al;
                if (MP <= 8) {
                    ah = *(const f16x8*)(abuf + (hl8 * MP + mrow8) * kRowH + 32 * kb + 8 * g4);
                } else {
                    ah = *(const f16x8*)(abuf + (0 * MP + mrow) * kRowH + 32 * kb + 8 * g4);
                    al = *(const f16x8*)(abuf + (1 * MP + mrow) * kRowH + 32 * kb + 8 * g4);
                }
#pragma unroll
                for (int j = 0; j < T; j++) {
                    // T is even for a pair: tile j takes group j & 1
                    if (NG == 2 && (j & 1) != q) continue;
                    const u32x4 wv = wcur[j][kb >> 2];
                    const uint32_t word = (kb & 3) == 0 ? wv.x : (kb & 3) == 1 ? wv.y
                                        : (kb & 3) == 2 ? wv.z : wv.w;
                    f16x8 b = nib_to_f16(word, nk);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, acc[j], 0, 0, 0);
                    if (MP > 8) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, acc[j], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < T; j++) {
            tot[j][0] = fmaf(acc[j][0], down, tot[j][0]);
            tot[j][1] = fmaf(acc[j][1], down, tot[j][1]);
            tot[j][2] = fmaf(acc[j][2], down, tot[j][2]);
            tot[j][3] = fmaf(acc[j][3], down, tot[j][3]);
        }
        // the next round overwrites this wave's A buffer
        __builtin_amdgcn_wave_barrier();
    };
    if (MP <= 5 && my_rounds == 2) {
        // the usual case at K = 4096: both rounds' weights and activations
        // are issued at once, so the wave waits for memory once (up to 5
        // rows: with 8 the second round's activations cost the registers of
        // a second block per CU, measured slower)
        // (each round's activations before its weights: loads complete in
        // issue order, so the A-prep waits for the activations only)
        ARaw a0, a1;
        __builtin_amdgcn_sched_barrier(0);
        load_a(wave, a0);
        load_w(wave, wcur);
        __builtin_amdgcn_sched_barrier(0);
        load_a(wave + W, a1);
        load_w(wave + W, wnxt);
        __builtin_amdgcn_sched_barrier(0);
        round_body(a0, wcur);
        __builtin_amdgcn_sched_barrier(0);
        round_body(a1, wnxt);
    } else {
        ARaw acur;
        // activations before weights: the A-prep waits for them, and loads
        // complete in issue order, so the weights stay in flight meanwhile
        if (my_rounds > 0) {
            load_a(wave, acur);
            load_w(wave, wcur);
        }
        for (int i = 0; i < my_rounds; i++) {
            const int r = wave + i * W;
            if (i > 0) load_a(r, acur);
            if (i + 1 < my_rounds) load_w(r + W, wnxt);
            round_body(acur, wcur);
            if (i + 1 < my_rounds) {
#pragma unroll
                for (int j = 0; j < T; j++) {
                    wcur[j][0] = wnxt[j][0];
                    wcur[j][1] = wnxt[j][1];
                }
            }
        }
    }

    if (PRO == kProRmsNorm) {
#pragma unroll
        for (int m = 0; m < MP; m++) {
            float v = wave_sum(ssq[m]);
            if (lane == 0) s_ssq[wave][m] = v;
        }
    }
    __syncthreads();                 // every wave is done with its A buffer
    // partials: red[wave][tile][row][col]; lane holds rows 4*g4 .. +3, col lane%16
    float* red = lds;
    if (MP <= 8) {
        // row r's hi sum (D row r, lane group g4 < 2) plus its lo sum (D row
        // r + 8, the lane 32 above)
#pragma unroll
        for (int j = 0; j < T; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) tot[j][v] += __shfl_down(tot[j][v], 32);
    }
#pragma unroll
    for (int j = 0; j < T; j++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            int row = 4 * g4 + v;
            if (row < MP) red[((wave * T + j) * MP + row) * 16 + (lane & 15)] = tot[j][v];
        }
    __syncthreads();
    constexpr int kOuts = T * MP * 16;
    for (int o = threadIdx.x; o < kOuts; o += 64 * W) {
        const int j = o / (MP * 16), row = (o / 16) % MP, col = o % 16;
        if (row >= M) continue;
        if (EPI == kEpiSwiGlu && (j & 1)) continue;     // the gate thread does the pair
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) v += red[((w * T + j) * MP + row) * 16 + col];
        float rs = 1.0f;
        if (PRO == kProRmsNorm) {
            float ss = 0.0f;
#pragma unroll
            for (int w = 0; w < W; w++) ss += s_ssq[w][row];
            rs = 1.0f / sqrtf(ss / (float)a.K + a.eps);
            v *= rs;
        }
        const int lt = logical_tile(L0 + j, paired, ff_tiles);
        if (EPI == kEpiSwiGlu) {
            float u = 0.0f;
#pragma unroll
            for (int w = 0; w < W; w++) u += red[((w * T + j + 1) * MP + row) * 16 + col];
            u *= rs;
            float act = v / (1.0f + __expf(-v)) * u;
            a.y[(size_t)row * a.ldy + lt * 16 + col] = act;
        } else {
            float* yp = a.y + (size_t)row * a.ldy + lt * 16 + col;
            *yp = EPI == kEpiAccumulate ? *yp + v : v;
        }
    }
}

// ------------------------------------------------------------ streaming GEMV
//
// Very wide outputs at K = 4096 (an lm_head over a 128k vocabulary) with up to
// 5 rows: a persistent grid, one 8-wave block per CU.  Wave w owns the
// 256-row slices w and w + 8 of K for the whole launch.  A block walks a
// contiguous run of column units (two layout tiles, 32 columns) and keeps the
// A operands of the current scale group in registers, in MFMA layout; they
// are rebuilt only when a unit enters a new group (every gs / 32 units), so
// the rows are prepared once per group rather than once per 32 columns.  The
// next unit's scales and weights are in flight while a unit is multiplied;
// the wave partials of a unit are summed in a fixed order behind one barrier
// (double-buffered), so results do not depend on timing.
//
// Measured against the block-per-tile kernel (7B rows, weights rotated over
// the MALL): 4096 x 128256 at 5 rows 61.5 -> 53.1 us, at 1 row 47.9 -> 46.3
// us.  Runs of about 3 units per block (4096 x 22016) lose to it (17.0 vs
// 20.7 us): a unit's decode, MFMAs and reduction on 2 waves per SIMD take
// about as long as its 64 KiB take to arrive, and the first unit waits for
// the rows' preparation.
constexpr int kStreamWaves = 8;
constexpr int kStreamT = 2;                           // layout tiles per unit
constexpr int kStreamK = 2 * kStreamWaves * kRoundK;  // 4096
constexpr int kXRow = kRoundK + 4;                    // padded fp32 row of a slice
constexpr int kStreamIdle = 1 << 30;                  // byte offset past any matrix taken

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int MP, int PRO, int EPI>
__global__ __launch_bounds__(64 * kStreamWaves, 1) void k_gemv_stream(MfmaArgs a, int nunits) {
    constexpr int W = kStreamWaves, T = kStreamT;
    constexpr int RW = 2;                        // slices per wave
    constexpr int R = W * RW;                    // 256-row slices of K
    static_assert(MP <= 5, "x slices of up to 5 rows in LDS");
    static_assert(EPI != kEpiSwiGlu, "one scale group per unit");
    __shared__ float s_x[R][MP][kXRow];          // x (times the RMSNorm weight), by slice
    __shared__ _Float16 s_ab[W][2 * MP * kRowH]; // A staging of one slice per wave
    __shared__ float s_red[2][W][T][MP][16];     // wave partials of a unit, double-buffered
    __shared__ float s_ssq[W][MP];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const NibConst nk = nib_consts();
    const int M = a.M;
    constexpr int nchunks = kStreamK / kChunkK;
    // XCD-aware: the blocks of one XCD take neighbouring runs of units, which
    // share scale rows (block b runs on XCD b % 8)
    const int nblk = gridDim.x;
    const int per_xcd = nblk / 8;
    const int sb = (int)blockIdx.x < per_xcd * 8
                       ? (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8)
                       : (int)blockIdx.x;
    const int u0 = (int)((long long)sb * nunits / nblk);
    const int u1 = (int)((long long)(sb + 1) * nunits / nblk);
    const int g4 = lane >> 4;
    const int hl8 = (lane >> 3) & 1;
    const int mrow8 = (lane & 7) < M ? (lane & 7) : M - 1;
    _Float16* abuf = s_ab[wave];

    auto group_of = [&](int u) __attribute__((always_inline)) { return u * T * 16 / a.gs; };
    // whether unit u (inside the run, after its first unit) enters a new group
    auto enters = [&](int u) __attribute__((always_inline)) {
        return u > u0 && u < u1 && group_of(u) != group_of(u - 1);
    };
    // the lane's 4 scales in each of the wave's slices, for the group of unit u
    typedef float4 SRow[RW];
    auto load_s = [&](int u, SRow& dst) __attribute__((always_inline)) {
        const float* row = a.scales_t + (size_t)group_of(u) * kStreamK;
#pragma unroll
        for (int i = 0; i < RW; i++)
            dst[i] = *(const float4*)(row + (wave + i * W) * kRoundK + 4 * lane);
    };
    // weights through a buffer resource: an idle unit (past the end of the
    // run) reads out of range, which returns zeros without touching memory,
    // so every unit issues the same loads and the compiler's waits count
    // them exactly (conditional loads made it wait for all of them)
    typedef u32x4 WBuf[RW][T][2];
    WBuf wa, wb;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.w, (short)0, (int)((size_t)a.N / 16 * nchunks * kChunkBytes), kBufWord3);
    auto load_w = [&](int u, WBuf& dst) __attribute__((always_inline)) {
        const int base = u < u1 ? u * T * nchunks * kChunkBytes : kStreamIdle;
#pragma unroll
        for (int i = 0; i < RW; i++)
#pragma unroll
            for (int j = 0; j < T; j++)
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const int vo = (j * nchunks + 2 * (wave + i * W) + c) * kChunkBytes + 16 * lane;
                    dst[i][j][c] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo + base, 0, 2));
                }
    };
    // a unit's loads: the scales of a group it enters (at most one pending:
    // a group spans at least two units), then its weights
    SRow sp;
    auto issue = [&](int u, WBuf& dst) __attribute__((always_inline)) {
        if (enters(u)) load_s(u, sp);
        load_w(u, dst);
    };

    // ---- prologue: the wave's slices of x and the first group's scales,
    // then the first two units' loads (loads complete in issue order, so the
    // preparation waits for these only)
    const bool work = u0 < u1;
    float amax = 0.0f;
    float ssq[MP];
#pragma unroll
    for (int m = 0; m < MP; m++) ssq[m] = 0.0f;
    SRow s0;
    {
        float4 xv[RW][MP], nwv[RW];
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int r = wave + i * W;
#pragma unroll
            for (int m = 0; m < MP; m++)
                // rows past M read row M - 1 (zeroed where used): no
                // branches between the loads
                xv[i][m] = *(const float4*)(a.x + (size_t)(m < M ? m : M - 1) * a.ldx + r * kRoundK +
                                            4 * lane);
            nwv[i] = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            if (PRO == kProRmsNorm) nwv[i] = *(const float4*)(a.nw + r * kRoundK + 4 * lane);
        }
        if (work) load_s(u0, s0);
        // in unit order, as the loop issues them (its waits assume it)
        __builtin_amdgcn_sched_barrier(0);
        load_w(u0, wa);
        __builtin_amdgcn_sched_barrier(0);
        issue(u0 + 1, wb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int r = wave + i * W;
#pragma unroll
            for (int m = 0; m < MP; m++) {
                const float4 t = m < M ? xv[i][m] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (PRO == kProRmsNorm) {
                    ssq[m] = fmaf(t.x, t.x, ssq[m]);
                    ssq[m] = fmaf(t.y, t.y, ssq[m]);
                    ssq[m] = fmaf(t.z, t.z, ssq[m]);
                    ssq[m] = fmaf(t.w, t.w, ssq[m]);
                }
                // the RMSNorm weight multiplies x once here (1 / rms is
                // applied to the sums at the end)
                const float4 n = nwv[i];
                const float4 v = make_float4(t.x * n.x, t.y * n.y, t.z * n.z, t.w * n.w);
                *(float4*)&s_x[r][m][4 * lane] = v;
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
        }
    }
    if (PRO == kProRmsNorm) {
#pragma unroll
        for (int m = 0; m < MP; m++) {
            const float v = wave_sum(ssq[m]);
            if (lane == 0) s_ssq[wave][m] = v;
        }
    }
    amax = wave_max_nonneg(amax);

    // ---- A operands from a group's scales: a[m][k] = x[m][k] s[k] 2^E as
    // hi + lo fp16 (hi rounded toward zero, lo the rounded remainder), each
    // lane converting its 4 columns of every row into the wave's staging
    // rows, read back in MFMA layout (A rows 0-7 the hi parts of rows 0-7,
    // rows 8-15 the lo parts).  2^E makes |a| < 2^15 over the wave's slices.
    f16x8 A[RW][8];
    float down;
    auto build = [&](const SRow& sr) __attribute__((always_inline)) {
        float smax = 0.0f;
#pragma unroll
        for (int i = 0; i < RW; i++)
            smax = fmaxf(smax, fmaxf(fmaxf(fabsf(sr[i].x), fabsf(sr[i].y)),
                                     fmaxf(fabsf(sr[i].z), fabsf(sr[i].w))));
        const float bound = amax * wave_max_nonneg(smax);
        int E = 0;
        if (bound > 0.0f && bound < __builtin_inff()) E = 14 - ilogbf(bound);
        E = E > 100 ? 100 : (E < -100 ? -100 : E);
        const float up = ldexpf(1.0f, E);
        down = ldexpf(1.0f, -E);
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int r = wave + i * W;
            const float s0 = sr[i].x * up, s1 = sr[i].y * up, s2 = sr[i].z * up, s3 = sr[i].w * up;
#pragma unroll
            for (int m = 0; m < MP; m++) {
                if (m < M) {
                    const float4 xv = *(const float4*)&s_x[r][m][4 * lane];
                    const float v0 = xv.x * s0, v1 = xv.y * s1, v2 = xv.z * s2, v3 = xv.w * s3;
                    const f16x2 h01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(v0, v1));
                    const f16x2 h23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(v2, v3));
                    const f16x2 l01 = __builtin_bit_cast(
                        f16x2, __builtin_amdgcn_cvt_pkrtz(v0 - (float)h01[0], v1 - (float)h01[1]));
                    const f16x2 l23 = __builtin_bit_cast(
                        f16x2, __builtin_amdgcn_cvt_pkrtz(v2 - (float)h23[0], v3 - (float)h23[1]));
                    *(uint2*)(abuf + (0 * MP + m) * kRowH + 4 * lane) =
                        make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
                    *(uint2*)(abuf + (1 * MP + m) * kRowH + 4 * lane) =
                        make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
                }
            }
            wave_lds_sync();
#pragma unroll
            for (int kb = 0; kb < 8; kb++)
                A[i][kb] = *(const f16x8*)(abuf + (hl8 * MP + mrow8) * kRowH + 32 * kb + 8 * g4);
            // the staging rows are read before the next slice overwrites them
            wave_lds_sync();
        }
    };
    wave_lds_sync();                 // s_x
    if (work) build(s0);
    __syncthreads();                 // s_ssq

    // the output this thread finishes for each unit, spread over the waves
    // so that no wave carries the whole epilogue; and its 1 / rms
    constexpr int kOuts = T * MP * 16;
    static_assert(kOuts <= 64 * W, "one output per thread");
    const int oe = lane * W + wave;
    const int oj = oe / (MP * 16), orow = (oe / 16) % MP, ocol = oe % 16;
    const bool outer = oe < kOuts && orow < M;
    float rs = 1.0f;
    if (PRO == kProRmsNorm && outer) {
        float ss = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) ss += s_ssq[w][orow];
        rs = 1.0f / sqrtf(ss / (float)kStreamK + a.eps);
    }

    auto unit = [&](int u, WBuf& w, int buf) __attribute__((always_inline)) {
        // idle units (past the run) only keep the loads in step
        const bool live = u < u1;
        if (enters(u)) build(sp);
        f32x4 acc[T];
#pragma unroll
        for (int j = 0; j < T; j++) acc[j] = (f32x4)(0.0f);
        if (live) {
#pragma unroll
            for (int i = 0; i < RW; i++)
#pragma unroll
                for (int kb = 0; kb < 8; kb++) {
#pragma unroll
                    for (int j = 0; j < T; j++) {
                        const u32x4 wv = w[i][j][kb >> 2];
                        const uint32_t word = (kb & 3) == 0 ? wv.x : (kb & 3) == 1 ? wv.y
                                            : (kb & 3) == 2 ? wv.z : wv.w;
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i][kb], nib_to_f16(word, nk),
                                                                        acc[j], 0, 0, 0);
                    }
                    // decode k block by k block (all at once would hold 16
                    // registers per tile and block)
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
        // the loads of unit u + 2 into the registers just consumed
        issue(u + 2, w);
        if (!live) return;
        // hi + lo halves (D rows r and r + 8, 32 lanes apart: lanes 0-31
        // take lane l + 32's value through v_permlane32_swap), then 2^-E
#pragma unroll
        for (int j = 0; j < T; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const auto sw = __builtin_amdgcn_permlane32_swap(
                    __float_as_uint(acc[j][v]), __float_as_uint(acc[j][v]), false, false);
                const float t = acc[j][v] + __uint_as_float(sw[1]);
                const int row = 4 * g4 + v;
                if (g4 < 2 && row < MP) s_red[buf][wave][j][row][lane & 15] = t * down;
            }
        __syncthreads();
        if (outer) {
            float v = 0.0f;
#pragma unroll
            for (int wv = 0; wv < W; wv++) v += s_red[buf][wv][oj][orow][ocol];
            v *= rs;
            float* yp = a.y + (size_t)orow * a.ldy + (u * T + oj) * 16 + ocol;
            *yp = EPI == kEpiAccumulate ? *yp + v : v;
        }
    };
    // whole pairs of units, the last padded with an idle unit: a unit
    // skipped inside the loop would make the compiler assume the next
    // unit's loads were the last ones issued and wait for all of them
    for (int u = u0; u < u1; u += 2) {
        unit(u, wa, 0);
        unit(u + 1, wb, 1);
    }
}

// Repack cogito's row-major nibbles (two's complement, flat) into layout 3.
// One thread per output u32 word.
__global__ void k_repack_mfma(const uint8_t* __restrict__ flat, int K, int N, int paired,
                              uint32_t* __restrict__ out) {
    size_t wi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t words = (size_t)K * N / 8;
    if (wi >= words) return;
    // word wi: layout tile L, chunk c, lane l, word j
    const int nchunks = K / kChunkK;
    size_t t = wi;
    const int j = (int)(t % 4); t /= 4;
    const int l = (int)(t % 64); t /= 64;
    const int c = (int)(t % nchunks); t /= nchunks;
    const int L = (int)t;
    const int lt = logical_tile(L, paired, N / 32);
    const int col = lt * 16 + (l & 15);
    const int kbase = 32 * (4 * c + j) + 8 * (l >> 4);
    uint32_t word = 0;
#pragma unroll
    for (int p = 0; p < 8; p++) {
        size_t idx = (size_t)(kbase + p) * N + col;
        unsigned byte = flat[idx >> 1];
        unsigned nib = (idx & 1) ? (byte >> 4) : (byte & 0xF);
        nib ^= 0x8u;                          // two's complement -> offset binary
        word |= nib << (4 * ((p >> 1) + 4 * (p & 1)));    // slot {0,4,1,5,2,6,3,7}[p]
    }
    out[wi] = word;
}

// Layout 3 -> fp32 W[K,N] (row-major), for cg_dequantize of a device weight.
__global__ void k_dequant_mfma(const uint32_t* __restrict__ w, const float* __restrict__ scales_t,
                               int K, int N, int gs, int paired, float* __restrict__ out) {
    size_t wi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t words = (size_t)K * N / 8;
    if (wi >= words) return;
    const int nchunks = K / kChunkK;
    size_t t = wi;
    const int j = (int)(t % 4); t /= 4;
    const int l = (int)(t % 64); t /= 64;
    const int c = (int)(t % nchunks); t /= nchunks;
    const int L = (int)t;
    const int lt = logical_tile(L, paired, N / 32);
    const int col = lt * 16 + (l & 15);
    const int kbase = 32 * (4 * c + j) + 8 * (l >> 4);
    const uint32_t word = w[wi];
#pragma unroll
    for (int p = 0; p < 8; p++) {
        int k = kbase + p;
        unsigned nib = (word >> (4 * ((p >> 1) + 4 * (p & 1)))) & 0xFu;
        float s = scales_t[(size_t)(col / gs) * K + k];
        out[(size_t)k * N + col] = (float)((int)nib - 8) * s;
    }
}

// Layout 3 -> cogito's row-major nibbles (two's complement, flat): the
// inverse of k_repack_mfma.  One thread per flat byte (two columns of one
// row, which sit in neighbouring lanes of the same layout word index).
__global__ void k_unpack_mfma(const uint32_t* __restrict__ w, int K, int N, int paired,
                              uint8_t* __restrict__ flat) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= (size_t)K * N / 2) return;
    const int nchunks = K / kChunkK, ff_tiles = N / 32;
    unsigned out = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const size_t idx = 2 * b + h;
        const int k = (int)(idx / N), col = (int)(idx % N);
        const int lt = col >> 4;
        const int L = paired ? (lt < ff_tiles ? 2 * lt : 2 * (lt - ff_tiles) + 1) : lt;
        const int c = k / kChunkK, kk = k % kChunkK;
        const int j = kk >> 5, l = ((kk & 31) >> 3) * 16 + (col & 15), p = kk & 7;
        const uint32_t word = w[(((size_t)L * nchunks + c) * 64 + l) * 4 + j];
        const unsigned nib = (word >> (4 * ((p >> 1) + 4 * (p & 1)))) & 0xFu;
        out |= (nib ^ 0x8u) << (4 * h);                 // offset binary -> two's complement
    }
    flat[b] = (uint8_t)out;
}

template <int MP, int T, int NG, int PRO, int EPI, int W = kWaves>
int launch_t(const MfmaArgs& a, int nblocks) {
    hipLaunchKernelGGL((k_gemv_mfma<MP, T, NG, PRO, EPI, W>), dim3(nblocks), dim3(64 * W), 0,
                       stream(), a);
    return launch_check("k_gemv_mfma");
}

// CUs of the current device: the streaming GEMV's grid.
int stream_blocks() {
    static int cus = 0;
    if (cus <= 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
            cus = n;
        if (cus <= 0) cus = 256;
    }
    return cus;
}

// Units on the busiest CU from which the streaming GEMV takes a product
// (0: never).
int g_stream_min_units = 8;

template <int MP, int PRO, int EPI>
int launch_stream(const MfmaArgs& a) {
    const int nunits = a.N / (16 * kStreamT);
    const int nb = stream_blocks() < nunits ? stream_blocks() : nunits;
    hipLaunchKernelGGL((k_gemv_stream<MP, PRO, EPI>), dim3(nb), dim3(64 * kStreamWaves), 0,
                       stream(), a, nunits);
    return launch_check("k_gemv_stream");
}

// Whether the streaming GEMV takes y = x @ W: K = 4096, up to 5 rows, one
// scale group per unit and at least two units per group, the matrix within
// the idle offset, and enough units on the busiest CU (ceil(units / CUs) >=
// the setting) to outweigh its preparation.
bool stream_takes(const MfmaArgs& a, int epi) {
    if (g_stream_min_units <= 0 || epi == kEpiSwiGlu || a.K != kStreamK || a.M > 5 ||
        a.gs % (32 * kStreamT) || (size_t)a.K * a.N / 2 >= (size_t)kStreamIdle ||
        a.N % (16 * kStreamT))
        return false;
    return a.N / (16 * kStreamT) > (g_stream_min_units - 1) * stream_blocks();
}

template <int PRO, int EPI>
int launch_stream_pe(const MfmaArgs& a) {
    if (a.M == 1) return launch_stream<1, PRO, EPI>(a);
    if (a.M == 2) return launch_stream<2, PRO, EPI>(a);
    if (a.M <= 4) return launch_stream<4, PRO, EPI>(a);
    return launch_stream<5, PRO, EPI>(a);
}

template <int MP, int PRO, int EPI>
int launch_mp(const MfmaArgs& a, int T) {
    const int tiles = a.N / 16;
    if constexpr (EPI == kEpiSwiGlu) {
        if (T == 4) return launch_t<MP, 4, 2, PRO, EPI>(a, tiles / 4);
        return launch_t<MP, 2, 2, PRO, EPI>(a, tiles / 2);
    } else {
        if constexpr (MP <= 8 && PRO == kProNone) {
            // 16 waves per block when a wave of 8 would have more than two
            // 256-row rounds (a shorter chain of memory waits), or two with
            // at most one block per CU (more waves in flight; with more
            // blocks the larger blocks lose to the tail).  The A buffers of
            // 16 waves fit LDS up to 8 rows; with the RMSNorm prologue 128
            // registers would spill.
            const int rounds = a.K / kRoundK;
            if (rounds > 2 * kWaves || (rounds > kWaves && tiles / T <= 256)) {
                if (T == 2) return launch_t<MP, 2, 1, PRO, EPI, 2 * kWaves>(a, tiles / 2);
                if (T == 1) return launch_t<MP, 1, 1, PRO, EPI, 2 * kWaves>(a, tiles);
            }
        }
        if (T == 4) return launch_t<MP, 4, 1, PRO, EPI>(a, tiles / 4);
        if (T == 2) return launch_t<MP, 2, 1, PRO, EPI>(a, tiles / 2);
        return launch_t<MP, 1, 1, PRO, EPI>(a, tiles);
    }
}

template <int PRO, int EPI>
int launch_pe(const MfmaArgs& a, int T) {
    if (a.M == 1) return launch_mp<1, PRO, EPI>(a, T);
    if (a.M == 2) return launch_mp<2, PRO, EPI>(a, T);
    if (a.M <= 4) return launch_mp<4, PRO, EPI>(a, T);
    // 5 rows (a chain of 4 drafts and the bonus position) keep 3 fewer rows
    // of activations in registers than 8
    if (a.M == 5) return launch_mp<5, PRO, EPI>(a, T);
    if constexpr (EPI == kEpiSwiGlu) {
        return launch_mp<8, PRO, EPI>(a, T);
    } else {
        if (a.M <= 8) return launch_mp<8, PRO, EPI>(a, T);
        return launch_mp<16, PRO, EPI>(a, T);
    }
}

// ------------------------------------------------------------------ GEMM
// y = x @ W for M >= 16 rows (batched verify, tree verify).  A block of 4
// waves covers two 128-column slots (two neighbouring scale groups, or the
// gate and up halves of the same 128 SwiGLU columns), each wave 4 column
// tiles of one slot, so one A fragment read from LDS feeds 4 tiles.  Per
// slot the activations are prepared once per 128-row step: x * nw * s (the
// scale of that slot's group at each k) times a per-row factor rstd * 2^E,
// split into hi + lo fp16 (22 significant bits); the MFMA sums are scaled by
// 2^-E at the end.  k_gemm_rows fixes the row factors before the GEMM from
// the whole row: max|x * nw| * rstd * max|s| * 2^E < 2^15.  The next step's
// activations and the weights two steps ahead are loaded while a step is
// multiplied.  K is split over blockIdx.z; k_gemm_reduce sums the splits in
// a fixed order and applies the epilogue (store, accumulate, SwiGLU of the
// gate|up pair).

constexpr int kGemmWaves = 4;
constexpr int kGemmTiles = 4;            // column tiles per wave
constexpr int kGemmRowH = kChunkK + 8;   // LDS pitch (halfs) of an A row

struct GemmArgs {
    const float* x;           // [M][ldx]
    int ldx, M, K, N, gs;
    const uint8_t* w;         // layout 3
    const float* scales_t;    // [N/gs][K]
    const float* nw;          // RMSNorm weights [K] or nullptr
    const float* rowscale;    // [M] rstd * 2^E (k_gemm_rows), or
    const float* unscale;     // [M] 2^-E       ... nullptr with stats:
    const float* stats;       // [M][nstat][2] partial (max|x*nw|, sum x^2) of x
    int nstat;                //   per 128 columns, written by the producer's epilogue
    float smax, eps;          // the row factors' scale bound and RMSNorm epsilon
    float* part;              // [ksplit][M][N] partial sums, logical columns (y itself
                              // for one split storing rows of N floats)
    int ksteps;               // 128-row chunks per split
    int ff;                   // SwiGLU pair: N / 2
    // one split of a gate|up pair: SwiGLU in the epilogue, straight into y
    float* y;                 // [M][ldy] (nullptr: partial sums into part)
    int ldy;
    float* stats_out;         // [M][ff / 128][2] of y, or nullptr
    const float* nw_next;     // the next linear's RMSNorm weights, or nullptr
};

template <int RT, int NG, int PRO>
__global__ __launch_bounds__(64 * kGemmWaves, 2) void k_gemm_int4(GemmArgs a) {
    constexpr int BM = 16 * RT;
    constexpr int RPT = BM / 8;                 // rows prepared per thread
    __shared__ _Float16 sa[2][2][BM][kGemmRowH];
    __shared__ float s_unscale[BM];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const NibConst nk = nib_consts();
    const int paired = NG == 2;
    const int nchunks = a.K / kChunkK;
    // XCD-aware order (block b runs on XCD b % 8): with several row blocks,
    // each XCD takes a contiguous run of (column block, row block) pairs, row
    // blocks fastest, so the row blocks of one column block run together on
    // one XCD and share its L2 copy of the weights (tree verify, 256 rows:
    // 14.25 -> 13.70 ms a step; with one row block the plain order measured
    // faster).  The tail past a multiple of 8 keeps the plain order.
    int bx = blockIdx.x, by = blockIdx.y;
    if (gridDim.y > 1) {
        const int gy = gridDim.y, lin = blockIdx.y * gridDim.x + blockIdx.x;
        const int per = gridDim.x * gy / 8;
        const int q = lin < 8 * per ? (lin % 8) * per + lin / 8 : lin;
        bx = q / gy;
        by = q % gy;
    }
    // slots: logical 128-column groups and their scale-group rows
    int slot_ok[2], grp[2], lcol[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        if (paired) {
            lcol[s] = (s ? a.ff : 0) + 128 * bx;
            slot_ok[s] = 1;
        } else {
            lcol[s] = 128 * (2 * bx + s);
            slot_ok[s] = lcol[s] < a.N;
        }
        grp[s] = slot_ok[s] ? lcol[s] / a.gs : 0;
    }
    const int row0 = by * BM;
    const int c0 = blockIdx.z * a.ksteps;
    const int c1 = min(nchunks, c0 + a.ksteps);
    // preparation: thread -> 4 k values at pk, rows pr + 8 i (a row's 32
    // threads are one half wave)
    const int pk = 4 * (threadIdx.x & 31), pr = threadIdx.x >> 5;
    int xrow[RPT];
    uint32_t rowmask[RPT];
    float rsc[RPT];
    if (a.stats) {
        // row factors from the producer's partial statistics (fixed order):
        // the same rule as k_gemm_rows
        // four lanes per row, each over every fourth partial (loads issued
        // together), combined by shuffles in a fixed order
        __shared__ float s_rsc[BM];
        static_assert(4 * BM <= 64 * kGemmWaves, "four threads per row");
        float A = 0.0f, S = 0.0f;
        const int sr = threadIdx.x >> 2, sq = threadIdx.x & 3;
        if (sr < BM) {
            const int row = min(row0 + sr, a.M - 1);
            const float2* st = (const float2*)(a.stats + (size_t)row * a.nstat * 2);
#pragma unroll 4
            for (int j = sq; j < a.nstat; j += 4) {
                const float2 v = st[j];
                A = fmaxf(A, v.x);
                S += v.y;
            }
        }
        A = fmaxf(A, __shfl_xor(A, 1));
        S += __shfl_xor(S, 1);
        A = fmaxf(A, __shfl_xor(A, 2));
        S += __shfl_xor(S, 2);
        if (sr < BM && sq == 0) {
            const float rstd = PRO == kProRmsNorm ? 1.0f / sqrtf(S / (float)a.K + a.eps) : 1.0f;
            const float bound = A * rstd * a.smax;
            int E = 0;
            if (bound > 0.0f && bound < __builtin_inff()) E = 14 - ilogbf(bound);
            E = E > 100 ? 100 : (E < -100 ? -100 : E);
            s_rsc[sr] = rstd * ldexpf(1.0f, E);
            s_unscale[sr] = ldexpf(1.0f, -E);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            xrow[i] = min(row0 + pr + 8 * i, a.M - 1);
            rowmask[i] = row0 + pr + 8 * i < a.M ? ~0u : 0u;
            rsc[i] = s_rsc[pr + 8 * i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            xrow[i] = min(row0 + pr + 8 * i, a.M - 1);
            rowmask[i] = row0 + pr + 8 * i < a.M ? ~0u : 0u;
            rsc[i] = a.rowscale[xrow[i]];
        }
        if (threadIdx.x < BM)
            s_unscale[threadIdx.x] = a.unscale[min(row0 + (int)threadIdx.x, a.M - 1)];
    }

    // ---- this wave's tiles: slot ws, tiles 4 (wave & 1) + j of the slot.  A
    // wave of a missing slot (odd number of 128-column slots) runs on tile 0
    // and stores nothing, so that every wave takes the same path.
    const int ws = wave >> 1;
    const int wave_ok = slot_ok[ws];
    // loads through buffer resources: a lane's 32-bit offset is fixed, the
    // step's advance is a uniform SGPR offset, so a step's loads take no
    // address arithmetic (the resources bound every access to its array)
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.w, (short)0, (int)((size_t)a.N / 16 * nchunks * kChunkBytes), kBufWord3);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.x, (short)0, (int)((size_t)a.M * a.ldx * 4), kBufWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.scales_t, (short)0, (int)((size_t)(a.N / a.gs) * a.K * 4), kBufWord3);
    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(PRO == kProRmsNorm ? a.nw : a.scales_t), (short)0, a.K * 4, kBufWord3);
    int wo[kGemmTiles];
#pragma unroll
    for (int j = 0; j < kGemmTiles; j++) {
        const int t = 4 * (wave & 1) + j;               // tile within the slot
        const int L = paired ? 2 * (8 * bx + t) + ws : 8 * (2 * bx + ws) + t;
        wo[j] = (wave_ok ? L : 0) * nchunks * kChunkBytes + 16 * lane;
    }
    // steps run in pairs; a step at or past c1 (odd count) prepares zeros and
    // reads the split's last chunk again
    const int cend = c0 + ((c1 - c0 + 1) & ~1);
    auto wload = [&](int c, u32x4 (&d)[kGemmTiles]) {
        const int off = min(c, c1 - 1) * kChunkBytes;
#pragma unroll
        for (int j = 0; j < kGemmTiles; j++)
            d[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo[j], off, 2));
    };
    u32x4 wb0[kGemmTiles], wb1[kGemmTiles];
    __builtin_amdgcn_sched_barrier(0);
    wload(c0, wb0);

    f32x4 acc[kGemmTiles][RT];
#pragma unroll
    for (int j = 0; j < kGemmTiles; j++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) acc[j][rt] = (f32x4)(0.0f);

    // prefetched preparation inputs
    float4 px[RPT], ps[2], pn = make_float4(1.f, 1.f, 1.f, 1.f);
    uint32_t plive;
    int xo[RPT], so[2];
#pragma unroll
    for (int i = 0; i < RPT; i++) xo[i] = (xrow[i] * a.ldx + pk) * 4;
#pragma unroll
    for (int s_ = 0; s_ < 2; s_++) so[s_] = (grp[s_] * a.K + pk) * 4;
    auto ld4 = [](const __amdgpu_buffer_rsrc_t& r, int vo, int so_) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so_, 0));
    };
    auto load_prep = [&](int c) {
        const int cc = min(c, c1 - 1);
        const int kb = cc * kChunkK * 4;
        if (PRO == kProRmsNorm) pn = ld4(rn, pk * 4, kb);
#pragma unroll
        for (int s_ = 0; s_ < 2; s_++) ps[s_] = ld4(rs, so[s_], kb);
#pragma unroll
        for (int i = 0; i < RPT; i++) px[i] = ld4(rx, xo[i], kb);
        plive = c < c1 ? ~0u : 0u;
    };
    // the same load order as at the end of a step pair, so that the loop
    // entry needs no stricter wait than the back edge
    __builtin_amdgcn_sched_barrier(0);
    load_prep(c0);
    __builtin_amdgcn_sched_barrier(0);
    wload(c0 + 1, wb1);
    __builtin_amdgcn_sched_barrier(0);

    // sched_barrier(0) keeps the phases in this order, so that the waits
    // for the loads of the next step fall where they are consumed
    auto step = [&](int c, u32x4 (&wcur)[kGemmTiles]) {
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();                       // the previous step's A reads are done
        const float4 n4 = pn;
        // x times the row factor, once per step for both slots; rows past M
        // and steps past c1 take the factor 0.  Their loads are clamped to
        // live data (a row past M reads row M - 1, a step past c1 the
        // split's last chunk), so a product is non-finite only where the
        // same values already enter a live row's sum, and a row past M
        // feeds only its own, unstored, outputs.
        float4 xv[RPT];
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const float r = (plive & rowmask[i]) ? rsc[i] : 0.0f;
            xv[i].x = px[i].x * r;
            xv[i].y = px[i].y * r;
            xv[i].z = px[i].z * r;
            xv[i].w = px[i].w * r;
        }
        // a missing slot (odd slot count) prepares from valid memory and is
        // never stored
#pragma unroll
        for (int s_ = 0; s_ < 2; s_++) {
            const float n0 = n4.x * ps[s_].x, n1 = n4.y * ps[s_].y;
            const float n2 = n4.z * ps[s_].z, n3 = n4.w * ps[s_].w;
#pragma unroll
            for (int i = 0; i < RPT; i++) {
                const float v0 = xv[i].x * n0, v1 = xv[i].y * n1;
                const float v2 = xv[i].z * n2, v3 = xv[i].w * n3;
                const f16x2 h01 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(v0, v1));
                const f16x2 h23 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(v2, v3));
                // hi: v rounded toward zero; lo: the exact remainder rounded
                // to fp16 (one v_fma_mixlo / v_fma_mixhi each: 600 -> 504
                // VALU instructions per step pair, with x times the row
                // factor once per step)
                f16x2 l01, l23;
                l01[0] = (_Float16)(v0 - (float)h01[0]);
                l01[1] = (_Float16)(v1 - (float)h01[1]);
                l23[0] = (_Float16)(v2 - (float)h23[0]);
                l23[1] = (_Float16)(v3 - (float)h23[1]);
                const int r_ = pr + 8 * i;
                *(uint2*)&sa[s_][0][r_][pk] = make_uint2(__builtin_bit_cast(uint32_t, h01),
                                                         __builtin_bit_cast(uint32_t, h23));
                *(uint2*)&sa[s_][1][r_][pk] = make_uint2(__builtin_bit_cast(uint32_t, l01),
                                                         __builtin_bit_cast(uint32_t, l23));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        load_prep(c + 1);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            f16x8 b[kGemmTiles];
#pragma unroll
            for (int j = 0; j < kGemmTiles; j++) {
                const uint32_t word = kb == 0 ? wcur[j].x : kb == 1 ? wcur[j].y
                                    : kb == 2 ? wcur[j].z : wcur[j].w;
                b[j] = nib_to_f16(word, nk);
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const int ar = rt * 16 + (lane & 15), ak = 32 * kb + 8 * (lane >> 4);
                const f16x8 ah = *(const f16x8*)&sa[ws][0][ar][ak];
                const f16x8 al = *(const f16x8*)&sa[ws][1][ar][ak];
#pragma unroll
                for (int j = 0; j < kGemmTiles; j++) {
                    acc[j][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b[j], acc[j][rt], 0, 0, 0);
                    acc[j][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b[j], acc[j][rt], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        wload(c + 2, wcur);
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int c = c0; c < cend; c += 2) {
        step(c, wb0);
        step(c + 1, wb1);
    }

    if (NG == 2 && a.y) {
        // one K split of a gate|up pair: the up waves (slot 1) hand their
        // sums to the gate waves through LDS (the A buffers are free once
        // every wave is past its last step), which apply SwiGLU with the
        // split reduction's arithmetic (0 + sum * 2^-E, then g / (1 +
        // exp(-g)) * u) and store y and the row statistics of its 128
        // columns
        float (*s_up)[128] = (float (*)[128])&sa[0][0][0][0];
        float (*s_st)[2] = (float (*)[2])&sa[0][0][0][0] + BM * 64;
        static_assert(BM * 128 * 4 + BM * 2 * 4 <= (int)sizeof(sa), "epilogue fits the A buffers");
        __syncthreads();
        if (ws == 1) {
#pragma unroll
            for (int j = 0; j < kGemmTiles; j++)
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int r_ = rt * 16 + 4 * (lane >> 4) + v;
                        s_up[r_][64 * (wave & 1) + 16 * j + (lane & 15)] =
                            0.0f + acc[j][rt][v] * s_unscale[r_];
                    }
        }
        __syncthreads();
        float am[RT][4], ss[RT][4];
        if (ws == 0) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    am[rt][v] = 0.0f;
                    ss[rt][v] = 0.0f;
                }
#pragma unroll
            for (int j = 0; j < kGemmTiles; j++) {
                const int c = 64 * (wave & 1) + 16 * j + (lane & 15);
                const int col = 128 * bx + c;
                const float nwc = a.nw_next ? a.nw_next[col] : 1.0f;
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int r_ = rt * 16 + 4 * (lane >> 4) + v;
                        const int row = row0 + r_;
                        const float g = 0.0f + acc[j][rt][v] * s_unscale[r_];
                        const float o = g / (1.0f + __expf(-g)) * s_up[r_][c];
                        if (row < a.M) a.y[(size_t)row * a.ldy + col] = o;
                        am[rt][v] = fmaxf(am[rt][v], fabsf(o * nwc));
                        ss[rt][v] = fmaf(o, o, ss[rt][v]);
                    }
            }
        }
        if (!a.stats_out) return;
        // per row: the 4 tiles in a lane, then the 16 lanes of its DPP row
        // (lane 15 of each row), then the two gate waves (wave 1 through LDS)
        if (ws == 0) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    am[rt][v] = row16_max_nonneg(am[rt][v]);
                    ss[rt][v] = row16_sum(ss[rt][v]);
                }
        }
        __syncthreads();                 // the gate waves' reads of s_up are done
        if (wave == 1 && (lane & 15) == 15) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r_ = rt * 16 + 4 * (lane >> 4) + v;
                    s_st[r_][0] = am[rt][v];
                    s_st[r_][1] = ss[rt][v];
                }
        }
        __syncthreads();
        if (wave == 0 && (lane & 15) == 15) {
            const int nst = a.ff / 128;
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r_ = rt * 16 + 4 * (lane >> 4) + v;
                    const int row = row0 + r_;
                    if (row < a.M) {
                        a.stats_out[((size_t)row * nst + bx) * 2] = fmaxf(am[rt][v], s_st[r_][0]);
                        a.stats_out[((size_t)row * nst + bx) * 2 + 1] = ss[rt][v] + s_st[r_][1];
                    }
                }
        }
        return;
    }
    if (!wave_ok) return;
    float* pp = a.part + (size_t)blockIdx.z * a.M * a.N;
#pragma unroll
    for (int j = 0; j < kGemmTiles; j++) {
        const int col = lcol[ws] + 16 * (4 * (wave & 1) + j) + (lane & 15);
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r_ = rt * 16 + 4 * (lane >> 4) + v;
                const int row = row0 + r_;
                if (row < a.M) pp[(size_t)row * a.N + col] = acc[j][rt][v] * s_unscale[r_];
            }
    }
}

// Row factors of the GEMM's activations: rstd (RMSNorm, else 1) times the
// power of two 2^E with max|x * nw| * rstd * smax * 2^E < 2^15, and 2^-E.
// One block per row; every thread's loads are issued together.
__global__ __launch_bounds__(256) void k_gemm_rows(const float* __restrict__ x, int ldx, int K,
                                                   const float* __restrict__ nw, int rms,
                                                   float eps, float smax,
                                                   float* __restrict__ rowscale,
                                                   float* __restrict__ unscale) {
    __shared__ float s_a[4], s_s[4];
    constexpr int U = 12;                   // float4 per thread in one batch (K <= 12288)
    const int m = blockIdx.x, t = threadIdx.x;
    const float* xr = x + (size_t)m * ldx;
    const int K4 = K / 4;
    float amax = 0.0f, ssq = 0.0f;
    for (int base = 0; base < K4; base += U * 256) {
        float4 v[U], w[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = min(base + t + 256 * u, K4 - 1);
            v[u] = *(const float4*)(xr + 4 * i);
            w[u] = nw ? *(const float4*)(nw + 4 * i) : make_float4(1.f, 1.f, 1.f, 1.f);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (base + t + 256 * u >= K4) continue;
            ssq = fmaf(v[u].x, v[u].x, fmaf(v[u].y, v[u].y, fmaf(v[u].z, v[u].z, fmaf(v[u].w, v[u].w, ssq))));
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[u].x * w[u].x), fabsf(v[u].y * w[u].y)),
                                     fmaxf(fabsf(v[u].z * w[u].z), fabsf(v[u].w * w[u].w))));
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o));
        ssq += __shfl_xor(ssq, o);
    }
    if ((t & 63) == 0) {
        s_a[t >> 6] = amax;
        s_s[t >> 6] = ssq;
    }
    __syncthreads();
    if (t == 0) {
        float A = 0.0f, S = 0.0f;
        for (int wv = 0; wv < 4; wv++) {
            A = fmaxf(A, s_a[wv]);
            S += s_s[wv];
        }
        const float rstd = rms ? 1.0f / sqrtf(S / (float)K + eps) : 1.0f;
        const float bound = A * rstd * smax;
        int E = 0;
        if (bound > 0.0f && bound < __builtin_inff()) E = 14 - ilogbf(bound);
        E = E > 100 ? 100 : (E < -100 ? -100 : E);
        rowscale[m] = rstd * ldexpf(1.0f, E);
        unscale[m] = ldexpf(1.0f, -E);
    }
}

// 0 + p[0] + p[mn] + ... + p[(n - 1) mn] left to right, eight splits' loads
// in flight together (one memory round trip per eight splits; past n the
// loads repeat split n - 1, which is in bounds, and add +0, which leaves the
// sum's bits alone: a sum that starts at +0 never becomes -0)
__device__ __forceinline__ float split_sum(const float* __restrict__ p, size_t mn, int n) {
    float v = 0.0f;
    for (int z0 = 0; z0 < n; z0 += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; j++) t[j] = p[(size_t)min(z0 + j, n - 1) * mn];
#pragma unroll
        for (int j = 0; j < 8; j++) v += z0 + j < n ? t[j] : 0.0f;
    }
    return v;
}

// The same for four neighbouring outputs (16-byte loads).
__device__ __forceinline__ void split_sum4(const float* __restrict__ p, size_t mn, int n,
                                           float (&v)[4]) {
    v[0] = v[1] = v[2] = v[3] = 0.0f;
    for (int z0 = 0; z0 < n; z0 += 8) {
        float4 t[8];
#pragma unroll
        for (int j = 0; j < 8; j++) t[j] = *(const float4*)(p + (size_t)min(z0 + j, n - 1) * mn);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const bool in = z0 + j < n;
            v[0] += in ? t[j].x : 0.0f;
            v[1] += in ? t[j].y : 0.0f;
            v[2] += in ? t[j].z : 0.0f;
            v[3] += in ? t[j].w : 0.0f;
        }
    }
}

// Sum of the K splits in order, and the epilogue.  With stats_out, also the
// (max|y * nw_next|, sum y^2) of every 128 stored outputs of a row (two
// waves; the output width is a multiple of 128): the next GEMM's row
// statistics without a pass over y.
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_reduce(const float* __restrict__ part, int ksplit,
                                                     int M, int N, float* __restrict__ y,
                                                     int ldy, float* __restrict__ stats_out,
                                                     const float* __restrict__ nw_next) {
    __shared__ float s_a[4], s_s[4];
    const int Nout = EPI == kEpiSwiGlu ? N / 2 : N;
    // 32-bit indices (M * Nout < 2^31, checked on the host): a 64-bit
    // division costs about a hundred instructions
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (!stats_out && i >= (unsigned)(M * Nout)) return;
    const bool live = i < (unsigned)(M * Nout);
    const int row = live ? (int)(i / (unsigned)Nout) : 0;
    const int col = live ? (int)(i - (unsigned)row * (unsigned)Nout) : 0;
    const size_t mn = (size_t)M * N;
    float out = 0.0f;
    if (live) {
        const float* p = part + (size_t)row * N + col;
        const float v = split_sum(p, mn, ksplit);
        float* yp = y + (size_t)row * ldy + col;
        if (EPI == kEpiSwiGlu) {
            const float u = split_sum(p + Nout, mn, ksplit);
            out = v / (1.0f + __expf(-v)) * u;
        } else {
            out = EPI == kEpiAccumulate ? *yp + v : v;
        }
        *yp = out;
    }
    if (!stats_out) return;
    float am = live ? fabsf(out * (nw_next ? nw_next[col] : 1.0f)) : 0.0f;
    float ss = live ? out * out : 0.0f;
    for (int o = 32; o > 0; o >>= 1) {
        am = fmaxf(am, __shfl_xor(am, o));
        ss += __shfl_xor(ss, o);
    }
    if ((threadIdx.x & 63) == 0) {
        s_a[threadIdx.x >> 6] = am;
        s_s[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    // threads 0 and 128 (each the first of its 128 outputs) store the pair
    // of waves they lead
    if ((threadIdx.x & 127) == 0 && live) {
        const int h = threadIdx.x >> 6;
        const int nblk = Nout / 128, blk = col / 128;
        stats_out[((size_t)row * nblk + blk) * 2] = fmaxf(s_a[h], s_a[h + 1]);
        stats_out[((size_t)row * nblk + blk) * 2 + 1] = s_s[h] + s_s[h + 1];
    }
}

// The same with four neighbouring outputs per thread: 16-byte loads of the
// splits and 16-byte stores of y (y 16-byte aligned, ldy % 4 == 0, N % 8 ==
// 0).  Each output is the same sum, in the same order, and the same epilogue
// as in k_gemm_reduce.  A half wave's 128 outputs are one row's 128-column
// statistics block (the output width is a multiple of 128), so each half
// reduces its (max, sum of squares) by DPP and its last lane stores them:
// no LDS, no barrier, where the scalar kernel used a chain of shuffles.
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_reduce4(const float* __restrict__ part, int ksplit,
                                                      int M, int N, float* __restrict__ y,
                                                      int ldy, float* __restrict__ stats_out,
                                                      const float* __restrict__ nw_next) {
    const int Nout = EPI == kEpiSwiGlu ? N / 2 : N;
    const unsigned e = 4 * (blockIdx.x * blockDim.x + threadIdx.x);   // first of 4 outputs
    const bool live = e < (unsigned)(M * Nout);
    if (!stats_out && !live) return;
    const int row = live ? (int)(e / (unsigned)Nout) : 0;
    const int col = live ? (int)(e - (unsigned)row * (unsigned)Nout) : 0;
    const size_t mn = (size_t)M * N;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live) {
        const float* p = part + (size_t)row * N + col;
        float v[4], u[4];
        split_sum4(p, mn, ksplit, v);
        float4* yp = (float4*)(y + (size_t)row * ldy + col);
        if (EPI == kEpiSwiGlu) {
            split_sum4(p + Nout, mn, ksplit, u);
#pragma unroll
            for (int c = 0; c < 4; c++) o[c] = v[c] / (1.0f + __expf(-v[c])) * u[c];
        } else if (EPI == kEpiAccumulate) {
            const float4 old = *yp;
            o[0] = old.x + v[0]; o[1] = old.y + v[1]; o[2] = old.z + v[2]; o[3] = old.w + v[3];
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) o[c] = v[c];
        }
        *yp = make_float4(o[0], o[1], o[2], o[3]);
    }
    if (!stats_out) return;
    float am = 0.0f, ss = 0.0f;
    if (live) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            am = fmaxf(am, fabsf(o[c] * (nw_next ? nw_next[col + c] : 1.0f)));
            ss = fmaf(o[c], o[c], ss);
        }
    }
    am = half_max_nonneg(am);
    ss = half_sum(ss);
    if ((threadIdx.x & 31) == 31 && live) {
        // the half's first output: 31 quads back
        const int nblk = Nout / 128, blk = (col - 124) / 128;
        stats_out[((size_t)row * nblk + blk) * 2] = am;
        stats_out[((size_t)row * nblk + blk) * 2 + 1] = ss;
    }
}

template <int RT, int NG>
int launch_gemm(const GemmArgs& a, dim3 grid) {
    if (a.nw)
        hipLaunchKernelGGL((k_gemm_int4<RT, NG, kProRmsNorm>), grid, dim3(64 * kGemmWaves), 0,
                           stream(), a);
    else
        hipLaunchKernelGGL((k_gemm_int4<RT, NG, kProNone>), grid, dim3(64 * kGemmWaves), 0,
                           stream(), a);
    return launch_check("k_gemm_int4");
}

}  // namespace

// Column tiles per block: two when that still gives >= 256 blocks (one per
// CU) and the pair shares a scale group (measured on the 7B shapes: two beat
// one by ~20% and four by ~25%, which drops below two blocks per CU), else
// one.  A gate|up pair always takes one gate and one up tile.
extern "C" int cgk_gemv_mfma_tiles(int N, int gs, int paired) {
    const int tiles = N / 16;
    if (paired) return 2;
    if (tiles / 2 >= 256 && gs % 32 == 0) return 2;
    return 1;
}

extern "C" int cgk_int4_repack_mfma(const uint8_t* flat, const float* scales, int K, int N,
                                    int gs, int paired, uint8_t* w, float* scales_t) {
    if (K % kRoundK || N % 16 || gs % 16 || N % gs || (paired && (N % 32))) {
        cgx_set_error("repack_mfma: unsupported shape K=%d N=%d gs=%d", K, N, gs);
        return -1;
    }
    size_t words = (size_t)K * N / 8;
    hipLaunchKernelGGL(k_repack_mfma, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                       stream(), flat, K, N, paired, (uint32_t*)w);
    if (launch_check("k_repack_mfma")) return -1;
    return cgk_int4_transpose_scales(scales, K, N / gs, scales_t);
}

extern "C" int cgk_int4_unpack_mfma(const uint8_t* w, const float* scales_t, int K, int N,
                                    int gs, int paired, uint8_t* flat, float* scales) {
    if (K % kRoundK || N % 16 || gs % 16 || N % gs || (paired && (N % 32))) {
        cgx_set_error("unpack_mfma: unsupported shape K=%d N=%d gs=%d", K, N, gs);
        return -1;
    }
    size_t bytes = (size_t)K * N / 2;
    hipLaunchKernelGGL(k_unpack_mfma, dim3((unsigned)((bytes + 255) / 256)), dim3(256), 0,
                       stream(), (const uint32_t*)w, K, N, paired, flat);
    if (launch_check("k_unpack_mfma")) return -1;
    // scales_t [N/gs][K] -> flat [K][N/gs]
    return cgk_int4_transpose_scales(scales_t, N / gs, K, scales);
}

extern "C" int cgk_int4_dequantize_mfma(const uint8_t* w, const float* scales_t, int K, int N,
                                        int gs, int paired, float* out) {
    size_t words = (size_t)K * N / 8;
    hipLaunchKernelGGL(k_dequant_mfma, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                       stream(), (const uint32_t*)w, scales_t, K, N, gs, paired, out);
    return launch_check("k_dequant_mfma");
}

// y = x @ W (layout 3) for M <= 16 rows per launch (larger M in chunks of 16).
// pro: 0 none, 1 RMSNorm of the rows (weights nw, eps); epi: 0 store,
// 1 accumulate (y += ...), 2 SwiGLU of a paired gate|up weight (y [M][N/2]).
extern "C" int cgk_gemv_mfma(const float* x, int ldx, int M, int K, int N, int gs,
                             const uint8_t* w, const float* scales_t, float* y, int ldy,
                             int pro, const float* nw, float eps, int epi) {
    const int paired = epi == kEpiSwiGlu;
    if (M < 1 || K % kRoundK || N % 16 || gs % 16 || N % gs || ldx < K ||
        (paired && N % 32) || (pro == kProRmsNorm && !nw) || pro < 0 || pro > 1 || epi < 0 ||
        epi > 2 || ldy < (paired ? N / 2 : N)) {
        cgx_set_error("gemv_mfma: unsupported shape M=%d K=%d N=%d gs=%d", M, K, N, gs);
        return -1;
    }
    if (((uintptr_t)x & 15) || (ldx & 3) || (nw && ((uintptr_t)nw & 15))) {
        cgx_set_error("gemv_mfma: x / norm weights must be 16-byte aligned with ldx %% 4 == 0");
        return -1;
    }
    const int T = cgk_gemv_mfma_tiles(N, gs, paired);
    // rows per launch: 16 (8 for the SwiGLU pair, whose A buffers are twice
    // as large); each launch streams W once
    const int mstep = paired ? 8 : 16;
    for (int m0 = 0; m0 < M; m0 += mstep) {
        MfmaArgs a;
        a.x = x + (size_t)m0 * ldx;
        a.ldx = ldx;
        a.M = M - m0 < mstep ? M - m0 : mstep;
        a.K = K; a.N = N; a.gs = gs;
        a.w = w; a.scales_t = scales_t;
        a.y = y + (size_t)m0 * ldy;
        a.ldy = ldy;
        a.nw = nw; a.eps = eps;
        a.ff = N / 2;
        int rc;
        if (stream_takes(a, epi)) {
            rc = pro == kProRmsNorm
                     ? (epi == kEpiAccumulate ? launch_stream_pe<kProRmsNorm, kEpiAccumulate>(a)
                                              : launch_stream_pe<kProRmsNorm, kEpiStore>(a))
                     : (epi == kEpiAccumulate ? launch_stream_pe<kProNone, kEpiAccumulate>(a)
                                              : launch_stream_pe<kProNone, kEpiStore>(a));
        } else if (pro == kProRmsNorm) {
            rc = epi == kEpiSwiGlu ? launch_pe<kProRmsNorm, kEpiSwiGlu>(a, T)
               : epi == kEpiAccumulate ? launch_pe<kProRmsNorm, kEpiAccumulate>(a, T)
               : launch_pe<kProRmsNorm, kEpiStore>(a, T);
        } else {
            rc = epi == kEpiSwiGlu ? launch_pe<kProNone, kEpiSwiGlu>(a, T)
               : epi == kEpiAccumulate ? launch_pe<kProNone, kEpiAccumulate>(a, T)
               : launch_pe<kProNone, kEpiStore>(a, T);
        }
        if (rc) return rc;
    }
    return 0;
}

// Test hook: the units on the busiest CU from which the streaming GEMV takes
// a product (0 never, 1 every product it supports); returns the previous
// value, and a negative argument only reads it.
extern "C" int cgx_gemv_stream_min_units(int units) {
    const int old = g_stream_min_units;
    if (units >= 0) g_stream_min_units = units;
    return old;
}

// 1 when cgk_gemm_int4 takes this product: 8 layout tiles per block within
// one scale group per A slot.
// Launches of at least this many blocks (four outputs a thread) take
// k_gemm_reduce4.
static int g_reduce4_min_blocks = 512;
// One K split of a gate|up pair applies SwiGLU in the GEMM (1), or stores
// partial sums for k_gemm_reduce (0).
static int g_gemm_swiglu_here = 1;

extern "C" int cgx_gemm_swiglu_here(int on) {
    const int old = g_gemm_swiglu_here;
    if (on >= 0) g_gemm_swiglu_here = on != 0;
    return old;
}

extern "C" int cgx_gemm_reduce4_min_blocks(int blocks) {
    const int old = g_reduce4_min_blocks;
    if (blocks >= 0) g_reduce4_min_blocks = blocks;
    return old;
}

extern "C" int cgk_gemm_int4_supported(int M, int K, int N, int gs, int paired) {
    return M >= 1 && K % kChunkK == 0 && N % 128 == 0 && gs % 128 == 0 &&
           (!paired || (N / 2) % 128 == 0);
}

extern "C" int cgk_gemm_int4(const float* x, int ldx, int M, int K, int N, int gs,
                             const uint8_t* w, const float* scales_t, float smax, float* y,
                             int ldy, int pro, const float* nw, float eps, int epi,
                             const float* stats_in, int nstat_in, float* stats_out,
                             const float* nw_next) {
    const int paired = epi == kEpiSwiGlu;
    if (!cgk_gemm_int4_supported(M, K, N, gs, paired) || ldx < K || (ldx & 3) ||
        ((uintptr_t)x & 15) || (pro == kProRmsNorm && (!nw || ((uintptr_t)nw & 15))) ||
        ldy < (paired ? N / 2 : N) || (size_t)M * N >= (1u << 31)) {
        cgx_set_error("gemm_int4: unsupported shape M=%d K=%d N=%d gs=%d", M, K, N, gs);
        return -1;
    }
    // row tiles per block: up to 3 (48 rows) for short batches; longer ones
    // run as blocks of 2 row tiles (32 rows), which doubles the blocks that
    // share the weights and leaves fewer K splits to reduce (measured on the
    // tree verify's 256 rows: 13.52 ms a step against 13.84 with 4 row tiles;
    // more blocks per launch or four blocks per CU were slower)
    const int RT = M > 48 ? 2 : (M + 15) / 16;
    const int BM = 16 * RT;
    const int rowblocks = (M + BM - 1) / BM;
    const int colblocks = paired ? N / 2 / 128 : (N / 128 + 1) / 2;
    const int nchunks = K / kChunkK;
    // two blocks per CU, splits of at least two chunks, and partial sums
    // (8 M bytes per column and split, written and read) at most about twice
    // the weight bytes (K / 2 per column): at 40 rows the blocks for every CU
    // are worth more than the partial traffic (measured), at 256 rows not
    int ksplit = (512 + colblocks * rowblocks - 1) / (colblocks * rowblocks);
    ksplit = ksplit > nchunks / 2 ? nchunks / 2 : ksplit;
    ksplit = ksplit > K / (4 * M) ? K / (4 * M) : ksplit;
    ksplit = ksplit < 1 ? 1 : (ksplit > 16 ? 16 : ksplit);
    const int ksteps = (nchunks + ksplit - 1) / ksplit;
    ksplit = (nchunks + ksteps - 1) / ksteps;
    // one split storing plain rows (the lm_head of a tree verify): the GEMM
    // writes y itself, and no reduction pass copies it; one split of a
    // gate|up pair (the tree verify's 256 rows): the GEMM applies SwiGLU and
    // writes y and its row statistics (tree verify 12.50 -> 12.36 ms a step)
    const bool swiglu_here = ksplit == 1 && paired && g_gemm_swiglu_here;
    const bool direct = (ksplit == 1 && epi == kEpiStore && !stats_out && ldy == N) ||
                        swiglu_here;
    const size_t row_bytes = (((size_t)M * 8) + 255) & ~(size_t)255;
    char* ws = (char*)cgx_scratch(CGX_SLOT_WS5,
                                  row_bytes + (direct ? 0 : (size_t)ksplit * M * N * 4));
    if (!ws) return -1;
    GemmArgs a;
    a.x = x; a.ldx = ldx; a.M = M; a.K = K; a.N = N; a.gs = gs;
    a.w = w; a.scales_t = scales_t;
    a.nw = pro == kProRmsNorm ? nw : nullptr;
    a.rowscale = (const float*)ws;
    a.unscale = (const float*)ws + M;
    a.stats = stats_in;
    a.nstat = nstat_in;
    a.smax = smax;
    a.eps = eps;
    a.part = direct ? y : (float*)(ws + row_bytes);
    a.ksteps = ksteps;
    a.ff = N / 2;
    a.y = swiglu_here ? y : nullptr;
    a.ldy = ldy;
    a.stats_out = swiglu_here ? stats_out : nullptr;
    a.nw_next = nw_next;
    if (!stats_in) {
        hipLaunchKernelGGL(k_gemm_rows, dim3(M), dim3(256), 0, stream(), x, ldx, K, a.nw,
                           pro == kProRmsNorm, eps, smax, (float*)ws, (float*)ws + M);
        if (launch_check("k_gemm_rows")) return -1;
    } else if (nstat_in < 1) {
        cgx_set_error("gemm_int4: row statistics without entries");
        return -1;
    }
    dim3 grid(colblocks, rowblocks, ksplit);
    int rc;
    if (paired) {
        rc = RT == 1 ? launch_gemm<1, 2>(a, grid) : RT == 2 ? launch_gemm<2, 2>(a, grid)
           : RT == 3 ? launch_gemm<3, 2>(a, grid) : launch_gemm<4, 2>(a, grid);
    } else {
        rc = RT == 1 ? launch_gemm<1, 1>(a, grid) : RT == 2 ? launch_gemm<2, 1>(a, grid)
           : RT == 3 ? launch_gemm<3, 1>(a, grid) : launch_gemm<4, 1>(a, grid);
    }
    if (rc || direct) return rc;
    const int Nout = paired ? N / 2 : N;
    const size_t outs = (size_t)M * Nout;
    const int blocks = (int)((outs + 255) / 256);
    // four outputs a thread where y's rows are 16-byte aligned (the
    // decoder's buffers) and the launch keeps at least 512 blocks: 16-byte
    // loads and stores, DPP statistics (tree verify, 256 rows: 12.94 ->
    // 12.54 ms a step).  Fewer outputs keep a thread each (the batch-8
    // verify, 40 rows and up to 16 splits, measured the same either way once
    // each thread's split loads were batched: 5.66 -> 5.45 ms a step).
    const int blocks4 = (int)((outs / 4 + 255) / 256);
    if (((uintptr_t)y & 15) == 0 && ldy % 4 == 0 && blocks4 >= g_reduce4_min_blocks) {
        if (epi == kEpiSwiGlu)
            hipLaunchKernelGGL(k_gemm_reduce4<kEpiSwiGlu>, dim3(blocks4), dim3(256), 0, stream(),
                               a.part, ksplit, M, N, y, ldy, stats_out, nw_next);
        else if (epi == kEpiAccumulate)
            hipLaunchKernelGGL(k_gemm_reduce4<kEpiAccumulate>, dim3(blocks4), dim3(256), 0,
                               stream(), a.part, ksplit, M, N, y, ldy, stats_out, nw_next);
        else
            hipLaunchKernelGGL(k_gemm_reduce4<kEpiStore>, dim3(blocks4), dim3(256), 0, stream(),
                               a.part, ksplit, M, N, y, ldy, stats_out, nw_next);
        return launch_check("k_gemm_reduce4");
    }
    if (epi == kEpiSwiGlu)
        hipLaunchKernelGGL(k_gemm_reduce<kEpiSwiGlu>, dim3(blocks), dim3(256), 0, stream(),
                           a.part, ksplit, M, N, y, ldy, stats_out, nw_next);
    else if (epi == kEpiAccumulate)
        hipLaunchKernelGGL(k_gemm_reduce<kEpiAccumulate>, dim3(blocks), dim3(256), 0, stream(),
                           a.part, ksplit, M, N, y, ldy, stats_out, nw_next);
    else
        hipLaunchKernelGGL(k_gemm_reduce<kEpiStore>, dim3(blocks), dim3(256), 0, stream(),
                           a.part, ksplit, M, N, y, ldy, stats_out, nw_next);
    return launch_check("k_gemm_reduce");
}

// max |s| over a scales array (host result, synchronising)
__global__ void k_absmax(const float* __restrict__ s, size_t n, unsigned int* out) {
    float m = 0.0f;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        m = fmaxf(m, fabsf(s[i]));
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(m));
}

extern "C" int cgk_absmax(const float* s, size_t n, float* out_host) {
    unsigned int* d = (unsigned int*)cgx_scratch(CGX_SLOT_OUT1, 16);
    if (!d) return -1;
    unsigned int zero = 0u, r = 0u;
    if (hipMemcpyAsync(d, &zero, 4, hipMemcpyHostToDevice, stream()) != hipSuccess) {
        cgx_set_error("absmax: copy failed");
        return -1;
    }
    hipLaunchKernelGGL(k_absmax, dim3(256), dim3(256), 0, stream(), s, n, d);
    if (launch_check("k_absmax")) return -1;
    if (hipMemcpyAsync(&r, d, 4, hipMemcpyDeviceToHost, stream()) != hipSuccess ||
        hipStreamSynchronize(stream()) != hipSuccess) {
        cgx_set_error("absmax: copy failed");
        return -1;
    }
    float f;
    memcpy(&f, &r, sizeof f);
    *out_host = f;
    return 0;
}
