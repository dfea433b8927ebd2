// attn_dec.hip -- flash decoding / verification over the INT4 KV cache on
// the gfx950 matrix cores (the speculative verify shape: a few query rows per
// KV head against a long cached context).
//
// Reference semantics (cogito-ml/cogito):
//   src/cuda/flash_attn_kernels.c:261-396  online softmax; GQA: query head h
//                                           reads KV head h * Hk / H; masked
//                                           scores are -FLT_MAX
//   src/quantize/int4.c:236-289            K/V value = nibble * scale, one
//                                           scale per (position, head, group)
// This kernel takes the cache with one scale group per head row (group ==
// head_dim, the cache the decoder builds); other groupings use k_attn.
//
// Arithmetic.  Scores S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x32_f16:
// the K and V nibbles are exact fp16 integers; Q (times the softmax scale)
// and P (times the V scale of its key) are each carried as hi + lo fp16
// (22 significant bits) after a power-of-two scaling into fp16 range; the
// products are exact and accumulate in fp32.  The K scale multiplies the
// fp32 score of its key.
//
// Work split.  Block = (key split, KV head, chunk of 16*RT query rows), 4
// waves; wave w takes the 32-key tiles w, w+4, ... of the split.  The launch
// picks RT (16 or 32 rows per block) and the split length from the shape
// (see cgk_attn_dec_batch).  A block loads its Q rows, then issues its first
// tile, and builds the Q operands while the tile is in flight (the barrier
// that publishes them orders LDS only); every tile is loaded by the same
// branch-free sequence (keys past the split's end are clamped and masked),
// the loop prefetches the next tile, and the last tile is peeled off so no
// load is issued past the split.  In the
// S^T orientation a lane holds one query row and 8 keys of a tile -- exactly
// the B operand of the P^T side, so P never moves.  V^T needs each lane to
// hold 8 keys of one head-dim column: the lane loads one u32 (8 columns) of
// each of its 8 keys and v_perm_b32 gathers nibble t of two keys at a time.
// Waves merge through LDS; splits merge in k_attn_dec_combine.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>

#include "cgx_internal.h"

namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kTile = 32;                  // keys per wave tile
constexpr int kSplitKeys = kWaves * kTile; // keys per block round
// launch shape: about this many blocks with 16 / 32 query rows per block,
// at most this many key splits (the combine reads every split's partial rows)
constexpr int kTargetBlocks1 = 256;
constexpr int kTargetBlocks2 = 384;
constexpr int kMaxSplits = 40;

inline hipStream_t stream() { return (hipStream_t)cgx_stream(); }

int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        cgx_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

enum { kMaskNone = 0, kMaskCausal = 1, kMaskTree = 4 };
constexpr int kMaxBatch = 16;

struct DecArgs {
    const float* Q;              // [Nq][H][D]
    const uint8_t* kc;           // [pos][Hk][D/2] two's complement nibbles
    const uint8_t* vc;
    const float* ks;             // [pos][Hk] (one group per head row)
    const float* vs;
    int Nq, Nk, H, Hk, D_;
    float scale;
    int mask_kind;
    int splits, keys_per_split;
    float* O;                    // [Nq][H][D] when splits == 1
    float* part_o;               // [splits][Nq*H][D]
    float* part_ml;              // [splits][Nq*H][2]
    unsigned long long anc[64];  // tree: ancestor bits over the last tw keys
    int tw;                      // tree window: the last tw keys (Nq <= tw <= 64) are
                                 // visible to a query row only through its anc bits
    // batch: B sequences, each with Nq query rows (Q, O: [B][Nq][H][D]) and
    // its own cache at kc + b * seq_kbytes (scales + b * seq_groups) of
    // nk[b] keys; blockIdx.z = b * chunks + row chunk
    int B, chunks;
    size_t seq_kbytes, seq_groups;
    int nk[kMaxBatch];
    // fused RoPE and cache append (k_attn_dec<..., true>): the Q rows come
    // from the raw projections and are rotated here; the Nq new keys of each
    // sequence (positions nk - Nq .. nk - 1) are rotated, quantised and
    // written to the cache by split nsplit_old, which attends over them from
    // LDS; splits below it cover the cached keys [0, nk - Nq)
    const float* qkv;            // [B][Nq][ldq]: q heads, k heads, v heads
    int ldq;
    const float2* rope;          // [B][Nq][D/2] (cos, sin) of each row's rotary position
    uint8_t* kcw;                // the caches (kc, vc, ks, vs), written
    uint8_t* vcw;
    float* ksw;
    float* vsw;
    int nsplit_old;
    // row statistics of O for the GEMM that reads it (D == 128: one entry
    // per output row and head, i.e. per 128 columns): (max|o|, sum o^2),
    // [B][Nq][H][2]; nullptr: none
    float* stats;
};

__device__ __forceinline__ int head_begin(int hk, int H, int Hk) { return (hk * H + Hk - 1) / Hk; }

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

// nibble slot of MFMA position p inside a u32 of 8 nibbles (see nib_pairs)
__device__ __forceinline__ int slot_of(int p) { return (p >> 1) + 4 * (p & 1); }

// Eight offset-binary nibbles of w as exact fp16 (o - 8), in position order
// p -> slot {0,4,1,5,2,6,3,7}[p].
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

// Nibble t (0..7) of two offset-binary words as an exact fp16 pair (o - 8).
__device__ __forceinline__ f16x2 nib_pair(uint32_t wlo, uint32_t whi, int t, const NibConst& nk) {
    const uint32_t b = (uint32_t)(t >> 1);
    const uint32_t sel = 0x0C000C00u | ((4u + b) << 16) | b;
    const uint32_t v = __builtin_amdgcn_perm(whi, wlo, sel);
    if (t & 1) {
        const f16x2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
        const f16x2 m72 = {(_Float16)-72.0f, (_Float16)-72.0f};
        return __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (v & nk.mhi) | nk.mag), s16, m72);
    }
    const f16x2 m1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    return __builtin_bit_cast(f16x2, (v & nk.mlo) | nk.mag) + m1032;
}

__device__ __forceinline__ void split16(float v, _Float16& hi, _Float16& lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// Sum / maximum (non-negative values) over each 32-lane half of the wave:
// scans over the 16-lane DPP rows, then row_bcast:15 adds row 0's total into
// row 1 and row 2's into row 3, so lanes 31 and 63 hold the halves' results.
__device__ __forceinline__ float half_sum(float v) {
#define CGX_DPP(CTRL, RMASK) \
    __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, RMASK, 0xF, true))
    v += CGX_DPP(0x111, 0xF);
    v += CGX_DPP(0x112, 0xF);
    v += CGX_DPP(0x114, 0xF);
    v += CGX_DPP(0x118, 0xF);
    v += CGX_DPP(0x142, 0xA);
    return v;
}
__device__ __forceinline__ float half_max_nonneg(float v) {
    v = fmaxf(v, CGX_DPP(0x111, 0xF));
    v = fmaxf(v, CGX_DPP(0x112, 0xF));
    v = fmaxf(v, CGX_DPP(0x114, 0xF));
    v = fmaxf(v, CGX_DPP(0x118, 0xF));
    v = fmaxf(v, CGX_DPP(0x142, 0xA));
    return v;
#undef CGX_DPP
}

// Workgroup barrier that orders LDS accesses only: global loads in flight
// stay in flight (__syncthreads() would wait for every one of them).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// key of MFMA position pos (0..31) of a tile: positions 8g..8g+3 are keys
// 4g..4g+3, positions 8g+4..8g+7 are keys 16+4g..16+4g+3 (the S^T rows a
// lane of group g holds)
__device__ __forceinline__ int key_of_pos(int g, int p) { return p < 4 ? 4 * g + p : 16 + 4 * g + p - 4; }

// Rotate-half RoPE with k_rope_append's operations (decoder.hip): value d of
// a head row from its own value and its partner's (d +- D/2), (c, s) of i =
// d mod D/2.  Each product rounds on its own, as in the reference's CPU code:
// contraction is off here (this file is otherwise built with it, and the
// _rn intrinsics lower to plain operations the backend would fuse).
__device__ __forceinline__ float rope_val(float own, float partner, float2 cs, bool second) {
#pragma clang fp contract(off)
    const float a = second ? partner * cs.y : own * cs.x;
    const float b = second ? own * cs.x : partner * cs.y;
    return second ? a + b : a - b;
}

// own c + partner s', each product rounded on its own (s' = -s gives the
// first half's own c - partner s, s' = s the second half's partner s + own c)
__device__ __forceinline__ float rope_sum(float own, float partner, float c, float s) {
#pragma clang fp contract(off)
    return own * c + partner * s;
}

template <int D, int RT, bool FUSED>
__global__ __launch_bounds__(64 * kWaves, 2) void k_attn_dec(DecArgs a) {
    constexpr int NC = D / 32;          // QK MFMAs per 16 keys (32 head-dim values each)
    constexpr int DPL = D / 4;          // head-dim values per lane group
    constexpr int ROWS = 16 * RT;
    // LDS: the Q^T operands (read back per tile, which keeps them out of
    // the register file), then, in the same bytes, the waves' partial O
    constexpr int kQBytes = RT * NC * 2 * 64 * (int)sizeof(f16x8);
    constexpr int kOBytes = kWaves * ROWS * (D + 4) * (int)sizeof(float);
    __shared__ __attribute__((aligned(16))) unsigned char s_raw[kOBytes > kQBytes ? kOBytes : kQBytes];
    f16x8 (*s_q)[NC][2][64] = (f16x8 (*)[NC][2][64])s_raw;
    float (*s_o)[ROWS][D + 4] = (float (*)[ROWS][D + 4])s_raw;
    __shared__ float s_m[kWaves][ROWS], s_l[kWaves][ROWS];
    __shared__ float s_w[kWaves][ROWS], s_M[ROWS], s_L[ROWS];
    // fused launches keep two more things in s_raw, past the Q operands
    // (s_o overwrites all of it only after the last tile): the rotary table
    // of the block's rows (read while the Q operands are built) and the new
    // keys in the cache's layout (up to 64 keys, read by the tiles)
    constexpr int kTblBytes = ROWS * (D / 2) * (int)sizeof(float2);
    constexpr int kNewKeys = 64;
    static_assert(!FUSED || kQBytes + kTblBytes + kNewKeys * (D + 8) <= (int)sizeof(s_raw),
                  "fused staging fits the block's LDS");
    // the table transposed: tbl[j][2 t + h] = (cos, sin) of frequency
    // DPL h + j of table row t, so that the lanes reading one j (every query
    // row, both halves) read neighbouring words, with no bank conflict
    float2 (*tbl)[2 * ROWS] = (float2 (*)[2 * ROWS])(s_raw + kQBytes);
    uint8_t (*st_k)[D / 2] = (uint8_t (*)[D / 2])(s_raw + kQBytes + kTblBytes);
    uint8_t (*st_v)[D / 2] = st_k + kNewKeys;
    float* st_ks = (float*)(st_v + kNewKeys);
    float* st_vs = st_ks + kNewKeys;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const NibConst nk = nib_consts();
    const int n = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int h0 = head_begin(hk, a.H, a.Hk), h1 = head_begin(hk + 1, a.H, a.Hk);
    const int R = (h1 - h0) * a.Nq;
    // the block's sequence and its cache
    const int sq = (int)blockIdx.z / a.chunks;
    const int row0 = ((int)blockIdx.z % a.chunks) * ROWS;
    const int Nk = a.B > 1 ? a.nk[sq] : a.Nk;
    const uint8_t* __restrict__ kcache = a.kc + (size_t)sq * a.seq_kbytes;
    const uint8_t* __restrict__ vcache = a.vc + (size_t)sq * a.seq_kbytes;
    const float* __restrict__ kscale = a.ks + (size_t)sq * a.seq_groups;
    const float* __restrict__ vscale = a.vs + (size_t)sq * a.seq_groups;
    const float* __restrict__ Qs = a.Q + (size_t)sq * a.Nq * a.H * D;
    const size_t orow0 = (size_t)sq * a.Nq * a.H;
    const int Hk = a.Hk;
    const size_t krow = (size_t)Hk * (D / 2);       // bytes between positions

    // fused: split nsplit_old is the new keys, the others the cached ones
    const bool new_split = FUSED && split == a.nsplit_old;
    const int nk_old = FUSED ? Nk - a.Nq : Nk;
    const int k_begin = new_split ? nk_old : split * a.keys_per_split;
    const int k_end = new_split ? Nk : min(nk_old, k_begin + a.keys_per_split);
    const int ntiles = (k_end - k_begin + kTile - 1) / kTile;
    // first key under the mask's bits: the new positions (chain), or the
    // tree window (the tree's nodes, of this call and of earlier calls)
    const int base = Nk - (a.mask_kind == kMaskTree ? a.tw : a.Nq);

    float m_run[RT], l_part[RT];
    f32x4 o[RT][8];                                  // O^T tiles t = 0..7
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        m_run[rt] = -__builtin_inff();
        l_part[rt] = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) o[rt][t] = (f32x4)(0.0f);
    }
    int ev_cur = 0;                                  // O is held times 2^ev_cur

    // -- loads of one tile: K rows (A operand: key n (+16 kh), head-dim part
    //    g), V words (A of V^T: column block n, keys of positions 8g..8g+7),
    //    K and V scales of the keys this lane scores
    struct TileData {
        uint32_t kw[2][NC];
        uint32_t vw[8];
        float sk[8], sv[8];
    };
    // one load sequence for every tile (a single code path keeps the
    // compiler's load counters exact, so a wait for one tile never waits for
    // the next): keys past k_end read the last key (its values are masked),
    // addresses are 32-bit offsets (key * row bytes) from uniform bases.
    // Lane (n, g) reads K rows n and 16 + n (head-dim part g), and the V word
    // and K / V scales of its keys 4g + koff(p), koff = {0, 1, 2, 3, 16, 17,
    // 18, 19} (key_of_pos); lanes n >= D/8 read V column block 0, whose O^T
    // rows are never stored.
    const int nb = n < D / 8 ? n : 0;
    const uint8_t* __restrict__ kbase = kcache + (size_t)hk * (D / 2);
    const uint8_t* __restrict__ vbase = vcache + (size_t)hk * (D / 2);
    const float* __restrict__ ksb = kscale + hk;
    const float* __restrict__ vsb = vscale + hk;
    const uint32_t krow32 = (uint32_t)krow;
    // (a split past a short sequence's cached keys reads position 0: valid
    // memory, never used)
    const int klast = max(k_end - 1, 0);
    auto load_tile = [&](int kt, TileData& t) {
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            const uint32_t key = (uint32_t)min(kt + 16 * kh + n, klast);
            const uint8_t* p = kbase + (key * krow32 + (uint32_t)((D / 8) * g));
            if (NC == 4) {
                u32x4 v = *(const u32x4*)p;
                t.kw[kh][0] = v.x; t.kw[kh][1 % NC] = v.y; t.kw[kh][2 % NC] = v.z; t.kw[kh][3 % NC] = v.w;
            } else if (NC == 2) {
                u32x2 v = *(const u32x2*)p;
                t.kw[kh][0] = v.x; t.kw[kh][1 % NC] = v.y;
            } else {
                t.kw[kh][0] = *(const uint32_t*)p;
            }
        }
        // the scores need K and its scales, the O update V and its scales:
        // loads complete in issue order, so the K scales come before V
        const int kl = kt + 4 * g;
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const uint32_t key = (uint32_t)min(kl + (p < 4 ? p : 12 + p), klast);
            t.sk[p] = ksb[key * (uint32_t)Hk];
        }
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const uint32_t key = (uint32_t)min(kl + (p < 4 ? p : 12 + p), klast);
            t.vw[p] = *(const uint32_t*)(vbase + (key * krow32 + (uint32_t)(4 * nb)));
            t.sv[p] = vsb[key * (uint32_t)Hk];
        }
    };
    // the same tile from the LDS staging of the new keys (key kt + j is row
    // kt + j - k_begin; rows past the last are clamped and masked)
    auto load_tile_lds = [&](int kt, TileData& t) {
        const int rlast = k_end - 1 - k_begin;
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            const int r = min(kt - k_begin + 16 * kh + n, rlast);
            const uint8_t* p = &st_k[r][(D / 8) * g];
#pragma unroll
            for (int c = 0; c < NC; c++) t.kw[kh][c] = *(const uint32_t*)(p + 4 * c);
        }
        const int kl = kt - k_begin + 4 * g;
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const int r = min(kl + (p < 4 ? p : 12 + p), rlast);
            t.sk[p] = st_ks[r];
            t.vw[p] = *(const uint32_t*)&st_v[r][4 * nb];
            t.sv[p] = st_vs[r];
        }
    };

    // ---- Q^T operands of the block's rows (B operand: row n, 8 positions per
    //      MFMA), built once per block and read back from LDS by every wave
    float qinv[RT];
    int rq[RT];
    bool rok[RT];
    unsigned long long anc_row[RT];
    int lim_row[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = row0 + 16 * rt + n;
        rok[rt] = r < R;
        rq[rt] = rok[rt] ? r % a.Nq : 0;
        anc_row[rt] = a.anc[rq[rt]];     // zero unless a tree mask
        // chain: keys up to the query's own position; tree: the cached prefix
        // (plus ancestor bits); no mask: every key
        lim_row[rt] = a.mask_kind == kMaskCausal ? Nk - a.Nq + rq[rt]
                    : a.mask_kind == kMaskTree ? Nk - a.tw - 1 : Nk;
    }
    // the Q rows are loaded first (the previous kernel just wrote them, they
    // come from cache), then the first tile: loads complete in issue order,
    // so the operand preparation below waits for Q only and overlaps the
    // tile's HBM latency.  Rows past R read row 0 (valid memory) and are
    // zeroed, so the loads are unconditional.
    float qv[RT][DPL];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = row0 + 16 * rt + n;
        const int h = h0 + (rok[rt] ? r / a.Nq : 0), q = rq[rt];
        if (FUSED) {
            // the raw q row (rotated below, once the rotary table is in LDS)
            const float* qp = a.qkv + ((size_t)sq * a.Nq + q) * a.ldq + (size_t)h * D + DPL * g;
#pragma unroll
            for (int i = 0; i < DPL; i += 4) {
                const float4 t = *(const float4*)(qp + i);
                qv[rt][i] = t.x; qv[rt][i + 1] = t.y; qv[rt][i + 2] = t.z; qv[rt][i + 3] = t.w;
            }
        } else {
            const float* qp = Qs + ((size_t)q * a.H + h) * D + DPL * g;
#pragma unroll
            for (int i = 0; i < DPL; i += 4) {
                const float4 t = *(const float4*)(qp + i);
                qv[rt][i] = t.x; qv[rt][i + 1] = t.y; qv[rt][i + 2] = t.z; qv[rt][i + 3] = t.w;
            }
        }
    }
    // unconditional, like the prefetch below: a wave without a tile reads the
    // split's last key (k_end >= 1 whenever the block runs)
    TileData td;
    // fused: the rotary table rows of the block's queries, loaded before the
    // first tile (loads complete in issue order, so the rotation below waits
    // for Q and the table only).  With Nq <= ROWS the table holds the Nq rows
    // of the sequence (indexed by q), else the block's rows (by r - row0).
    constexpr int kTblQuads = D / 4;                    // float4 = two (cos, sin)
    constexpr int kTblLoads = (ROWS * kTblQuads + 64 * kWaves - 1) / (64 * kWaves);
    const bool tbl_by_q = a.Nq <= ROWS;
    const int tbl_rows = tbl_by_q ? a.Nq : ROWS;
    float4 tv[FUSED ? kTblLoads : 1];
    if (FUSED) {
#pragma unroll
        for (int j = 0; j < kTblLoads; j++) {
            const int e = min((int)threadIdx.x + j * 64 * kWaves, tbl_rows * kTblQuads - 1);
            const int i = e / kTblQuads, c = e % kTblQuads;
            const int q = tbl_by_q ? i : (row0 + i < R ? (row0 + i) % a.Nq : 0);
            tv[j] = *(const float4*)(a.rope + ((size_t)sq * a.Nq + q) * (D / 2) + 2 * c);
        }
    }
    // the new-key split: the raw K / V values of its rows (a batch of up to
    // kStage rows a wave, all loads in flight before the first is used)
    constexpr int kStage = 4;
    const int half = D / 2;
    const int sl = lane < half ? lane : half - 1;       // lane -> dims 2 sl, 2 sl + 1
    const int e0 = 2 * sl;
    const bool k_second = e0 >= half;
    const int e_par = k_second ? e0 - half : e0 + half, i_rot = k_second ? e0 - half : e0;
    float sv0[kStage], sv1[kStage], su0[kStage], su1[kStage];
    float2 sc0[kStage], sc1[kStage];
    auto stage_load = [&](int rbase) {
#pragma unroll
        for (int b = 0; b < kStage; b++) {
            const int rr = min(rbase + b * kWaves, 2 * a.Nq - 1);
            const int pnew = rr >> 1;
            const bool isv = rr & 1;
            const size_t qrow = (size_t)sq * a.Nq + pnew;
            const float* src = a.qkv + qrow * a.ldq + (size_t)(a.H + (isv ? Hk : 0) + hk) * D;
            sv0[b] = src[e0];
            sv1[b] = src[e0 + 1];
            su0[b] = src[e_par];
            su1[b] = src[e_par + 1];
            sc0[b] = a.rope[qrow * half + i_rot];
            sc1[b] = a.rope[qrow * half + i_rot + 1];
        }
    };
    // the staged rows: K rotated, K and V quantised as k_rope_append does
    // (absmax / 7 per head row, floor 1e-8, roundf, clamp to [-8, 7]) into
    // LDS, and, by the block of row chunk 0, into the cache
    auto stage_store = [&](int rbase) {
        const bool writer = (int)blockIdx.z % a.chunks == 0;
#pragma unroll
        for (int b = 0; b < kStage; b++) {
            const int rr = rbase + b * kWaves;
            if (rr >= 2 * a.Nq) break;                 // wave-uniform
            const int pnew = rr >> 1;
            const bool isv = rr & 1;
            float v0 = sv0[b], v1 = sv1[b];
            if (!isv) {
                v0 = rope_val(v0, su0[b], sc0[b], k_second);
                v1 = rope_val(v1, su1[b], sc1[b], k_second);
            }
            float mx = lane < half ? fmaxf(fabsf(v0), fabsf(v1)) : 0.0f;
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0x111, 0xF, 0xF, true)));
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0x112, 0xF, 0xF, true)));
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0x114, 0xF, 0xF, true)));
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0x118, 0xF, 0xF, true)));
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0x142, 0xA, 0xF, true)));
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0x143, 0xC, 0xF, true)));
            mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 63));
            float sc = __fdiv_rn(mx, 7.0f);
            if (sc < 1e-8f) sc = 1.0f;
            int q0 = (int)roundf(__fdiv_rn(v0, sc)), q1 = (int)roundf(__fdiv_rn(v1, sc));
            q0 = q0 > 7 ? 7 : (q0 < -8 ? -8 : q0);
            q1 = q1 > 7 ? 7 : (q1 < -8 ? -8 : q1);
            const uint8_t byte = (uint8_t)((q0 & 0xF) | ((q1 & 0xF) << 4));
            const size_t th = (size_t)(nk_old + pnew) * Hk + hk;   // (position, head)
            if (lane < half) {
                (isv ? st_v : st_k)[pnew][lane] = byte;
                if (writer) {
                    uint8_t* cw = (isv ? a.vcw : a.kcw) + (size_t)sq * a.seq_kbytes;
                    cw[th * half + lane] = byte;
                }
            }
            if (lane == 0) {
                (isv ? st_vs : st_ks)[pnew] = sc;
                if (writer) ((isv ? a.vsw : a.ksw) + (size_t)sq * a.seq_groups)[th] = sc;
            }
        }
    };
    if (new_split) stage_load(wave);
    if (!new_split) load_tile(k_begin + wave * kTile, td);
    if (FUSED) {
#pragma unroll
        for (int j = 0; j < kTblLoads; j++) {
            const int e = (int)threadIdx.x + j * 64 * kWaves;
            if (e < tbl_rows * kTblQuads) {
                // entries i, i + 1 of row t (i even: the same half)
                const int t = e / kTblQuads, i = 2 * (e % kTblQuads);
                const int h = i / DPL, jj = i % DPL;
                tbl[jj][2 * t + h] = make_float2(tv[j].x, tv[j].y);
                tbl[jj + 1][2 * t + h] = make_float2(tv[j].z, tv[j].w);
            }
        }
    }
    if (new_split) {
        // wave w takes rows w, w + 4, ... of the 2 Nq (key, value) rows
        for (int rb = wave;;) {
            stage_store(rb);
            rb += kWaves * kStage;
            if (rb >= 2 * a.Nq) break;
            stage_load(rb);
        }
    }
    if (FUSED) {
        // rotate the Q rows: lane (n, g) holds dims DPL g .. DPL g + DPL - 1,
        // its partners (d +- D/2) are in lane group g ^ 2, i.e. the lane 32
        // apart; v_permlane32_swap exchanges the two halves of the wave
        lds_barrier();                               // the rotary table is in LDS
        // value d: own c - partner s (first half) or partner s + own c
        // (second half), i.e. own c + partner s' with s' = -s / s: negation
        // and the order of an addition's operands are exact
        const uint32_t sflip = g >= 2 ? 0u : 0x80000000u;
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int col = 2 * (tbl_by_q ? rq[rt] : 16 * rt + n) + (g & 1);
#pragma unroll
            for (int i = 0; i < DPL; i++) {
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(qv[rt][i]),
                                                                 __float_as_uint(qv[rt][i]),
                                                                 false, false);
                const float partner = __uint_as_float(g >= 2 ? sw[0] : sw[1]);
                const float2 cs = tbl[i][col];
                const float sn = __uint_as_float(__float_as_uint(cs.y) ^ sflip);
                qv[rt][i] = rope_sum(qv[rt][i], partner, cs.x, sn);
            }
        }
    }
    {
        // rows are per lane (n); every wave computes the row exponent of its
        // lanes' rows for all RT (cheap), the fp16 splits are divided: wave w
        // builds the operands of row tile rt for head-dim chunks c with
        // (rt * NC + c) % kWaves == w
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const float keep = rok[rt] ? 1.0f : 0.0f;
            float qmax = 0.0f;
#pragma unroll
            for (int i = 0; i < DPL; i++) {
                qv[rt][i] *= keep;
                qmax = fmaxf(qmax, fabsf(qv[rt][i]));
            }
            qmax *= a.scale;
            qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
            qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
            int E = 0;
            if (qmax > 0.0f && qmax < __builtin_inff()) E = 14 - ilogbf(qmax);
            E = E > 100 ? 100 : (E < -100 ? -100 : E);
            const float up = ldexpf(1.0f, E) * a.scale;
            qinv[rt] = ldexpf(1.0f, -E);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                if ((rt * NC + c) % kWaves != wave) continue;
                f16x8 hv, lv;
#pragma unroll
                for (int p = 0; p < 8; p++) {
                    const float v = qv[rt][8 * c + slot_of(p)] * up;
                    _Float16 hi, lo;
                    split16(v, hi, lo);
                    hv[p] = hi;
                    lv[p] = lo;
                }
                s_q[rt][c][0][lane] = hv;
                s_q[rt][c][1][lane] = lv;
            }
        }
    }
    // the Q^T operands are in LDS; the first tile's loads stay in flight
    lds_barrier();

    // keys below open_end are visible to every row: the chain's cached
    // prefix, the tree's prefix below its window, every key without a mask
    const int open_end = a.mask_kind == kMaskNone ? Nk : base;
    // one tile: scores, online softmax, O update.  The loop prefetches the
    // next tile while it computes; the last tile is peeled off so that no
    // load is issued past the split (each path keeps exact load counters).
    auto process = [&](TileData& td, const int tile) {
        const int kt = k_begin + tile * kTile;
        // wave-uniform: the wave's first tile (O and l are still zero), and a
        // whole tile under no mask
        const bool first = tile == wave;
        const bool open = kt + kTile <= k_end && kt + kTile <= open_end;
        uint32_t (&kw)[2][NC] = td.kw;
        uint32_t (&vw)[8] = td.vw;
        float (&sk)[8] = td.sk;
        float (&sv)[8] = td.sv;

        // the Q^T operands are re-read from LDS every tile (an opaque lane
        // index keeps the compiler from hoisting them into 64 VGPRs)
        int ql = lane;
        asm volatile("" : "+v"(ql));
        // -- S^T = K Q^T (lane: row n, keys 4g+i of each 16-key half)
        f32x4 s[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) s[rt][0] = s[rt][1] = (f32x4)(0.0f);
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const f16x8 ka = nib_to_f16(kw[kh][c] ^ 0x88888888u, nk);
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    s[rt][kh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, s_q[rt][c][0][ql], s[rt][kh], 0, 0, 0);
                    s[rt][kh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, s_q[rt][c][1][ql], s[rt][kh], 0, 0, 0);
                }
            }

        // -- V^T operands (positions 8g..8g+7 = the lane's keys), exponent of P~
        float svmax = 0.0f;
#pragma unroll
        for (int p = 0; p < 8; p++) svmax = fmaxf(svmax, fabsf(sv[p]));
        svmax = fmaxf(svmax, __shfl_xor(svmax, 16));
        svmax = fmaxf(svmax, __shfl_xor(svmax, 32));
        // P~ = P * s_v * 2^ev stays below 2^15; ev only ever decreases, so
        // rescaling O by 2^(ev - ev_cur) cannot overflow
        int ev = 0;
        if (svmax > 0.0f && svmax < __builtin_inff()) ev = 14 - ilogbf(svmax);
        ev = ev > 60 ? 60 : (ev < -60 ? -60 : ev);
        if (!first && ev > ev_cur) ev = ev_cur;
        const float evup = ldexpf(1.0f, ev);
        const float evshift = first ? 1.0f : ldexpf(1.0f, ev - ev_cur);
        ev_cur = ev;
        float svup[8];
#pragma unroll
        for (int p = 0; p < 8; p++) svup[p] = sv[p] * evup;
#pragma unroll
        for (int p = 0; p < 8; p++) vw[p] ^= 0x88888888u;

        f16x8 ph[RT], pl[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            // scores, mask, online softmax for row (rt, n)
            float val[8];
            float tmax = -__builtin_inff();
            if (open) {
                // rows past R score 0 against their zeroed Q and are never stored
#pragma unroll
                for (int p = 0; p < 8; p++) {
                    val[p] = s[rt][p >> 2][p & 3] * qinv[rt] * sk[p];
                    tmax = fmaxf(tmax, val[p]);
                }
            } else {
#pragma unroll
                for (int p = 0; p < 8; p++) {
                    const int kk = kt + key_of_pos(g, p);
                    const bool exists = kk < k_end;
                    // keys <= lim_row are visible; a tree row also sees its
                    // ancestors among the new keys
                    const unsigned rel = (unsigned)(kk - base);
                    const bool anc_bit = rel < 64u && ((anc_row[rt] >> (rel & 63u)) & 1ull);
                    const bool vis = rok[rt] && (kk <= lim_row[rt] || anc_bit);
                    const float sc = s[rt][p >> 2][p & 3] * qinv[rt] * sk[p];
                    val[p] = !exists ? -__builtin_inff() : (vis ? sc : -FLT_MAX);
                    tmax = fmaxf(tmax, val[p]);
                }
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float m_new = fmaxf(m_run[rt], tmax);
            const float alpha = m_new == -__builtin_inff() ? 1.0f : __expf(m_run[rt] - m_new);
            m_run[rt] = m_new;
            float psum = 0.0f;
#pragma unroll
            for (int p = 0; p < 8; p++) {
                const float pv = m_new == -__builtin_inff() ? 0.0f : __expf(val[p] - m_new);
                psum += pv;
                _Float16 hi, lo;
                split16(pv * svup[p], hi, lo);
                ph[rt][p] = hi;
                pl[rt][p] = lo;
            }
            if (first) {
                l_part[rt] = psum;           // O is zero: nothing to rescale
            } else {
                l_part[rt] = l_part[rt] * alpha + psum;
                const float oscale = alpha * evshift;
#pragma unroll
                for (int t = 0; t < 8; t++) o[rt][t] *= oscale;
            }
        }
        // -- O^T += V^T P^T (tile t: head-dim columns 8m + t); the V^T operand
        //    of a tile serves every row tile
#pragma unroll
        for (int t = 0; t < 8; t++) {
            f16x8 va;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                f16x2 pr = nib_pair(vw[2 * j], vw[2 * j + 1], t, nk);
                va[2 * j] = pr[0];
                va[2 * j + 1] = pr[1];
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                o[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph[rt], o[rt][t], 0, 0, 0);
                o[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl[rt], o[rt][t], 0, 0, 0);
            }
        }
    };
    if (new_split) {
        // at most 64 new keys: one tile each for waves 0 and 1
        if (wave < ntiles) {
            load_tile_lds(k_begin + wave * kTile, td);
            process(td, wave);
        }
    } else {
        TileData tn;
        int tile = wave;
        for (; tile + kWaves < ntiles; tile += kWaves) {
            load_tile(k_begin + (tile + kWaves) * kTile, tn);
            process(td, tile);
            td = tn;
        }
        if (tile < ntiles) process(td, tile);
    }

    // ---- per wave: true-unit O, row max and sum -> LDS (s_o reuses the
    // bytes of s_q: every wave is past its last read of the Q operands)
    __syncthreads();
    const float oun = ldexpf(1.0f, -ev_cur);
    // rows of this block that exist (R may end inside it)
    const int nvalid = min(ROWS, R - row0);
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        float l = l_part[rt];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        const int row = 16 * rt + n;
        if (g == 0) {
            s_m[wave][row] = m_run[rt];
            s_l[wave][row] = l;
        }
        // lane holds O^T[m = 4g + i][row] of tile t: head-dim 8m + t, so for
        // each i its 8 tiles are 8 consecutive columns
        if (row < nvalid) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int d0 = 8 * (4 * g + i);
                if (d0 < D) {
                    float4* dst = (float4*)&s_o[wave][row][d0];
                    dst[0] = make_float4(o[rt][0][i] * oun, o[rt][1][i] * oun, o[rt][2][i] * oun,
                                         o[rt][3][i] * oun);
                    dst[1] = make_float4(o[rt][4][i] * oun, o[rt][5][i] * oun, o[rt][6][i] * oun,
                                         o[rt][7][i] * oun);
                }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < nvalid) {
        const int row = threadIdx.x;
        float M = -__builtin_inff();
#pragma unroll
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, s_m[w][row]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float wgt = s_m[w][row] == -__builtin_inff() ? 0.0f : __expf(s_m[w][row] - M);
            s_w[w][row] = wgt;
            L += s_l[w][row] * wgt;
        }
        s_M[row] = M;
        s_L[row] = L;
    }
    __syncthreads();
    // four consecutive columns per thread
    constexpr int kQuads = D / 4;
    const size_t nrow = (size_t)a.B * a.Nq * a.H;
    for (int e = threadIdx.x; e < nvalid * kQuads; e += 64 * kWaves) {
        const int row = e / kQuads, d = 4 * (e % kQuads);
        const int r = row0 + row;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float4 v = *(const float4*)&s_o[w][row][d];
            const float wg = s_w[w][row];
            acc.x += v.x * wg; acc.y += v.y * wg; acc.z += v.z * wg; acc.w += v.w * wg;
        }
        const int h = h0 + r / a.Nq, q = r % a.Nq;
        const size_t orow = orow0 + (size_t)q * a.H + h;
        if (a.splits == 1) {
            const float L = s_L[row];
            const float4 out = L > 0.0f ? make_float4(acc.x / L, acc.y / L, acc.z / L, acc.w / L)
                                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            *(float4*)&a.O[orow * D + d] = out;
            if (D == 128 && a.stats) {
                // a row's 32 quads are one half wave (rows start at multiples
                // of 32 threads), which reduces them by DPP
                float am = fmaxf(fmaxf(fabsf(out.x), fabsf(out.y)), fmaxf(fabsf(out.z), fabsf(out.w)));
                float ss = fmaf(out.w, out.w, fmaf(out.z, out.z, fmaf(out.y, out.y, out.x * out.x)));
                am = half_max_nonneg(am);
                ss = half_sum(ss);
                if ((threadIdx.x & 31) == 31) *(float2*)&a.stats[orow * 2] = make_float2(am, ss);
            }
        } else {
            *(float4*)&a.part_o[((size_t)split * nrow + orow) * D + d] = acc;
            if (d == 0) {
                *(float2*)&a.part_ml[((size_t)split * nrow + orow) * 2] =
                    make_float2(s_M[row], s_L[row]);
            }
        }
    }
}

// Merge the splits: one block per output row, one thread per head-dim value.
// Every split's (max, sum) pair is loaded at once into LDS; each thread then
// forms the maximum, the weights and the weighted sum in split order (the
// same fixed order for every column), and reads the partial rows eight splits
// at a time with independent loads.
// With stats (D == 128: two waves), also the row's (max|o|, sum o^2).
__global__ void k_attn_dec_combine(const float* __restrict__ part_o,
                                   const float* __restrict__ part_ml, int splits, int nrow,
                                   int D, float* __restrict__ O, float* __restrict__ stats) {
    const int row = blockIdx.x, d = threadIdx.x;
    __shared__ float s_m[128], s_l[128], s_w[128];
    for (int s = d; s < splits; s += blockDim.x) {
        const float2 ml = *(const float2*)(part_ml + ((size_t)s * nrow + row) * 2);
        s_m[s] = ml.x;
        s_l[s] = ml.y;
    }
    __syncthreads();
    float M = -__builtin_inff();
    for (int s = 0; s < splits; s++) M = fmaxf(M, s_m[s]);
    for (int s = d; s < splits; s += blockDim.x)
        s_w[s] = s_m[s] == -__builtin_inff() ? 0.0f : __expf(s_m[s] - M);
    __syncthreads();
    float L = 0.0f;
    for (int s = 0; s < splits; s++) L += s_l[s] * s_w[s];
    float acc = 0.0f;
    int s = 0;
    for (; s + 8 <= splits; s += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = part_o[((size_t)(s + j) * nrow + row) * D + d];
#pragma unroll
        for (int j = 0; j < 8; j++) acc += v[j] * s_w[s + j];
    }
    for (; s < splits; s++) acc += part_o[((size_t)s * nrow + row) * D + d] * s_w[s];
    const float o = L > 0.0f ? acc / L : 0.0f;
    O[(size_t)row * D + d] = o;
    if (!stats) return;
    float am = half_max_nonneg(fabsf(o)), ss = half_sum(o * o);
    // halves 0..3 (lanes 31, 63 of waves 0 and 1) -> s_m / s_l (free again)
    __syncthreads();
    if ((d & 31) == 31) {
        s_m[d >> 5] = am;
        s_l[d >> 5] = ss;
    }
    __syncthreads();
    if (d == 0)
        *(float2*)&stats[(size_t)row * 2] =
            make_float2(fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3])),
                        (s_l[0] + s_l[1]) + (s_l[2] + s_l[3]));
}

template <int D, int RT, bool FUSED = false>
int launch(const DecArgs& a, dim3 grid) {
    hipLaunchKernelGGL((k_attn_dec<D, RT, FUSED>), grid, dim3(64 * kWaves), 0, stream(), a);
    return launch_check("k_attn_dec");
}

}  // namespace

// 1 when the decode kernel takes this attention (INT4 cache, one scale group
// per head row, head_dim 32/64/128, chain / tree / no mask, batch 1).
extern "C" int cgk_attn_dec_supported(int D, int gs, int B, int mask_kind) {
    return (D == 32 || D == 64 || D == 128) && gs == D && B == 1 &&
           (mask_kind == kMaskNone || mask_kind == kMaskCausal || mask_kind == kMaskTree);
}

// Launch shape and launch of one call: rows per block (RT), key splits over
// the keys the splits stream (the cached keys when fused; the new keys are
// one more split), the split combine.  `a` holds the shape and pointers.
static int launch_dec(DecArgs& a, int nk_split_max, bool fused, float* O) {
    const int B = a.B, Nq = a.Nq, H = a.H, Hk = a.Hk, D = a.D_;
    const int R = (H / Hk) * Nq;
    // rows per block: 32 (RT = 2) dequantises each K/V tile once for both
    // 16-row halves, 16 (RT = 1) gives twice the blocks.  RT = 2 when RT = 1
    // would have more than 1024 block rounds of work.  Measured on the 7B head
    // shape (H 32, Hk 8, D 128), attention plus combine per call: the 5-row
    // chain at batch 1 (528 rounds) 14.1 us at RT = 1 against 16.6 at RT = 2;
    // batch 8 (4224) 33.6 against 39.8; the 64-node tree at batch 4 (8704)
    // 47.4 against 51.4.  The block targets were measured the same way.
    const int total_rounds = (a.Nk + kSplitKeys - 1) / kSplitKeys;
    const long rounds1 = (long)total_rounds * Hk * B * ((R + 15) / 16);
    const int RT = (R > 16 && rounds1 > 1024) ? 2 : 1;
    const int target_blocks = RT == 2 ? kTargetBlocks2 : kTargetBlocks1;
    const int chunks = (R + 16 * RT - 1) / (16 * RT);
    a.chunks = chunks;
    // keys per split: whole block rounds; about target_blocks blocks, at most
    // kMaxSplits splits before a split takes more rounds (rounded down, so a
    // context just past a multiple of the split size adds a split rather than
    // doubling every split); the splits follow the longest sequence, shorter
    // ones leave their last splits empty
    const int split_rounds = (nk_split_max + kSplitKeys - 1) / kSplitKeys;
    const int nrb = Hk * B * chunks;    // blocks of one split
    int maxsp = target_blocks / nrb;
    maxsp = maxsp < 1 ? 1 : (maxsp > kMaxSplits ? kMaxSplits : maxsp);
    const int rps = split_rounds / maxsp > 1 ? split_rounds / maxsp : 1;
    int kps = kSplitKeys * rps;
    while ((nk_split_max + kps - 1) / kps > 127) kps += kSplitKeys;
    const int nsplit = (nk_split_max + kps - 1) / kps;
    const int splits = fused ? nsplit + 1 : nsplit;
    a.nsplit_old = nsplit;
    a.splits = splits;
    a.keys_per_split = kps;
    a.O = O;
    const int nrow = B * Nq * H;
    if (splits > 1) {
        a.part_o = (float*)cgx_scratch(CGX_SLOT_WS2, (size_t)splits * nrow * D * 4);
        a.part_ml = (float*)cgx_scratch(CGX_SLOT_WS3, (size_t)splits * nrow * 2 * 4);
        if (!a.part_o || !a.part_ml) return -1;
    } else {
        a.part_o = a.part_ml = nullptr;
    }
    dim3 grid(splits, Hk, chunks * B);
    int rc;
    if (fused) {
        if (RT == 2) {
            if (D == 128) rc = launch<128, 2, true>(a, grid);
            else if (D == 64) rc = launch<64, 2, true>(a, grid);
            else rc = launch<32, 2, true>(a, grid);
        } else {
            if (D == 128) rc = launch<128, 1, true>(a, grid);
            else if (D == 64) rc = launch<64, 1, true>(a, grid);
            else rc = launch<32, 1, true>(a, grid);
        }
    } else if (RT == 2) {
        if (D == 128) rc = launch<128, 2>(a, grid);
        else if (D == 64) rc = launch<64, 2>(a, grid);
        else rc = launch<32, 2>(a, grid);
    } else {
        if (D == 128) rc = launch<128, 1>(a, grid);
        else if (D == 64) rc = launch<64, 1>(a, grid);
        else rc = launch<32, 1>(a, grid);
    }
    if (rc) return rc;
    if (splits > 1) {
        hipLaunchKernelGGL(k_attn_dec_combine, dim3(nrow), dim3(D), 0, stream(), a.part_o,
                           a.part_ml, splits, nrow, D, O, D == 128 ? a.stats : nullptr);
        if (launch_check("k_attn_dec_combine")) return -1;
    }
    return 0;
}

static int fill_args(DecArgs& a, const uint8_t* kc, const uint8_t* vc, const float* ks,
                     const float* vs, int B, const int* nk, size_t seq_kbytes,
                     size_t seq_groups, int Nq, int H, int Hk, int D, float scale,
                     int mask_kind, const unsigned long long* anc, int tw, int* nkmax_out) {
    int nkmax = 0, nkmin = 1 << 30;
    for (int b = 0; b < B && b < kMaxBatch; b++) {
        nkmax = nk[b] > nkmax ? nk[b] : nkmax;
        nkmin = nk[b] < nkmin ? nk[b] : nkmin;
    }
    if (mask_kind == kMaskTree && tw <= 0) tw = Nq;
    if (B < 1 || B > kMaxBatch || Nq <= 0 || nkmin < Nq || Hk <= 0 || H % Hk ||
        (mask_kind == kMaskTree && (Nq > 64 || !anc || tw < Nq || tw > 64 || nkmin < tw)) ||
        (D != 32 && D != 64 && D != 128)) {
        cgx_set_error("attn_dec: unsupported shape B=%d Nq=%d Nk=%d..%d H=%d Hk=%d D=%d", B, Nq,
                      nkmin, nkmax, H, Hk, D);
        return -1;
    }
    if (((uintptr_t)kc & 15) || (seq_kbytes & 15)) {
        cgx_set_error("attn_dec: the K cache must be 16-byte aligned");
        return -1;
    }
    memset(&a, 0, sizeof(a));
    a.kc = kc; a.vc = vc; a.ks = ks; a.vs = vs;
    a.Nq = Nq; a.Nk = nkmax; a.H = H; a.Hk = Hk; a.D_ = D;
    a.scale = scale;
    a.mask_kind = mask_kind;
    a.tw = mask_kind == kMaskTree ? tw : Nq;
    for (int i = 0; i < 64; i++) a.anc[i] = (mask_kind == kMaskTree && i < Nq) ? anc[i] : 0ull;
    a.B = B;
    a.seq_kbytes = seq_kbytes;
    a.seq_groups = seq_groups;
    for (int b = 0; b < kMaxBatch; b++) a.nk[b] = b < B ? nk[b] : 0;
    *nkmax_out = nkmax;
    return 0;
}

// Batched form: B sequences, each Nq query rows against its own cache
// (sequence b at kc + b * seq_kbytes, scales + b * seq_groups) of nk[b] keys.
extern "C" int cgk_attn_dec_batch(const float* Q, const uint8_t* kc, const uint8_t* vc,
                                  const float* ks, const float* vs, int B, const int* nk,
                                  size_t seq_kbytes, size_t seq_groups, int Nq, int H, int Hk,
                                  int D, float scale, int mask_kind,
                                  const unsigned long long* anc, int tw, float* O,
                                  float* stats) {
    DecArgs a;
    int nkmax;
    if (fill_args(a, kc, vc, ks, vs, B, nk, seq_kbytes, seq_groups, Nq, H, Hk, D, scale,
                  mask_kind, anc, tw, &nkmax))
        return -1;
    if (((uintptr_t)Q & 15) || ((uintptr_t)O & 15)) {
        cgx_set_error("attn_dec: Q, O and the K cache must be 16-byte aligned");
        return -1;
    }
    a.Q = Q;
    a.stats = D == 128 ? stats : nullptr;
    return launch_dec(a, nkmax, false, O);
}

// Fused RoPE, cache append and attention: qkv [B][Nq][ldq] are the raw
// projections of the step's rows (q heads, k heads, v heads), rope [B][Nq][D/2]
// the (cos, sin) of each row's rotary position (cgk_embed_rope); nk[b] counts
// the new keys, which this call rotates, quantises and writes to positions
// nk[b] - Nq .. nk[b] - 1 of the cache (one scale per head row).
extern "C" int cgk_attn_dec_rope(const float* qkv, int ldq, const float* rope, uint8_t* kc,
                                 uint8_t* vc, float* ks, float* vs, int B, const int* nk,
                                 size_t seq_kbytes, size_t seq_groups, int Nq, int H, int Hk,
                                 int D, float scale, int mask_kind,
                                 const unsigned long long* anc, int tw, float* O,
                                 float* stats) {
    DecArgs a;
    int nkmax;
    if (fill_args(a, kc, vc, ks, vs, B, nk, seq_kbytes, seq_groups, Nq, H, Hk, D, scale,
                  mask_kind, anc, tw, &nkmax))
        return -1;
    if (Nq > 64 || ((uintptr_t)qkv & 15) || (ldq & 3) || ((uintptr_t)rope & 15) ||
        ((uintptr_t)O & 15) || ldq < (H + 2 * Hk) * D) {
        cgx_set_error("attn_dec_rope: %d rows (at most 64), or qkv / rope / O not 16-byte "
                      "aligned with ldq %% 4 == 0", Nq);
        return -1;
    }
    a.qkv = qkv;
    a.ldq = ldq;
    a.rope = (const float2*)rope;
    a.kcw = kc; a.vcw = vc; a.ksw = ks; a.vsw = vs;
    a.stats = D == 128 ? stats : nullptr;
    int nk_old_max = 0;
    for (int b = 0; b < B; b++) nk_old_max = nk[b] - Nq > nk_old_max ? nk[b] - Nq : nk_old_max;
    return launch_dec(a, nk_old_max, true, O);
}

extern "C" int cgk_attn_dec(const float* Q, const uint8_t* kc, const uint8_t* vc, const float* ks,
                            const float* vs, int Nq, int Nk, int H, int Hk, int D, float scale,
                            int mask_kind, const unsigned long long* anc, float* O) {
    return cgk_attn_dec_batch(Q, kc, vc, ks, vs, 1, &Nk, 0, 0, Nq, H, Hk, D, scale, mask_kind,
                              anc, Nq, O, nullptr);
}
