// eos.hpp -- the two exactness building blocks of the samplers, shared by
// accept.hip and filter.hip (both compiled with -ffp-contract=off):
//
//  1. exp_glibc(): expf evaluated exactly as glibc >= 2.28 does on x86-64
//     with FMA (the table-driven method of ARM's optimized-routines).
//  2. Exact ordered summation ("EOS"): the value of `s = 0; for i: s += x[i]`
//     in binary32 round-to-nearest-even for non-negative x, computed by a
//     1024-thread workgroup, with find-first queries on the running sum.
//
// Header-only; everything has internal linkage in each including file.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kCh = 32;                      // elements per thread per round
constexpr int kRound = kThreads * kCh;       // 32768 elements per round
constexpr int kMaxRounds = 8;                // rows up to 262144 elements
constexpr int kDirty = -1000;                // binade marker of a replayed chunk
constexpr int kDirtySlots = 96;              // dirty chunks staged in LDS per round

// ------------------------------------------------------------ exact expf

// 2^(i/32) rounded to binary64, stored minus (i << 47) so that adding
// (k << 47) for an integer k yields the bits of 2^(k/32).
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
    0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
    0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
    0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
    0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
    0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// Branch-free: the main path runs on the argument clamped into the range
// where it applies and the out-of-range results are selected afterwards, so
// several evaluations can be in flight in one thread.
// tab: kExp2Tab, or a copy of it (a workgroup's copy in LDS reads faster
// than the constant table at a lane-dependent index)
__device__ __forceinline__ float exp_glibc_t(float x, const uint64_t* tab) {
    const bool over = !(x <= 0x1.62e42ep6f);       // NaN included
    const bool under = x < -0x1.9fe368p6f;
    const float special = x != x ? x + x : (over ? __builtin_inff() : 0.0f);
    x = fminf(fmaxf(x, -0x1.9fe368p6f), 0x1.62e42ep6f);
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    double r = fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki & 31] + (ki << 47);
    double s = __longlong_as_double((long long)t);
    double z = fma(c0, r, c1);
    double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return over || under ? special : (float)y;
}

__device__ __forceinline__ float exp_glibc(float x) { return exp_glibc_t(x, kExp2Tab); }

// ------------------------------------------------- fast, certified expf
// exp(x) for x in [kExpFastMin, 0]: x log2(e) = n + f by a two-part
// Cody-Waite reduction in fp32, 2^f by v_exp_f32, times 2^n exactly.  Its
// distance to exp_glibc(x) is at most kExpFastRel * exp_glibc(x) over that
// whole range (checked on every fp32 input by the GPU test of
// cgx_exp_fast_maxerr_dev); outside it the samplers use exp_glibc itself.
constexpr float kExpFastMin = -87.0f;
constexpr float kExpFastRel = 0x1p-20f;

__device__ __forceinline__ float exp_fast(float x) {
    const float kL2eHi = 0x1.715476p+0f;        // log2(e) rounded to fp32
    const float kL2eLo = 0x1.4ae0bep-26f;       // log2(e) - kL2eHi
    const float n = rintf(x * kL2eHi);
    const float f = fmaf(x, kL2eLo, fmaf(x, kL2eHi, -n));
    return ldexpf(__builtin_amdgcn_exp2f(f), (int)n);
}

// A cheaper exp(x) for x in [kExpFastMin, 0], for sums that only feed
// bounds: 2^(x log2(e)) by v_exp_f32 on the rounded product (no reduction;
// the product's rounding, up to 2^-18 in the exponent at |x| = 87, dominates
// the error).  Its distance to exp_glibc(x) is at most kExpStatRel *
// exp_glibc(x) over that range (checked on every fp32 input by the GPU test
// of cgx_exp_stat_maxerr_dev, with a factor-2 margin).
constexpr float kExpStatRel = 0x1p-16f;

__device__ __forceinline__ float exp_stat(float x) {
    return __builtin_amdgcn_exp2f(x * 0x1.715476p+0f);
}

// exp of x as cogito computes it (exp_glibc), or its certified approximation
__device__ __forceinline__ float exp_cert(float x) {
    return (x >= kExpFastMin && x <= 0.0f) ? exp_fast(x) : exp_glibc(x);
}

// Absolute error bounds, relative to the approximation, of
//   e~ = exp_cert(a)                        against expf(a)
//   p~ = e~ * fl(1 / S)                     against fl(expf(a) / S)
//   r~ = max(0, p~ - q~) (fp32 subtraction) against max(0, fl(p - q))
// (exp_cert within 2^-20; each fp32 rounding adds at most 2^-24)
constexpr float kExpErr = kExpFastRel * (1.0f + 0x1p-10f);
constexpr float kProbRel = kExpFastRel * (1.0f + 0x1p-10f) + 0x1p-21f;
constexpr float kResRel = kProbRel + 0x1p-21f;
// the same with exp_stat in place of exp_cert (sums that feed only bounds)
constexpr float kStatProbRel = kExpStatRel * (1.0f + 0x1p-10f) + 0x1p-21f;
constexpr float kStatResRel = kStatProbRel + 0x1p-21f;

// ------------------------------------------------------ element generators

struct RowSrc {                 // raw fp32 row
    const float* p;
    __device__ float operator()(int j) const { return p[j]; }
};

struct ScaledSrc {              // row / T (the filtered distribution's first step)
    const float* p;
    float T;
    __device__ float operator()(int j) const { return T == 1.0f ? p[j] : __fdiv_rn(p[j], T); }
};

template <class S>
struct ExpGen {                 // expf((src - m) / T), speculative.c:61
    S src;
    float m, T;
    __device__ float operator()(int j) const {
        const float d = __fsub_rn(src(j), m);
        return exp_glibc(T == 1.0f ? d : __fdiv_rn(d, T));   // d / 1 == d exactly
    }
};

template <class G>
struct DivGen {                 // g / S, speculative.c:64
    G g;
    float S;
    __device__ float operator()(int j) const { return __fdiv_rn(g(j), S); }
};

template <class A, class B>
struct ResidualGen {            // fmaxf(0, p - q), speculative.c:153
    A p;
    B q;
    __device__ float operator()(int j) const { return fmaxf(0.0f, __fsub_rn(p(j), q(j))); }
};

// --------------------------------------------------------- block helpers

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

struct Mono {                    // effect of a run of additions on (n, parity)
    int q0, q1;                  // increment (in ulps) for input parity 0 / 1; a run
                                 // stays in one binade, so under 2^24
    int c0, c1;                  // output parity for input parity 0 / 1
};

__device__ __forceinline__ Mono mono_id() { return Mono{0, 0, 0, 1}; }

__device__ __forceinline__ Mono mono_then(const Mono& a, const Mono& b) {
    Mono r;
    r.q0 = a.q0 + (a.c0 ? b.q1 : b.q0);
    r.c0 = a.c0 ? b.c1 : b.c0;
    r.q1 = a.q1 + (a.c1 ? b.q1 : b.q0);
    r.c1 = a.c1 ? b.c1 : b.c0;
    return r;
}

struct SegMono {
    Mono m;
    int head;                    // chunk index of the segment's first chunk
    int flag;                    // a segment starts inside this range
};

// Field-wise selects throughout: a conditional copy of the whole struct is
// not split into registers by the compiler and goes through scratch memory.
__device__ __forceinline__ SegMono seg_then(const SegMono& a, const SegMono& b) {
    const Mono ab = mono_then(a.m, b.m);
    const bool f = b.flag != 0;
    SegMono r;
    r.m.q0 = f ? b.m.q0 : ab.q0;
    r.m.q1 = f ? b.m.q1 : ab.q1;
    r.m.c0 = f ? b.m.c0 : ab.c0;
    r.m.c1 = f ? b.m.c1 : ab.c1;
    r.head = f ? b.head : a.head;
    r.flag = a.flag | b.flag;
    return r;
}

__device__ __forceinline__ SegMono seg_pick(bool c, const SegMono& a, const SegMono& b) {
    SegMono r;
    r.m.q0 = c ? a.m.q0 : b.m.q0;
    r.m.q1 = c ? a.m.q1 : b.m.q1;
    r.m.c0 = c ? a.m.c0 : b.m.c0;
    r.m.c1 = c ? a.m.c1 : b.m.c1;
    r.head = c ? a.head : b.head;
    r.flag = c ? a.flag : b.flag;
    return r;
}

__device__ __forceinline__ SegMono shfl_up_seg(const SegMono& v, int d) {
    SegMono o;
    o.m.q0 = __shfl_up(v.m.q0, d);
    o.m.q1 = __shfl_up(v.m.q1, d);
    o.m.c0 = __shfl_up(v.m.c0, d);
    o.m.c1 = __shfl_up(v.m.c1, d);
    o.head = __shfl_up(v.head, d);
    o.flag = __shfl_up(v.flag, d);
    return o;
}

// binade index of a non-negative value: floor(log2 v) for normal binary32
// magnitudes, -127 for the subnormal range [0, 2^-126) (one "binade" whose
// ulp is 2^-149 and which contains 0).
__device__ __forceinline__ int binade_of(double v) {
    if (v < 0x1p-126) return -127;
    return ilogb(v);
}

// The same for a binary32 value, from its bits: the exponent field minus the
// bias (zero and subnormals: -127); +inf, NaN and negative values lie in no
// binade.
__device__ __forceinline__ int binade_bits(float s) {
    const int e = (int)(__float_as_uint(s) >> 23);
    return e >= 255 ? 0x7fffffff : e - 127;
}

// Inside binade b the bits of a non-negative binary32 value are its count of
// ulps u_b plus a constant, so for s in b: the parity of s / u_b is the low
// bit, and s + q u_b (while it stays in b) is the bit pattern plus q.
__device__ __forceinline__ unsigned parity_bits(float s) { return __float_as_uint(s) & 1u; }
__device__ __forceinline__ float add_ulps(float s, int q) {
    return __uint_as_float(__float_as_uint(s) + (unsigned)q);
}

struct EosShared {
    double wsum[kWaves];
    SegMono wseg[kWaves];
    SegMono wpre[kWaves];        // wave w: aggregate of waves 0..w-1
    Mono incl[kThreads];
    int binade[kThreads];
    int head[kThreads];
    int seg_last[kThreads];
    float cstart[kMaxRounds][kThreads];
    float cend[kMaxRounds][kThreads];
    int item_c[kThreads];        // walk items: first chunk of each segment / dirty chunk
    int wcount[kWaves];
    int n_items;
    int dirty_slot[kThreads];    // staging slot of a dirty chunk (-1: none)
    alignas(16) float dirty_vals[kDirtySlots][kCh];
    float total;
    int result;
    float fval;
    float rval;
};

// Row staging for stores.  A thread's chunk is kCh consecutive elements, so
// writing it straight to memory makes every store instruction write 64
// partial cache lines (one per lane).  Instead a row of at most kRound values
// moves from the chunks to lane-consecutive positions through LDS (each wave
// its own 64 chunks, with a pitch of kCh + 1 floats so the lanes' writes
// along their chunks and the wave's reads of 64 consecutive values fall in
// distinct banks) and is stored 256 contiguous bytes per instruction.  The
// staging area overlaps EosShared (EosLds): it is used only where no EOS
// state is live, behind barriers on both sides.
constexpr int kTrPitch = kCh + 1;
constexpr int kTrWave = 64 * kTrPitch;

union EosLds {
    EosShared sh;
    float tr[kWaves * kTrWave];
};

// p[t*kCh + k] = q[k] for the elements below n (n <= kRound).
__device__ __forceinline__ void store_vals(float* p, int n, const float (&q)[kCh], float* tr) {
    const int l = lane_id(), w = wave_id();
    const int wb = w * 64 * kCh;
    float* tw = tr + w * kTrWave;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kCh; k++) tw[l * kTrPitch + k] = q[k];
    // a wave reads back only its own area, and one wave's LDS accesses
    // complete in order
#pragma unroll
    for (int i = 0; i < kCh; i++) {
        const int e = 64 * i + l;
        if (wb + e < n) p[wb + e] = tw[(e / kCh) * kTrPitch + e % kCh];
    }
    __syncthreads();
}

__device__ __forceinline__ float block_max_f(float v, EosShared& sh) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    __syncthreads();
    if (lane_id() == 0) sh.cend[0][wave_id()] = v;
    __syncthreads();
    float r = sh.cend[0][0];
    for (int w = 1; w < kWaves; w++) r = fmaxf(r, sh.cend[0][w]);
    __syncthreads();
    return r;
}

template <class G>
__device__ __forceinline__ float gen_max(const G& g, int n, EosShared& sh) {
    // max scan of speculative.c:55-56 (the value; -0/+0 ties do not change
    // any later result)
    float v = -__builtin_inff();
    for (int j = threadIdx.x; j < n; j += kThreads) v = fmaxf(v, g(j));
    return block_max_f(v, sh);
}

// Sequential replay of one chunk by the walker wave: lanes evaluate the 32
// elements in parallel, then the adds run in order.
template <class G>
__device__ __forceinline__ float replay_chunk_wave(const G& g, int base, int n, float s) {
    int j = base + lane_id();
    float x = (lane_id() < kCh && j < n) ? g(j) : 0.0f;
    // lane k's value straight into a scalar operand: only the adds are serial
#pragma unroll
    for (int k = 0; k < kCh; k++)
        s = __fadd_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k)));
    return s;
}

__device__ __forceinline__ double readlane_f64(double v, int k) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), k);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), k);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// ----------------------------------------------------- DPP wave scans
// Inclusive scans over the 64 lanes with DPP: row_shr 1, 2, 4, 8 inside each
// row of 16 lanes, then row_bcast:15 and row_bcast:31 across rows.  Data only
// flows from lower to higher lanes, so non-commutative operators are fine.
template <int CTRL, int RMASK>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, RMASK, 0xF, false);
}
template <int CTRL, int RMASK>
__device__ __forceinline__ double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = dpp_i<CTRL, RMASK>((int)(b & 0xffffffffll));
    const int hi = dpp_i<CTRL, RMASK>((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
// lane receives a value at this step of the scan
__device__ __forceinline__ bool dpp_step_valid(int step) {
    const int l = lane_id();
    switch (step) {
        case 0: return (l & 15) >= 1;
        case 1: return (l & 15) >= 2;
        case 2: return (l & 15) >= 4;
        case 3: return (l & 15) >= 8;
        case 4: return (l >> 4) & 1;         // rows 1 and 3 from lane 15 / 47
        default: return l >= 32;             // rows 2 and 3 from lane 31
    }
}

__device__ __forceinline__ double wave_incl_sum_d(double x) {
    double o;
    o = dpp_d<0x111, 0xF>(x); if (dpp_step_valid(0)) x += o;
    o = dpp_d<0x112, 0xF>(x); if (dpp_step_valid(1)) x += o;
    o = dpp_d<0x114, 0xF>(x); if (dpp_step_valid(2)) x += o;
    o = dpp_d<0x118, 0xF>(x); if (dpp_step_valid(3)) x += o;
    o = dpp_d<0x142, 0xA>(x); if (dpp_step_valid(4)) x += o;
    o = dpp_d<0x143, 0xC>(x); if (dpp_step_valid(5)) x += o;
    return x;
}

template <int CTRL, int RMASK>
__device__ __forceinline__ SegMono dpp_seg(const SegMono& v) {
    SegMono o;
    o.m.q0 = dpp_i<CTRL, RMASK>(v.m.q0);
    o.m.q1 = dpp_i<CTRL, RMASK>(v.m.q1);
    o.m.c0 = dpp_i<CTRL, RMASK>(v.m.c0);
    o.m.c1 = dpp_i<CTRL, RMASK>(v.m.c1);
    o.head = dpp_i<CTRL, RMASK>(v.head);
    o.flag = dpp_i<CTRL, RMASK>(v.flag);
    return o;
}

__device__ __forceinline__ SegMono wave_incl_seg(SegMono v) {
    SegMono o;
    o = dpp_seg<0x111, 0xF>(v); v = seg_pick(dpp_step_valid(0), seg_then(o, v), v);
    o = dpp_seg<0x112, 0xF>(v); v = seg_pick(dpp_step_valid(1), seg_then(o, v), v);
    o = dpp_seg<0x114, 0xF>(v); v = seg_pick(dpp_step_valid(2), seg_then(o, v), v);
    o = dpp_seg<0x118, 0xF>(v); v = seg_pick(dpp_step_valid(3), seg_then(o, v), v);
    o = dpp_seg<0x142, 0xA>(v); v = seg_pick(dpp_step_valid(4), seg_then(o, v), v);
    o = dpp_seg<0x143, 0xC>(v); v = seg_pick(dpp_step_valid(5), seg_then(o, v), v);
    return v;
}

// Staged values of a dirty chunk, or the generator when it was not staged.
typedef float vf4 __attribute__((ext_vector_type(4)));

// s + v.x + v.y + v.z + v.w, in order (fp32)
__device__ __forceinline__ float add4(float s, vf4 v) {
    s = __fadd_rn(s, v.x);
    s = __fadd_rn(s, v.y);
    s = __fadd_rn(s, v.z);
    return __fadd_rn(s, v.w);
}

// A staged chunk: every lane reads all of it (one address: a broadcast) and
// runs the same additions in its own registers, so the serial chain carries
// no cross-lane moves.
template <class G>
__device__ __forceinline__ float replay_chunk_staged(const G& g, int slot, int base, int n,
                                                     float s, EosShared& sh) {
    if (slot < 0) return replay_chunk_wave(g, base, n, s);
    const vf4* p = (const vf4*)sh.dirty_vals[slot];
    vf4 v[kCh / 4];
#pragma unroll
    for (int i = 0; i < kCh / 4; i++) v[i] = p[i];
#pragma unroll
    for (int i = 0; i < kCh / 4; i++) s = add4(s, v[i]);
    return s;
}

// Monoid element of one chunk in binade b from exact values (fp32 / int32:
// y = x * 2^(23-b) is exact and below 2^24, so floor and fraction are exact).
template <class XF>
__device__ __forceinline__ Mono fold_chunk(XF xk, int b) {
    const int e = b == -127 ? 149 : 23 - b;
    // Without a tie (y exactly halfway between integers) every increment is
    // rint(y), whatever the running value; the increments are integers whose
    // running total stays below 2^24 (the run stays in one binade), so their
    // fp32 sum is exact.
    {
        float qs = 0.0f;
        bool tie = false;
#pragma unroll
        for (int k = 0; k < kCh; k++) {
            const float y = ldexpf(xk(k), e);
            const float r = rintf(y);
            tie |= fabsf(y - r) == 0.5f;
            qs += r;
        }
        if (!tie) {
            const int q = (int)qs;
            return Mono{q, q, q & 1, (q + 1) & 1};
        }
    }
    int c0 = 0, c1 = 1;
    int q0 = 0, q1 = 0;
#pragma unroll
    for (int k = 0; k < kCh; k++) {
        const float y = ldexpf(xk(k), e);
        const float f = floorf(y);
        const float fr = y - f;
        const int fi = (int)f;
        if (fr == 0.5f) {
            const int fo = fi & 1;
            q0 += fi + ((c0 ^ fo) & 1);
            q1 += fi + ((c1 ^ fo) & 1);
            c0 = 0;
            c1 = 0;
        } else {
            const int qi = fi + (fr > 0.5f ? 1 : 0);
            const int qo = qi & 1;
            q0 += qi;
            q1 += qi;
            c0 ^= qo;
            c1 ^= qo;
        }
    }
    return Mono{q0, q1, c0, c1};
}

// Segmented scan, walk and exact chunk boundaries of one round, shared by the
// exact and the certified front ends.  `own`/`clean`/`b` are this chunk's
// monoid element and binade; sh.binade, sh.dirty_slot and sh.dirty_vals are
// written and synchronised by the caller.
template <class G>
__device__ __forceinline__ float eos_tail(const Mono& own, bool clean, int b, const G& g, int rd,
                                          int n, float s_round, EosShared& sh) {
    const int t = threadIdx.x;
    // segmented scan of the monoid elements (segments = runs of one binade)
    const bool is_head = !clean || t == 0 || sh.binade[t - 1] != b;
    SegMono v;
    v.m = clean ? own : mono_id();
    v.head = t;
    v.flag = is_head ? 1 : 0;
    v = wave_incl_seg(v);
    if (lane_id() == 63) sh.wseg[wave_id()] = v;
    __syncthreads();
    // the waves' aggregates scanned by wave 0 (lane w: waves 0..w), so each
    // wave combines one exclusive prefix instead of looping over the waves
    // before it (chunk 0 heads wave 0's range: every prefix has a head)
    if (wave_id() == 0) {
        SegMono a{mono_id(), 0, 0};
        if (lane_id() < kWaves) {
            const SegMono& src = sh.wseg[lane_id()];
            a.m.q0 = src.m.q0;
            a.m.q1 = src.m.q1;
            a.m.c0 = src.m.c0;
            a.m.c1 = src.m.c1;
            a.head = src.head;
            a.flag = src.flag;
        }
        a = wave_incl_seg(a);
        if (lane_id() < kWaves - 1) sh.wpre[lane_id() + 1] = a;
    }
    __syncthreads();
    if (wave_id() > 0) v = seg_then(sh.wpre[wave_id()], v);
    sh.incl[t] = v.m;
    sh.head[t] = v.head;
    const bool is_last = t == kThreads - 1 || sh.binade[t + 1] != sh.binade[t] ||
                         sh.binade[t] == kDirty;
    if (clean && is_last) sh.seg_last[v.head] = t;

    // walk items: every dirty chunk, and the first chunk of every run of
    // clean chunks in one binade (the segment heads above), in order
    {
        const unsigned long long bal = __ballot(is_head);
        const int below = __popcll(bal & ((1ull << lane_id()) - 1ull));
        __syncthreads();
        if (lane_id() == 0) sh.wcount[wave_id()] = __popcll(bal);
        __syncthreads();
        int off = 0, tot = 0;
        for (int w = 0; w < kWaves; w++) {
            const int cw = sh.wcount[w];
            off += w < wave_id() ? cw : 0;
            tot += cw;
        }
        if (is_head) sh.item_c[off + below] = t;
        if (t == 0) sh.n_items = tot;
    }
    __syncthreads();

    // walk: one wave; each item's data sits in one lane and is read with
    // readlane, so the serial chain is only the running value
    if (wave_id() == 0) {
        float s = s_round;
        const int n_items = sh.n_items;
        for (int ib = 0; ib < n_items; ib += 64) {
            const int idx = ib + lane_id();
            const int my_c = idx < n_items ? sh.item_c[idx] : 0;
            const int my_b = sh.binade[my_c];
            const int my_e = my_b != kDirty ? sh.seg_last[my_c] : my_c;
            const int my_slot = sh.dirty_slot[my_c];
            int my_q0 = 0, my_q1 = 0;
            if (my_b != kDirty) {
                my_q0 = sh.incl[my_e].q0;
                my_q1 = sh.incl[my_e].q1;
            }
            const int cnt = n_items - ib < 64 ? n_items - ib : 64;
            for (int k = 0; k < cnt; k++) {
                const int c = __builtin_amdgcn_readlane(my_c, k);
                const int bc = __builtin_amdgcn_readlane(my_b, k);
                const int e = __builtin_amdgcn_readlane(my_e, k);
                if (bc == kDirty) {
                    if (lane_id() == 0) sh.cstart[rd][c] = s;
                    s = replay_chunk_staged(g, __builtin_amdgcn_readlane(my_slot, k),
                                            rd * kRound + c * kCh, n, s, sh);
                    if (lane_id() == 0) sh.cend[rd][c] = s;
                } else if (binade_bits(s) != bc) {
                    // a clean run whose start is not in the binade its chunks
                    // assumed (excluded by the error bound, handled exactly
                    // anyway): replay it chunk by chunk from the generator
                    for (int i = c; i <= e; i++) {
                        if (lane_id() == 0) {
                            sh.binade[i] = kDirty;
                            sh.cstart[rd][i] = s;
                        }
                        s = replay_chunk_wave(g, rd * kRound + i * kCh, n, s);
                        if (lane_id() == 0) sh.cend[rd][i] = s;
                    }
                } else {
                    if (lane_id() == 0) sh.cstart[rd][c] = s;
                    const int q0 = __builtin_amdgcn_readlane(my_q0, k),
                              q1 = __builtin_amdgcn_readlane(my_q1, k);
                    s = add_ulps(s, parity_bits(s) ? q1 : q0);
                }
            }
        }
        if (lane_id() == 0) sh.total = s;
    }
    __syncthreads();

    // exact chunk boundaries for every clean chunk
    const int bt = sh.binade[t];
    if (bt != kDirty) {
        const int h = sh.head[t];
        const float sh0 = sh.cstart[rd][h];
        const unsigned par = parity_bits(sh0);
        Mono ex = mono_id();
        if (t != h) {
            ex.q0 = sh.incl[t - 1].q0;
            ex.q1 = sh.incl[t - 1].q1;
            ex.c0 = sh.incl[t - 1].c0;
            ex.c1 = sh.incl[t - 1].c1;
        }
        // the run stays in binade bt, so every boundary is s + q ulps
        const float s0 = add_ulps(sh0, par ? ex.q1 : ex.q0);
        const int par2 = par ? ex.c1 : ex.c0;
        const float s1 = add_ulps(s0, par2 ? own.q1 : own.q0);
        if (t != h) sh.cstart[rd][t] = s0;
        sh.cend[rd][t] = s1;
    }
    const float total = sh.total;
    __syncthreads();
    return total;
}

// Binade of a chunk from the fp64 guide: [lo, hi] certainly contains the
// sequential running value throughout the chunk (err_pre/err_end: absolute
// error bounds of the guide values before / through this chunk).
__device__ __forceinline__ int guide_binade(double gs, double err_pre, double err_end,
                                            float s_round, EosShared& sh, bool* clean) {
    const int t = threadIdx.x;
    const double inc = wave_incl_sum_d(gs);
    if (lane_id() == 63) sh.wsum[wave_id()] = inc;
    __syncthreads();
    double wpre = 0.0;
    for (int w = 0; w < wave_id(); w++) wpre += sh.wsum[w];
    const double p_end = (double)s_round + wpre + inc;
    const double p_start = p_end - gs;
    // k sequential fp32 additions of non-negative values stay within
    // (1 +- 2^-24)^k <= 1 +- k 2^-24 (1 + 2^-7) of the real sum (k <= 2^15 + 33)
    const double delta = (double)(t * kCh + kCh + 1) * 0x1p-24 * (1.0 + 0x1p-7) + 0x1p-40;
    const double lo = t == 0 ? (double)s_round : (p_start - err_pre) * (1.0 - delta);
    const double hi = (p_end + err_end) * (1.0 + delta);
    const int b = binade_of(lo > 0.0 ? lo : 0.0);
    *clean = binade_of(hi) == b;
    return b;
}

// One round of the exact ordered sum: this thread's kCh values x (elements
// rd*kRound + t*kCh + k, zero past n), starting from the exact running value
// s_round.  Returns the exact value after the round; leaves the exact running
// value at every chunk boundary of the round in sh.cstart/sh.cend[rd].  `g`
// regenerates elements for the rare replays of chunks that were not staged.
template <class G>
__device__ __forceinline__ float eos_round(const float (&x)[kCh], const G& g, int rd, int n,
                                           float s_round, EosShared& sh) {
    const int t = threadIdx.x;
    double gs = 0.0;
#pragma unroll
    for (int k = 0; k < kCh; k++) gs += (double)x[k];
    bool clean;
    const int b = guide_binade(gs, 0.0, 0.0, s_round, sh, &clean);
    const Mono own = clean ? fold_chunk([&](int k) { return x[k]; }, b) : mono_id();
    sh.binade[t] = clean ? b : kDirty;

    // dirty chunks: stage their values for the walk (slots in chunk order)
    {
        const unsigned long long bal = __ballot(!clean);
        const int below = __popcll(bal & ((1ull << lane_id()) - 1ull));
        if (lane_id() == 0) sh.wcount[wave_id()] = __popcll(bal);
        __syncthreads();
        int off = 0;
#pragma unroll
        for (int w = 0; w < kWaves - 1; w++) off += w < wave_id() ? sh.wcount[w] : 0;
        const int slot = off + below;
        const bool staged = !clean && slot < kDirtySlots;
        sh.dirty_slot[t] = staged ? slot : -1;
        if (staged) {
#pragma unroll
            for (int k = 0; k < kCh; k++) sh.dirty_vals[slot][k] = x[k];
        }
    }
    __syncthreads();
    return eos_tail(own, clean, b, g, rd, n, s_round, sh);
}

// This thread's chunk g(base .. base + kCh - 1), zero past n.
template <class G>
__device__ __forceinline__ void chunk_vals(const G& g, int base, int n, float (&x)[kCh]) {
#pragma unroll
    for (int k = 0; k < kCh; k++) x[k] = (base + k < n) ? g(base + k) : 0.0f;
}

// raw rows: 16-byte loads when the chunk is whole and aligned (a lane's 32
// consecutive values in 8 loads rather than 32 strided ones)
__device__ __forceinline__ void chunk_vals(const RowSrc& g, int base, int n, float (&x)[kCh]) {
    if (base + kCh <= n && ((uintptr_t)(g.p + base) & 15u) == 0) {
        const float4* q = reinterpret_cast<const float4*>(g.p + base);
#pragma unroll
        for (int j = 0; j < kCh / 4; j++) {
            const float4 v = q[j];
            x[4 * j] = v.x;
            x[4 * j + 1] = v.y;
            x[4 * j + 2] = v.z;
            x[4 * j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < kCh; k++) x[k] = (base + k < n) ? g.p[base + k] : 0.0f;
    }
}

// Exact ordered sum of at most two chunks (n <= 64): one wave evaluates the
// elements (lane j: element j) and adds them in order with real fp32
// additions -- the reference's sum itself -- leaving the chunk boundaries as
// the general path does.
template <class G>
__device__ float eos_sum_small(const G& g, int n, EosShared& sh) {
    if (wave_id() == 0) {
        const int l = lane_id();
        const float x = l < n ? g(l) : 0.0f;
        float s = 0.0f;
        for (int c = 0; c * kCh < n; c++) {
            if (l == 0) sh.cstart[0][c] = s;
            const int end = min(n, (c + 1) * kCh);
            for (int j = c * kCh; j < end; j++)
                s = __fadd_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j)));
            if (l == 0) sh.cend[0][c] = s;
        }
        if (l == 0) sh.total = s;
    }
    __syncthreads();
    const float total = sh.total;
    __syncthreads();
    return total;
}

// Exact ordered sum of g(0..n-1).  Leaves the exact running value at every
// chunk boundary in sh.cstart / sh.cend (rounds x threads) for gen_find.
template <class G>
__device__ __forceinline__ float eos_sum(const G& g, int n, EosShared& sh) {
    if (n <= 2 * kCh) return eos_sum_small(g, n, sh);
    const int t = threadIdx.x;
    const int rounds = (n + kRound - 1) / kRound;
    float s_round = 0.0f;
    for (int rd = 0; rd < rounds; rd++) {
        float x[kCh];
        chunk_vals(g, rd * kRound + t * kCh, n, x);
        s_round = eos_round(x, g, rd, n, s_round, sh);
    }
    return s_round;
}

// Same for n <= kRound with this thread's values already in registers.
template <class G>
__device__ __forceinline__ float eos_sum_vals(const float (&x)[kCh], const G& g, int n,
                                              EosShared& sh) {
    if (n <= 2 * kCh) return eos_sum_small(g, n, sh);
    return eos_round(x, g, 0, n, 0.0f, sh);
}

// First i in [0, n) with r < (exact running sum through i); `dflt` if none.
// Must follow eos_sum over the same generator.  The running sum is
// non-decreasing, so at most one chunk has start <= r < end; one wave
// replays it (lanes evaluate, readlane feeds the serial adds).
template <class G>
__device__ __forceinline__ int gen_find_val(const G& g, int n, float r, int dflt, float total,
                                            float* val, EosShared& sh) {
    const int t = threadIdx.x;
    const int rounds = (n + kRound - 1) / kRound;
    if (t == 0) {
        sh.result = -1;
        sh.rval = total;
    }
    __syncthreads();
    for (int rd = 0; rd < rounds; rd++) {
        const float s0 = sh.cstart[rd][t], s1 = sh.cend[rd][t];
        const int base = rd * kRound + t * kCh;
        // the first chunk also takes r below its start (r < 0)
        if (base < n && (!(r < s0) || (rd == 0 && t == 0)) && (r < s1)) sh.result = rd * kThreads + t;
    }
    __syncthreads();
    const int hit = sh.result;
    if (wave_id() == 0) {
        int res = dflt;
        float rv = total;
        if (hit >= 0) {
            const int rd = hit / kThreads, c = hit % kThreads;
            const int base = rd * kRound + c * kCh;
            const int j = base + lane_id();
            const float x = (lane_id() < kCh && j < n) ? g(j) : 0.0f;
            float s = sh.cstart[rd][c];
            for (int k = 0; k < kCh && base + k < n; k++) {
                s = __fadd_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k)));
                if (r < s) {
                    res = base + k;
                    rv = s;
                    break;
                }
            }
        }
        if (lane_id() == 0) {
            sh.result = res;
            sh.rval = rv;
        }
    }
    __syncthreads();
    const int res = sh.result;
    *val = sh.rval;
    __syncthreads();
    return res;
}

template <class G>
__device__ __forceinline__ int gen_find(const G& g, int n, float r, int dflt, EosShared& sh) {
    float v;
    return gen_find_val(g, n, r, dflt, 0.0f, &v, sh);
}

// Broadcast g(j) for one index to the block.
template <class G>
__device__ __forceinline__ float gen_at(const G& g, int j, EosShared& sh) {
    if (threadIdx.x == 0) sh.fval = g(j);
    __syncthreads();
    float v = sh.fval;
    __syncthreads();
    return v;
}

// ------------------------------------------- single-round row helpers
// For rows of at most kRound elements each thread holds its kCh elements
// (t*kCh + k) in registers, so every pass after the first read works from
// registers; the values are bit-identical to the generators' (same
// operations in the same order).

// Row values of `src` for this thread (pad: elements past n).
template <class S>
__device__ __forceinline__ void load_vals(const S& src, int n, float pad, float (&x)[kCh]) {
    const int base = threadIdx.x * kCh;
#pragma unroll
    for (int k = 0; k < kCh; k++) x[k] = base + k < n ? src(base + k) : pad;
}

// raw rows: 16-byte loads where the thread's 32 elements are whole and aligned
__device__ __forceinline__ void load_vals(const RowSrc& src, int n, float pad, float (&x)[kCh]) {
    const int base = threadIdx.x * kCh;
    if (base + kCh <= n && ((uintptr_t)src.p & 15u) == 0) {
        const float4* q = reinterpret_cast<const float4*>(src.p + base);
#pragma unroll
        for (int j = 0; j < kCh / 4; j++) {
            const float4 v = q[j];
            x[4 * j] = v.x;
            x[4 * j + 1] = v.y;
            x[4 * j + 2] = v.z;
            x[4 * j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < kCh; k++) x[k] = base + k < n ? src.p[base + k] : pad;
    }
}

// scaled rows: the raw row's 16-byte loads, then the division (x / 1 == x)
__device__ __forceinline__ void load_vals(const ScaledSrc& src, int n, float pad,
                                          float (&x)[kCh]) {
    load_vals(RowSrc{src.p}, n, pad, x);
    if (src.T == 1.0f) return;
    const int base = threadIdx.x * kCh;
#pragma unroll
    for (int k = 0; k < kCh; k++) x[k] = base + k < n ? __fdiv_rn(x[k], src.T) : pad;
}

__device__ __forceinline__ float vals_max(const float (&x)[kCh], EosShared& sh) {
    float v = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < kCh; k++) v = fmaxf(v, x[k]);
    return block_max_f(v, sh);
}

// e = expf((x - m) / T) (ExpGen), zero past n
__device__ __forceinline__ void vals_exp(const float (&x)[kCh], float m, float T, int n,
                                         float (&e)[kCh]) {
    const int base = threadIdx.x * kCh;
    if (T == 1.0f) {   // d / 1 == d exactly: the division is skipped
#pragma unroll
        for (int k = 0; k < kCh; k++)
            e[k] = base + k < n ? exp_glibc(__fsub_rn(x[k], m)) : 0.0f;
        return;
    }
#pragma unroll
    for (int k = 0; k < kCh; k++)
        e[k] = base + k < n ? exp_glibc(__fdiv_rn(__fsub_rn(x[k], m), T)) : 0.0f;
}

// the value of element j (any thread's) broadcast to the block
__device__ __forceinline__ float vals_at(const float (&x)[kCh], int j, EosShared& sh) {
    if ((int)threadIdx.x == j / kCh) {
#pragma unroll
        for (int k = 0; k < kCh; k++)
            if (k == j % kCh) sh.fval = x[k];
    }
    __syncthreads();
    const float v = sh.fval;
    __syncthreads();
    return v;
}

// cg_sample_temperature on register values of a row (n <= kRound), `src`
// regenerating elements for replays.
template <class S>
__device__ __forceinline__ int sample_temperature_vals_m(const float (&x)[kCh], float m,
                                                         const S& src, int V, float T, float u,
                                                         EosShared& sh) {
    float e[kCh];
    vals_exp(x, m, T, V, e);
    ExpGen<S> eg{src, m, T};
    const float S_ = eos_sum_vals(e, eg, V, sh);
    DivGen<ExpGen<S>> pg{eg, S_};
#pragma unroll
    for (int k = 0; k < kCh; k++) e[k] = __fdiv_rn(e[k], S_);   // (0 / S = 0 past V)
    eos_sum_vals(e, pg, V, sh);
    return gen_find(pg, V, u, V - 1, sh);
}

// the same with the row maximum computed here
template <class S>
__device__ __forceinline__ int sample_temperature_vals(const float (&x)[kCh], const S& src, int V,
                                                       float T, float u, EosShared& sh) {
    return sample_temperature_vals_m(x, vals_max(x, sh), src, V, T, u, sh);
}

// cg_sample_temperature on the values of `src` (speculative.c:54-75).
template <class S>
__device__ __forceinline__ int sample_temperature_gen(const S& src, int V, float T, float u,
                                      EosShared& sh) {
    if (V <= kRound) {
        float x[kCh];
        load_vals(src, V, -__builtin_inff(), x);
        return sample_temperature_vals(x, src, V, T, u, sh);
    }
    float m = gen_max(src, V, sh);
    ExpGen<S> e{src, m, T};
    float S_ = eos_sum(e, V, sh);
    DivGen<ExpGen<S>> p{e, S_};
    eos_sum(p, V, sh);
    return gen_find(p, V, u, V - 1, sh);
}

// cg_sample_corrected on two probability sources (speculative.c:148-172).
template <class P, class Q>
__device__ __forceinline__ int sample_corrected_gen(const P& p, const Q& q, int V, float u,
                                    EosShared& sh) {
    ResidualGen<P, Q> r{p, q};
    float R = eos_sum(r, V, sh);
    if (R < 1e-10f) return sample_temperature_gen(p, V, 1.0f, u, sh);
    return gen_find(r, V, __fmul_rn(u, R), 0, sh);
}

// The same with both probability rows in registers (n <= kRound).
template <class P, class Q>
__device__ __forceinline__ int sample_corrected_vals(const float (&pv)[kCh], const float (&qv)[kCh],
                                                     const P& p, const Q& q, int V, float u,
                                                     EosShared& sh) {
    ResidualGen<P, Q> r{p, q};
    float rv[kCh];
#pragma unroll
    for (int k = 0; k < kCh; k++) rv[k] = fmaxf(0.0f, __fsub_rn(pv[k], qv[k]));
    const float R = eos_sum_vals(rv, r, V, sh);
    if (R < 1e-10f) return sample_temperature_vals(pv, p, V, 1.0f, u, sh);
    return gen_find(r, V, __fmul_rn(u, R), 0, sh);
}

}  // namespace
