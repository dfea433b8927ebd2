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

__device__ __forceinline__ float exp_glibc(float x) {
    if (!(x <= 0x1.62e42ep6f)) return x != x ? x + x : __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
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
    uint64_t t = kExp2Tab[ki & 31] + (ki << 47);
    double s = __longlong_as_double((long long)t);
    double z = fma(c0, r, c1);
    double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// ------------------------------------------------------ element generators

struct RowSrc {                 // raw fp32 row
    const float* p;
    __device__ float operator()(int j) const { return p[j]; }
};

template <class S>
struct ExpGen {                 // expf((src - m) / T), speculative.c:61
    S src;
    float m, T;
    __device__ float operator()(int j) const {
        return exp_glibc(__fdiv_rn(__fsub_rn(src(j), m), T));
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
    double q0, q1;               // increment (in ulps) for input parity 0 / 1
    int c0, c1;                  // output parity for input parity 0 / 1
};

__device__ __forceinline__ Mono mono_id() { return Mono{0.0, 0.0, 0, 1}; }

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

__device__ __forceinline__ SegMono seg_then(const SegMono& a, const SegMono& b) {
    SegMono r;
    r.flag = a.flag | b.flag;
    if (b.flag) {
        r.m = b.m;
        r.head = b.head;
    } else {
        r.m = mono_then(a.m, b.m);
        r.head = a.head;
    }
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

__device__ __forceinline__ double ulp_scale(int b) {   // 1 / ulp
    return b == -127 ? 0x1p149 : ldexp(1.0, 23 - b);
}

__device__ __forceinline__ double ulp_of(int b) {
    return b == -127 ? 0x1p-149 : ldexp(1.0, b - 23);
}

__device__ __forceinline__ int parity_of(float s, int b) {
    double n = (double)s * ulp_scale(b);
    return (int)((long long)n & 1);
}

struct EosShared {
    double wsum[kWaves];
    SegMono wseg[kWaves];
    Mono incl[kThreads];
    int binade[kThreads];
    int head[kThreads];
    int seg_last[kThreads];
    float cstart[kMaxRounds][kThreads];
    float cend[kMaxRounds][kThreads];
    float total;
    int result;
    float fval;
    float rval;
};

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
#pragma unroll
    for (int k = 0; k < kCh; k++) s = __fadd_rn(s, __shfl(x, k));
    return s;
}

// Exact ordered sum of g(0..n-1).  Leaves the exact running value at every
// chunk boundary in sh.cstart / sh.cend (rounds x threads) for gen_find.
template <class G>
__device__ __forceinline__ float eos_sum(const G& g, int n, EosShared& sh) {
    const int t = threadIdx.x;
    const int rounds = (n + kRound - 1) / kRound;
    float s_round = 0.0f;
    for (int rd = 0; rd < rounds; rd++) {
        const int base = rd * kRound + t * kCh;
        float x[kCh];
#pragma unroll
        for (int k = 0; k < kCh; k++) x[k] = (base + k < n) ? g(base + k) : 0.0f;

        // fp64 guide: exclusive / inclusive prefix of chunk sums
        double gs = 0.0;
#pragma unroll
        for (int k = 0; k < kCh; k++) gs += (double)x[k];
        double inc = gs;
        for (int d = 1; d < 64; d <<= 1) {
            double o = __shfl_up(inc, d);
            if (lane_id() >= d) inc += o;
        }
        if (lane_id() == 63) sh.wsum[wave_id()] = inc;
        __syncthreads();
        double wpre = 0.0;
        for (int w = 0; w < wave_id(); w++) wpre += sh.wsum[w];
        double p_end = (double)s_round + wpre + inc;
        double p_start = p_end - gs;
        double delta = (double)(t * kCh + kCh + 1) * 0x1p-24 * (1.0 + 0x1p-20) + 0x1p-40;
        double lo = t == 0 ? (double)s_round : p_start * (1.0 - delta);
        double hi = p_end * (1.0 + delta);
        int b = binade_of(lo);
        bool clean = binade_of(hi) == b;

        // own monoid element under binade b
        Mono own = mono_id();
        if (clean) {
            double sc = ulp_scale(b);
            int c0 = 0, c1 = 1;
            double q0 = 0.0, q1 = 0.0;
#pragma unroll
            for (int k = 0; k < kCh; k++) {
                double y = (double)x[k] * sc;
                double f = floor(y);
                double fr = y - f;
                if (fr == 0.5) {
                    int fo = (int)((long long)f & 1);
                    q0 += f + (double)((c0 ^ fo) & 1);
                    q1 += f + (double)((c1 ^ fo) & 1);
                    c0 = 0;
                    c1 = 0;
                } else {
                    double q = f + (fr > 0.5 ? 1.0 : 0.0);
                    int qo = (int)((long long)q & 1);
                    q0 += q;
                    q1 += q;
                    c0 ^= qo;
                    c1 ^= qo;
                }
            }
            own = Mono{q0, q1, c0, c1};
        }
        sh.binade[t] = clean ? b : kDirty;
        __syncthreads();
        bool is_head = !clean || t == 0 || sh.binade[t - 1] != b;
        SegMono v;
        v.m = clean ? own : mono_id();
        v.head = t;
        v.flag = is_head ? 1 : 0;
        for (int d = 1; d < 64; d <<= 1) {
            SegMono o = shfl_up_seg(v, d);
            if (lane_id() >= d) v = seg_then(o, v);
        }
        if (lane_id() == 63) sh.wseg[wave_id()] = v;
        __syncthreads();
        if (wave_id() > 0) {
            SegMono pre = sh.wseg[0];
            for (int w = 1; w < wave_id(); w++) pre = seg_then(pre, sh.wseg[w]);
            v = seg_then(pre, v);
        }
        sh.incl[t] = v.m;
        sh.head[t] = v.head;
        bool is_last = t == kThreads - 1 || sh.binade[t + 1] != sh.binade[t] ||
                       sh.binade[t] == kDirty;
        if (clean && is_last) sh.seg_last[v.head] = t;
        __syncthreads();

        // walk: one wave, segments in O(1), replayed chunks in order
        if (wave_id() == 0) {
            float s = s_round;
            int c = 0;
            while (c < kThreads) {
                int bc = sh.binade[c];
                if (bc != kDirty && binade_of((double)s) != bc) {
                    // cannot happen under the error bound; stay exact anyway
                    bc = kDirty;
                    int e = sh.seg_last[c];
                    for (int i = c; i <= e; i++) sh.binade[i] = kDirty;
                }
                if (bc == kDirty) {
                    if (lane_id() == 0) sh.cstart[rd][c] = s;
                    s = replay_chunk_wave(g, rd * kRound + c * kCh, n, s);
                    if (lane_id() == 0) sh.cend[rd][c] = s;
                    c++;
                } else {
                    int e = sh.seg_last[c];
                    if (lane_id() == 0) sh.cstart[rd][c] = s;
                    Mono me = sh.incl[e];
                    double q = parity_of(s, bc) ? me.q1 : me.q0;
                    s = (float)((double)s + q * ulp_of(bc));
                    c = e + 1;
                }
            }
            if (lane_id() == 0) sh.total = s;
        }
        __syncthreads();

        // exact chunk boundaries for every clean chunk
        int bt = sh.binade[t];
        if (bt != kDirty) {
            int h = sh.head[t];
            float sh0 = sh.cstart[rd][h];
            int par = parity_of(sh0, bt);
            Mono ex = (t == h) ? mono_id() : sh.incl[t - 1];
            double u = ulp_of(bt);
            double s0 = (double)sh0 + (par ? ex.q1 : ex.q0) * u;
            int par2 = par ? ex.c1 : ex.c0;
            double s1 = s0 + (par2 ? own.q1 : own.q0) * u;
            if (t != h) sh.cstart[rd][t] = (float)s0;
            sh.cend[rd][t] = (float)s1;
        }
        s_round = sh.total;
        __syncthreads();
    }
    return s_round;
}

// First i in [0, n) with r < (exact running sum through i); `dflt` if none.
// Must follow eos_sum over the same generator.
template <class G>
__device__ __forceinline__ int gen_find(const G& g, int n, float r, int dflt, EosShared& sh) {
    const int t = threadIdx.x;
    const int rounds = (n + kRound - 1) / kRound;
    if (t == 0) sh.result = dflt;
    __syncthreads();
    for (int rd = 0; rd < rounds; rd++) {
        float s0 = sh.cstart[rd][t], s1 = sh.cend[rd][t];
        // the first chunk also takes r below its start (r < 0)
        if ((!(r < s0) || (rd == 0 && t == 0)) && (r < s1)) {
            int base = rd * kRound + t * kCh;
            float s = s0;
            for (int k = 0; k < kCh && base + k < n; k++) {
                s = __fadd_rn(s, g(base + k));
                if (r < s) {
                    sh.result = base + k;
                    break;
                }
            }
        }
    }
    __syncthreads();
    int res = sh.result;
    __syncthreads();
    return res;
}

// gen_find that also returns the exact running sum through the found index
// (`*val`); {dflt, total} when no index qualifies.  Must follow eos_sum over
// the same generator, whose result is `total`.
template <class G>
__device__ __forceinline__ int gen_find_val(const G& g, int n, float r, int dflt, float total,
                                            float* val, EosShared& sh) {
    const int t = threadIdx.x;
    const int rounds = (n + kRound - 1) / kRound;
    if (t == 0) {
        sh.result = dflt;
        sh.rval = total;
    }
    __syncthreads();
    for (int rd = 0; rd < rounds; rd++) {
        float s0 = sh.cstart[rd][t], s1 = sh.cend[rd][t];
        // the first chunk also takes r below its start (r < 0)
        if ((!(r < s0) || (rd == 0 && t == 0)) && (r < s1)) {
            int base = rd * kRound + t * kCh;
            float s = s0;
            for (int k = 0; k < kCh && base + k < n; k++) {
                s = __fadd_rn(s, g(base + k));
                if (r < s) {
                    sh.result = base + k;
                    sh.rval = s;
                    break;
                }
            }
        }
    }
    __syncthreads();
    int res = sh.result;
    *val = sh.rval;
    __syncthreads();
    return res;
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

// cg_sample_temperature on the values of `src` (speculative.c:54-75).
template <class S>
__device__ __forceinline__ int sample_temperature_gen(const S& src, int V, float T, float u,
                                      EosShared& sh) {
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

}  // namespace
