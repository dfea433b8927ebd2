// accept.hip -- acceptance sampling for speculative decoding on gfx950,
// bit-identical to cogito's CPU samplers on the same logits and uniforms.
//
// Reference (cogito-ml/cogito, src/inference/speculative.c):
//   cg_acceptance_prob      :49-52   q < 1e-10 ? 1 : fminf(1, p / q)
//   cg_sample_temperature   :54-75   max; expf((l - max) / T); running fp32
//                                    sum; p /= sum; first i with u < cumsum
//   cg_sample_corrected     :148-172 r = fmaxf(0, p - q); running sum R;
//                                    R < 1e-10 -> cg_sample_temperature(p);
//                                    first i with u*R < cumsum(r)
//
// Two building blocks make the GPU results equal to the CPU's bit for bit:
//
//  1. exp_glibc(): expf evaluated exactly as glibc >= 2.28 does on x86-64
//     with FMA (the table-driven method of ARM's optimized-routines: x*N/ln2
//     = k + r, 2^(k/N) from a 32-entry table of 2^(i/32) rounded to binary64,
//     a cubic in r, one final rounding to binary32).  Checked exhaustively
//     against the host libm on [-104, 0] (tests/test_accept_oracle.py pins
//     the same formula on the CPU; tests/test_gpu_accept.py on the GPU).
//
//  2. Exact ordered summation ("EOS"): the value of the reference's loop
//     `s = 0; for i: s += x[i]` (binary32, round-to-nearest-even) for
//     non-negative x, computed in parallel.  While s stays inside one binade
//     [2^b, 2^(b+1)) every addition rounds to a multiple of u_b = 2^(b-23),
//     so s advances by the integer q_i = rne(x_i / u_b); only exact ties
//     depend on the running value, through its parity.  Each thread folds
//     its chunk of 32 elements into a 2-state monoid element (increment and
//     output parity for input parity 0 and 1); a block-wide segmented scan
//     composes them.  Chunks where s may cross a binade -- located with an
//     fp64 prefix sum and the rigorous bound |s_i - P_i| <= i*2^-24*s_i --
//     are replayed sequentially with real fp32 adds by one wave.  The walk
//     over segments and replayed chunks yields the exact running value at
//     every chunk boundary; a CDF search then replays one chunk.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cgx_internal.h"

#include "eos.hpp"

namespace {

inline hipStream_t stream() { return (hipStream_t)cgx_stream(); }

int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        cgx_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

// ------------------------------------------------------------- kernels

__global__ __launch_bounds__(kThreads) void k_exact_expf(const float* x, float* y, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = exp_glibc(x[i]);
}

// Largest relative distance between exp_fast and exp_glibc over every fp32
// in [lo, hi] (lo < hi <= 0), as an ordered-int max of the error's bits.
__global__ void k_exp_fast_maxerr(float lo, float hi, unsigned int* out) {
    // negative floats: the bit pattern grows with |x|; hi = 0 starts at -0.0
    const unsigned int ulo = __float_as_uint(hi) | 0x80000000u, uhi = __float_as_uint(lo);
    float worst = 0.0f;
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;
         i <= (unsigned long long)(uhi - ulo); i += (unsigned long long)gridDim.x * blockDim.x) {
        const float x = __uint_as_float(ulo + (unsigned int)i);
        const float g = exp_glibc(x), f = exp_fast(x);
        if (g > 0.0f) worst = fmaxf(worst, fabsf(f - g) / g);
    }
    atomicMax(out, __float_as_uint(worst));
}

// The same for exp_stat.
__global__ void k_exp_stat_maxerr(float lo, float hi, unsigned int* out) {
    const unsigned int ulo = __float_as_uint(hi) | 0x80000000u, uhi = __float_as_uint(lo);
    float worst = 0.0f;
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;
         i <= (unsigned long long)(uhi - ulo); i += (unsigned long long)gridDim.x * blockDim.x) {
        const float x = __uint_as_float(ulo + (unsigned int)i);
        const float g = exp_glibc(x), f = exp_stat(x);
        if (g > 0.0f) worst = fmaxf(worst, fabsf(f - g) / g);
    }
    atomicMax(out, __float_as_uint(worst));
}

__global__ __launch_bounds__(kThreads) void k_ordered_sum(const float* x, int n, float* out) {
    __shared__ EosShared sh;
    float s = eos_sum(RowSrc{x}, n, sh);
    if (threadIdx.x == 0) out[0] = s;
}

// ------------------------------------------- certified single-row draw
// cg_sample_temperature (speculative.c:54-75) returns the first k with
// u < C_k, C_k the binary32 running sum of p_j = fl(e_j / S), e_j =
// expf(a_j) and S the binary32 running sum of the e_j.  For a row held in
// registers the draw is first decided from approximations with rigorous
// bounds:
//   e~_j  exp_fast(a_j), within 2^-20 of e_j on [kExpFastMin, 0]; 0 below,
//         where e_j < 2^-125;
//   sums  fp32 within a thread (32 terms: within 31 * 2^-24 of the real
//         sum), fp64 across threads;
//   S     within B_S = sum_j min(e_j, h_S) of the real sum: a rounding to
//         nearest moves a sum by at most half an ulp of its result (h_S:
//         half an ulp of S's largest possible binade) and by at most the
//         term added;
//   C_k   within R_k = sum_{j<=k} min(p_j, h_C) of sum_{j<=k} p_j, each p_j
//         within 2^-24 p_j + 2^-150 of e_j / S.
// That gives an interval for every C_k.  With k the first index whose
// estimate exceeds u, the token is k once the interval of C_{k-1} lies at or
// below u and that of C_k above it (u at or above every estimate: V-1, once
// C_{V-2} is certainly <= u).  Anything else -- u within the bounds of a
// step, a non-finite row, an argument above 0 or NaN (T outside (0, inf]) --
// is decided by the exact sums.
//
// The bounds are worst cases of the running sums' roundings (up to about
// V 2^-24 of a sum on a diffuse row), so they settle u only where its CDF
// step is wider than that.  A gate sends rows whose expected step (sum of
// p^2, estimated from a quarter of the row) is below 8 V 2^-24 to the exact
// sums at once, from a cheap exponential (2^(d log2(e) / T), v_exp_f32) and
// one reduction: on diffuse rows (p ~ 1 / V) the bounds would settle only a
// few draws in a hundred.
struct CertShared {
    double ew[kWaves], mw[kWaves], bw[kWaves];
    float g1[kWaves], g2[kWaves];
    int cand;
    int tok;
};

// draws of k_sample_temperature(_rows) the exact sums decided (test statistics)
__device__ unsigned long long g_row_fallbacks;

__device__ __forceinline__ float wave_incl_sum_f(float x) {
    float o;
#define CGX_STEP(CTRL, RMASK, S)                                                     \
    o = __int_as_float(dpp_i<CTRL, RMASK>(__float_as_int(x)));                      \
    if (dpp_step_valid(S)) x += o;
    CGX_STEP(0x111, 0xF, 0)
    CGX_STEP(0x112, 0xF, 1)
    CGX_STEP(0x114, 0xF, 2)
    CGX_STEP(0x118, 0xF, 3)
    CGX_STEP(0x142, 0xA, 4)
    CGX_STEP(0x143, 0xC, 5)
#undef CGX_STEP
    return x;
}

// The token from the row's register values x (element t*kCh + k) and their
// maximum m; where the exact sums decide, -1 (the gate: x still holds the
// row) or -2 (after the certified pass, which no longer keeps x) --
// block-uniform.
__device__ __forceinline__ int sample_temperature_cert(const float (&x)[kCh], float m, int V,
                                                       float T, float u, CertShared& cs) {
    const int t = threadIdx.x, l = lane_id(), w = wave_id(), base = t * kCh;
    // gate, on every 4th element scaled by 4 plus the maximum's own term 1
    // (on the rows worth certifying a few top terms dominate the sum of
    // squares); padding: 2^-inf = 0; a non-finite m or T makes the sums NaN
    // or the arguments positive, which the certified pass rejects
    const float sc = 0x1.715476p+0f / T;
    float g1 = 0.0f, g2 = 0.0f;
#pragma unroll
    for (int k = 0; k < kCh; k += 4) {
        const float g = __builtin_amdgcn_exp2f(__fsub_rn(x[k], m) * sc);
        g1 += g;
        g2 = fmaf(g, g, g2);
    }
    g1 = wave_incl_sum_f(g1);
    g2 = wave_incl_sum_f(g2);
    if (l == 63) {
        cs.g1[w] = g1;
        cs.g2[w] = g2;
    }
    if (t == 0) cs.cand = 0x7fffffff;
    __syncthreads();
    float G1 = 0.0f, G2 = 0.0f;
    for (int i = 0; i < kWaves; i++) {
        G1 += cs.g1[i];
        G2 += cs.g2[i];
    }
    G1 = fmaf(4.0f, G1, 1.0f);
    G2 = fmaf(4.0f, G2, 1.0f);
    if (!(G2 * 0x1p24f >= 8.0f * (float)V * G1 * G1)) return -1;

    // the reference's arguments (x / 1 == x), their certified exponentials
    // and the thread's fp32 sum; an argument that is NaN or above 0 (a
    // non-finite row or T outside (0, inf]) sends the row to the exact path
    float e[kCh];
    float es = 0.0f;
    int bad = 0;
#pragma unroll
    for (int k = 0; k < kCh; k++) {
        const float d = __fsub_rn(x[k], m);
        const float a = T == 1.0f ? d : __fdiv_rn(d, T);
        const bool in = base + k < V;
        bad |= in && !(a <= 0.0f);
        e[k] = in && a >= kExpFastMin ? exp_fast(a) : 0.0f;
        es += e[k];
    }
    const double ein = wave_incl_sum_d((double)es);
    if (l == 63) cs.ew[w] = ein;
    if (__syncthreads_or(bad)) return -2;
    double eoff = 0.0, E = 0.0;
    for (int i = 0; i < kWaves; i++) {
        const double v = cs.ew[i];
        if (i < w) eoff += v;
        E += v;
    }
    const double ex0 = eoff + (ein - (double)es);   // sum of the e~ before this thread

    // Bounds that need only E (>= 1: the row maximum's term is exactly 1).
    // dl covers exp_fast (2^-20) and the fp32 sums (31 * 2^-24) with room for
    // the fp64 roundings; S and every C_k stay within a factor (1 +- V 2^-23)
    // of their real sums (V <= 2^15).
    const double Vd = (double)V, dl = 0x1p-18, abs_e = Vd * 0x1p-125;
    const double S_hi0 = (E * (1.0 + dl) + abs_e) * (1.0 + Vd * 0x1p-23);
    const double S_lo0 = E * (1.0 - dl) * (1.0 - Vd * 0x1p-23);
    const float hS = ldexpf(1.0f, binade_of(S_hi0) - 24);
    // p_j <= kap e~_j + 2^-124, so min(p_j, h_C) <= kap min(e~_j, tau) + 2^-124
    const double kap = (1.0 + dl) / S_lo0;
    const double C_hi0 = (kap * E * (1.0 + dl) + Vd * 0x1p-124) * (1.0 + Vd * 0x1p-23);
    const double hC = ldexp(1.0, binade_of(C_hi0) - 24);
    const float tau = (float)(hC / kap * (1.0 + 0x1p-22));   // >= hC / kap after rounding
    float ms = 0.0f, bs = 0.0f;
#pragma unroll
    for (int k = 0; k < kCh; k++) {
        ms += fminf(e[k], tau);
        bs += fminf(e[k], hS);
    }
    const double min_ = wave_incl_sum_d((double)ms);
    const double bin = wave_incl_sum_d((double)bs);
    // candidate: the first index whose estimate (prefix / E) exceeds u
    const double r = (double)u * E;
    if (base < V && ex0 + (double)es > r && (ex0 <= r || t == 0)) {
        float p = 0.0f;
        int kk = -1;
#pragma unroll
        for (int k = 0; k < kCh; k++) {
            p += e[k];
            if (kk < 0 && base + k < V && ex0 + (double)p > r) kk = k;
        }
        if (kk >= 0) atomicMin(&cs.cand, base + kk);
    }
    if (l == 63) {
        cs.mw[w] = min_;
        cs.bw[w] = bin;
    }
    __syncthreads();
    double moff = 0.0, B = 0.0;
    for (int i = 0; i < kWaves; i++) {
        if (i < w) moff += cs.mw[i];
        B += cs.bw[i];
    }
    const double mx0 = moff + (min_ - (double)ms);
    const int cand = cs.cand;
    const bool none = cand == 0x7fffffff;
    const int kc = none ? V - 1 : cand;
    if (t == kc / kCh) {
        const double BS = B * (1.0 + 0x1p-17) + abs_e;
        const double S_lo = E * (1.0 - dl) - BS, S_hi = E * (1.0 + dl) + abs_e + BS;
        // this thread's prefixes through kc - 1 and through kc (the same fp32
        // additions as above)
        const int kl = kc - base;
        float pe = 0.0f, pm = 0.0f, pe0 = 0.0f, pm0 = 0.0f, pe1 = 0.0f, pm1 = 0.0f;
#pragma unroll
        for (int k = 0; k < kCh; k++) {
            pe += e[k];
            pm += fminf(e[k], tau);
            if (k == kl - 1) {
                pe0 = pe;
                pm0 = pm;
            }
            if (k == kl) {
                pe1 = pe;
                pm1 = pm;
            }
        }
        const double Pe0 = ex0 + (double)pe0, Pm0 = mx0 + (double)pm0;
        const double Pe1 = ex0 + (double)pe1, Pm1 = mx0 + (double)pm1;
        const double n0 = (double)kc, n1 = n0 + 1.0;     // terms through kc - 1, kc
        const double kAbs = 0x1p-45;                     // the fp64 sums' absolute error
        const double R0 = kap * Pm0 * (1.0 + dl) + n0 * 0x1p-124;
        const double R1 = kap * Pm1 * (1.0 + dl) + n1 * 0x1p-124;
        const double up0 = (Pe0 * (1.0 + dl) + abs_e) * (1.0 + 0x1p-24) / S_lo * (1.0 + 0x1p-40) +
                           n0 * 0x1p-150 + R0 + kAbs;
        const double lo1 = Pe1 * (1.0 - dl) * (1.0 - 0x1p-24) / S_hi * (1.0 - 0x1p-40) -
                           n1 * 0x1p-150 - R1 - kAbs;
        const double ud = (double)u;
        const bool ok = (kc == 0 || up0 <= ud) && (none || lo1 > ud);
        cs.tok = ok ? kc : -2;
    }
    __syncthreads();
    return cs.tok;
}

// cg_sample_temperature on one row: certified decision first (cert) on rows
// held in registers, the exact sums where it does not settle the draw
__device__ __forceinline__ int sample_row(const float* logits, int V, float T, float u,
                                          int cert, EosShared& sh, CertShared& cs) {
    int tok;
    if (V <= kRound) {
        float x[kCh];
        load_vals(RowSrc{logits}, V, -__builtin_inff(), x);
        const float m = vals_max(x, sh);
        tok = cert ? sample_temperature_cert(x, m, V, T, u, cs) : -1;
        if (tok < 0) {
            if (cert && threadIdx.x == 0) atomicAdd(&g_row_fallbacks, 1ull);
            // the row again (L2-resident) where the certified pass let it go
            if (tok == -2) load_vals(RowSrc{logits}, V, -__builtin_inff(), x);
            tok = sample_temperature_vals_m(x, m, RowSrc{logits}, V, T, u, sh);
        }
    } else {
        tok = sample_temperature_gen(RowSrc{logits}, V, T, u, sh);
    }
    return tok;
}

__global__ __launch_bounds__(kThreads) void k_sample_temperature(const float* logits, int V,
                                                                 float T, float u, int cert,
                                                                 int* out) {
    __shared__ EosShared sh;
    __shared__ CertShared cs;
    const int tok = sample_row(logits, V, T, u, cert, sh, cs);
    if (threadIdx.x == 0) out[0] = tok;
}

// One block per row: row r at logits + r * ld, its draw u[r] (device)
__global__ __launch_bounds__(kThreads) void k_sample_temperature_rows(const float* logits,
                                                                      size_t ld, int V,
                                                                      float T, const float* u,
                                                                      int cert, int* out) {
    __shared__ EosShared sh;
    __shared__ CertShared cs;
    const int r = blockIdx.x;
    const int tok = sample_row(logits + (size_t)r * ld, V, T, u[r], cert, sh, cs);
    if (threadIdx.x == 0) out[r] = tok;
}

__global__ __launch_bounds__(kThreads) void k_sample_corrected(const float* q, const float* p,
                                                               int V, float u, int* out) {
    __shared__ EosShared sh;
    int tok = sample_corrected_gen(RowSrc{p}, RowSrc{q}, V, u, sh);
    if (threadIdx.x == 0) out[0] = tok;
}

__global__ __launch_bounds__(kThreads) void k_temperature_probs(const float* logits, int V,
                                                                float T, float* probs) {
    __shared__ EosShared sh;
    RowSrc src{logits};
    float m = gen_max(src, V, sh);
    ExpGen<RowSrc> e{src, m, T};
    float S_ = eos_sum(e, V, sh);
    for (int j = threadIdx.x; j < V; j += kThreads) probs[j] = __fdiv_rn(e(j), S_);
}

// One block per (position, chain).  Position i < gamma: target row i and
// draft row i -> acceptance ratio of the drafted token and, speculatively,
// the correction token with draw i+1.  Position gamma: the bonus token from
// target row gamma with draw gamma.
__global__ __launch_bounds__(kThreads) void k_verify_rows(
    const float* __restrict__ target, const float* __restrict__ draft,
    const int* __restrict__ tokens, const float* __restrict__ u, int gamma, int V,
    float T, float* __restrict__ accept_prob, int* __restrict__ correction,
    int* __restrict__ bonus) {
    __shared__ EosShared sh;
    const int pos = blockIdx.x, chain = blockIdx.y;
    const float* trow = target + ((size_t)chain * (gamma + 1) + pos) * V;
    const float* uu = u + (size_t)chain * (gamma + 1);
    if (pos == gamma) {
        int tok = sample_temperature_gen(RowSrc{trow}, V, T, uu[gamma], sh);
        if (threadIdx.x == 0) bonus[chain] = tok;
        return;
    }
    const float* drow = draft + ((size_t)chain * gamma + pos) * V;
    RowSrc ts{trow}, ds{drow};
    const int x = tokens[(size_t)chain * gamma + pos];
    if (V <= kRound) {
        // both rows in registers: one read of each row, one expf per element
        float tv[kCh], dv[kCh];
        load_vals(ts, V, -__builtin_inff(), tv);
        load_vals(ds, V, -__builtin_inff(), dv);
        const float mt = vals_max(tv, sh), md = vals_max(dv, sh);
        vals_exp(tv, mt, T, V, tv);
        vals_exp(dv, md, T, V, dv);
        ExpGen<RowSrc> et{ts, mt, T}, ed{ds, md, T};
        const float St = eos_sum_vals(tv, et, V, sh);
        const float Sd = eos_sum_vals(dv, ed, V, sh);
#pragma unroll
        for (int k = 0; k < kCh; k++) {
            tv[k] = __fdiv_rn(tv[k], St);
            dv[k] = __fdiv_rn(dv[k], Sd);
        }
        DivGen<ExpGen<RowSrc>> pt{et, St}, pd{ed, Sd};
        float a = 0.0f;   // a draft token outside [0, V) is rejected
        if (x >= 0 && x < V) {
            const float px = vals_at(tv, x, sh), qx = vals_at(dv, x, sh);
            a = qx < 1e-10f ? 1.0f : fminf(1.0f, __fdiv_rn(px, qx));
        }
        if (threadIdx.x == 0) accept_prob[(size_t)chain * gamma + pos] = a;
        const int tok = sample_corrected_vals(tv, dv, pt, pd, V, uu[pos + 1], sh);
        if (threadIdx.x == 0) correction[(size_t)chain * gamma + pos] = tok;
        return;
    }
    float mt = gen_max(ts, V, sh);
    float md = gen_max(ds, V, sh);
    ExpGen<RowSrc> et{ts, mt, T}, ed{ds, md, T};
    float St = eos_sum(et, V, sh);
    float Sd = eos_sum(ed, V, sh);
    DivGen<ExpGen<RowSrc>> pt{et, St}, pd{ed, Sd};
    float a = 0.0f;   // a draft token outside [0, V) is rejected
    if (x >= 0 && x < V) {
        float px = gen_at(pt, x, sh), qx = gen_at(pd, x, sh);
        a = qx < 1e-10f ? 1.0f : fminf(1.0f, __fdiv_rn(px, qx));
    }
    if (threadIdx.x == 0) accept_prob[(size_t)chain * gamma + pos] = a;
    int tok = sample_corrected_gen(pt, pd, V, uu[pos + 1], sh);
    if (threadIdx.x == 0) correction[(size_t)chain * gamma + pos] = tok;
}

// k_verify_rows over dense (filtered) distributions: one block per
// (position < gamma, chain); p rows [chain][gamma + 1][V] (the last row of a
// chain is not read), q rows [chain][gamma][V].
__global__ __launch_bounds__(kThreads) void k_verify_rows_dist(
    const float* __restrict__ p, const float* __restrict__ q, const int* __restrict__ tokens,
    const float* __restrict__ u, int gamma, int V, float* __restrict__ accept_prob,
    int* __restrict__ correction) {
    __shared__ EosShared sh;
    const int pos = blockIdx.x, chain = blockIdx.y;
    const size_t r = (size_t)chain * gamma + pos;
    RowSrc pt{p + ((size_t)chain * (gamma + 1) + pos) * V}, pd{q + r * V};
    int x = tokens[r];
    float a = 0.0f;   // a draft token outside [0, V) is rejected
    if (x >= 0 && x < V) {
        float px = pt(x), qx = pd(x);
        a = qx < 1e-10f ? 1.0f : fminf(1.0f, __fdiv_rn(px, qx));
    }
    if (threadIdx.x == 0) accept_prob[r] = a;
    const float ud = u[(size_t)chain * (gamma + 1) + pos + 1];
    int tok;
    if (V <= kRound) {
        // both rows in registers (16-byte loads), the residual formed there
        float pv[kCh], qv[kCh];
        load_vals(pt, V, 0.0f, pv);
        load_vals(pd, V, 0.0f, qv);
        tok = sample_corrected_vals(pv, qv, pt, pd, V, ud, sh);
    } else {
        tok = sample_corrected_gen(pt, pd, V, ud, sh);
    }
    if (threadIdx.x == 0) correction[r] = tok;
}

// First rejected position (u[i] < a[i] accepts, speculative.c draw order),
// then the emitted tokens.
__global__ void k_verify_combine(const int* __restrict__ tokens, const float* __restrict__ u,
                                 const float* __restrict__ accept_prob,
                                 const int* __restrict__ correction,
                                 const int* __restrict__ bonus, int gamma, int batch,
                                 int* __restrict__ out_tokens, int* __restrict__ n_accepted) {
    int chain = blockIdx.x * blockDim.x + threadIdx.x;
    if (chain >= batch) return;
    const float* uu = u + (size_t)chain * (gamma + 1);
    const float* a = accept_prob + (size_t)chain * gamma;
    const int* x = tokens + (size_t)chain * gamma;
    int* out = out_tokens + (size_t)chain * (gamma + 1);
    int n = gamma;
    for (int i = 0; i < gamma; i++) {
        if (!(uu[i] < a[i])) {
            n = i;
            break;
        }
        out[i] = x[i];
    }
    out[n] = n < gamma ? correction[(size_t)chain * gamma + n] : bonus[chain];
    for (int i = n + 1; i <= gamma; i++) out[i] = -1;
    n_accepted[chain] = n;
}

}  // namespace

// -------------------------------------------------------------- launchers

extern "C" int cgk_exp_fast_maxerr(float lo, float hi, unsigned int* out_dev) {
    if (!(lo < hi) || hi > 0.0f || lo < -104.0f) {
        cgx_set_error("exp_fast_maxerr: range must satisfy -104 <= lo < hi <= 0");
        return -1;
    }
    hipLaunchKernelGGL(k_exp_fast_maxerr, dim3(4096), dim3(256), 0, stream(), lo, hi, out_dev);
    return launch_check("k_exp_fast_maxerr");
}

extern "C" int cgk_exp_stat_maxerr(float lo, float hi, unsigned int* out_dev) {
    if (!(lo < hi) || hi > 0.0f || lo < kExpFastMin) {
        cgx_set_error("exp_stat_maxerr: range must satisfy %g <= lo < hi <= 0", kExpFastMin);
        return -1;
    }
    hipLaunchKernelGGL(k_exp_stat_maxerr, dim3(4096), dim3(256), 0, stream(), lo, hi, out_dev);
    return launch_check("k_exp_stat_maxerr");
}

extern "C" int cgk_exact_expf(const float* x, float* y, int n) {
    hipLaunchKernelGGL(k_exact_expf, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0,
                       stream(), x, y, n);
    return launch_check("k_exact_expf");
}

static int check_v(int V) {
    if (V <= 0 || V > kRound * kMaxRounds) {
        cgx_set_error("vocabulary size %d outside [1, %d]", V, kRound * kMaxRounds);
        return -1;
    }
    return 0;
}

extern "C" int cgk_ordered_sum(const float* x, int n, float* out) {
    if (check_v(n)) return -1;
    hipLaunchKernelGGL(k_ordered_sum, dim3(1), dim3(kThreads), 0, stream(), x, n, out);
    return launch_check("k_ordered_sum");
}

static int g_row_cert = 1;

// Certified decision of the single-row draws on (default) or off; returns the
// previous setting (-1 only reads it).
extern "C" int cgx_sample_row_certified(int on) {
    const int prev = g_row_cert;
    if (on >= 0) g_row_cert = on != 0;
    return prev;
}

// Single-row draws since the library loaded whose certified decision left
// the token to the exact sums (synchronises the library's stream).
extern "C" long long cgx_sample_row_fallbacks(void) {
    if (cgx_ensure_init()) return -1;
    unsigned long long v = 0;
    hipError_t e = hipStreamSynchronize(stream());
    if (e == hipSuccess)
        e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_row_fallbacks), sizeof v, 0,
                                hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        cgx_set_error("cgx_sample_row_fallbacks: %s", hipGetErrorString(e));
        return -1;
    }
    return (long long)v;
}

extern "C" int cgk_sample_temperature(const float* logits, int V, float T, float u,
                                      int* out) {
    if (check_v(V)) return -1;
    hipLaunchKernelGGL(k_sample_temperature, dim3(1), dim3(kThreads), 0, stream(), logits,
                       V, T, u, g_row_cert, out);
    return launch_check("k_sample_temperature");
}

extern "C" int cgk_sample_temperature_rows(const float* logits, int rows, int V, float T,
                                           const float* u, int* out, size_t ld) {
    if (check_v(V)) return -1;
    if (rows < 1 || (rows > 1 && ld < (size_t)V)) {
        cgx_set_error("sample rows: %d rows of %d values at stride %zu", rows, V, ld);
        return -1;
    }
    hipLaunchKernelGGL(k_sample_temperature_rows, dim3(rows), dim3(kThreads), 0, stream(),
                       logits, ld, V, T, u, g_row_cert, out);
    return launch_check("k_sample_temperature_rows");
}

extern "C" int cgk_sample_corrected(const float* q, const float* p, int V, float u,
                                    int* out) {
    if (check_v(V)) return -1;
    hipLaunchKernelGGL(k_sample_corrected, dim3(1), dim3(kThreads), 0, stream(), q, p, V,
                       u, out);
    return launch_check("k_sample_corrected");
}

extern "C" int cgk_temperature_probs(const float* logits, int V, float T, float* probs) {
    if (check_v(V)) return -1;
    hipLaunchKernelGGL(k_temperature_probs, dim3(1), dim3(kThreads), 0, stream(), logits, V,
                       T, probs);
    return launch_check("k_temperature_probs");
}

extern "C" int cgk_verify_chain(const float* target, const float* draft, const int* tokens,
                                const float* u, int batch, int gamma, int V, float T,
                                float* accept_prob, int* correction, int* bonus,
                                int* out_tokens, int* n_accepted) {
    if (check_v(V)) return -1;
    if (gamma < 1 || batch < 1 || batch > 65535) {
        cgx_set_error("verify: gamma %d / batch %d out of range", gamma, batch);
        return -1;
    }
    hipLaunchKernelGGL(k_verify_rows, dim3(gamma + 1, batch), dim3(kThreads), 0, stream(),
                       target, draft, tokens, u, gamma, V, T, accept_prob, correction,
                       bonus);
    if (launch_check("k_verify_rows")) return -1;
    hipLaunchKernelGGL(k_verify_combine, dim3((batch + 63) / 64), dim3(64), 0, stream(),
                       tokens, u, accept_prob, correction, bonus, gamma, batch, out_tokens,
                       n_accepted);
    return launch_check("k_verify_combine");
}

extern "C" int cgk_verify_chain_dist(const float* p, const float* q, const int* tokens,
                                     const float* u, int batch, int gamma, int V,
                                     const int* bonus, float* accept_prob, int* correction,
                                     int* out_tokens, int* n_accepted) {
    if (check_v(V)) return -1;
    if (gamma < 1 || batch < 1 || batch > 65535) {
        cgx_set_error("verify: gamma %d / batch %d out of range", gamma, batch);
        return -1;
    }
    hipLaunchKernelGGL(k_verify_rows_dist, dim3(gamma, batch), dim3(kThreads), 0, stream(), p,
                       q, tokens, u, gamma, V, accept_prob, correction);
    if (launch_check("k_verify_rows_dist")) return -1;
    hipLaunchKernelGGL(k_verify_combine, dim3((batch + 63) / 64), dim3(64), 0, stream(),
                       tokens, u, accept_prob, correction, bonus, gamma, batch, out_tokens,
                       n_accepted);
    return launch_check("k_verify_combine");
}
