// verify.hip -- the verify composition (accept tests, first reject, correction
// or bonus draw) as a chunk-parallel pipeline over many workgroups per row,
// bit-identical to cogito's sequential samplers:
//
//   cg_sample_temperature  src/inference/speculative.c:54-75
//   cg_acceptance_prob     speculative.c:49-52
//   cg_sample_corrected    speculative.c:148-172
//
// Every sum the reference forms is a left-to-right binary32 sum; its exact
// value is reproduced with the binade argument of eos.hpp (inside one binade
// every addition advances the running value by rne(x / ulp) ulps, ties aside),
// but the elements are not evaluated exactly up front.  Each element gets a
// fast approximation with a rigorous error bound (exp_fast, a rounded
// reciprocal); the approximation decides the rounding whenever no
// half-integer lies within the bound of x / ulp, and the element is
// re-evaluated exactly (glibc-identical expf, IEEE division) only otherwise.
//
// Rows are cut into segments of 4096 elements (one 256-thread workgroup, 16
// elements -- one chunk -- per thread).  Per row and pass:
//   stats : segment maximum and an approximate segment sum with an error
//           bound (against the segment's own maximum, rescaled later)
//   fold  : the row maximum; exact arguments; the binade of every chunk from
//           the approximate prefix (guide) and its bound; chunk summaries
//           (ulp increments per input parity); a segmented scan into runs of
//           one binade; chunks that may cross a binade are staged exactly
//   walk  : one wave per row composes the runs and replays the staged chunks
//           with real fp32 additions: the exact running value at every
//           segment and run start, and the row sum
// Pass 1 covers every target and draft row; the decisions then pick, per
// chain, the one row (bonus: target row gamma, probabilities p = e / S) or
// row pair (first reject j: residual max(0, p - q)) whose CDF is searched,
// pass 2 sums it the same way, and the find replays the one chunk that holds
// the draw.  Chains with non-finite rows, or a residual mass below 1e-10
// (the reference then samples softmax(p)), are finished by the single-block
// exact kernel at the end.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "cgx_internal.h"

#include "eos.hpp"

namespace {

namespace vp {

constexpr int kT = 256;                  // threads per segment workgroup
constexpr int kW = kT / 64;
constexpr int kC = 16;                   // elements per chunk (per thread)
constexpr int kSeg = kT * kC;            // 4096 elements per segment
constexpr int kItemCap = 64;             // runs per segment (more: exact replay)
constexpr int kDirtyCap = kT;            // staged chunks per segment (all of them)
constexpr int kWalkItems = 256;          // walk: runs held in LDS per batch
constexpr int kMaxGamma = 64;
constexpr int kCompactMaxBlocks = 256;   // pass-2 folds with wave-shared exact evaluations
constexpr int kMaxSegs = 64;             // segments per row (V <= 262144)

enum { kKindExp = 0, kKindProb = 1, kKindRes = 2 };

inline hipStream_t stream() { return (hipStream_t)cgx_stream(); }

int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        cgx_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

// One walk item: a run of clean chunks of one binade (total effect on the
// running value) or a run of chunks whose exact values are staged (chunks
// that may cross a binade).  A run ends where the next item starts.
struct Item {
    int chunk;      // first chunk (within the segment)
    int binade;     // kDirty for staged chunks
    int q0, q1;     // run increments in ulps for input parity 0 / 1
    int c;          // output parities: bit 0 for input parity 0, bit 1 for 1
    int slot;       // staging slot of the first staged chunk
    int end;        // one past the run's last chunk
    int pad;
};

// Monoid of a run of additions inside one binade, integer form (a run never
// advances more than 2^24 ulps: it stays in its binade).
struct MI {
    int q0, q1, c;
};

__device__ __forceinline__ MI mi_id() { return MI{0, 0, 2}; }

__device__ __forceinline__ MI mi_then(const MI& a, const MI& b) {
    const int a0 = a.c & 1, a1 = (a.c >> 1) & 1;
    const int b0 = b.c & 1, b1 = (b.c >> 1) & 1;
    MI r;
    r.q0 = a.q0 + (a0 ? b.q1 : b.q0);
    r.q1 = a.q1 + (a1 ? b.q1 : b.q0);
    r.c = (a0 ? b1 : b0) | ((a1 ? b1 : b0) << 1);
    return r;
}

struct SMI {
    MI m;
    int flag;       // a run starts inside this range
};

__device__ __forceinline__ SMI smi_then(const SMI& a, const SMI& b) {
    if (b.flag) return b;
    return SMI{mi_then(a.m, b.m), a.flag};
}

template <int CTRL, int RMASK>
__device__ __forceinline__ SMI dpp_smi(const SMI& v) {
    SMI o;
    o.m.q0 = dpp_i<CTRL, RMASK>(v.m.q0);
    o.m.q1 = dpp_i<CTRL, RMASK>(v.m.q1);
    o.m.c = dpp_i<CTRL, RMASK>(v.m.c);
    o.flag = dpp_i<CTRL, RMASK>(v.flag);
    return o;
}

__device__ __forceinline__ SMI wave_incl_smi(SMI v) {
    SMI o;
    o = dpp_smi<0x111, 0xF>(v); if (dpp_step_valid(0)) v = smi_then(o, v);
    o = dpp_smi<0x112, 0xF>(v); if (dpp_step_valid(1)) v = smi_then(o, v);
    o = dpp_smi<0x114, 0xF>(v); if (dpp_step_valid(2)) v = smi_then(o, v);
    o = dpp_smi<0x118, 0xF>(v); if (dpp_step_valid(3)) v = smi_then(o, v);
    o = dpp_smi<0x142, 0xA>(v); if (dpp_step_valid(4)) v = smi_then(o, v);
    o = dpp_smi<0x143, 0xC>(v); if (dpp_step_valid(5)) v = smi_then(o, v);
    return v;
}

// Binade of a non-negative fp32 from its bits (-127: zero and subnormals),
// and s advanced by a run summary in its binade b.  Inside a binade s / ulp
// is 2^23 + mantissa (bits for b = -127), so the parity is the low bit and
// adding q ulps adds q to the bit pattern (reaching 2^(b+1) exactly included).
__device__ __forceinline__ int binade_bits(float s) {
    const int ex = (int)(__float_as_uint(s) >> 23);
    return ex == 0 ? -127 : ex - 127;
}

__device__ __forceinline__ float mi_apply(float s, const MI& m) {
    // branch-free choice of the increment (a select here became a
    // dynamically indexed pair in scratch memory inside the walk's loop)
    const unsigned int u = __float_as_uint(s);
    const unsigned int q0 = (unsigned int)m.q0, q1 = (unsigned int)m.q1;
    return __uint_as_float(u + (q0 ^ ((q0 ^ q1) & (0u - (u & 1u)))));
}

// ------------------------------------------------------------- workspace

struct Rows {            // pass-1 rows: per chain target 0..gamma, draft 0..gamma-1
    const float* target;
    const float* draft;
    int gamma, V;
    size_t ldt;          // floats between consecutive target rows (V unless strided)
    __device__ const float* row(int r) const {
        const int per = 2 * gamma + 1, c = r / per, i = r % per;
        return i <= gamma ? target + ((size_t)c * (gamma + 1) + i) * ldt
                          : draft + ((size_t)c * gamma + (i - gamma - 1)) * V;
    }
};

struct Task {            // pass-2 row of a chain
    int kind;            // kKindProb (bonus), kKindRes (first reject), -1: finished elsewhere
    int ra, rb;          // pass-1 rows: target (and draft for kKindRes)
    int j;               // output position
    float u;             // the draw
    int pad[3];
};

struct Work {
    int R1, chains, nseg;
    float* seg_m;        // [R1][nseg] segment maxima
    double* seg_gh;      // [R1][nseg][2] approximate sums G, H (see k_seg_stats)
    int* seg_bad;        // [R1][nseg] NaN or +inf present
    float* row_m;        // [R1]
    float* row_S;        // [R1 + chains] row sums
    int* cnt;            // [Rall][nseg][2] items, staged chunks (-1: overflow)
    Item* items;         // [Rall][nseg][kItemCap]
    float* dirty;        // [Rall][nseg][kDirtyCap][kC]
    float* seg_start;    // [Rall][nseg + 1] exact running value (last: row sum)
    float* item_start;   // [Rall][nseg][kItemCap]
    float* dirty_start;  // [Rall][nseg][kDirtyCap] exact value at each staged chunk start
    double* task_ge;     // [chains][nseg][2] residual guide sums, bounds
    MI* chunk_mi;        // [chains][nseg][kT] pass-2 chunk summaries (identity if staged)
    Task* task;          // [chains]
    int* flags;          // [chains] 1: non-finite row, 2: residual mass < 1e-10
    // certified decisions (null: every pass-1 row is summed exactly)
    int* need;           // [chains][R1 / chains + 1]: count, then the rows to sum exactly
    int* pre;            // [chains][gamma] accept test: 1 accept, 0 reject, -1 open
};

__device__ __forceinline__ size_t segi(const Work& w, int row, int seg) {
    return (size_t)row * w.nseg + seg;
}

// Row values of one pass: exact element values, and approximations with
// absolute error bounds, computed from the exact exponent arguments.
template <int KIND>
struct Eval {
    const float* a;
    const float* b;
    float ma, mb, Sa, Sb, ia, ib, T;
    int V;
    const uint64_t* tab;     // exp_glibc's table (kExp2Tab or a copy in LDS)

    __device__ __forceinline__ float arg(float x, float m) const {
        return T == 1.0f ? __fsub_rn(x, m) : __fdiv_rn(__fsub_rn(x, m), T);
    }
    // exact value from arguments
    __device__ __forceinline__ float exact(float A, float B) const {
        if constexpr (KIND == kKindExp) {
            return exp_glibc_t(A, tab);
        } else if constexpr (KIND == kKindProb) {
            return __fdiv_rn(exp_glibc_t(A, tab), Sa);
        } else {
            return fmaxf(0.0f, __fsub_rn(__fdiv_rn(exp_glibc_t(A, tab), Sa),
                                         __fdiv_rn(exp_glibc_t(B, tab), Sb)));
        }
    }
    // approximation and its bound: exp_fast on [-87, 0]; below, expf is
    // under 2^-125 and the approximation 0 (absolute bound); 2^-140 covers
    // subnormal quotients
    __device__ __forceinline__ float2 approx(float A, float B) const {
        const bool oa = A >= kExpFastMin;
        const float ea = oa ? exp_fast(A) : 0.0f;
        if constexpr (KIND == kKindExp) {
            return make_float2(ea, oa ? ea * kExpErr : 0x1p-125f);
        } else if constexpr (KIND == kKindProb) {
            const float p = ea * ia;
            return make_float2(p, (oa ? p * kProbRel : 0x1p-124f * ia) + 0x1p-140f);
        } else {
            const bool ob = B >= kExpFastMin;
            const float eb = ob ? exp_fast(B) : 0.0f;
            const float p = ea * ia, q = eb * ib;
            const float abs_err = (oa ? 0.0f : 0x1p-124f * ia) + (ob ? 0.0f : 0x1p-124f * ib);
            return make_float2(fmaxf(0.0f, p - q), kResRel * (p + q) + abs_err + 0x1p-140f);
        }
    }
    // a residual's approximation and bound from exp_stat (within kExpStatRel
    // on [-87, 0]): for sums that feed only the guide's bounds
    __device__ __forceinline__ float2 approx_stat(float A, float B) const {
        static_assert(KIND == kKindRes, "residual rows only");
        const bool oa = A >= kExpFastMin, ob = B >= kExpFastMin;
        const float ea = oa ? exp_stat(A) : 0.0f;
        const float eb = ob ? exp_stat(B) : 0.0f;
        const float p = ea * ia, q = eb * ib;
        const float abs_err = (oa ? 0.0f : 0x1p-124f * ia) + (ob ? 0.0f : 0x1p-124f * ib);
        return make_float2(fmaxf(0.0f, p - q), kStatResRel * (p + q) + abs_err + 0x1p-140f);
    }
    // exact value of element j, from memory
    __device__ __forceinline__ float at(int j) const {
        if (j < 0 || j >= V) return 0.0f;
        const float A = arg(a[j], ma);
        const float B = KIND == kKindRes ? arg(b[j], mb) : 0.0f;
        return exact(A, B);
    }
    // this thread's chunk: raw values, exact arguments from them, or both
    __device__ __forceinline__ void raw(int base, float (&X)[kC], float (&Y)[kC]) const;
    __device__ __forceinline__ void args_of(int base, const float (&X)[kC], const float (&Y)[kC],
                                            float (&A)[kC], float (&B)[kC]) const;
    __device__ __forceinline__ void args(int base, float (&A)[kC], float (&B)[kC]) const;
};

// this thread's chunk of a row as stored (-inf past V)
__device__ __forceinline__ void load_raw(const float* p, int base, int V, float (&x)[kC]) {
    if (base + kC <= V && ((uintptr_t)(p + base) & 15u) == 0) {
        const float4* q = reinterpret_cast<const float4*>(p + base);
#pragma unroll
        for (int i = 0; i < kC / 4; i++) {
            const float4 v = q[i];
            x[4 * i] = v.x;
            x[4 * i + 1] = v.y;
            x[4 * i + 2] = v.z;
            x[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < kC; k++) x[k] = base + k < V ? p[base + k] : -__builtin_inff();
    }
}

// exact args of a chunk from its raw values (-inf past V: value 0)
__device__ __forceinline__ void make_args(const float (&x)[kC], float m, float T, int base,
                                          int V, float (&A)[kC]) {
    if (T == 1.0f) {
#pragma unroll
        for (int k = 0; k < kC; k++)
            A[k] = base + k < V ? __fsub_rn(x[k], m) : -__builtin_inff();
    } else {
#pragma unroll
        for (int k = 0; k < kC; k++)
            A[k] = base + k < V ? __fdiv_rn(__fsub_rn(x[k], m), T) : -__builtin_inff();
    }
}

template <int KIND>
__device__ __forceinline__ void Eval<KIND>::raw(int base, float (&X)[kC], float (&Y)[kC]) const {
    load_raw(a, base, V, X);
    if constexpr (KIND == kKindRes) load_raw(b, base, V, Y);
}

template <int KIND>
__device__ __forceinline__ void Eval<KIND>::args_of(int base, const float (&X)[kC],
                                                    const float (&Y)[kC], float (&A)[kC],
                                                    float (&B)[kC]) const {
    make_args(X, ma, T, base, V, A);
    if constexpr (KIND == kKindRes) make_args(Y, mb, T, base, V, B);
}

template <int KIND>
__device__ __forceinline__ void Eval<KIND>::args(int base, float (&A)[kC], float (&B)[kC]) const {
    float X[kC], Y[kC];
    raw(base, X, Y);
    args_of(base, X, Y, A, B);
}

// Summary of one chunk in binade b from its approximations (v, bound er) and
// exact arguments: exact, re-evaluating the elements the bound cannot decide.
// LDS ordering inside one wave (the wave's own LDS writes, then its reads):
// wavefront-scope fences around a wave barrier.
__device__ __forceinline__ void walk_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One wave's list of elements to evaluate exactly (64 per round).
struct WaveList {
    float a[64], b[64], r[64];
};

// Exact values of the elements flagged in `need` (bit k: element k of this
// lane's chunk), replacing v[k].  The wave evaluates them 64 at a time: the
// flagged elements are listed in LDS in lane order, each lane evaluates one,
// and the owners read their results back -- one exact evaluation per lane
// and round instead of every flagged position of every lane in turn.  A
// wave-uniform call.
template <int KIND>
__device__ __forceinline__ void exact_compact(const Eval<KIND>& ev, const float (&A)[kC],
                                              const float (&B)[kC], unsigned need,
                                              float (&v)[kC], WaveList& wl) {
    const int l = lane_id();
    const int cnt = __popc(need);
    int off = cnt;                            // inclusive prefix over the wave
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(off, o);
        if (l >= o) off += t;
    }
    const int total = __shfl(off, 63);
    off -= cnt;
    for (int r0 = 0; r0 < total; r0 += 64) {
        int idx = off - r0;
#pragma unroll
        for (int k = 0; k < kC; k++) {
            if ((need >> k) & 1u) {
                if (idx >= 0 && idx < 64) {
                    wl.a[idx] = A[k];
                    if constexpr (KIND == kKindRes) wl.b[idx] = B[k];
                }
                idx++;
            }
        }
        walk_sync();
        if (l < total - r0) wl.r[l] = ev.exact(wl.a[l], KIND == kKindRes ? wl.b[l] : 0.0f);
        walk_sync();
        idx = off - r0;
#pragma unroll
        for (int k = 0; k < kC; k++) {
            if ((need >> k) & 1u) {
                if (idx >= 0 && idx < 64) v[k] = wl.r[idx];
                idx++;
            }
        }
        walk_sync();
    }
}

// The certified fold of a clean chunk in binade b, in two halves around the
// wave's exact evaluations.  chunk_need: y = v / ulp and its bound, by a
// power-of-two scale (exact; ldexp, as the scale itself can exceed the fp32
// range for tiny binades); an element whose bound holds a half-integer (ties
// included) is flagged for its exact value.
__device__ __forceinline__ int chunk_scale(int b) { return b == -127 ? 149 : 23 - b; }

__device__ __forceinline__ unsigned chunk_need(const float (&v)[kC], const float (&er)[kC],
                                               int b) {
    const int e = chunk_scale(b);
    unsigned need = 0;
#pragma unroll
    for (int k = 0; k < kC; k++) {
        const float y = ldexpf(v[k], e);
        if (fabsf(y - rintf(y)) + ldexpf(er[k], e) >= 0.5f) need |= 1u << k;
    }
    return need;
}

// chunk_fold: with every flagged element exact, each element's rounding to
// the binade's ulp is decided (ties by the running parity).
__device__ __forceinline__ MI chunk_fold(const float (&v)[kC], int b, bool any) {
    const int e = chunk_scale(b);
    if (!any) {                               // no element near a half-integer
        int q = 0;
#pragma unroll
        for (int k = 0; k < kC; k++) q += (int)rintf(ldexpf(v[k], e));
        return MI{q, q, (q & 1) | (((q & 1) ^ 1) << 1)};
    }
    int q0 = 0, q1 = 0, c0 = 0, c1 = 1;
#pragma unroll
    for (int k = 0; k < kC; k++) {
        const float y = ldexpf(v[k], e);
        const float f = floorf(y);
        const float fr = y - f;
        const int fi = (int)f;
        if (fr == 0.5f) {
            // a tie rounds to the even neighbour: the running parity decides
            const int fo = fi & 1;
            q0 += fi + ((c0 ^ fo) & 1);
            q1 += fi + ((c1 ^ fo) & 1);
            c0 = 0;
            c1 = 0;
        } else {
            const int qi = fi + (fr > 0.5f ? 1 : 0);
            q0 += qi;
            q1 += qi;
            c0 ^= qi & 1;
            c1 ^= qi & 1;
        }
    }
    return MI{q0, q1, c0 | (c1 << 1)};
}

constexpr int kExactBatch = 4;           // exact evaluations in flight per lane

// The certified fold of a clean chunk with each lane evaluating its own
// flagged elements, four at a time (four independent evaluation chains in
// flight instead of one long dependent chain per element).
template <int KIND>
__device__ __forceinline__ MI fold_chunk16(const Eval<KIND>& ev, const float (&A)[kC],
                                           const float (&B)[kC], float (&v)[kC],
                                           const float (&er)[kC], int b) {
    const unsigned need = chunk_need(v, er, b);
    if (!need) return chunk_fold(v, b, false);
#pragma unroll
    for (int k0 = 0; k0 < kC; k0 += kExactBatch) {
        if ((need >> k0) & ((1u << kExactBatch) - 1u)) {
            float ex[kExactBatch];
#pragma unroll
            for (int j = 0; j < kExactBatch; j++) ex[j] = ev.exact(A[k0 + j], B[k0 + j]);
#pragma unroll
            for (int j = 0; j < kExactBatch; j++)
                v[k0 + j] = (need >> (k0 + j)) & 1u ? ex[j] : v[k0 + j];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    return chunk_fold(v, b, true);
}

// ------------------------------------------------------ block reductions

__device__ __forceinline__ float block_max256(float v, float* s_w) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    __syncthreads();
    if (lane_id() == 0) s_w[wave_id()] = v;
    __syncthreads();
    float r = s_w[0];
    for (int w = 1; w < kW; w++) r = fmaxf(r, s_w[w]);
    return r;
}

__device__ __forceinline__ double block_sum256_d(double v, double* s_w) {
    v = wave_incl_sum_d(v);
    __syncthreads();
    if (lane_id() == 63) s_w[wave_id()] = v;
    __syncthreads();
    double r = 0.0;
    for (int w = 0; w < kW; w++) r += s_w[w];
    return r;
}

// inclusive fp64 scan over the block, and the block total
__device__ __forceinline__ double block_incl256_d(double v, double* s_w, double* total) {
    v = wave_incl_sum_d(v);
    __syncthreads();
    if (lane_id() == 63) s_w[wave_id()] = v;
    __syncthreads();
    double pre = 0.0, tot = 0.0;
    for (int w = 0; w < kW; w++) {
        pre += w < wave_id() ? s_w[w] : 0.0;
        tot += s_w[w];
    }
    *total = tot;
    return pre + v;
}

template <int CTRL, int RMASK>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(dpp_i<CTRL, RMASK>(__float_as_int(v)));
}

// inclusive fp32 scan over the wave (DPP; row_shr 1, 2, 4, 8, row_bcast 15, 31)
__device__ __forceinline__ float wave_incl_sum_f(float x) {
    float o;
    o = dppf<0x111, 0xF>(x); if (dpp_step_valid(0)) x += o;
    o = dppf<0x112, 0xF>(x); if (dpp_step_valid(1)) x += o;
    o = dppf<0x114, 0xF>(x); if (dpp_step_valid(2)) x += o;
    o = dppf<0x118, 0xF>(x); if (dpp_step_valid(3)) x += o;
    o = dppf<0x142, 0xA>(x); if (dpp_step_valid(4)) x += o;
    o = dppf<0x143, 0xC>(x); if (dpp_step_valid(5)) x += o;
    return x;
}

// inclusive fp32 scans of two values over the block; each result is within
// 2^-19 relative of the exact prefix (at most 10 roundings of partial sums
// of non-negative values)
__device__ __forceinline__ void block_incl256_f2(float a, float b, float* s_w, float* ia,
                                                 float* ib) {
    a = wave_incl_sum_f(a);
    b = wave_incl_sum_f(b);
    __syncthreads();
    if (lane_id() == 63) {
        s_w[wave_id()] = a;
        s_w[kW + wave_id()] = b;
    }
    __syncthreads();
    float pa = 0.0f, pb = 0.0f;
    for (int w = 0; w < wave_id(); w++) {
        pa += s_w[w];
        pb += s_w[kW + w];
    }
    *ia = pa + a;
    *ib = pb + b;
}

// first thread (lowest index) with pred, or kT
__device__ __forceinline__ int block_first256(bool pred, int* s_w) {
    const unsigned long long bal = __ballot(pred);
    __syncthreads();
    if (lane_id() == 0) s_w[wave_id()] = bal ? wave_id() * 64 + __builtin_ctzll(bal) : kT;
    __syncthreads();
    int r = kT;
    for (int w = 0; w < kW; w++) r = min(r, s_w[w]);
    return r;
}

// One segment's term of a row guide: c G with c = exp(-(m - ms) / T), and
// its error bound (see exp_prefix).
__device__ __forceinline__ void guide_term(double G, double H, float ms, bool mine, float m,
                                           float T, double* cg, double* eb) {
    *cg = *eb = 0.0;
    if (mine && G > 0.0) {
        const double D = ((double)m - (double)ms) / (double)T;
        const bool ok = D <= 87.0;
        const double c = ok ? (double)exp_fast(-(float)D) : 0.0;
        *cg = c * G;
        const double cu = ok ? c * (1.0 + 0x1p-19 + 0x1p-23 * D) : 0x1p-125;
        // G's terms within kExpStatRel (2^-16) of exp_glibc, their fp32
        // per-thread sums within 2^-20, exp_glibc within 2^-24 of exp:
        // 2^-15 of G covers them with room to spare
        static_assert(kExpStatRel <= 0x1p-16f, "the bound below assumes exp_stat within 2^-16");
        *eb = cu * (0x1p-22 * 1.01 * H + (0x1p-23 * 1.01 * D + 0x1p-15) * G) +
              (cu - c) * G + 0x1p-136;
    }
}

// ------------------------------------------------- certified decisions

// The fp32 values a positive binary64 bound admits: the least fp32 value
// >= x, the greatest <= x (x a normal fp32 magnitude).
__device__ __forceinline__ float f32_at_least(double x) {
    const float f = (float)x;
    return (double)f < x ? __uint_as_float(__float_as_uint(f) + 1u) : f;
}
__device__ __forceinline__ float f32_at_most(double x) {
    const float f = (float)x;
    return (double)f > x ? __uint_as_float(__float_as_uint(f) - 1u) : f;
}

struct PreShared {
    float m[2 * kMaxGamma + 1];
    float lo[2 * kMaxGamma + 1], hi[2 * kMaxGamma + 1];
};

// Chain c's certified decisions, from its segment stats alone (one block
// per chain after k_seg_stats; its waves share the rows).
// Each row's maximum m (exact) and an interval [lo, hi] of fp32 values
// holding its sum S, the reference's sequential fp32 sum of
// e_i = expf((x_i - m) / T): the guide c G within E (as in exp_prefix), and
// at most V - 1 roundings of a sum of non-negative values, which stay within
// (1 -/+ V 2^-24) of the real sum; S >= 1 (the maximum's element is
// expf(0) = 1) and S <= V.  An accept test u < a, a = min(1, p(x) / q(x)),
// p(x) = e_t(x) / S_t and q(x) = e_d(x) / S_d in fp32 (a = 1 if
// q(x) < 1e-10), is settled when u lies outside the interval of a those
// bounds allow: rounded division and min are monotone.  Listed for the exact
// sums are the rows the chain's outcome can still depend on: both rows of
// every open test before the first settled reject k, then both rows of
// test k, or the bonus row gamma when no test is a settled reject.  A chain
// with a non-finite row lists none (the fallback takes it).
__device__ void pre_decide_chain(const Rows& rows, const int* __restrict__ tokens,
                                 const float* __restrict__ u, float T, const Work& w, int c,
                                 PreShared& sh) {
    const int l = lane_id(), gamma = rows.gamma, V = rows.V;
    const int per = 2 * gamma + 1;
    const double ku = (double)V * 0x1p-24;
    int bad = 0;
    for (int i = wave_id(); i < per; i += (int)(blockDim.x / 64)) {
        const int r = c * per + i;
        float ms = -__builtin_inff();
        double G = 0.0, H = 0.0;
        if (l < w.nseg) {
            const size_t si = segi(w, r, l);
            ms = w.seg_m[si];
            G = w.seg_gh[2 * si];
            H = w.seg_gh[2 * si + 1];
            bad |= w.seg_bad[si];
        }
        float m = ms;
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        double cg, eb;
        guide_term(G, H, ms, l < w.nseg, m, T, &cg, &eb);
        for (int o = 32; o > 0; o >>= 1) {
            cg += __shfl_xor(cg, o);
            eb += __shfl_xor(eb, o);
        }
        bad |= !(m > -__builtin_inff());
        const double E = eb * (1.0 + 0x1p-40);
        const double lo = fmax((cg - E) * (1.0 - ku), 1.0);
        const double hi = fmin((cg + E) * (1.0 + ku / (1.0 - ku)) + 0x1p-140, (double)V);
        if (l == 0) {
            w.row_m[r] = m;
            sh.m[i] = m;
            sh.lo[i] = f32_at_least(lo);
            sh.hi[i] = f32_at_most(hi);
        }
    }
    bad = __syncthreads_or(bad);
    if (wave_id() != 0) return;
    int st = -1;
    if (l < gamma) {
        const int x = tokens[(size_t)c * gamma + l];
        st = 0;   // a draft token outside [0, V): a = 0, rejected
        if (x >= 0 && x < V && !bad) {
            const int it = l, id = gamma + 1 + l;
            const float at = __fdiv_rn(__fsub_rn(rows.row(c * per + it)[x], sh.m[it]), T);
            const float ad = __fdiv_rn(__fsub_rn(rows.row(c * per + id)[x], sh.m[id]), T);
            const float et = exp_glibc(at), ed = exp_glibc(ad);
            const float plo = __fdiv_rn(et, sh.hi[it]), phi = __fdiv_rn(et, sh.lo[it]);
            const float qlo = __fdiv_rn(ed, sh.hi[id]), qhi = __fdiv_rn(ed, sh.lo[id]);
            float alo = 1.0f, ahi = 1.0f;
            if (!(qhi < 1e-10f)) {
                alo = fminf(1.0f, __fdiv_rn(plo, qhi));
                if (!(qlo < 1e-10f)) ahi = fminf(1.0f, __fdiv_rn(phi, qlo));
            }
            const float uu = u[(size_t)c * (gamma + 1) + l];
            st = uu < alo ? 1 : (!(uu < ahi) ? 0 : -1);
        }
        w.pre[(size_t)c * gamma + l] = st;
    }
    const unsigned long long rej = __ballot(l < gamma && st == 0);
    const unsigned long long open = __ballot(l < gamma && st < 0);
    const int k = rej ? __builtin_ctzll(rej) : gamma;
    if (l == 0) {
        int* nd = w.need + (size_t)c * (per + 1);
        int n = 0;
        if (!bad) {
            if (k < gamma) {
                nd[1 + n++] = c * per + k;
                nd[1 + n++] = c * per + gamma + 1 + k;
            } else {
                nd[1 + n++] = c * per + gamma;
            }
            const unsigned long long below = k >= 64 ? ~0ull : (1ull << k) - 1ull;
            for (unsigned long long o = open & below; o; o &= o - 1) {
                const int i = __builtin_ctzll(o);
                nd[1 + n++] = c * per + i;
                nd[1 + n++] = c * per + gamma + 1 + i;
            }
        }
        nd[0] = n;
    }
}

constexpr int kPreThreads = 1024;        // k_pre_decide: up to 16 rows at a time

__global__ __launch_bounds__(kPreThreads) void k_pre_decide(Rows rows,
                                                            const int* __restrict__ tokens,
                                                            const float* __restrict__ u, float T,
                                                            Work w) {
    __shared__ PreShared sh;
    pre_decide_chain(rows, tokens, u, T, w, blockIdx.x, sh);
}

// ------------------------------------------------------- stats (pass 1)

// Per segment of a pass-1 row: its maximum m_s and, against m_s, the
// approximate sum G = sum g_i of g_i = exp(a'_i), a'_i = (x_i - m_s) / T as
// rounded, and H = sum g_i |a'_i|.  With c = exp((m_s - m) / T) for the row
// maximum m, the row's exact elements e_i = expf((x_i - m) / T) satisfy
//   |sum e_i - c G| <= c (2^-22 1.01 H + (2^-23 1.01 D + 2^-18) G) + 2^-136,
// D = (m - m_s) / T: the two rounded arguments differ from (x - m)/T and
// (x - m_s)/T by at most 2^-23 |a| each, expf and exp_cert add 2^-23 and
// 2^-20 relative, the fp32 partial sums 2^-20, subnormal results 2^-149 each.
__global__ __launch_bounds__(kT) void k_seg_stats(Rows rows, float T, Work w) {
    __shared__ float s_f[kW];
    __shared__ double s_d[kW];
    const int seg = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
    const float* p = rows.row(r);
    const int base = seg * kSeg + t * kC, V = rows.V;
    float x[kC];
    bool bad = false;
    float mx = -__builtin_inff();
    if (base + kC <= V && ((uintptr_t)(p + base) & 15u) == 0) {
        const float4* q = reinterpret_cast<const float4*>(p + base);
#pragma unroll
        for (int i = 0; i < kC / 4; i++) {
            const float4 v = q[i];
            x[4 * i] = v.x;
            x[4 * i + 1] = v.y;
            x[4 * i + 2] = v.z;
            x[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < kC; k++) x[k] = base + k < V ? p[base + k] : -__builtin_inff();
    }
#pragma unroll
    for (int k = 0; k < kC; k++) {
        bad |= !(x[k] <= FLT_MAX) && !(x[k] == -__builtin_inff());   // NaN or +inf
        mx = fmaxf(mx, x[k]);
    }
    const float ms = block_max256(mx, s_f);
    float g = 0.0f, h = 0.0f;
    if (ms > -__builtin_inff()) {
        // exp_stat (within kExpStatRel of exp_glibc: these sums only feed
        // the guide's bounds) on the clamped argument everywhere (arguments
        // are <= 0), without a branch per element; exp_glibc afterwards for
        // the rare arguments below its range
        float a[kC], e[kC];
        bool slow = false;
        if (T == 1.0f) {
#pragma unroll
            for (int k = 0; k < kC; k++) a[k] = __fsub_rn(x[k], ms);
        } else {
#pragma unroll
            for (int k = 0; k < kC; k++) a[k] = __fdiv_rn(__fsub_rn(x[k], ms), T);
        }
#pragma unroll
        for (int k = 0; k < kC; k++) {
            const bool live = x[k] > -__builtin_inff();
            const float f = exp_stat(fmaxf(a[k], kExpFastMin));
            e[k] = live ? f : 0.0f;
            a[k] = live ? a[k] : 0.0f;
            slow |= live && !(a[k] >= kExpFastMin && a[k] <= 0.0f);
        }
        if (slow) {
#pragma unroll
            for (int k = 0; k < kC; k++)
                if (x[k] > -__builtin_inff() && !(a[k] >= kExpFastMin && a[k] <= 0.0f))
                    e[k] = exp_glibc(a[k]);
        }
#pragma unroll
        for (int k = 0; k < kC; k++) {
            g += e[k];
            h += e[k] * fabsf(a[k]);
        }
    }
    const double G = block_sum256_d((double)g, s_d);
    const double H = block_sum256_d((double)h, s_d);
    const int nbad = __syncthreads_or(bad);
    if (t == 0) {
        const size_t i = segi(w, r, seg);
        w.seg_m[i] = ms;
        w.seg_gh[2 * i] = G;
        w.seg_gh[2 * i + 1] = H;
        w.seg_bad[i] = nbad;
    }
}

// guide of a pass-1 row over segments [0, seg) from its segment stats: sum of
// c G and its bound.  seg < 64, so wave 0 holds every term (lane s: segment
// s's G, H and maximum ms, loaded by the caller); c = exp(-D) with exp_fast on
// the fp32-rounded D (relative error 2^-20 + 2^-24 D), or 0 below 2^-125.
__device__ __forceinline__ void exp_prefix(double G, double H, float ms, bool mine, float m,
                                           float T, double* s_d, double* P, double* E) {
    if (wave_id() == 0) {
        double cg, eb;
        guide_term(G, H, ms, mine, m, T, &cg, &eb);
        for (int o = 32; o > 0; o >>= 1) {
            cg += __shfl_xor(cg, o);
            eb += __shfl_xor(eb, o);
        }
        if (threadIdx.x == 0) {
            s_d[0] = cg;
            s_d[1] = eb * (1.0 + 0x1p-40);
        }
    }
    __syncthreads();
    *P = s_d[0];
    *E = s_d[1];
    __syncthreads();
}

// the stats of segment t of pass-1 row r (thread t < nseg)
struct SegStats {
    float m;
    double G, H;
};

__device__ __forceinline__ SegStats seg_stats_of(const Work& w, int r) {
    SegStats st{-__builtin_inff(), 0.0, 0.0};
    if ((int)threadIdx.x < w.nseg) {
        const size_t i = segi(w, r, threadIdx.x);
        st.m = w.seg_m[i];
        st.G = w.seg_gh[2 * i];
        st.H = w.seg_gh[2 * i + 1];
    }
    return st;
}

// ------------------------------------------------------------ the fold

struct FoldShared {
    uint64_t tab[32];        // exp_glibc's table
    WaveList wl[kW];
    float f[kW];
    float f2[2 * kW];
    double d[kW];
    int i[kW];
    SMI wagg[kW];
    int bin[kT];
    int nitems, ndirty;
};

// One segment of a row through the certified fold: items and staged chunks
// for the walk.  COMPACT: exact evaluations listed and shared across the
// wave (fewer per lane: the shorter latency when the grid is small); else
// each lane evaluates its own (fewer instructions: the higher throughput on
// a large grid).  X/Y: this thread's chunk as loaded (raw); P0/E0: guide of
// the row before this segment and its bound.
template <bool COMPACT, int KIND>
__device__ void fold_segment(const Eval<KIND>& ev, const Work& w, int row, int seg,
                             const float (&X)[kC], const float (&Y)[kC], double P0, double E0,
                             FoldShared& sh) {
    const int t = threadIdx.x;
    const int base = seg * kSeg + t * kC;
    float A[kC], B[kC];
    ev.args_of(base, X, Y, A, B);
    float v[kC], er[kC];
    float gs = 0.0f, ge = 0.0f;
#pragma unroll
    for (int k = 0; k < kC; k++) {
        const float2 q = ev.approx(A[k], B[k]);
        v[k] = q.x;
        er[k] = q.y;
        gs += q.x;
        ge += q.y;
    }
    ge += gs * 0x1p-19f;                      // rounding of the 16-term fp32 sum
    float pe, ee;
    block_incl256_f2(gs, ge, sh.f2, &pe, &ee);
    // fp32 scan roundings: 2^-19 relative of each prefix
    const double Pend = P0 + (double)pe, Pst = Pend - (double)gs;
    const double Eend = (E0 + (double)ee * (1.0 + 0x1p-18)) * (1.0 + 0x1p-30) +
                        (double)pe * 0x1p-18 + Pend * 0x1p-40;
    const double Est = Eend + (double)gs * 0x1p-18;
    // k sequential fp32 additions of non-negative values stay within
    // [(1 - 2^-24)^k, (1 + 2^-24)^k] of the real sum: >= 1 - ku, <= 1 + ku / (1 - ku)
    const double ks = (double)base * 0x1p-24, ke = (double)(base + kC) * 0x1p-24;
    double lo = base == 0 ? 0.0 : (Pst - Est) * (1.0 - ks);
    if (!(lo > 0.0)) lo = 0.0;
    const double hi = (Pend + Eend) * (1.0 + ke / (1.0 - ke)) + 0x1p-140;
    const int b = binade_of(lo);
    const bool clean = binade_of(hi) == b;
    MI own;
    if constexpr (COMPACT) {
        const unsigned need = clean ? chunk_need(v, er, b) : 0u;
        exact_compact(ev, A, B, need, v, sh.wl[wave_id()]);
        own = clean ? chunk_fold(v, b, need != 0u) : mi_id();
    } else {
        own = clean ? fold_chunk16(ev, A, B, v, er, b) : mi_id();
    }
    if constexpr (KIND != kKindExp)   // pass 2: the find resolves a clean run from these
        w.chunk_mi[((size_t)(row - w.R1) * w.nseg + seg) * kT + t] = own;
    sh.bin[t] = clean ? b : kDirty;
    __syncthreads();
    const bool head = t == 0 || sh.bin[t - 1] != sh.bin[t];
    const bool tail = t == kT - 1 || sh.bin[t + 1] != sh.bin[t];
    const bool last = clean && tail;

    // item index (heads in order) and staging slot (dirty chunks in order)
    const unsigned long long hb = __ballot(head), db = __ballot(!clean);
    const unsigned long long below = (1ull << lane_id()) - 1ull;
    if (lane_id() == 0) sh.i[wave_id()] = __popcll(hb) | (__popcll(db) << 16);
    SMI sv{own, head ? 1 : 0};
    sv = wave_incl_smi(sv);
    if (lane_id() == 63) sh.wagg[wave_id()] = sv;
    __syncthreads();
    int hoff = 0, doff = 0, htot = 0, dtot = 0;
    SMI pre{mi_id(), 0};
    for (int ww = 0; ww < kW; ww++) {
        const int hc = sh.i[ww] & 0xffff, dc = sh.i[ww] >> 16;
        if (ww < wave_id()) {
            hoff += hc;
            doff += dc;
            pre = smi_then(pre, sh.wagg[ww]);
        }
        htot += hc;
        dtot += dc;
    }
    if (wave_id() > 0) sv = smi_then(pre, sv);
    const int item = hoff + __popcll(hb & below) + (head ? 0 : -1);
    const int slot = doff + __popcll(db & below);     // consecutive within a dirty run
    const bool over = htot > kItemCap;
    const size_t si = segi(w, row, seg);
    Item* it = w.items + si * kItemCap;
    if (!over) {
        if (head) {
            it[item].chunk = t;
            it[item].binade = clean ? b : kDirty;
            it[item].slot = clean ? -1 : slot;
        }
        if (tail) it[item].end = t + 1;
        if (last) {
            it[item].q0 = sv.m.q0;
            it[item].q1 = sv.m.q1;
            it[item].c = sv.m.c;
        }
        // staged chunks: every element exact (0 past V: argument -inf)
        if constexpr (COMPACT) {
            exact_compact(ev, A, B, clean ? 0u : (1u << kC) - 1u, v, sh.wl[wave_id()]);
            if (!clean) {
                float* dv = w.dirty + (si * kDirtyCap + slot) * kC;
#pragma unroll
                for (int k0 = 0; k0 < kC; k0 += 4)
                    *(float4*)(dv + k0) = make_float4(v[k0], v[k0 + 1], v[k0 + 2], v[k0 + 3]);
            }
        } else if (!clean) {
            float* dv = w.dirty + (si * kDirtyCap + slot) * kC;
#pragma unroll
            for (int k0 = 0; k0 < kC; k0 += kExactBatch) {
                float ex[kExactBatch];
#pragma unroll
                for (int j = 0; j < kExactBatch; j++) ex[j] = ev.exact(A[k0 + j], B[k0 + j]);
                *(float4*)(dv + k0) = make_float4(ex[0], ex[1], ex[2], ex[3]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    if (t == 0) {
        w.cnt[2 * si] = over ? -1 : htot;
        w.cnt[2 * si + 1] = over ? -1 : dtot;
    }
}

__device__ __forceinline__ Eval<kKindExp> pass1_eval(const Rows& rows, int r, float m, float T) {
    Eval<kKindExp> ev;
    ev.a = rows.row(r);
    ev.b = nullptr;
    ev.ma = m;
    ev.mb = 0.0f;
    ev.Sa = ev.Sb = 1.0f;
    ev.ia = ev.ib = 1.0f;
    ev.T = T;
    ev.V = rows.V;
    ev.tab = kExp2Tab;
    return ev;
}

template <int KIND>
__device__ __forceinline__ Eval<KIND> task_eval(const Rows& rows, const Work& w, const Task& tk,
                                                float T) {
    Eval<KIND> ev;
    ev.a = rows.row(tk.ra);
    ev.b = KIND == kKindRes ? rows.row(tk.rb) : nullptr;
    ev.ma = w.row_m[tk.ra];
    ev.mb = KIND == kKindRes ? w.row_m[tk.rb] : 0.0f;
    ev.Sa = w.row_S[tk.ra];
    ev.Sb = KIND == kKindRes ? w.row_S[tk.rb] : 1.0f;
    ev.ia = 1.0f / ev.Sa;
    ev.ib = 1.0f / ev.Sb;
    ev.T = T;
    ev.V = rows.V;
    ev.tab = kExp2Tab;
    return ev;
}

// Every global load of the block is issued first (the chunk and the row's
// segment stats), so their latencies overlap.
// The k-th pass-1 row of chain c to sum exactly, and how many there are:
// every row of the chain, or the list the certified decisions left.
__device__ __forceinline__ int need_count(const Rows& rows, const Work& w, int c) {
    const int per = 2 * rows.gamma + 1;
    return w.need ? w.need[(size_t)c * (per + 1)] : per;
}
__device__ __forceinline__ int need_row(const Rows& rows, const Work& w, int c, int k) {
    const int per = 2 * rows.gamma + 1;
    return w.need ? w.need[(size_t)c * (per + 1) + 1 + k] : c * per + k;
}

__device__ __forceinline__ void fold1_row(const Rows& rows, float T, const Work& w, int r,
                                          int seg, FoldShared& sh) {
    // the segment stats first: loads complete in issue order, so the row
    // maximum and the guide wait for them only while the chunk arrives
    const SegStats st = seg_stats_of(w, r);
    float X[kC], Y[kC];
    load_raw(rows.row(r), seg * kSeg + threadIdx.x * kC, rows.V, X);
    const float m = block_max256(st.m, sh.f);        // the row maximum
    if (seg == 0 && threadIdx.x == 0) w.row_m[r] = m;
    double P0, E0;
    exp_prefix(st.G, st.H, st.m, (int)threadIdx.x < seg, m, T, sh.d, &P0, &E0);
    Eval<kKindExp> ev = pass1_eval(rows, r, m, T);
    ev.tab = sh.tab;
    fold_segment<false>(ev, w, r, seg, X, Y, P0, E0, sh);
}

// Block (seg, k * chains + c) folds segment seg of chain c's k-th listed row
// (every pass-1 row, or those the certified decisions left; blocks past the
// list end at once, and come last in dispatch order).
__global__ __launch_bounds__(kT) void k_seg_fold1(Rows rows, float T, Work w) {
    __shared__ FoldShared sh;
    const int c = blockIdx.y % w.chains, k = blockIdx.y / w.chains;
    if (k >= need_count(rows, w, c)) return;
    if (threadIdx.x < 32) sh.tab[threadIdx.x] = kExp2Tab[threadIdx.x];   // read after a barrier
    fold1_row(rows, T, w, need_row(rows, w, c, k), blockIdx.x, sh);
}

// The decisions of chain c, by one wave: non-finite rows (NaN, +inf, all
// -inf) go to the exact single-block path; otherwise the accept tests of the
// drafted tokens, the first reject j and the chain's pass-2 task (the
// residual of pair j, or the bonus from target row gamma).  Every caller
// computes the same decisions for a finite chain; the one with `write`
// stores them (the others' task for a chain with non-finite rows is not used:
// the kernels after this one read the stored task).
__device__ Task decide_chain(const Rows& rows, const int* __restrict__ tokens,
                             const float* __restrict__ u, float T, const Work& w, int c,
                             bool write, float* __restrict__ accept_prob,
                             int* __restrict__ out_tokens, int* __restrict__ n_accepted) {
    const int l = lane_id(), gamma = rows.gamma, V = rows.V;
    const int per = 2 * gamma + 1;
    // only the storing caller checks for non-finite rows: a chain that has
    // them is finished by the fallback whatever the others compute for it.
    // (A finite row's sum cannot overflow: every element is at most 1.)
    int bad = 0;
    if (write) {
        for (int r = l; r < per; r += 64) {
            const int rr = c * per + r;
            bad |= !(w.row_m[rr] > -__builtin_inff());
            for (int s = 0; s < w.nseg; s++) bad |= w.seg_bad[segi(w, rr, s)];
        }
        bad = __any(bad);
    }
    const float* uu = u + (size_t)c * (gamma + 1);
    bool reject = false;
    // a test the certified decisions settled stands; an open one is taken
    // exactly (its rows were summed exactly)
    const int pre = w.pre && l < gamma ? w.pre[(size_t)c * gamma + l] : -1;
    if (pre >= 0) {
        reject = pre == 0;
    } else if (l < gamma) {
        const int x = tokens[(size_t)c * gamma + l];
        float a = 0.0f;   // a draft token outside [0, V) is rejected
        if (x >= 0 && x < V) {
            const int rt = c * per + l, rd = c * per + gamma + 1 + l;
            const float at = __fdiv_rn(__fsub_rn(rows.row(rt)[x], w.row_m[rt]), T);
            const float ad = __fdiv_rn(__fsub_rn(rows.row(rd)[x], w.row_m[rd]), T);
            const float px = __fdiv_rn(exp_glibc(at), w.row_S[rt]);
            const float qx = __fdiv_rn(exp_glibc(ad), w.row_S[rd]);
            a = qx < 1e-10f ? 1.0f : fminf(1.0f, __fdiv_rn(px, qx));
        }
        if (write && !bad && accept_prob) accept_prob[(size_t)c * gamma + l] = a;
        reject = !(uu[l] < a);
    }
    const unsigned long long rb = __ballot(reject);
    const int j = rb ? __builtin_ctzll(rb) : gamma;
    Task tk;
    tk.kind = bad ? -1 : (j < gamma ? kKindRes : kKindProb);
    tk.ra = c * per + j;
    tk.rb = c * per + gamma + 1 + (j < gamma ? j : 0);
    tk.j = j;
    tk.u = uu[j < gamma ? j + 1 : gamma];
    tk.pad[0] = tk.pad[1] = tk.pad[2] = 0;
    if (!write) return tk;
    if (bad) {
        if (l == 0) {
            w.flags[c] = 1;
            w.task[c].kind = -1;
        }
        return tk;
    }
    int* out = out_tokens + (size_t)c * (gamma + 1);
    for (int i = l; i <= gamma; i += 64) {
        if (i < j) out[i] = tokens[(size_t)c * gamma + i];
        else if (i > j) out[i] = -1;
    }
    if (l == 0) {
        n_accepted[c] = j;
        w.flags[c] = 0;
        w.task[c] = tk;
    }
    return tk;
}

// residual guide sums of the first-reject row pairs (pass-2 stats).  Each
// block first takes its chain's decisions (the segment-0 block stores them
// for the kernels after this one), so no separate launch decides.
__global__ __launch_bounds__(kT) void k_res_stats(Rows rows, const int* __restrict__ tokens,
                                                  const float* __restrict__ u, float T, Work w,
                                                  float* __restrict__ accept_prob,
                                                  int* __restrict__ out_tokens,
                                                  int* __restrict__ n_accepted) {
    __shared__ double s_d[kW];
    __shared__ Task s_task;
    const int seg = blockIdx.x, c = blockIdx.y;
    if (wave_id() == 0) {
        const Task t0 = decide_chain(rows, tokens, u, T, w, c, seg == 0, accept_prob, out_tokens,
                                     n_accepted);
        if (lane_id() == 0) s_task = t0;
    }
    __syncthreads();
    const Task tk = s_task;
    if (tk.kind != kKindRes) return;
    const Eval<kKindRes> ev = task_eval<kKindRes>(rows, w, tk, T);
    const int base = seg * kSeg + threadIdx.x * kC;
    float A[kC], B[kC];
    ev.args(base, A, B);
    // the task row's segment sums feed only the pass-2 guide and its bound,
    // where the sequential sum's k 2^-24 dwarfs the exponential's error
    float gs = 0.0f, ge = 0.0f;
#pragma unroll
    for (int k = 0; k < kC; k++) {
        const float2 q = ev.approx_stat(A[k], B[k]);
        gs += q.x;
        ge += q.y;
    }
    ge += gs * 0x1p-19f;
    const double G = block_sum256_d((double)gs, s_d);
    const double E = block_sum256_d((double)ge, s_d);
    if (threadIdx.x == 0) {
        const size_t i = (size_t)c * w.nseg + seg;
        w.task_ge[2 * i] = G;
        w.task_ge[2 * i + 1] = E * (1.0 + 0x1p-30) + G * 0x1p-40;
    }
}

template <bool COMPACT>
__global__ __launch_bounds__(kT) void k_seg_fold2(Rows rows, float T, Work w) {
    __shared__ FoldShared sh;
    const int seg = blockIdx.x, c = blockIdx.y;
    const Task tk = w.task[c];
    if (tk.kind < 0) return;
    if (threadIdx.x < 32) sh.tab[threadIdx.x] = kExp2Tab[threadIdx.x];   // read after a barrier
    const int base = seg * kSeg + threadIdx.x * kC;
    float X[kC], Y[kC];
    if (tk.kind == kKindProb) {
        // p_i = e_i / S: the pass-1 guide of row ra, divided by S
        Eval<kKindProb> ev = task_eval<kKindProb>(rows, w, tk, T);
        ev.tab = sh.tab;
        const SegStats st = seg_stats_of(w, tk.ra);   // before the chunk (issue order)
        ev.raw(base, X, Y);
        double P, E;
        exp_prefix(st.G, st.H, st.m, (int)threadIdx.x < seg, ev.ma, T, sh.d, &P, &E);
        const double P0 = P / (double)ev.Sa;
        const double E0 = E / (double)ev.Sa + P0 * 0x1p-22;
        fold_segment<COMPACT>(ev, w, w.R1 + c, seg, X, Y, P0, E0, sh);
    } else {
        Eval<kKindRes> ev = task_eval<kKindRes>(rows, w, tk, T);
        ev.tab = sh.tab;
        double g = 0.0, e = 0.0;                       // before the chunk (issue order)
        if ((int)threadIdx.x < seg) {
            const size_t i = (size_t)c * w.nseg + threadIdx.x;
            g = w.task_ge[2 * i];
            e = w.task_ge[2 * i + 1];
        }
        ev.raw(base, X, Y);
        const double P0 = block_sum256_d(g, sh.d);
        const double E0 = block_sum256_d(e, sh.d);
        fold_segment<COMPACT>(ev, w, w.R1 + c, seg, X, Y, P0, E0, sh);
    }
}

// ------------------------------------------------------------- the walk

// s + x_0 + x_1 + ... + x_63 in order (fp32), x_k held by lane k; padding
// lanes hold +0.0, which leaves a non-negative s unchanged.  Fully unrolled:
// the readlanes do not depend on s, only the additions chain.
__device__ __forceinline__ float add64(float s, float x) {
#pragma unroll
    for (int k = 0; k < 64; k++)
        s = __fadd_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k)));
    return s;
}

// Exact running value through elements [j0, j1) of a row (one wave: exact
// values 64 at a time, the next batch loaded before the current one is added).
template <int KIND>
__device__ float replay_exact(const Eval<KIND>& ev, int j0, int j1, float s) {
    float x = j0 + lane_id() < j1 ? ev.at(j0 + lane_id()) : 0.0f;
    for (int j = j0; j < j1; j += 64) {
        const float xn = j + 64 + lane_id() < j1 ? ev.at(j + 64 + lane_id()) : 0.0f;
        s = add64(s, x);
        x = xn;
    }
    return s;
}

constexpr int kWalkStaged = kDirtyCap * kC;   // walk: staged values held in LDS per batch

// 16 bytes a lane from global memory straight into LDS: lane i's bytes land
// at dst + 16 i (dst wave-uniform), no registers and no wait at issue
__device__ __forceinline__ void load_lds16(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

// One step of a walk: a stretch of consecutive clean runs (their summaries
// composed: adding q ulps adds q to the bit pattern, across binades too), a
// dirty run (its staged chunks replayed), or a segment replayed exactly.
struct WalkOp {
    int kind;            // kOpClean, kOpDirty, kOpExact
    int j0, j1;          // element range (for an exact replay)
    int q0, q1, c;       // clean: the stretch's composed summary
    int bin0, bin1;      // clean: binade of its first and last run
    int nd;              // dirty: staged chunks
    int sidx;            // dirty: index of its first chunk in dirty_start
    int r0, r1;          // its runs (batch indices), first and last
};
enum { kOpClean = 0, kOpDirty = 1, kOpExact = 2 };
constexpr int kWalkOps = kWalkItems + kMaxSegs;

struct WalkShared {
    alignas(16) Item items[kWalkItems];
    alignas(16) float staged[kWalkStaged + 2 * kC];   // + 2 chunks: reads ahead past the last
    alignas(16) WalkOp ops[kWalkOps];
    int segof[kWalkItems];       // segment of each run
    int item_op[kWalkItems];     // op of each run
    int heads[kWalkItems];       // ops begun by runs 0..j (inclusive)
    MI item_pre[kWalkItems];     // composed summaries of the stretch's runs before it
    float op_start[kWalkOps];    // exact value at each op's start
    int op_slow[kWalkOps];       // 1: replayed exactly run by run (starts stored then)
    int seg_first[kMaxSegs];     // first run of each segment of the batch
    int seg_ovb[kMaxSegs];       // overflowed segments of the batch before it
};

// One wave per row: exact value at every segment and item start, row sum.
// Segments are walked in batches; a batch's runs and staged values are
// gathered into LDS first, all loads in flight together, so the serial chain
// of additions waits on global memory once per batch, not once per staged run.
// The walk runs in one wave: its LDS traffic (and the LDS-bound loads,
// waited for with s_waitcnt) needs ordering inside the wave only, so the walk
// also runs as one wave of a larger block.

// The walk of a short row (few segments): one step per run and segment, the
// starts (with STARTS) kept in lanes and stored 64 at a time.
template <bool STARTS, int KIND>
__device__ void walk_row_runs(const Eval<KIND>& ev, const Work& w, int row, WalkShared& sh) {
    const int l = lane_id();
    // every segment's counts (nseg <= 64; lane l: segment l), and their
    // prefix sums; a segment whose runs overflowed (-1) is replayed exactly
    int c = 0, dc = 0;
    if (l < w.nseg) {
        c = w.cnt[2 * segi(w, row, l)];
        dc = w.cnt[2 * segi(w, row, l) + 1];
    }
    int io = c > 0 ? c : 0, so = c >= 0 && dc > 0 ? dc * kC : 0;
    for (int o = 1; o < 64; o <<= 1) {
        const int a = __shfl_up(io, o), b = __shfl_up(so, o);
        if (l >= o) {
            io += a;
            so += b;
        }
    }
    const float* rdirty = w.dirty + segi(w, row, 0) * kDirtyCap * kC;
    const Item* ritems = w.items + segi(w, row, 0) * kItemCap;
    float s = 0.0f;
    float seg_st = 0.0f;      // lane g: start of segment g
    int g0 = 0;
    while (g0 < w.nseg) {
        // batch [g0, g1): as many segments as fit (lane l holds the prefix
        // counts through segment l, so the fitting segments form a ballot)
        const int ib = g0 > 0 ? __builtin_amdgcn_readlane(io, g0 - 1) : 0;
        const int sb = g0 > 0 ? __builtin_amdgcn_readlane(so, g0 - 1) : 0;
        const unsigned long long fit = __ballot(l >= g0 && l < w.nseg && io - ib <= kWalkItems &&
                                                so - sb <= kWalkStaged);
        const int g1 = max(g0 + 1, 64 - __clzll(fit));
        // gather the batch's runs and staged values into LDS, every load in
        // flight together (counts from the lanes' prefix sums: no LDS read
        // between the loads).  Runs and staged values of consecutive segments
        // land back to back, in walk order.
        for (int seg = g0; seg < g1; seg++) {
            const int sa = seg > 0 ? __builtin_amdgcn_readlane(so, seg - 1) : 0;
            const int sz = __builtin_amdgcn_readlane(so, seg) - sa;         // floats
            const float* ssrc = rdirty + (size_t)seg * kDirtyCap * kC;
            float* sdst = sh.staged + (sa - sb);
            for (int f = 0; f < sz; f += 256)
                if (f + 4 * l < sz) load_lds16(ssrc + f + 4 * l, sdst + f);
            const int ia = seg > 0 ? __builtin_amdgcn_readlane(io, seg - 1) : 0;
            const int iz = (__builtin_amdgcn_readlane(io, seg) - ia) * (int)(sizeof(Item) / 4);
            const int* isrc = (const int*)(ritems + (size_t)seg * kItemCap);
            int* idst = (int*)(sh.items + (ia - ib));
            for (int f = 0; f < iz; f += 256)
                if (f + 4 * l < iz) load_lds16(isrc + f + 4 * l, idst + f);
        }
        __builtin_amdgcn_s_waitcnt(0);
        walk_sync();
        // One stream over the batch.  A segment's runs are read into lanes
        // (lane i: run i) one segment ahead, and inside a dirty run the next
        // two staged chunks are read ahead, all independent of the running
        // value, so the serial chain holds only the additions and register
        // reads.  Staged chunks are consumed in order: a dirty run's chunks
        // are the next ones in the stream.  (Read-ahead buffers live inside
        // one loop only: a buffer carried across loop levels is copied at
        // each entry, and a copy waits for its reads.)
        Item nxt = Item{};
        {
            const int n0 = __builtin_amdgcn_readlane(c, g0);
            if (l < n0) nxt = sh.items[l];
        }
        const vf4* sp = (const vf4*)sh.staged;
        int q = 0;                // staged chunks consumed
        for (int seg = g0; seg < g1; seg++) {
            const size_t si = segi(w, row, seg);
            const int segbase = seg * kSeg;
            if (STARTS) seg_st = l == seg ? s : seg_st;
            const int n = __builtin_amdgcn_readlane(c, seg);
            const Item mine = nxt;
            if (seg + 1 < g1) {
                const int n1 = __builtin_amdgcn_readlane(c, seg + 1);
                if (l < n1) nxt = sh.items[__builtin_amdgcn_readlane(io, seg) - ib + l];
            }
            if (n < 0) {
                s = replay_exact(ev, segbase, min(segbase + kSeg, ev.V), s);
                continue;
            }
            float item_st = 0.0f;     // lane i: start of run i (n <= kItemCap = 64)
            for (int i = 0; i < n; i++) {
                Item it;
                it.chunk = __builtin_amdgcn_readlane(mine.chunk, i);
                it.binade = __builtin_amdgcn_readlane(mine.binade, i);
                it.end = __builtin_amdgcn_readlane(mine.end, i);
                if (STARTS) item_st = l == i ? s : item_st;
                if (it.binade == kDirty) {
                    it.slot = __builtin_amdgcn_readlane(mine.slot, i);
                    float* out = w.dirty_start + si * kDirtyCap + it.slot;
                    const int nd = it.end - it.chunk;
                    float dst = 0.0f;    // lane k % 64: start of staged chunk k
                    // chunk k of the run in X (k even) or Y (k odd); each
                    // buffer is reloaded with chunk k + 2 right after its
                    // additions, so neither is copied while its read is in
                    // flight
                    const vf4* rp = sp + 4 * q;
                    vf4 x0 = rp[0], x1 = rp[1], x2 = rp[2], x3 = rp[3];
                    vf4 y0 = rp[4], y1 = rp[5], y2 = rp[6], y3 = rp[7];
                    auto step = [&](vf4& v0, vf4& v1, vf4& v2, vf4& v3, int k) {
                        if (STARTS) dst = l == (k & 63) ? s : dst;
                        s = add4(add4(add4(add4(s, v0), v1), v2), v3);
                        const vf4* np = rp + 4 * (k + 2);
                        v0 = np[0];
                        v1 = np[1];
                        v2 = np[2];
                        v3 = np[3];
                        __builtin_amdgcn_sched_barrier(0);   // reads issued here
                        if (STARTS && ((k & 63) == 63 || k == nd - 1) && l <= (k & 63))
                            out[(k & ~63) + l] = dst;
                    };
                    int k = 0;
                    for (; k + 1 < nd; k += 2) {
                        step(x0, x1, x2, x3, k);
                        step(y0, y1, y2, y3, k + 1);
                    }
                    if (k < nd) step(x0, x1, x2, x3, k);
                    q += nd;
                } else if (binade_bits(s) != it.binade) {
                    // the run's start is not in the binade its chunks assumed
                    // (excluded by the bounds; replayed exactly anyway)
                    s = replay_exact(ev, segbase + it.chunk * kC,
                                     min(segbase + it.end * kC, ev.V), s);
                } else {
                    s = mi_apply(s, MI{__builtin_amdgcn_readlane(mine.q0, i),
                                       __builtin_amdgcn_readlane(mine.q1, i),
                                       __builtin_amdgcn_readlane(mine.c, i)});
                }
            }
            if (STARTS && l < n) w.item_start[si * kItemCap + l] = item_st;
        }
        walk_sync();
        g0 = g1;
    }
    if (STARTS && l < w.nseg) w.seg_start[(size_t)row * (w.nseg + 1) + l] = seg_st;
    if (l == 0) {
        if (STARTS) w.seg_start[(size_t)row * (w.nseg + 1) + w.nseg] = s;
        w.row_S[row] = s;
    }
}

// The walk of a long row.  Per batch of segments: the runs and staged values are gathered into LDS
// (all loads in flight together); then, in parallel, the runs become a list
// of ops -- consecutive clean runs composed into one stretch, a dirty run,
// or a segment whose runs overflowed -- so that the serial chain takes one
// step per op instead of one per run and segment.  Ops are read 64 at a time
// into lanes; the staged chunks of a dirty run are consumed in stream order
// (two read ahead).  With STARTS the starts of the runs inside a stretch
// follow afterwards, in parallel, from the stretch's start and the composed
// summaries of the runs before them.
template <bool STARTS, int KIND>
__device__ void walk_row_ops(const Eval<KIND>& ev, const Work& w, int row, WalkShared& sh) {
    const int l = lane_id();
    // every segment's counts (nseg <= 64; lane l: segment l), and their
    // prefix sums; a segment whose runs overflowed (-1) is replayed exactly
    int c = 0, dc = 0;
    if (l < w.nseg) {
        c = w.cnt[2 * segi(w, row, l)];
        dc = w.cnt[2 * segi(w, row, l) + 1];
    }
    const bool lane_over = l < w.nseg && c < 0;
    int io = c > 0 ? c : 0, so = c >= 0 && dc > 0 ? dc * kC : 0;
    int ov = lane_over ? 1 : 0;               // overflowed segments through l
    for (int o = 1; o < 64; o <<= 1) {
        const int a = __shfl_up(io, o), b = __shfl_up(so, o), d = __shfl_up(ov, o);
        if (l >= o) {
            io += a;
            so += b;
            ov += d;
        }
    }
    const float* rdirty = w.dirty + segi(w, row, 0) * kDirtyCap * kC;
    const Item* ritems = w.items + segi(w, row, 0) * kItemCap;
    float s = 0.0f;
    int g0 = 0;
    while (g0 < w.nseg) {
        // batch [g0, g1): as many segments as fit (lane l holds the prefix
        // counts through segment l, so the fitting segments form a ballot)
        const int ib = g0 > 0 ? __builtin_amdgcn_readlane(io, g0 - 1) : 0;
        const int sb = g0 > 0 ? __builtin_amdgcn_readlane(so, g0 - 1) : 0;
        const int ob = g0 > 0 ? __builtin_amdgcn_readlane(ov, g0 - 1) : 0;
        const unsigned long long fit = __ballot(l >= g0 && l < w.nseg && io - ib <= kWalkItems &&
                                                so - sb <= kWalkStaged);
        const int g1 = max(g0 + 1, 64 - __clzll(fit));
        const int nit = __builtin_amdgcn_readlane(io, g1 - 1) - ib;
        for (int seg = g0; seg < g1; seg++) {
            const int sa = seg > 0 ? __builtin_amdgcn_readlane(so, seg - 1) : 0;
            const int sz = __builtin_amdgcn_readlane(so, seg) - sa;         // floats
            const float* ssrc = rdirty + (size_t)seg * kDirtyCap * kC;
            float* sdst = sh.staged + (sa - sb);
            for (int f = 0; f < sz; f += 256)
                if (f + 4 * l < sz) load_lds16(ssrc + f + 4 * l, sdst + f);
            const int ia = seg > 0 ? __builtin_amdgcn_readlane(io, seg - 1) : 0;
            const int iz = (__builtin_amdgcn_readlane(io, seg) - ia) * (int)(sizeof(Item) / 4);
            const int* isrc = (const int*)(ritems + (size_t)seg * kItemCap);
            int* idst = (int*)(sh.items + (ia - ib));
            for (int f = 0; f < iz; f += 256)
                if (f + 4 * l < iz) load_lds16(isrc + f + 4 * l, idst + f);
        }
        // per segment of the batch (lane l: segment l): its runs' segment,
        // first run and the overflowed segments before it
        if (l >= g0 && l < g1) {
            const int e0 = io - (c > 0 ? c : 0) - ib;
            for (int i = 0; i < c; i++) sh.segof[e0 + i] = l;
            sh.seg_first[l] = e0;
            sh.seg_ovb[l] = ov - (lane_over ? 1 : 0) - ob;
        }
        __builtin_amdgcn_s_waitcnt(0);
        walk_sync();

        // ---- the ops, in parallel: lane l takes runs kIPL l .. kIPL l + kIPL - 1.
        // A run begins an op unless it is clean and follows a clean run of
        // the same or the next segment (every segment that is not replayed
        // exactly has a run, so a larger step passes such a segment).
        constexpr int kIPL = kWalkItems / 64;
        Item it[kIPL];
        int sg[kIPL];
        bool head[kIPL];
        SMI loc[kIPL];                            // inclusive summaries in the lane
        int nhead = 0;
        SMI acc{mi_id(), 0};
#pragma unroll
        for (int i = 0; i < kIPL; i++) {
            const int j = kIPL * l + i;
            const bool live = j < nit;
            it[i] = live ? sh.items[j] : Item{};
            sg[i] = live ? sh.segof[j] : 0;
            const bool dirty = it[i].binade == kDirty;
            bool h = true;
            if (live && j > 0) {
                const bool pdirty = (i > 0 ? it[i - 1].binade : sh.items[j - 1].binade) == kDirty;
                const int ps = i > 0 ? sg[i - 1] : sh.segof[j - 1];
                h = dirty || pdirty || sg[i] - ps > 1;
            }
            head[i] = live && h;
            nhead += head[i] ? 1 : 0;
            const MI m = (live && !dirty) ? MI{it[i].q0, it[i].q1, it[i].c} : mi_id();
            acc = smi_then(acc, SMI{m, head[i] ? 1 : 0});
            loc[i] = acc;
        }
        int hx = nhead;                           // heads through this lane
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(hx, o);
            if (l >= o) hx += t;
        }
        const int nheads = __shfl(hx, 63);
        hx -= nhead;
        const SMI lin = wave_incl_smi(acc);       // lanes' aggregates, scanned
        SMI before;                               // through the lanes below
        before.m.q0 = __shfl_up(lin.m.q0, 1);
        before.m.q1 = __shfl_up(lin.m.q1, 1);
        before.m.c = __shfl_up(lin.m.c, 1);
        before.flag = __shfl_up(lin.flag, 1);
        if (l == 0) before = SMI{mi_id(), 0};
        const int next_head = __shfl_down(head[0] ? 1 : 0, 1);   // next lane's first run
#pragma unroll
        for (int i = 0; i < kIPL; i++) {
            const int j = kIPL * l + i;
            if (j < nit) {
                if (head[i]) hx++;
                const int seg = sg[i];
                const int op = hx - 1 + sh.seg_ovb[seg];
                sh.heads[j] = hx;
                sh.item_op[j] = op;
                sh.item_pre[j] = head[i] ? mi_id()
                                         : (i > 0 ? smi_then(before, loc[i - 1]) : before).m;
                const bool last = j + 1 >= nit || (i + 1 < kIPL ? head[i + 1] : next_head != 0);
                WalkOp& o = sh.ops[op];
                const int segbase = seg * kSeg;
                if (head[i]) {
                    o.kind = it[i].binade == kDirty ? kOpDirty : kOpClean;
                    o.j0 = segbase + it[i].chunk * kC;
                    o.bin0 = it[i].binade;
                    o.nd = it[i].end - it[i].chunk;
                    o.sidx = (int)(segi(w, row, seg) * kDirtyCap) + it[i].slot;
                    o.r0 = j;
                }
                if (last) {
                    const SMI incl = smi_then(before, loc[i]);
                    o.q0 = incl.m.q0;
                    o.q1 = incl.m.q1;
                    o.c = incl.m.c;
                    o.bin1 = it[i].binade;
                    o.j1 = min(segbase + it[i].end * kC, ev.V);
                    o.r1 = j;
                }
            }
        }
        walk_sync();
        // overflowed segments: one exact op each, after the heads of the
        // runs before it (lane l: segment l)
        if (l >= g0 && l < g1 && lane_over) {
            const int e = sh.seg_first[l];
            const int op = (e > 0 ? sh.heads[e - 1] : 0) + sh.seg_ovb[l];
            WalkOp& o = sh.ops[op];
            o.kind = kOpExact;
            o.j0 = l * kSeg;
            o.j1 = min(l * kSeg + kSeg, ev.V);
            o.r0 = 0;
            o.r1 = -1;
        }
        const int nops = nheads + (__builtin_amdgcn_readlane(ov, g1 - 1) - ob);
        walk_sync();

        // ---- the serial chain: 64 ops at a time in lanes
        const vf4* sp = (const vf4*)sh.staged;
        int q = 0;                                // staged chunks consumed
        for (int p0 = 0; p0 < nops; p0 += 64) {
            const WalkOp mo = p0 + l < nops ? sh.ops[p0 + l] : WalkOp{};
            float ost = 0.0f;                     // lane k: start of op p0 + k
            int slow = 0;                         // lane k: op p0 + k replayed run by run
            const int pn = min(64, nops - p0);
            for (int k = 0; k < pn; k++) {
                if (STARTS) ost = l == k ? s : ost;
                const int kind = __builtin_amdgcn_readlane(mo.kind, k);
                if (kind == kOpDirty) {
                    const int nd = __builtin_amdgcn_readlane(mo.nd, k);
                    float* out = w.dirty_start + __builtin_amdgcn_readlane(mo.sidx, k);
                    float dst = 0.0f;    // lane kk % 64: start of staged chunk kk
                    // chunk kk of the run in X (kk even) or Y (kk odd); each
                    // buffer is reloaded with chunk kk + 2 right after its
                    // additions, so neither is copied while its read is in
                    // flight
                    const vf4* rp = sp + 4 * q;
                    vf4 x0 = rp[0], x1 = rp[1], x2 = rp[2], x3 = rp[3];
                    vf4 y0 = rp[4], y1 = rp[5], y2 = rp[6], y3 = rp[7];
                    auto step = [&](vf4& v0, vf4& v1, vf4& v2, vf4& v3, int kk) {
                        if (STARTS) dst = l == (kk & 63) ? s : dst;
                        s = add4(add4(add4(add4(s, v0), v1), v2), v3);
                        const vf4* np = rp + 4 * (kk + 2);
                        v0 = np[0];
                        v1 = np[1];
                        v2 = np[2];
                        v3 = np[3];
                        __builtin_amdgcn_sched_barrier(0);   // reads issued here
                        if (STARTS && ((kk & 63) == 63 || kk == nd - 1) && l <= (kk & 63))
                            out[(kk & ~63) + l] = dst;
                    };
                    int kk = 0;
                    for (; kk + 1 < nd; kk += 2) {
                        step(x0, x1, x2, x3, kk);
                        step(y0, y1, y2, y3, kk + 1);
                    }
                    if (kk < nd) step(x0, x1, x2, x3, kk);
                    q += nd;
                    continue;
                }
                bool fast = false;
                if (kind == kOpClean &&
                    binade_bits(s) == __builtin_amdgcn_readlane(mo.bin0, k)) {
                    const float sn = mi_apply(s, MI{__builtin_amdgcn_readlane(mo.q0, k),
                                                    __builtin_amdgcn_readlane(mo.q1, k),
                                                    __builtin_amdgcn_readlane(mo.c, k)});
                    // the stretch ends in its last run's binade (the bounds
                    // exclude anything else)
                    if (binade_bits(sn) == __builtin_amdgcn_readlane(mo.bin1, k)) {
                        s = sn;
                        fast = true;
                    }
                }
                if (!fast) {
                    // an overflowed segment, or a stretch that left the
                    // binades its runs assumed (excluded by the bounds):
                    // exact replay, run by run so that every start is exact
                    const int r0 = __builtin_amdgcn_readlane(mo.r0, k);
                    const int r1 = __builtin_amdgcn_readlane(mo.r1, k);
                    if (r1 < r0) {
                        s = replay_exact(ev, __builtin_amdgcn_readlane(mo.j0, k),
                                         __builtin_amdgcn_readlane(mo.j1, k), s);
                    } else {
                        slow = l == k ? 1 : slow;
                        for (int r = r0; r <= r1; r++) {
                            const int seg = sh.segof[r];
                            const Item ir = sh.items[r];
                            if (STARTS && l == 0) {
                                w.item_start[segi(w, row, seg) * kItemCap +
                                             (r - sh.seg_first[seg])] = s;
                                if (r == sh.seg_first[seg])
                                    w.seg_start[(size_t)row * (w.nseg + 1) + seg] = s;
                            }
                            s = replay_exact(ev, seg * kSeg + ir.chunk * kC,
                                             min(seg * kSeg + ir.end * kC, ev.V), s);
                        }
                    }
                }
            }
            if (STARTS && p0 + l < nops) {
                sh.op_start[p0 + l] = ost;
                sh.op_slow[p0 + l] = slow;
            }
        }
        if (STARTS) {
            walk_sync();
            // run starts: the stretch's start advanced by the runs before it;
            // segment starts: the segment's first run, or its exact op
            for (int j = l; j < nit; j += 64) {
                const int op = sh.item_op[j];
                if (sh.op_slow[op]) continue;
                const int seg = sh.segof[j];
                const int first = sh.seg_first[seg];
                const float st = mi_apply(sh.op_start[op], sh.item_pre[j]);
                w.item_start[segi(w, row, seg) * kItemCap + (j - first)] = st;
                if (j == first) w.seg_start[(size_t)row * (w.nseg + 1) + seg] = st;
            }
            if (l >= g0 && l < g1 && lane_over) {
                const int e = sh.seg_first[l];
                const int op = (e > 0 ? sh.heads[e - 1] : 0) + sh.seg_ovb[l];
                w.seg_start[(size_t)row * (w.nseg + 1) + l] = sh.op_start[op];
            }
        }
        walk_sync();
        g0 = g1;
    }
    if (l == 0) {
        if (STARTS) w.seg_start[(size_t)row * (w.nseg + 1) + w.nseg] = s;
        w.row_S[row] = s;
    }
}

// One wave walks a row: the exact value at every segment, run and
// staged-chunk start is stored for the find with STARTS; without, only the
// row sum.  A row of many segments takes the op list (its parallel set-up
// pays once the clean runs it merges across segment boundaries are many);
// a short row steps through its runs directly.
constexpr int kOpWalkMinSegs = 16;

template <bool STARTS, int KIND>
__device__ __forceinline__ void walk_row(const Eval<KIND>& ev, const Work& w, int row,
                                         WalkShared& sh) {
    if (w.nseg >= kOpWalkMinSegs) walk_row_ops<STARTS>(ev, w, row, sh);
    else walk_row_runs<STARTS>(ev, w, row, sh);
}

// Block k * chains + c walks chain c's k-th listed row.
__global__ __launch_bounds__(64) void k_walk1(Rows rows, float T, Work w) {
    __shared__ WalkShared sh;
    const int c = blockIdx.x % w.chains, k = blockIdx.x / w.chains;
    if (k >= need_count(rows, w, c)) return;
    const int r = need_row(rows, w, c, k);
    walk_row<false>(pass1_eval(rows, r, w.row_m[r], T), w, r, sh);
}




// --------------------------------------------------------------- the find

struct FindShared {
    FoldShared fold;
    int item;
    float sst[kMaxSegs], send[kMaxSegs];   // segment starts and ends
    int scnt[kMaxSegs];                      // runs per segment (-1: replayed exactly)
    Item it[kItemCap];                       // the segment's runs,
    float ist[kItemCap], iend[kItemCap];     // their starts and ends
    float dst[kT];                           // a staged run's chunk starts
};

// First element i of the row with thr < (running value after i), from the
// walk's exact starts; dflt when the row sum does not exceed thr.
template <int KIND>
__device__ int find_row(const Eval<KIND>& ev, const Work& w, int row, float thr, int dflt,
                        FindShared& sh) {
    const int t = threadIdx.x;
    const float* ss = w.seg_start + (size_t)row * (w.nseg + 1);
    // each search step loads everything its successor needs from the step's
    // answer in one round trip: the segments' starts, ends and run counts,
    // then the segment's runs with their starts and ends, then a staged
    // run's chunk starts (the choices travel through LDS)
    if (t < w.nseg) {
        sh.sst[t] = ss[t];
        sh.send[t] = ss[t + 1];
        sh.scnt[t] = w.cnt[2 * segi(w, row, t)];
    }
    const int seg = block_first256(t < w.nseg && thr < sh.send[t < w.nseg ? t : 0], sh.fold.i);
    if (seg >= w.nseg) return dflt;
    const size_t si = segi(w, row, seg);
    const int n = sh.scnt[seg];
    const int segbase = seg * kSeg;
    int j0 = segbase, j1 = min(segbase + kSeg, ev.V);
    float s0 = sh.sst[seg];
    if (n >= 0) {
        const Item* its = w.items + si * kItemCap;
        const float* is = w.item_start + si * kItemCap;
        const float segend = sh.send[seg];
        if (t < n) {
            sh.it[t] = its[t];
            sh.ist[t] = is[t];
            sh.iend[t] = t + 1 < n ? is[t + 1] : segend;
        }
        const int i = block_first256(t < n && thr < sh.iend[t < n ? t : 0], sh.fold.i);
        if (i >= n) return dflt;
        const Item it = sh.it[i];
        const int cnext = i + 1 < n ? sh.it[i + 1].chunk : kT;
        s0 = sh.ist[i];
        if (it.binade == kDirty) {
            // staged run: the walk left the exact start of each of its chunks
            const int nc = cnext - it.chunk;
            const float* ds = w.dirty_start + si * kDirtyCap + it.slot;
            float cend = 0.0f;
            if (t < nc) {
                sh.dst[t] = ds[t];
                cend = t + 1 < nc ? ds[t + 1] : sh.iend[i];
            }
            const int ch = block_first256(t < nc && thr < cend, sh.fold.i);
            if (ch >= nc) return dflt;
            s0 = sh.dst[ch];
            j0 = segbase + (it.chunk + ch) * kC;
            j1 = min(j0 + kC, ev.V);
        } else {
            // clean run [c0, c1): exact chunk ends from the chunk summaries
            // that the fold left (the same summaries the run's total came from)
            const int c0 = it.chunk, c1 = cnext;
            const bool mine = t >= c0 && t < c1;
            const MI own = mine ? w.chunk_mi[((size_t)(row - w.R1) * w.nseg + seg) * kT + t]
                                : mi_id();
            SMI sv{own, 0};
            sv = wave_incl_smi(sv);
            __syncthreads();
            if (lane_id() == 63) sh.fold.wagg[wave_id()] = sv;
            __syncthreads();
            MI pre = mi_id();
#pragma unroll
            for (int ww = 0; ww < kW - 1; ww++)
                if (ww < wave_id()) pre = mi_then(pre, sh.fold.wagg[ww].m);
            const MI incl = mi_then(pre, sv.m);
            const float cend = mine ? mi_apply(s0, incl) : 0.0f;
            sh.dst[t] = cend;
            const int ch = block_first256(mine && thr < cend, sh.fold.i);
            if (ch >= c1) return dflt;
            // start of chunk ch: the end of chunk ch - 1, or the run's start
            s0 = ch > c0 ? sh.dst[ch - 1] : s0;
            j0 = segbase + ch * kC;
            j1 = min(j0 + kC, ev.V);
        }
    }
    // exact replay of [j0, j1) from s0 by wave 0 (padding lanes add +0.0 and
    // cannot be the first to exceed thr)
    if (wave_id() == 0) {
        int hit = -1;
        float s = s0;
        for (int j = j0; j < j1 && hit < 0; j += 64) {
            const float x = j + lane_id() < j1 ? ev.at(j + lane_id()) : 0.0f;
#pragma unroll
            for (int k = 0; k < 64; k++) {
                s = __fadd_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k)));
                if (hit < 0 && thr < s) hit = j + k;
            }
        }
        if (lane_id() == 0) sh.item = hit;
    }
    __syncthreads();
    return sh.item < 0 ? dflt : sh.item;
}

// Pass 2 of a chain: wave 0 walks the task row (exact starts, the sum R),
// then the block finds the draw in it -- one launch for both.
__global__ __launch_bounds__(kT) void k_walk2(Rows rows, float T, Work w,
                                              int* __restrict__ out_tokens) {
    __shared__ union {
        WalkShared walk;
        FindShared find;
    } sh;
    const int c = blockIdx.x;
    const Task tk = w.task[c];
    if (tk.kind < 0) return;
    const int row = w.R1 + c;
    if (wave_id() == 0) {
        if (tk.kind == kKindProb)
            walk_row<true>(task_eval<kKindProb>(rows, w, tk, T), w, row, sh.walk);
        else
            walk_row<true>(task_eval<kKindRes>(rows, w, tk, T), w, row, sh.walk);
    }
    __syncthreads();          // the walk's starts and sum, for every wave
    const float R = w.row_S[row];
    int tok;
    if (tk.kind == kKindRes) {
        if (R < 1e-10f) {
            // speculative.c:157-160: softmax of p instead (exact path)
            if (threadIdx.x == 0) w.flags[c] = 2;
            return;
        }
        tok = find_row(task_eval<kKindRes>(rows, w, tk, T), w, row, __fmul_rn(tk.u, R), 0,
                       sh.find);
    } else {
        tok = find_row(task_eval<kKindProb>(rows, w, tk, T), w, row, tk.u, rows.V - 1, sh.find);
    }
    if (threadIdx.x == 0) out_tokens[(size_t)c * (rows.gamma + 1) + tk.j] = tok;
}

// ------------------------------------------------------------ fallback

// Chains the pipeline left (non-finite rows, residual mass < 1e-10): the
// exact single-block samplers of eos.hpp, positions in order.
__global__ __launch_bounds__(kThreads) void k_verify_fallback(
    Rows rows, const int* __restrict__ tokens, const float* __restrict__ u, float T, Work w,
    float* __restrict__ accept_prob, int* __restrict__ out_tokens,
    int* __restrict__ n_accepted) {
    __shared__ EosShared sh;
    const int c = blockIdx.x, gamma = rows.gamma, V = rows.V, per = 2 * gamma + 1;
    const int flag = w.flags[c];
    if (flag == 0) return;
    const float* uu = u + (size_t)c * (gamma + 1);
    int* out = out_tokens + (size_t)c * (gamma + 1);
    if (flag == 2) {
        // the accept tests stand; only the correction draw changes
        const Task tk = w.task[c];
        RowSrc ts{rows.row(tk.ra)}, ds{rows.row(tk.rb)};
        ExpGen<RowSrc> et{ts, w.row_m[tk.ra], T}, ed{ds, w.row_m[tk.rb], T};
        DivGen<ExpGen<RowSrc>> pt{et, w.row_S[tk.ra]}, pd{ed, w.row_S[tk.rb]};
        const int tok = sample_corrected_gen(pt, pd, V, tk.u, sh);
        if (threadIdx.x == 0) out[tk.j] = tok;
        return;
    }
    int j = gamma;
    for (int i = 0; i < gamma; i++) {
        RowSrc ts{rows.row(c * per + i)}, ds{rows.row(c * per + gamma + 1 + i)};
        const float mt = gen_max(ts, V, sh), md = gen_max(ds, V, sh);
        ExpGen<RowSrc> et{ts, mt, T}, ed{ds, md, T};
        const float St = eos_sum(et, V, sh), Sd = eos_sum(ed, V, sh);
        DivGen<ExpGen<RowSrc>> pt{et, St}, pd{ed, Sd};
        const int x = tokens[(size_t)c * gamma + i];
        float a = 0.0f;   // a draft token outside [0, V) is rejected
        if (x >= 0 && x < V) {
            const float px = gen_at(pt, x, sh), qx = gen_at(pd, x, sh);
            a = qx < 1e-10f ? 1.0f : fminf(1.0f, __fdiv_rn(px, qx));
        }
        if (threadIdx.x == 0) accept_prob[(size_t)c * gamma + i] = a;
        if (j == gamma && !(uu[i] < a)) {
            j = i;
            const int tok = sample_corrected_gen(pt, pd, V, uu[i + 1], sh);
            if (threadIdx.x == 0) out[i] = tok;
        }
    }
    if (j == gamma) {
        const int tok = sample_temperature_gen(RowSrc{rows.row(c * per + gamma)}, V, T,
                                               uu[gamma], sh);
        if (threadIdx.x == 0) out[gamma] = tok;
    }
    if (threadIdx.x == 0) {
        for (int i = 0; i < gamma + 1; i++) {
            if (i < j) out[i] = tokens[(size_t)c * gamma + i];
            else if (i > j) out[i] = -1;
        }
        n_accepted[c] = j;
    }
}

}  // namespace vp
}  // namespace

// ------------------------------------------------------------- launcher

// pass-1 workgroups (segments x rows) from which calls without accept_prob
// take the certified decisions
static int g_lean_min_blocks = 2048;

extern "C" int cgx_verify_lean_min_blocks(int blocks) {
    const int old = g_lean_min_blocks;
    if (blocks >= 0) g_lean_min_blocks = blocks;
    return old;
}

// (the pass-1 grids take one row per y index: at most 65535 rows)
extern "C" int cgk_verify_pipe_supported(int batch, int gamma, int V, float T) {
    return batch >= 1 && gamma >= 0 && gamma <= vp::kMaxGamma &&
           (long long)batch * (2 * gamma + 1) <= 65535 && V >= 1 &&
           V <= kRound * kMaxRounds && T > 0.0f && T <= FLT_MAX;
}

// Workspace of the allocation-free entry point (cgk_verify_pipe_static): a
// file-scope device array.  Each GPU it is used on holds its own copy at its
// own address until the process ends; host code reaches it only through the
// address hipGetSymbolAddress returns with that device current.
constexpr size_t kStaticWsBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kStaticWsBytes];
constexpr int kMaxDevices = 64;
static void* g_static_ws[kMaxDevices];

extern "C" int cgk_verify_static_init(int device) {
    if (device < 0 || device >= kMaxDevices) {
        cgx_set_error("verify workspace: device %d outside 0..%d", device, kMaxDevices - 1);
        return -1;
    }
    if (g_static_ws[device]) return 0;
    // the symbol's address on `device`: that device current for the lookup,
    // the caller's current device restored after it
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) {
        (void)hipGetLastError();
        cgx_set_error("verify workspace: no current device");
        return -1;
    }
    if (cur != device && hipSetDevice(device) != hipSuccess) {
        (void)hipGetLastError();
        cgx_set_error("verify workspace: device %d cannot be made current", device);
        return -1;
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != device) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        cgx_set_error("verify workspace: hipGetSymbolAddress failed on device %d: %s", device,
                      hipGetErrorString(e));
        return -1;
    }
    g_static_ws[device] = p;
    return 0;
}

// ws_fixed: a caller-provided workspace of ws_cap bytes instead of the
// library's grow-only scratch.
static int verify_pipe(const float* target, size_t ldt, const float* draft, const int* tokens,
                       const float* u, int batch, int gamma, int V, float T, float* accept_prob,
                       int* out_tokens, int* n_accepted, char* ws_fixed = nullptr,
                       size_t ws_cap = 0) {
    using namespace vp;
    if (!cgk_verify_pipe_supported(batch, gamma, V, T)) {
        cgx_set_error("verify: batch %d, gamma %d, V %d, T %g outside the pipeline's range",
                      batch, gamma, V, (double)T);
        return -1;
    }
    const int nseg = (V + kSeg - 1) / kSeg;
    const int R1 = batch * (2 * gamma + 1), Rall = R1 + batch;
    // workspace carve (256-byte aligned pieces)
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) & ~(size_t)255;
        return o;
    };
    const size_t o_segm = take((size_t)R1 * nseg * 4);
    const size_t o_seggh = take((size_t)R1 * nseg * 16);
    const size_t o_segbad = take((size_t)R1 * nseg * 4);
    const size_t o_rowm = take((size_t)R1 * 4);
    const size_t o_rowS = take((size_t)Rall * 4);
    const size_t o_cnt = take((size_t)Rall * nseg * 8);
    const size_t o_items = take((size_t)Rall * nseg * kItemCap * sizeof(Item));
    const size_t o_dirty = take((size_t)Rall * nseg * kDirtyCap * kC * 4);
    const size_t o_sst = take((size_t)Rall * (nseg + 1) * 4);
    const size_t o_ist = take((size_t)Rall * nseg * kItemCap * 4);
    const size_t o_dst = take((size_t)Rall * nseg * kDirtyCap * 4);
    const size_t o_tge = take((size_t)batch * nseg * 16);
    const size_t o_cmi = take((size_t)batch * nseg * kT * sizeof(MI));
    const size_t o_task = take((size_t)batch * sizeof(Task));
    const size_t o_flags = take((size_t)batch * 4);
    const size_t o_ap = take((size_t)batch * gamma * 4);
    const size_t o_n = take((size_t)batch * 4);
    const size_t o_need = take((size_t)batch * (2 * gamma + 2) * 4);
    const size_t o_pre = take((size_t)batch * gamma * 4 + 4);
    if (ws_fixed && off > ws_cap) {
        cgx_set_error("verify: batch %d, gamma %d, V %d needs %zu bytes of workspace, above "
                      "the static maximum of %zu", batch, gamma, V, off, ws_cap);
        return -1;
    }
    char* ws = ws_fixed ? ws_fixed : (char*)cgx_scratch(CGX_SLOT_WS4, off);
    if (!ws) return -1;
    Work w;
    w.R1 = R1;
    w.chains = batch;
    w.nseg = nseg;
    w.seg_m = (float*)(ws + o_segm);
    w.seg_gh = (double*)(ws + o_seggh);
    w.seg_bad = (int*)(ws + o_segbad);
    w.row_m = (float*)(ws + o_rowm);
    w.row_S = (float*)(ws + o_rowS);
    w.cnt = (int*)(ws + o_cnt);
    w.items = (Item*)(ws + o_items);
    w.dirty = (float*)(ws + o_dirty);
    w.seg_start = (float*)(ws + o_sst);
    w.item_start = (float*)(ws + o_ist);
    w.dirty_start = (float*)(ws + o_dst);
    w.chunk_mi = (MI*)(ws + o_cmi);
    w.task_ge = (double*)(ws + o_tge);
    w.task = (Task*)(ws + o_task);
    w.flags = (int*)(ws + o_flags);
    // Without accept_prob only the emitted tokens are asked for: the accept
    // tests the segment stats settle need no exact sums (certified decisions),
    // and the exact fold and walk run only over the rows still needed.
    // (Only where the pass-1 grid is large: on a small one every kernel runs
    // at its latency, and the extra launch costs more than the work saved.)
    const bool lean = accept_prob == nullptr && gamma > 0 &&
                      (long long)nseg * R1 >= g_lean_min_blocks;
    w.need = lean ? (int*)(ws + o_need) : nullptr;
    w.pre = lean ? (int*)(ws + o_pre) : nullptr;
    float* ap = accept_prob ? accept_prob : (float*)(ws + o_ap);
    if (!n_accepted) n_accepted = (int*)(ws + o_n);
    Rows rows{target, draft, gamma, V, ldt};
    hipStream_t st = stream();
    hipLaunchKernelGGL(k_seg_stats, dim3(nseg, R1), dim3(kT), 0, st, rows, T, w);
    if (launch_check("k_seg_stats")) return -1;
    if (lean) {
        const int nt = min(kPreThreads, 64 * (2 * gamma + 1));
        hipLaunchKernelGGL(k_pre_decide, dim3(batch), dim3(nt), 0, st, rows, tokens, u, T, w);
        if (launch_check("k_pre_decide")) return -1;
    }
    hipLaunchKernelGGL(k_seg_fold1, dim3(nseg, R1), dim3(kT), 0, st, rows, T, w);
    if (launch_check("k_seg_fold1")) return -1;
    hipLaunchKernelGGL(k_walk1, dim3(R1), dim3(64), 0, st, rows, T, w);
    if (launch_check("k_walk1")) return -1;
    hipLaunchKernelGGL(k_res_stats, dim3(nseg, batch), dim3(kT), 0, st, rows, tokens, u, T, w,
                       lean ? nullptr : ap, out_tokens, n_accepted);
    if (launch_check("k_res_stats")) return -1;
    // a grid of at most one block per CU runs at its blocks' latency: the
    // wave-shared exact evaluations then; the per-lane ones on a larger grid
    if ((long long)nseg * batch <= kCompactMaxBlocks)
        hipLaunchKernelGGL(k_seg_fold2<true>, dim3(nseg, batch), dim3(kT), 0, st, rows, T, w);
    else
        hipLaunchKernelGGL(k_seg_fold2<false>, dim3(nseg, batch), dim3(kT), 0, st, rows, T, w);
    if (launch_check("k_seg_fold2")) return -1;
    hipLaunchKernelGGL(k_walk2, dim3(batch), dim3(kT), 0, st, rows, T, w, out_tokens);
    if (launch_check("k_walk2")) return -1;
    hipLaunchKernelGGL(k_verify_fallback, dim3(batch), dim3(kThreads), 0, st, rows, tokens, u,
                       T, w, ap, out_tokens, n_accepted);
    return launch_check("k_verify_fallback");
}

extern "C" int cgk_verify_pipe(const float* target, const float* draft, const int* tokens,
                               const float* u, int batch, int gamma, int V, float T,
                               float* accept_prob, int* out_tokens, int* n_accepted) {
    return verify_pipe(target, (size_t)V, draft, tokens, u, batch, gamma, V, T, accept_prob,
                       out_tokens, n_accepted);
}

// The same pipeline with its workspace in the static array of the current
// device: no allocation, every call on one GPU shares the array.
extern "C" int cgk_verify_pipe_static(int device, const float* target, const float* draft,
                                      const int* tokens, const float* u, int batch, int gamma,
                                      int V, float T, float* accept_prob, int* out_tokens,
                                      int* n_accepted) {
    if (cgk_verify_static_init(device)) return -1;
    return verify_pipe(target, (size_t)V, draft, tokens, u, batch, gamma, V, T, accept_prob,
                       out_tokens, n_accepted, (char*)g_static_ws[device], kStaticWsBytes);
}

// cg_sample_temperature on `rows` rows at once through the same pipeline: a
// verify with no drafted tokens is exactly the bonus draw from target row 0
// (speculative.c:54-75).  Row r at logits + r * ld; u: one draw per row
// (device); out: one token per row.
extern "C" int cgk_sample_temperature_pipe(const float* logits, int rows, int V, float T,
                                           const float* u, int* out, size_t ld) {
    return verify_pipe(logits, ld, logits, nullptr, u, rows, 0, V, T, nullptr, out, nullptr);
}
