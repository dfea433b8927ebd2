// filter.hip -- top-k and top-p (nucleus) filtering on gfx950, bit-identical
// to cogito's CPU samplers (src/inference/speculative.c).
//
//   cg_sample_top_k  :122-146  insertion top-k with strict '>' against a
//                              -1e30 floor (ties: the lower index is kept
//                              and ordered first), then cg_sample_temperature
//                              over the k values at T = 1
//   cg_sample_top_p  :77-120   softmax (T = 1); O(V^2) selection sort that
//                              swaps on every strictly larger element; first
//                              i with cumsum >= p; r = u * cumsum; scan
//
// Top-k: one workgroup per row.  A 4-pass radix select over order-preserving
// 32-bit keys finds the k-th largest key; elements above it plus the
// lowest-index ties at it are the reference's list, which a bitonic sort in
// LDS orders by (value desc, index asc).
//
// Top-p: probabilities (exact expf and ordered sum), a radix sort of the
// values (rowsort.hip), the exact sequential cumsum over the sorted values for
// the cutoff and the draw, and the reference's tie order for the one tie group
// that matters.  The selection sort's order of equal values is not stable
// but follows a rule that depends only on counts: let the members of the
// group of value v be i_1 < ... < i_n and g_t the number of elements > v
// after i_t and before i_(t+1) (g_n: after i_n).  Start with R = [], then
// for t = 1..n append i_t and rotate R left by g_t (mod t).  R is the order
// in which the sort emits the group.  (Each pass of the sort moves the chain
// of strict running maxima one record slot to the right; for the smallest
// value v present, only its leading run moves, and each pass that consumes an
// element > v behind that run rotates it by one.)
#include <hip/hip_runtime.h>

#include <cfloat>
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

constexpr int kTopKMax = 4096;         // top-k: list held in LDS
constexpr float kTopKFloor = -1e30f;   // speculative.c:128

// Order-preserving key of a float; -0 and +0 map to the same key.
__device__ __forceinline__ uint32_t order_key(float x) {
    uint32_t b = __float_as_uint(x);
    if ((b & 0x7fffffffu) == 0) b = 0;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Largest float below x: `s >= x` is `x_below < s` for finite fp32 s.
__device__ __forceinline__ float float_below(float x) {
    if (x != x || x == -__builtin_inff()) return x;
    if (x == 0.0f) return -0x1p-149f;
    uint32_t b = __float_as_uint(x);
    return __uint_as_float(x > 0.0f ? b - 1 : b + 1);
}

// Exclusive block scan of one int per thread (1024 threads); *total gets the
// sum.  `lds` holds kWaves ints.
__device__ __forceinline__ int block_excl_scan(int v, int* total, int* lds) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    __syncthreads();
    if (lane == 63) lds[w] = x;
    __syncthreads();
    int off = 0, tot = 0;
    for (int i = 0; i < kWaves; i++) {
        int s = lds[i];
        if (i < w) off += s;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return off + x - v;
}

__device__ __forceinline__ int block_sum_int(int v, int* lds) {
    int tot;
    block_excl_scan(v, &tot, lds);
    return tot;
}

// Sums of four ints over the block (`lds` holds kWaves int4).
__device__ __forceinline__ int4 block_sum_int4(int4 v, int4* lds) {
    for (int o = 32; o > 0; o >>= 1) {
        v.x += __shfl_xor(v.x, o);
        v.y += __shfl_xor(v.y, o);
        v.z += __shfl_xor(v.z, o);
        v.w += __shfl_xor(v.w, o);
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    int4 r = make_int4(0, 0, 0, 0);
    for (int w = 0; w < kWaves; w++) {
        const int4 a = lds[w];
        r.x += a.x;
        r.y += a.y;
        r.z += a.z;
        r.w += a.w;
    }
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------- top-p

// z / T, elementwise (the filtered distribution's first step).
__global__ void k_scale(const float* __restrict__ x, float* __restrict__ z, size_t n, float T) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) z[i] = __fdiv_rn(x[i], T);
}

// Softmax at T = 1 of each row of z = x / T (speculative.c:81-90): max,
// expf(z - max), running fp32 sum, division.  The rows of x are divided by T
// as they are read (k_scale's operation, so z is never stored).
__global__ __launch_bounds__(kThreads) void k_probs_rows(const float* __restrict__ x, int V,
                                                         float T, float* __restrict__ probs) {
    __shared__ EosLds lds;
    EosShared& sh = lds.sh;
    ScaledSrc src{x + (size_t)blockIdx.x * V, T};
    float* pr = probs + (size_t)blockIdx.x * V;
    if (V <= kRound) {
        // one round: the row and its exponentials stay in registers; the
        // probabilities are written through the staging area
        float x[kCh], e[kCh];
        load_vals(src, V, -__builtin_inff(), x);
        const float m = vals_max(x, sh);
        vals_exp(x, m, 1.0f, V, e);
        const float S = eos_sum_vals(e, ExpGen<ScaledSrc>{src, m, 1.0f}, V, sh);
#pragma unroll
        for (int k = 0; k < kCh; k++) e[k] = __fdiv_rn(e[k], S);
        store_vals(pr, V, e, lds.tr);
        return;
    }
    float m = gen_max(src, V, sh);
    ExpGen<ScaledSrc> e{src, m, 1.0f};
    // the exponentials are evaluated once, into the output row, and summed
    // from there
    for (int j = threadIdx.x; j < V; j += kThreads) pr[j] = e(j);
    __threadfence_block();
    __syncthreads();
    float S = eos_sum(RowSrc{pr}, V, sh);
    for (int j = threadIdx.x; j < V; j += kThreads) pr[j] = __fdiv_rn(pr[j], S);
}

// The tie group {j : p[j] == v} in index order: member indices -> wi[0..m),
// number of elements > v before each member -> wc[0..m).  Returns m; the
// count of elements > v in the whole row goes to *gt_total.
__device__ int tie_members(const float* p, int V, float v, int* wi, int* wc, int* gt_total,
                           int* lds) {
    const int per = (V + kThreads - 1) / kThreads;
    const int lo = threadIdx.x * per, hi = min(V, lo + per);
    int eq = 0, gt = 0;
    for (int j = lo; j < hi; j++) {
        float x = p[j];
        eq += x == v;
        gt += x > v;
    }
    int m, gtt;
    int e = block_excl_scan(eq, &m, lds);
    int g = block_excl_scan(gt, &gtt, lds);
    for (int j = lo; j < hi; j++) {
        float x = p[j];
        if (x == v) {
            wi[e] = j;
            wc[e] = g;
            e++;
        } else if (x > v) {
            g++;
        }
    }
    __syncthreads();
    *gt_total = gtt;
    return m;
}

// g_t of the tie rule for 1-based t.
__device__ __forceinline__ int tie_gap(const int* wc, int m, int gtt, int t) {
    return (t < m ? wc[t] : gtt) - wc[t - 1];
}

// Length of the shortest prefix of the non-negative values s[0..V) (whole
// chunks of kCh, V <= kRound; this thread's chunk in x, zero past V) whose
// sequential fp32 sum certainly exceeds thr, V when none: the fp64 sum P
// through chunk t bounds the fp32 running sum from below by P (1 - delta_t),
// the bound of the exact sum's guide for (t + 1) kCh additions of
// non-negative values.
__device__ __forceinline__ int certified_prefix(const float (&x)[kCh], int V, float thr,
                                                EosShared& sh) {
    const int t = threadIdx.x;
    double gs = 0.0;
#pragma unroll
    for (int k = 0; k < kCh; k++) gs += (double)x[k];
    const double inc = wave_incl_sum_d(gs);
    if (t == 0) sh.result = kThreads;
    if (lane_id() == 63) sh.wsum[wave_id()] = inc;
    __syncthreads();
    double wpre = 0.0;
    for (int w = 0; w < wave_id(); w++) wpre += sh.wsum[w];
    const double delta = (double)(t * kCh + kCh + 1) * 0x1p-24 * (1.0 + 0x1p-7) + 0x1p-40;
    if (t * kCh < V && (wpre + inc) * (1.0 - delta) > (double)thr) atomicMin(&sh.result, t);
    __syncthreads();
    const int first = sh.result;
    __syncthreads();
    return first >= kThreads ? V : min(V, (first + 1) * kCh);
}

// Cutoff, draw and the filtered distribution of top-p over one row: `probs`
// (index order) and `sorted` (descending).  Rows r with (r + 1) % tok_every
// == 0 draw a token (tokens[r / tok_every], draw u[(r / tok_every) *
// u_stride]; tok_every 0: none); every row writes its distribution when
// dist is given.  ws holds 2V ints per row.
__global__ __launch_bounds__(kThreads) void k_top_p_finish(
    const float* __restrict__ probs, const float* __restrict__ sorted, int V, float top_p,
    const float* __restrict__ u, int u_stride, int* __restrict__ tokens, int tok_every,
    float* __restrict__ dist, int* __restrict__ ws) {
    __shared__ EosShared sh;
    __shared__ int lds[kWaves];
    __shared__ int4 lds4[kWaves];
    __shared__ int s_tok;
    const int row = blockIdx.x;
    const float* pr = probs + (size_t)row * V;
    const float* sr = sorted + (size_t)row * V;
    int* wi = ws + (size_t)row * 2 * V;
    int* wc = wi + V;
    RowSrc s{sr};
    // The cumsum of the descending values: a sequential sum is a prefix of
    // the longer one, so only the certified prefix that passes the threshold
    // is summed (the cutoff and the draw lie inside it); this also keeps the
    // exact sum away from the binade boundary at 1 that the whole row's sum
    // approaches.  The whole row when no prefix is certified (or V > kRound).
    const float thr = float_below(top_p);       // cumsum >= top_p <=> thr < cumsum
    int n = V;
    float total;
    if (V <= kRound) {
        // the sorted row is read once for the certified prefix and its exact
        // sum
        float x[kCh];
        load_vals(s, V, 0.0f, x);
        n = certified_prefix(x, V, thr, sh);
        const int base = threadIdx.x * kCh;
#pragma unroll
        for (int k = 0; k < kCh; k++) x[k] = base + k < n ? x[k] : 0.0f;
        total = eos_sum_vals(x, s, n, sh);
    } else {
        total = eos_sum(s, n, sh);
    }
    if (n < V && !(thr < total)) {              // excluded by the bound; kept as a guard
        n = V;
        total = eos_sum(s, n, sh);
    }
    float C;
    const int ci = gen_find_val(s, n, thr, -1, total, &C, sh);
    const int cutoff = ci < 0 ? V : ci + 1;

    // The token (speculative.c:109-115: r = u * cumsum; first i < cutoff with
    // r < cumsum) is the sorted entry at `pos`; the distribution keeps the
    // first `cutoff` sorted entries, divided by the kept mass C.  One pass
    // over the row in index order serves both: it writes the distribution
    // (every element >= vc kept, right unless the tie group of vc is cut),
    // finds the element holding the token's value and counts the elements
    // above and equal to both values.
    const bool want_tok = tokens && tok_every > 0 && (row + 1) % tok_every == 0;
    const int ti = want_tok ? row / tok_every : 0;
    int pos = 0;
    if (want_tok) {
        const float r = __fmul_rn(u[(size_t)ti * u_stride], C);
        pos = gen_find(s, n, r, 0, sh);
        if (pos >= cutoff) pos = 0;
    }
    const float v = want_tok ? sr[pos] : 0.0f;
    const float vc = sr[cutoff - 1];
    float* dr = dist ? dist + (size_t)row * V : nullptr;
    // counts of the elements == v, > v, > vc, == vc; rows of at most kRound
    // elements keep their values in registers for the writes below
    int4 c = make_int4(0, 0, 0, 0);
    float xv[kCh];
    auto count = [&](int j, float x) {
        if (want_tok && x == v) s_tok = j;
        c.x += x == v;
        c.y += x > v;
        c.z += x > vc;
        c.w += x == vc;
    };
    if (V <= kRound) {
#pragma unroll
        for (int i = 0; i < kCh; i++) {
            const int j = (int)threadIdx.x + i * kThreads;
            xv[i] = j < V ? pr[j] : -1.0f;
        }
#pragma unroll
        for (int i = 0; i < kCh; i++)
            if ((int)threadIdx.x + i * kThreads < V) count((int)threadIdx.x + i * kThreads, xv[i]);
    } else {
        for (int j = threadIdx.x; j < V; j += kThreads) count(j, pr[j]);
    }
    const int4 cnt = block_sum_int4(c, lds4);

    if (want_tok) {
        // a value held by one element: that element (s_tok, written by it);
        // otherwise the reference's emission order of the tie group
        if (cnt.x > 1) {
            const int rank = pos - cnt.y;
            int gtt;
            int m = tie_members(pr, V, v, wi, wc, &gtt, lds);
            if (threadIdx.x == 0) {
                // walk the rotations backwards from the final slot `rank`
                int p = rank, tok = wi[0];
                for (int t = m; t >= 1; t--) {
                    p = (int)(((long long)p + tie_gap(wc, m, gtt, t)) % t);
                    if (p == t - 1) {
                        tok = wi[t - 1];
                        break;
                    }
                }
                s_tok = tok;
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) tokens[ti] = s_tok;
    }
    if (!dr) return;

    // the kept elements are those > vc and, when the whole tie group of vc
    // is kept, those == vc
    const int kept_in_group = cutoff - cnt.z;
    const bool whole = kept_in_group >= cnt.w;
    auto keep = [&](float x) { return (x > vc || (whole && x == vc)) ? __fdiv_rn(x, C) : 0.0f; };
    if (V <= kRound) {
#pragma unroll
        for (int i = 0; i < kCh; i++) {
            const int j = (int)threadIdx.x + i * kThreads;
            if (j < V) dr[j] = keep(xv[i]);
        }
    } else {
        for (int j = threadIdx.x; j < V; j += kThreads) dr[j] = keep(pr[j]);
    }
    __syncthreads();
    if (whole) return;
    // the first kept_in_group members of the group in the sort's emission
    // order are kept
    int gtt;
    int m = tie_members(pr, V, vc, wi, wc, &gtt, lds);
    const float val = __fdiv_rn(vc, C);
    for (int tt = threadIdx.x; tt < m; tt += kThreads) {
        int p = tt;
        for (int t = tt + 1; t <= m; t++) {
            int g = tie_gap(wc, m, gtt, t) % t;
            p = (p - g + t) % t;
        }
        if (p < kept_in_group) dr[wi[tt]] = val;
    }
}

// ---------------------------------------------------------------- top-k

__device__ __forceinline__ unsigned long long topk_entry(uint32_t key, int j) {
    return ((unsigned long long)key << 32) | (0xFFFFFFFFu - (uint32_t)j);
}

// Top-k over one row of z (k < V, k <= kTopKMax), then either a token
// (cg_sample_top_k; with top_p < 1 the nucleus rule over the list) or the
// filtered distribution (dense row).
__global__ __launch_bounds__(kThreads) void k_top_k(const float* __restrict__ z, int V, int k,
                                                    int kpow2, float top_p,
                                                    const float* __restrict__ u, int u_stride,
                                                    int* __restrict__ tokens, int tok_every,
                                                    float* __restrict__ dist,
                                                    int* __restrict__ lidx,
                                                    float* __restrict__ lp,
                                                    const unsigned long long* __restrict__ gcand,
                                                    const int* __restrict__ gstate) {
    __shared__ EosShared sh;
    __shared__ unsigned long long cand[kTopKMax];
    // radix passes: one histogram per wave (fewer same-address atomics), in
    // the candidate buffer, which is filled only after the passes
    static_assert(kWaves * 256 * sizeof(int) <= sizeof(cand), "histograms fit in cand");
    int (*hist)[256] = reinterpret_cast<int (*)[256]>(cand);
    __shared__ int lds[kWaves];
    __shared__ int s_digit, s_need, s_ncand;
    const int row = blockIdx.x, t = threadIdx.x, wv = t >> 6;
    const float* zr = z + (size_t)row * V;
    const uint32_t kfloor = order_key(kTopKFloor);

    // The row is read in coalesced sweeps of kU values per thread, whose loads
    // are all in flight before any is used.
    constexpr int kU = 8;
    auto sweep = [&](auto&& fn) {
        for (int j0 = t; j0 < V; j0 += kThreads * kU) {
            float xs[kU];
#pragma unroll
            for (int q = 0; q < kU; q++) {
                const int j = j0 + q * kThreads;
                xs[q] = j < V ? zr[j] : kTopKFloor;
            }
#pragma unroll
            for (int q = 0; q < kU; q++) fn(xs[q], j0 + q * kThreads);
        }
    };

    // candidates gathered by the multi-workgroup pass (k_topk_hist /
    // k_topk_collect): every eligible key in or above the k-th largest key's
    // 12-bit bin, in any order (the sort below orders them)
    const int gn = gcand ? gstate[4 * row] : -1;
    if (gn >= 0) {
        for (int i = t; i < gn; i += kThreads) cand[i] = gcand[(size_t)row * kTopKMax + i];
        if (t == 0) s_ncand = gn;
    } else {
        // radix select of the k-th largest key among eligible elements (value >
        // -1e30: never inserted otherwise; NaN never is); the first pass also
        // counts them
        uint32_t prefix = 0, pmask = 0;
        int need = k, E = 0, ties = 0;
        bool all = false;
        for (int pass = 0; pass < 4; pass++) {
            const int shift = 24 - 8 * pass;
            for (int i = t; i < kWaves * 256; i += kThreads) (&hist[0][0])[i] = 0;
            __syncthreads();
            int elig = 0;
            sweep([&](float x, int) {
                const uint32_t key = order_key(x);
                if (x > kTopKFloor && (key & pmask) == prefix) {
                    atomicAdd(&hist[wv][(key >> shift) & 255], 1);
                    elig++;
                }
            });
            if (pass == 0) {
                E = block_sum_int(elig, lds);
                all = E <= k;
                if (all) break;
            }
            __syncthreads();
            // digit of the need-th largest: thread i holds bin 255 - i; an
            // exclusive scan from the top bin down finds the bin where the count
            // reaches `need`
            int h = 0;
            if (t < 256) {
    #pragma unroll
                for (int w = 0; w < kWaves; w++) h += hist[w][255 - t];
            }
            int above;
            const int excl = block_excl_scan(h, &above, lds);
            if (t < 256 && excl < need && need <= excl + h) {
                s_digit = 255 - t;
                s_need = need - excl;
                s_ncand = h;                // after the last pass: the keys equal to T
            }
            __syncthreads();
            prefix |= (uint32_t)s_digit << shift;
            pmask |= 0xFFu << shift;
            need = s_need;
            ties = s_ncand;
            __syncthreads();
        }
        const uint32_t T = prefix;              // key of the k-th largest

        // collect: every eligible key > T, then the first `need` keys == T by
        // index.  When every key == T fits next to the others, all of them are
        // collected and the sort by (value desc, index asc) keeps the first
        // `need`; otherwise each thread scans its own range in index order.
        const bool all_ties = all || (k - need) + ties <= kTopKMax;
        if (t == 0) s_ncand = 0;
        __syncthreads();
        sweep([&](float x, int j) {
            const uint32_t key = order_key(x);
            if (x > kTopKFloor && (all || key > T || (all_ties && key == T)))
                cand[atomicAdd(&s_ncand, 1)] = topk_entry(key, j);
        });
        if (!all && !all_ties) {
            const int per = (V + kThreads - 1) / kThreads;
            const int lo = t * per, hi = min(V, lo + per);
            int eq = 0;
            for (int j = lo; j < hi; j++) eq += (zr[j] > kTopKFloor && order_key(zr[j]) == T);
            int tot;
            int r = block_excl_scan(eq, &tot, lds);
            for (int j = lo; j < hi && r < need; j++) {
                float x = zr[j];
                if (x > kTopKFloor && order_key(x) == T) {
                    cand[atomicAdd(&s_ncand, 1)] = topk_entry(order_key(x), j);
                    r++;
                }
            }
        }

    }
    __syncthreads();
    const int ncand = s_ncand;
    // sort size: a power of two holding the list and every candidate
    int spow2 = kpow2;
    while (spow2 < ncand) spow2 <<= 1;
    // unfilled slots keep the reference's initial (-1e30, 0); sort padding last
    for (int i = ncand + t; i < spow2; i += kThreads)
        cand[i] = i < k ? topk_entry(kfloor, 0) : 0ull;
    __syncthreads();
    for (int kk = 2; kk <= spow2; kk <<= 1) {
        for (int jj = kk >> 1; jj > 0; jj >>= 1) {
            for (int p = t; p < spow2 / 2; p += kThreads) {
                int i = 2 * jj * (p / jj) + (p % jj);
                int l = i + jj;
                unsigned long long a = cand[i], b = cand[l];
                bool desc = (i & kk) == 0;
                if (desc ? (a < b) : (a > b)) {
                    cand[i] = b;
                    cand[l] = a;
                }
            }
            __syncthreads();
        }
    }
    // decode in place into vals[kTopKMax] | idx[kTopKMax]
    float rv[kTopKMax / kThreads];
    int ri[kTopKMax / kThreads];
#pragma unroll
    for (int q = 0; q < kTopKMax / kThreads; q++) {
        int i = t + q * kThreads;
        rv[q] = 0.0f;
        ri[q] = 0;
        if (i < k) {
            unsigned long long c = cand[i];
            uint32_t key = (uint32_t)(c >> 32);
            int j = (int)(0xFFFFFFFFu - (uint32_t)c);
            if (key == kfloor) {
                rv[q] = kTopKFloor;
                ri[q] = 0;
            } else {
                rv[q] = zr[j];
                ri[q] = j;
            }
        }
    }
    __syncthreads();
    float* vals = (float*)cand;
    int* idx = (int*)cand + kTopKMax;
#pragma unroll
    for (int q = 0; q < kTopKMax / kThreads; q++) {
        int i = t + q * kThreads;
        if (i < k) {
            vals[i] = rv[q];
            idx[i] = ri[q];
        }
    }
    __syncthreads();

    const bool use_p = top_p < 1.0f;
    RowSrc vs{vals};
    // this row's token (rows r with (r + 1) % tok_every == 0): tokens[ti]
    // with the draw u[ti * u_stride]
    const bool want_tok = tokens && tok_every > 0 && (row + 1) % tok_every == 0;
    const int ti = want_tok ? row / tok_every : 0;
    const bool more = dist || lidx;      // a distribution or list after the token
    if (want_tok && !use_p) {
        int j = sample_temperature_gen(vs, k, 1.0f, u[(size_t)ti * u_stride], sh);
        if (t == 0) tokens[ti] = idx[j];
        if (!more) return;
        __syncthreads();
    }
    // list probabilities: cg_sample_temperature's softmax at T = 1
    float m = gen_max(vs, k, sh);
    ExpGen<RowSrc> e{vs, m, 1.0f};
    float S = eos_sum(e, k, sh);
    DivGen<ExpGen<RowSrc>> pr{e, S};
    int keep = k;
    float mass = 1.0f;
    if (use_p) {
        float tot = eos_sum(pr, k, sh);
        int ci = gen_find_val(pr, k, float_below(top_p), -1, tot, &mass, sh);
        keep = ci < 0 ? k : ci + 1;
    }
    if (want_tok && use_p) {
        int j = gen_find(pr, k, __fmul_rn(u[(size_t)ti * u_stride], mass), 0, sh);
        if (j >= keep) j = 0;
        if (t == 0) tokens[ti] = idx[j];
        if (!more) return;
        __syncthreads();
    }
    if (lidx) {
        // the list itself: entry j of the row is (idx[j], probability); past
        // the top-p cutoff, and for the (-1e30, 0) fillers, the probability
        // is 0
        for (int j = t; j < k; j += kThreads) {
            float v = j < keep ? (use_p ? __fdiv_rn(pr(j), mass) : pr(j)) : 0.0f;
            lidx[(size_t)row * k + j] = idx[j];
            lp[(size_t)row * k + j] = v;
        }
        return;
    }
    if (!dist) return;
    float* dr = dist + (size_t)row * V;
    for (int j = t; j < V; j += kThreads) dr[j] = 0.0f;
    __syncthreads();
    // list indices are distinct except the (-1e30, 0) fillers, whose
    // probability is 0 and which are never written
    for (int j = t; j < keep; j += kThreads) {
        float v = use_p ? __fdiv_rn(pr(j), mass) : pr(j);
        if (v != 0.0f) dr[idx[j]] = v;
    }
}

// ------------------------------------------ top-k over many workgroups
// Rows of 16384 values and more: each row is cut into tiles of kTK values,
// one 256-thread workgroup per (tile, row).  k_topk_hist adds the tile's
// histogram of the top kHBits bits of the eligible keys into the row's;
// k_topk_collect finds, from the row's histogram, the bin of the k-th
// largest key and appends every eligible key of its tile in or above that
// bin to the row's candidate list (the sort in k_top_k orders them); a row
// whose bin would overflow the list (kTopKMax) is marked and k_top_k selects
// from the row itself.

constexpr int kTK = 4096;                 // values per tile
constexpr int kTKThreads = 256;
constexpr int kHBits = 12, kHBins = 1 << kHBits;
constexpr int kTKState = 4;               // per row: candidates (-1: select in k_top_k)

__global__ void k_topk_zero(int* __restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

__global__ __launch_bounds__(kTKThreads) void k_topk_hist(const float* __restrict__ z, int V,
                                                         int* __restrict__ hist) {
    __shared__ int h[kHBins];
    const int row = blockIdx.y, tile = blockIdx.x, t = threadIdx.x;
    for (int i = t; i < kHBins; i += kTKThreads) h[i] = 0;
    __syncthreads();
    const float* zr = z + (size_t)row * V + (size_t)tile * kTK;
    const int n = min(kTK, V - tile * kTK);
    float xs[kTK / kTKThreads];
#pragma unroll
    for (int q = 0; q < kTK / kTKThreads; q++) {
        const int j = q * kTKThreads + t;
        xs[q] = j < n ? zr[j] : kTopKFloor;
    }
#pragma unroll
    for (int q = 0; q < kTK / kTKThreads; q++)
        if (xs[q] > kTopKFloor) atomicAdd(&h[order_key(xs[q]) >> (32 - kHBits)], 1);
    __syncthreads();
    int* gh = hist + (size_t)row * kHBins;
    for (int i = t; i < kHBins; i += kTKThreads)
        if (h[i]) atomicAdd(&gh[i], h[i]);
}

__global__ __launch_bounds__(kTKThreads) void k_topk_collect(const float* __restrict__ z, int V,
                                                            int k, const int* __restrict__ hist,
                                                            int* __restrict__ state,
                                                            unsigned long long* __restrict__ gcand) {
    constexpr int kPer = kHBins / kTKThreads;          // bins per thread
    constexpr int kW = kTKThreads / 64;
    __shared__ int s_w[kW];
    __shared__ int s_bin, s_fast;
    const int row = blockIdx.y, tile = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const int* gh = hist + (size_t)row * kHBins;
    // thread t holds bins kHBins-1-kPer*t downwards; the exclusive scan in
    // thread order counts the keys above them
    int hb[kPer], hs = 0;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        hb[q] = gh[kHBins - 1 - kPer * t - q];
        hs += hb[q];
    }
    int x = hs;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) s_w[t >> 6] = x;
    if (t == 0) {
        s_bin = 0;                                     // at most k eligible: take them all
        s_fast = 1;
    }
    __syncthreads();
    int excl = x - hs, tot = 0;
    for (int w = 0; w < kW; w++) {
        if (w < (t >> 6)) excl += s_w[w];
        tot += s_w[w];
    }
    if (tot > k) {
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            if (excl < k && k <= excl + hb[q]) {
                s_bin = kHBins - 1 - kPer * t - q;
                s_fast = excl + hb[q] <= kTopKMax;
            }
            excl += hb[q];
        }
    }
    __syncthreads();
    if (!s_fast) {
        if (tile == 0 && t == 0) state[(size_t)row * kTKState] = -1;
        return;
    }
    const uint32_t bin = (uint32_t)s_bin;
    const float* zr = z + (size_t)row * V + (size_t)tile * kTK;
    const int n = min(kTK, V - tile * kTK);
#pragma unroll
    for (int q = 0; q < kTK / kTKThreads; q++) {
        const int j = q * kTKThreads + t;
        if (j >= n) continue;
        const float v = zr[j];
        const uint32_t key = order_key(v);
        if (v > kTopKFloor && (key >> (32 - kHBits)) >= bin) {
            const int pos = atomicAdd(&state[(size_t)row * kTKState], 1);
            gcand[(size_t)row * kTopKMax + pos] = topk_entry(key, tile * kTK + j);
        }
    }
}

// Launch of k_top_k, through the multi-workgroup candidate pass for long rows.
int launch_top_k(const float* z, int rows, int V, int k, int kpow2, float top_p, const float* u,
                 int u_stride, int* tokens, int tok_every, float* dist, int* lidx, float* lp) {
    const unsigned long long* gcand = nullptr;
    const int* gstate = nullptr;
    if (V >= 4 * kTK) {
        const size_t hn = (size_t)rows * (kHBins + kTKState);
        char* w = (char*)cgx_scratch(CGX_SLOT_WS6, hn * 4 + (size_t)rows * kTopKMax * 8 + 256);
        if (!w) return -1;
        int* hist = (int*)w;
        int* state = hist + (size_t)rows * kHBins;
        unsigned long long* cand =
            (unsigned long long*)(((uintptr_t)(w + hn * 4) + 255) & ~(uintptr_t)255);
        hipLaunchKernelGGL(k_topk_zero, dim3((unsigned)((hn + 255) / 256)), dim3(256), 0,
                           stream(), hist, hn);
        const dim3 grid((V + kTK - 1) / kTK, rows);
        hipLaunchKernelGGL(k_topk_hist, grid, dim3(kTKThreads), 0, stream(), z, V, hist);
        hipLaunchKernelGGL(k_topk_collect, grid, dim3(kTKThreads), 0, stream(), z, V, k, hist,
                           state, cand);
        if (launch_check("k_topk_collect")) return -1;
        gcand = cand;
        gstate = state;
    }
    hipLaunchKernelGGL(k_top_k, dim3(rows), dim3(kThreads), 0, stream(), z, V, k, kpow2, top_p,
                       u, u_stride, tokens, tok_every, dist, lidx, lp, gcand, gstate);
    return launch_check("k_top_k");
}

// ----------------------------------------------------- typical sampling
//
// cg_sample_typical is declared by cogito (include/cg_speculative.h:186)
// and never defined; this build defines it (decision D16) in the reference
// samplers' style: the softmax of cg_sample_top_p; L_i = (float)log p_i;
// H = sum_i fl(p_i * -L_i) left to right in fp32; tokens ordered by
// (|fl(-L_i - H)| ascending, index ascending); the first tokens of that order
// up to cumsum >= typical_p; the draw r = u * (kept mass) scans them.

// log of a positive finite float in binary64 by a fixed sequence of IEEE
// operations (no FMA; this file is built without contraction): x = m 2^k,
// m in [sqrt(1/2), sqrt(2)), log m = 2 atanh((m - 1) / (m + 1)) by the odd
// series to s^25.  The CPU restatement evaluates the same sequence, so both
// give the same bits.
__device__ double typ_log(float x) {
    const double kLn2 = 0x1.62e42fefa39efp-1;
    const double kSqrt2 = 0x1.6a09e667f3bcdp+0;
    const double kC[13] = {1.0,        1.0 / 3.0,  1.0 / 5.0,  1.0 / 7.0,  1.0 / 9.0,
                           1.0 / 11.0, 1.0 / 13.0, 1.0 / 15.0, 1.0 / 17.0, 1.0 / 19.0,
                           1.0 / 21.0, 1.0 / 23.0, 1.0 / 25.0};
    const unsigned long long b = (unsigned long long)__double_as_longlong((double)x);
    int k = (int)((b >> 52) & 0x7ff) - 1023;
    double m = __longlong_as_double(
        (long long)((b & 0x000fffffffffffffull) | 0x3ff0000000000000ull));
    if (m > kSqrt2) {
        m = __dmul_rn(m, 0.5);
        k += 1;
    }
    const double s = __ddiv_rn(__dsub_rn(m, 1.0), __dadd_rn(m, 1.0));
    const double s2 = __dmul_rn(s, s);
    double q = kC[12];
#pragma unroll
    for (int j = 11; j >= 0; j--) q = __dadd_rn(kC[j], __dmul_rn(s2, q));
    return __dadd_rn(__dmul_rn((double)k, kLn2), __dmul_rn(2.0, __dmul_rn(s, q)));
}

__global__ void k_typ_log(const float* __restrict__ x, double* __restrict__ y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = typ_log(x[i]);
}

// Per row: -L_i and the entropy terms, H by the exact ordered sum, then the
// sort key of each token (its score's bits; +inf for p_i = 0).
__global__ __launch_bounds__(kThreads) void k_typ_scores(const float* __restrict__ probs, int V,
                                                         float* __restrict__ nl,
                                                         float* __restrict__ terms,
                                                         uint32_t* __restrict__ keys) {
    __shared__ EosShared sh;
    const size_t rb = (size_t)blockIdx.x * V;
    const float* pr = probs + rb;
    for (int j = threadIdx.x; j < V; j += kThreads) {
        const float x = pr[j];
        const float n = x > 0.0f ? -(float)typ_log(x) : 0.0f;
        nl[rb + j] = n;
        terms[rb + j] = x > 0.0f ? __fmul_rn(x, n) : 0.0f;
    }
    __threadfence_block();
    __syncthreads();
    const float H = eos_sum(RowSrc{terms + rb}, V, sh);
    for (int j = threadIdx.x; j < V; j += kThreads) {
        const float sc = pr[j] > 0.0f ? fabsf(__fsub_rn(nl[rb + j], H)) : __builtin_inff();
        keys[rb + j] = __float_as_uint(sc);
    }
}

struct PermSrc {                 // probabilities in the typical order
    const float* p;
    const uint32_t* o;
    __device__ float operator()(int j) const { return p[o[j]]; }
};

// Cutoff over the typical order, then the draw (tokens) or the filtered
// distribution (dist, dense rows).
__global__ __launch_bounds__(kThreads) void k_typ_finish(const float* __restrict__ probs,
                                                         const uint32_t* __restrict__ perm,
                                                         int V, float typical_p,
                                                         const float* __restrict__ u,
                                                         int* __restrict__ tokens,
                                                         float* __restrict__ dist) {
    __shared__ EosShared sh;
    const int row = blockIdx.x;
    const size_t rb = (size_t)row * V;
    PermSrc g{probs + rb, perm + rb};
    const float total = eos_sum(g, V, sh);
    float C;
    const int ci = gen_find_val(g, V, float_below(typical_p), -1, total, &C, sh);
    const int cutoff = ci < 0 ? V : ci + 1;
    if (tokens) {
        // speculative.c:109-115's scan over the kept tokens
        int pos = gen_find(g, V, __fmul_rn(u[row], C), 0, sh);
        if (pos >= cutoff) pos = 0;
        if (threadIdx.x == 0) tokens[row] = (int)perm[rb + pos];
        return;
    }
    float* dr = dist + rb;
    for (int j = threadIdx.x; j < V; j += kThreads) dr[j] = 0.0f;
    __threadfence_block();
    __syncthreads();
    for (int j = threadIdx.x; j < cutoff; j += kThreads) {
        const int i = (int)perm[rb + j];
        dr[i] = __fdiv_rn(probs[rb + i], C);
    }
}

}  // namespace

// -------------------------------------------------------------- launchers

extern "C" int cgk_typ_log(const float* x, double* y, int n) {
    hipLaunchKernelGGL(k_typ_log, dim3((n + 255) / 256), dim3(256), 0, stream(), x, y, n);
    return launch_check("k_typ_log");
}

// Typical sampling of `rows` rows of logits [rows][V] (T = 1): tokens[row]
// drawn with u[row], or dense distributions.  Uses scratch slot WS0.
extern "C" int cgk_typical_rows(const float* logits, int rows, int V, float typical_p,
                                const float* u, int* tokens, float* dist) {
    if (rows <= 0 || V <= 0 || rows > 65535 || (!tokens == !dist)) {
        cgx_set_error("typical: invalid arguments");
        return -1;
    }
    if (V > kRound * kMaxRounds) {
        cgx_set_error("typical: vocabulary size %d above %d", V, kRound * kMaxRounds);
        return -1;
    }
    const size_t n = (size_t)rows * V;
    const size_t a = (n * 4 + 255) & ~(size_t)255;
    const size_t sb = cgk_row_sort_ws(rows, V, 1);
    char* w = (char*)cgx_scratch(CGX_SLOT_WS0, 6 * a + sb);
    if (!w) return -1;
    float* probs = (float*)w;
    float* nl = (float*)(w + a);
    float* terms = (float*)(w + 2 * a);
    uint32_t* keys = (uint32_t*)(w + 3 * a);
    uint32_t* skeys = (uint32_t*)(w + 4 * a);
    uint32_t* perm = (uint32_t*)(w + 5 * a);
    void* sws = w + 6 * a;
    hipLaunchKernelGGL(k_probs_rows, dim3(rows), dim3(kThreads), 0, stream(), logits, V, 1.0f,
                       probs);
    if (launch_check("k_probs_rows")) return -1;
    hipLaunchKernelGGL(k_typ_scores, dim3(rows), dim3(kThreads), 0, stream(), probs, V, nl, terms,
                       keys);
    if (launch_check("k_typ_scores")) return -1;
    if (cgk_row_sort(keys, nullptr, rows, V, 0, skeys, perm, sws, sb)) return -1;
    hipLaunchKernelGGL(k_typ_finish, dim3(rows), dim3(kThreads), 0, stream(), probs, perm, V,
                       typical_p, u, tokens, dist);
    return launch_check("k_typ_finish");
}

// Top-k lists of `rows` rows of z [rows][V] (1 <= top_k < V): lidx/lp
// [rows][top_k], entry j = the j-th of cg_sample_top_k's list (value desc,
// index asc) and its probability (softmax of the list at T = 1, then the
// top-p cutoff and renormalisation when top_p < 1; 0 past the cutoff and for
// the -1e30 fillers).
extern "C" int cgk_topk_lists(const float* z, int rows, int V, int top_k, float top_p, int* lidx,
                              float* lp) {
    if (rows <= 0 || V <= 0 || rows > 65535 || top_k < 1 || top_k >= V || top_k > kTopKMax ||
        !lidx || !lp) {
        cgx_set_error("topk_lists: invalid arguments (rows %d, V %d, k %d)", rows, V, top_k);
        return -1;
    }
    if (V > kRound * kMaxRounds) {
        cgx_set_error("topk_lists: vocabulary size %d above %d", V, kRound * kMaxRounds);
        return -1;
    }
    int kpow2 = 64;
    while (kpow2 < top_k) kpow2 <<= 1;
    return launch_top_k(z, rows, V, top_k, kpow2, top_p, nullptr, 0, nullptr, 0, nullptr, lidx,
                        lp);
}

extern "C" int cgk_scale(const float* x, float* z, size_t n, float T) {
    if (!n) return 0;
    hipLaunchKernelGGL(k_scale, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream(), x,
                       z, n, T);
    return launch_check("k_scale");
}

// Top-k / top-p over `rows` rows of z [rows][V]: dense filtered
// distributions of every row (dist != NULL) and tokens of the rows r with
// (r + 1) % tok_every == 0 (tokens[r / tok_every], drawn with
// u[(r / tok_every) * u_stride]), in the same launches.
extern "C" int cgk_filter_rows_ex(const float* z, int rows, int V, int top_k, float top_p,
                                  const float* u, int u_stride, int* tokens, int tok_every,
                                  float* dist) {
    return cgk_filter_rows_t(z, 1.0f, nullptr, rows, V, top_k, top_p, u, u_stride, tokens,
                             tok_every, dist);
}

// The same over rows of x at temperature T (z = x / T): the top-p path
// divides as it reads; the top-k path first writes z into zbuf ([rows][V]).
extern "C" int cgk_filter_rows_t(const float* x, float T, float* zbuf, int rows, int V,
                                 int top_k, float top_p, const float* u, int u_stride,
                                 int* tokens, int tok_every, float* dist) {
    if (!tokens) tok_every = 0;
    if (rows <= 0 || V <= 0 || rows > 65535 || (!tok_every && !dist) || tok_every < 0 ||
        (tok_every && !u)) {
        cgx_set_error("filter: invalid arguments");
        return -1;
    }
    if (V > kRound * kMaxRounds) {
        cgx_set_error("filter: vocabulary size %d above %d", V, kRound * kMaxRounds);
        return -1;
    }
    if (top_k > 0 && top_k < V) {
        if (top_k > kTopKMax) {
            cgx_set_error("top-k: k = %d above the supported %d", top_k, kTopKMax);
            return -1;
        }
        int kpow2 = 64;
        while (kpow2 < top_k) kpow2 <<= 1;
        const float* z = x;
        if (T != 1.0f) {
            if (!zbuf) {
                cgx_set_error("filter: top-k at T != 1 needs a workspace for x / T");
                return -1;
            }
            if (cgk_scale(x, zbuf, (size_t)rows * V, T)) return -1;
            z = zbuf;
        }
        return launch_top_k(z, rows, V, top_k, kpow2, top_p, u, u_stride, tokens, tok_every,
                            dist, nullptr, nullptr);
    }
    // the descending sort of each row's probabilities (rowsort.hip, on the
    // values' bit patterns, monotone for non-negative floats) shares its
    // workspace with the finish's
    size_t n = (size_t)rows * V;
    size_t wsb = n * 8;
    const size_t sb = cgk_row_sort_ws(rows, V, 0);
    if (sb > wsb) wsb = sb;
    char* w = (char*)cgx_scratch(CGX_SLOT_WS0, n * 8 + wsb);
    if (!w) return -1;
    float* probs = (float*)w;
    float* sorted = probs + n;
    int* ws = (int*)(sorted + n);
    hipLaunchKernelGGL(k_probs_rows, dim3(rows), dim3(kThreads), 0, stream(), x, V, T, probs);
    if (launch_check("k_probs_rows")) return -1;
    if (cgk_row_sort((const uint32_t*)probs, nullptr, rows, V, 1, (uint32_t*)sorted, nullptr, ws,
                     wsb))
        return -1;
    hipLaunchKernelGGL(k_top_p_finish, dim3(rows), dim3(kThreads), 0, stream(), probs, sorted,
                       V, top_p, u, u_stride, tokens, tok_every, dist, ws);
    return launch_check("k_top_p_finish");
}

// One token per row drawn with u[row] (tokens != NULL), or dense filtered
// distributions (dist != NULL).
extern "C" int cgk_filter_rows(const float* z, int rows, int V, int top_k, float top_p,
                               const float* u, int* tokens, float* dist) {
    if (!tokens == !dist) {
        cgx_set_error("filter: invalid arguments");
        return -1;
    }
    return cgk_filter_rows_ex(z, rows, V, top_k, top_p, u, 1, tokens, tokens ? 1 : 0, dist);
}
