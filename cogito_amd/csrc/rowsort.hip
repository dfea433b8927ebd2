// rowsort.hip -- stable radix sort of rows of 32-bit keys, optionally
// carrying a 32-bit payload, with several workgroups per row (gfx950).
//
// The samplers that order a whole vocabulary row (top-p by probability,
// typical sampling by score) sort with it, so no row size is bounded by LDS.
// Least-significant-digit first, 8-bit digits, four passes, over tiles of
// 2048 keys (rows of more than 65536 keys: 4096) (grid: tiles x rows):
//   k_rs_hist     the tile's digit counts -> hist[row][tile][256];
//   k_rs_scatter  the tile's output offsets (counts of every tile before it,
//                 and of the digits before its own in the sort order), the
//                 stable rank of each key among the tile's keys of its digit,
//                 and the scatter.
// Rows of up to 65536 keys (at most kFuseTiles tiles) take one histogram
// launch and four scatters: each scatter also counts the next pass's digits
// by the tile its keys land in (LDS counts, added to the next pass's
// histogram with global atomics), and the histogram launch clears those
// histograms.  Longer rows take a histogram launch before every scatter.
// Ranks come from wave-level digit matching: eight ballots give each lane the
// mask of lanes holding the same digit, so one lane per digit group touches
// the LDS counters (no atomics, no contention when most keys share a digit,
// as the high byte of probabilities does).  A tile's keys are ordered (wave,
// item, lane), which is their order in the row, so every pass is stable.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cgx_internal.h"

namespace {

constexpr int kT = 256;                 // threads per block (4 waves)
constexpr int kWv = kT / 64;
constexpr int kBins = 256;
constexpr int kMaxTiles = 1024;         // rows up to 4 M keys (tiles of 4096)
constexpr int kSmallRow = 65536;        // rows up to this many keys: 8 keys a thread
constexpr int kHistBatch = 16;          // tile counts loaded per round trip
constexpr int kFuseTiles = 32;          // tiles of rows whose scatters count the next digits

// Keys per thread for a row of n keys: short rows take smaller tiles, so more
// workgroups share a row and each walks fewer keys in sequence.
inline int row_items(int n) { return n <= kSmallRow ? 8 : 16; }

inline hipStream_t stream() { return (hipStream_t)cgx_stream(); }

int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        cgx_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

// Lanes (among the valid ones) whose 8-bit digit equals this lane's.
__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool valid) {
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const bool bit = (d >> b) & 1u;
        const uint64_t v = __ballot(bit);
        m &= bit ? v : ~v;
    }
    return m;
}

// Position of item q of lane `lane` in wave w of tile `tile`.
template <int kItems>
__device__ __forceinline__ int tile_pos(int tile, int w, int q, int lane) {
    return tile * (kT * kItems) + w * (kItems * 64) + q * 64 + lane;
}

// zero: `zsets` further histograms of the grid's size, cleared (one entry per
// thread each)
template <int kItems>
__global__ __launch_bounds__(kT) void k_rs_hist(const uint32_t* __restrict__ keys, int n,
                                                int shift, int ntiles,
                                                uint32_t* __restrict__ hist,
                                                uint32_t* __restrict__ zero, int zsets) {
    __shared__ uint32_t h[kBins];
    const int row = blockIdx.y, tile = blockIdx.x, t = threadIdx.x;
    const int lane = t & 63, w = t >> 6;
    const size_t gsz = (size_t)gridDim.x * gridDim.y * kT;
    const size_t g = ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * kT + t;
    for (int z = 0; z < zsets; z++) zero[g + z * gsz] = 0u;
    h[t] = 0;
    __syncthreads();
    const uint32_t* src = keys + (size_t)row * n;
    uint32_t kk[kItems];
#pragma unroll
    for (int q = 0; q < kItems; q++) {
        const int p = tile_pos<kItems>(tile, w, q, lane);
        kk[q] = p < n ? src[p] : 0u;
    }
#pragma unroll
    for (int q = 0; q < kItems; q++) {
        const bool valid = tile_pos<kItems>(tile, w, q, lane) < n;
        const uint32_t d = (kk[q] >> shift) & 255u;
        const uint64_t m = match_digit(d, valid);
        if (valid && lane == __ffsll((unsigned long long)m) - 1)
            atomicAdd(&h[d], (uint32_t)__popcll(m));
    }
    __syncthreads();
    hist[((size_t)row * ntiles + tile) * kBins + t] = h[t];
}

// Exclusive sum over the 256 threads of the block (one value each).
__device__ __forceinline__ uint32_t block_excl_256(uint32_t v, uint32_t* part) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) part[w] = x;
    __syncthreads();
    uint32_t off = 0;
#pragma unroll
    for (int i = 0; i < kWv; i++) off += i < w ? part[i] : 0u;
    __syncthreads();
    return off + x - v;
}

// kNext: also count the next pass's digits (shift + 8) by destination tile
// into hnext (ntiles <= kFuseTiles).
template <int kItems, bool kDesc, bool kPay, bool kNext>
__global__ __launch_bounds__(kT) void k_rs_scatter(const uint32_t* __restrict__ kin,
                                                   const uint32_t* __restrict__ pin, int n,
                                                   int shift, int ntiles,
                                                   const uint32_t* __restrict__ hist,
                                                   uint32_t* __restrict__ kout,
                                                   uint32_t* __restrict__ pout,
                                                   uint32_t* __restrict__ hnext) {
    __shared__ uint32_t wcnt[kWv][kBins];
    __shared__ uint32_t goff[kBins];
    __shared__ uint32_t ord[kBins];
    __shared__ uint32_t part[kWv];
    __shared__ uint32_t h2[kNext ? kFuseTiles : 1][kBins];
    const int row = blockIdx.y, tile = blockIdx.x, t = threadIdx.x;
    const int lane = t & 63, w = t >> 6;
    const size_t rb = (size_t)row * n;
    if (kNext)
        for (int e = t; e < ntiles * kBins; e += kT) h2[e / kBins][e % kBins] = 0u;

    // keys first, so their loads are in flight during the offset arithmetic
    uint32_t kk[kItems], pp[kItems], rk[kItems];
#pragma unroll
    for (int q = 0; q < kItems; q++) {
        const int p = tile_pos<kItems>(tile, w, q, lane);
        kk[q] = p < n ? kin[rb + p] : 0u;
        if (kPay) pp[q] = p < n ? (pin ? pin[rb + p] : (uint32_t)p) : 0u;
    }

    // digit d = t: keys of d in earlier tiles, and in the whole row; the
    // tiles' counts are loaded kHistBatch at a time, so a row of up to
    // kHistBatch tiles costs one round trip
    const uint32_t* hr = hist + (size_t)row * ntiles * kBins;
    uint32_t pre = 0, tot = 0;
    for (int b0 = 0; b0 < ntiles; b0 += kHistBatch) {
        uint32_t c[kHistBatch];
#pragma unroll
        for (int i = 0; i < kHistBatch; i++)
            c[i] = b0 + i < ntiles ? hr[(size_t)(b0 + i) * kBins + t] : 0u;
#pragma unroll
        for (int i = 0; i < kHistBatch; i++) {
            tot += c[i];
            pre += b0 + i < tile ? c[i] : 0u;
        }
    }
    // digits in sort order: position o(d) = d (ascending) or 255 - d
    ord[kDesc ? 255 - t : t] = tot;
    for (int i = 0; i < kWv; i++) wcnt[i][t] = 0;
    __syncthreads();
    const uint32_t before = block_excl_256(ord[t], part);
    ord[t] = before;
    __syncthreads();
    goff[t] = ord[kDesc ? 255 - t : t] + pre;

    // stable rank of each key among the tile's keys of its digit, per wave
    const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
    for (int q = 0; q < kItems; q++) {
        const bool valid = tile_pos<kItems>(tile, w, q, lane) < n;
        const uint32_t d = (kk[q] >> shift) & 255u;
        const uint64_t m = match_digit(d, valid);
        rk[q] = 0;
        if (valid) {
            const uint32_t c = wcnt[w][d];
            rk[q] = c + (uint32_t)__popcll(m & lt);
            if (lane == __ffsll((unsigned long long)m) - 1) wcnt[w][d] = c + (uint32_t)__popcll(m);
        }
    }
    __syncthreads();
    // earlier waves' counts per digit
    {
        uint32_t r = 0;
#pragma unroll
        for (int i = 0; i < kWv; i++) {
            const uint32_t c = wcnt[i][t];
            wcnt[i][t] = r;
            r += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kItems; q++) {
        if (tile_pos<kItems>(tile, w, q, lane) >= n) continue;
        const uint32_t d = (kk[q] >> shift) & 255u;
        const uint32_t pos = goff[d] + wcnt[w][d] + rk[q];
        if (pos >= (uint32_t)n) continue;   // unreachable with consistent counts
        kout[rb + pos] = kk[q];
        if (kPay) pout[rb + pos] = pp[q];
        if (kNext) atomicAdd(&h2[pos / (kT * kItems)][(kk[q] >> (shift + 8)) & 255u], 1u);
    }
    if (kNext) {
        __syncthreads();
        uint32_t* hn = hnext + (size_t)row * ntiles * kBins;
        for (int e = t; e < ntiles * kBins; e += kT) {
            const uint32_t c = h2[e / kBins][e % kBins];
            if (c) atomicAdd(&hn[e], c);
        }
    }
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

template <int kItems, bool kNext>
int launch_scatter(dim3 grid, const uint32_t* ks, const uint32_t* ps, int n, int shift, int ntiles,
                   const uint32_t* hist, int desc, uint32_t* kd, uint32_t* pd, uint32_t* hnext) {
    if (desc && pd)
        hipLaunchKernelGGL((k_rs_scatter<kItems, true, true, kNext>), grid, dim3(kT), 0, stream(),
                           ks, ps, n, shift, ntiles, hist, kd, pd, hnext);
    else if (desc)
        hipLaunchKernelGGL((k_rs_scatter<kItems, true, false, kNext>), grid, dim3(kT), 0,
                           stream(), ks, ps, n, shift, ntiles, hist, kd, pd, hnext);
    else if (pd)
        hipLaunchKernelGGL((k_rs_scatter<kItems, false, true, kNext>), grid, dim3(kT), 0,
                           stream(), ks, ps, n, shift, ntiles, hist, kd, pd, hnext);
    else
        hipLaunchKernelGGL((k_rs_scatter<kItems, false, false, kNext>), grid, dim3(kT), 0,
                           stream(), ks, ps, n, shift, ntiles, hist, kd, pd, hnext);
    return launch_check("k_rs_scatter");
}

// hist: four histograms of rows x ntiles x kBins when kFused, else one.
template <int kItems, bool kFused>
int row_sort_passes(const uint32_t* kin, const uint32_t* pin, int rows, int n, int desc,
                    uint32_t* kout, uint32_t* pout, uint32_t* const kb[2], uint32_t* const pb[2],
                    uint32_t* hist) {
    const int ntiles = (n + kT * kItems - 1) / (kT * kItems);
    const dim3 grid(ntiles, rows);
    const size_t hsz = (size_t)rows * ntiles * kBins;
    const uint32_t* ks = kin;
    const uint32_t* ps = pin;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 8 * pass;
        uint32_t* kd = pass == 3 ? kout : kb[pass & 1];
        uint32_t* pd = pass == 3 ? pout : pb[pass & 1];
        if (!kFused || pass == 0) {
            hipLaunchKernelGGL(k_rs_hist<kItems>, grid, dim3(kT), 0, stream(), ks, n, shift,
                               ntiles, hist, hist + hsz, kFused ? 3 : 0);
            if (launch_check("k_rs_hist")) return -1;
        }
        const uint32_t* h = kFused ? hist + pass * hsz : hist;
        int rc;
        if constexpr (kFused)
            rc = pass < 3 ? launch_scatter<kItems, true>(grid, ks, ps, n, shift, ntiles, h, desc,
                                                         kd, pd, hist + (pass + 1) * hsz)
                          : launch_scatter<kItems, false>(grid, ks, ps, n, shift, ntiles, h,
                                                          desc, kd, pd, nullptr);
        else
            rc = launch_scatter<kItems, false>(grid, ks, ps, n, shift, ntiles, h, desc, kd, pd,
                                               nullptr);
        if (rc) return -1;
        ks = kd;
        ps = pd;
    }
    return 0;
}

size_t row_tiles(int n) {
    const size_t tile = (size_t)kT * row_items(n);
    return ((size_t)n + tile - 1) / tile;
}

}  // namespace

extern "C" size_t cgk_row_sort_ws(int rows, int n, int with_payload) {
    const size_t ntiles = row_tiles(n);
    const size_t nhist = row_items(n) == 8 ? 4 : 1;
    const size_t buf = align256((size_t)rows * n * 4);
    return (with_payload ? 4 : 2) * buf + align256(nhist * rows * ntiles * kBins * 4);
}

extern "C" int cgk_row_sort(const uint32_t* kin, const uint32_t* pin, int rows, int n, int desc,
                            uint32_t* kout, uint32_t* pout, void* ws, size_t ws_bytes) {
    if (rows <= 0 || rows > 65535 || n <= 0 || !kin || !kout || !ws) {
        cgx_set_error("row sort: invalid arguments (rows %d, n %d)", rows, n);
        return -1;
    }
    const int ntiles = (int)row_tiles(n);
    const int pay = pout != nullptr;
    if (ntiles > kMaxTiles || ws_bytes < cgk_row_sort_ws(rows, n, pay)) {
        cgx_set_error("row sort: %d keys per row need %d tiles (at most %d) or the workspace "
                      "is too small", n, ntiles, kMaxTiles);
        return -1;
    }
    const size_t buf = align256((size_t)rows * n * 4);
    char* w = (char*)ws;
    uint32_t* const kb[2] = {(uint32_t*)w, (uint32_t*)(w + buf)};
    uint32_t* const pb[2] = {pay ? (uint32_t*)(w + 2 * buf) : nullptr,
                             pay ? (uint32_t*)(w + 3 * buf) : nullptr};
    uint32_t* hist = (uint32_t*)(w + (pay ? 4 : 2) * buf);
    static_assert((kSmallRow + kT * 8 - 1) / (kT * 8) <= kFuseTiles, "short rows fit the fused counts");
    return row_items(n) == 8
        ? row_sort_passes<8, true>(kin, pin, rows, n, desc, kout, pout, kb, pb, hist)
        : row_sort_passes<16, false>(kin, pin, rows, n, desc, kout, pout, kb, pb, hist);
}
