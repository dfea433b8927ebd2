// decoder.hip -- the small kernels of the synthetic decoder stack that sit
// between the INT4 GEMVs (int4.hip) and attention (attn.hip):
//
//   k_embed        embedding rows of the step's tokens (token ids on device)
//   k_rope_append  RoPE of the step's Q and K (cg_apply_rope arithmetic,
//                  src/attention/flash_attn.c:335-360) and the INT4 KV-cache
//                  append of K and V (src/quantize/int4.c:155-231), one
//                  workgroup per (token, head)
//   k_fill_normal  seeded weights: a counter-based hash (lowbias32) gives
//                  four 16-bit uniforms per value; their centred sum scaled
//                  to unit variance (Irwin-Hall, n = 4) times std.  Integer
//                  arithmetic up to one int->float conversion and one
//                  multiply, so a CPU restatement produces the same bits.
//
// Block order of a layer (pre-norm, no bias, src/layers/transformer.c:26-149):
//   x += o_proj(attn(rope(qkv_proj(rmsnorm(x)))))
//   x += down(silu(gate(rmsnorm(x))) * up(rmsnorm(x)))
// with the RMSNorms fused into the following GEMV and the residual adds into
// the GEMV epilogue.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "cgx_internal.h"

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

__global__ void k_embed(const float* __restrict__ table, const int* __restrict__ tokens,
                        int M, int d, int V, float* __restrict__ x) {
    int m = blockIdx.y;
    int tok = tokens[m];
    tok = tok < 0 ? 0 : (tok >= V ? V - 1 : tok);
    const float* row = table + (size_t)tok * d;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        x[(size_t)m * d + i] = row[i];
}

constexpr int kMaxBatch = 16;
constexpr int kMaxTreeRows = 64;

// Token rows of B sequences, M each (row r = b * M + m): sequence b's rows
// sit at positions pos0[b] + m of its own cache (kc + b * seq_kbytes, scales
// + b * seq_groups).
struct RopeBatch {
    int M;
    int pos0[kMaxBatch];
    size_t seq_kbytes, seq_groups;
    int has_rel;                 // tree rows: rotary position pos0 + rel[row]
    int rel[kMaxTreeRows];
};

// Embedding rows of the step's tokens, and the rotary table of each row:
// cs[r][i] = (cos, sin) of the row's rotary position times frequency i (i <
// D/2), with k_rope_append's arithmetic, so that the fused attention
// (attn_dec.hip) rotates Q and K to the same bits.  Block (x, r); blocks with
// x == 0 also fill row r's table.
__global__ void k_embed_rope(const float* __restrict__ table, const int* __restrict__ tokens,
                             int d, int V, float* __restrict__ x, RopeBatch rb, int D,
                             float theta, float2* __restrict__ cs) {
    const int m = blockIdx.y;
    int tok = tokens[m];
    tok = tok < 0 ? 0 : (tok >= V ? V - 1 : tok);
    const float* row = table + (size_t)tok * d;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        x[(size_t)m * d + i] = row[i];
    if (blockIdx.x == 0) {
        const int sq = m / rb.M;
        const int rpos = rb.pos0[sq] + (rb.has_rel ? rb.rel[m % rb.M] : m % rb.M);
        for (int i = threadIdx.x; i < D / 2; i += blockDim.x) {
            float freq = __fdiv_rn(1.0f, powf(theta, __fdiv_rn((float)(2 * i), (float)D)));
            float angle = __fmul_rn((float)rpos, freq);
            cs[(size_t)m * (D / 2) + i] = make_float2(cosf(angle), sinf(angle));
        }
    }
}

// cs[r][i] = (cos, sin) of (pos0 + r) times frequency i, as k_embed_rope.
__global__ void k_rope_table(int rows, int D, int pos0, float theta, float2* __restrict__ cs) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= rows * (D / 2)) return;
    const int r = e / (D / 2), i = e % (D / 2);
    float freq = __fdiv_rn(1.0f, powf(theta, __fdiv_rn((float)(2 * i), (float)D)));
    float angle = __fmul_rn((float)(pos0 + r), freq);
    cs[e] = make_float2(cosf(angle), sinf(angle));
}

// One workgroup of D/2 threads per (token row, head): heads [0, H) are query
// heads (rotated into q_out), heads [H, H + Hk) are KV heads (K rotated, then
// K and V quantised into the cache row of the token's position).
// With cs (k_embed_rope's table of the same rows) the rotation takes its
// (cos, sin) from there, as the fused attention does, so both write the same
// cache bits.
__global__ void k_rope_append(const float* __restrict__ qkv, int ld, int H, int Hk, int D,
                              int gs, RopeBatch rb, float theta, const float2* __restrict__ cs,
                              float* __restrict__ q_out, uint8_t* __restrict__ kc,
                              uint8_t* __restrict__ vc, float* __restrict__ ks,
                              float* __restrict__ vs) {
    __shared__ float sk[256], sv[256];
    const int m = blockIdx.x, head = blockIdx.y, i = threadIdx.x, half = D / 2;
    const int sq = m / rb.M;
    // cache slot pos0 + row; rotary position the same, or pos0 + rel[row]
    // for a tree row (its depth below the verified prefix)
    const int pos = rb.pos0[sq] + m % rb.M;
    const int rpos = rb.has_rel ? rb.pos0[sq] + rb.rel[m % rb.M] : pos;
    kc += (size_t)sq * rb.seq_kbytes;
    vc += (size_t)sq * rb.seq_kbytes;
    ks += (size_t)sq * rb.seq_groups;
    vs += (size_t)sq * rb.seq_groups;
    const float* row = qkv + (size_t)m * ld;
    // the head's values first, so that their latency overlaps the rotary
    // angle's evaluation (a query head: its two halves; a KV head: K's
    // halves and V's)
    const bool is_q = head < H;
    const int hk = head - H;
    const float* k = is_q ? row + head * D : row + H * D + hk * D;
    const float* v = is_q ? k : row + (H + Hk) * D + hk * D;
    const float k0 = k[i], k1 = k[i + half];
    const float v0 = v[i], v1 = v[i + half];
    float c, s;
    if (cs) {
        const float2 t = cs[(size_t)m * half + i];
        c = t.x;
        s = t.y;
    } else {
        float freq = __fdiv_rn(1.0f, powf(theta, __fdiv_rn((float)(2 * i), (float)D)));
        float angle = __fmul_rn((float)rpos, freq);
        c = cosf(angle);
        s = sinf(angle);
    }
    if (is_q) {
        float* o = q_out + ((size_t)m * H + head) * D;
        o[i] = __fsub_rn(__fmul_rn(k0, c), __fmul_rn(k1, s));
        o[i + half] = __fadd_rn(__fmul_rn(k0, s), __fmul_rn(k1, c));
        return;
    }
    sk[i] = __fsub_rn(__fmul_rn(k0, c), __fmul_rn(k1, s));
    sk[i + half] = __fadd_rn(__fmul_rn(k0, s), __fmul_rn(k1, c));
    sv[i] = v0;
    sv[i + half] = v1;
    __syncthreads();
    // quantise: thread i packs dims 2i, 2i+1 (same group: gs is even).  The
    // group absmax (order-free) is a shuffle reduction over the gs/2 threads
    // of the group when they are a power of two inside one wave, else a scan.
    const int ngh = D / gs, g = (2 * i) / gs;
    float mk = fmaxf(fabsf(sk[2 * i]), fabsf(sk[2 * i + 1]));
    float mv = fmaxf(fabsf(sv[2 * i]), fabsf(sv[2 * i + 1]));
    const int gt = gs / 2;
    if ((gt & (gt - 1)) == 0 && gt <= 64) {
        for (int o = 1; o < gt; o <<= 1) {
            mk = fmaxf(mk, __shfl_xor(mk, o));
            mv = fmaxf(mv, __shfl_xor(mv, o));
        }
    } else {
        for (int e = g * gs; e < (g + 1) * gs; e++) {
            mk = fmaxf(mk, fabsf(sk[e]));
            mv = fmaxf(mv, fabsf(sv[e]));
        }
    }
    float sck = __fdiv_rn(mk, 7.0f), scv = __fdiv_rn(mv, 7.0f);
    if (sck < 1e-8f) sck = 1.0f;
    if (scv < 1e-8f) scv = 1.0f;
    const size_t th = (size_t)pos * Hk + hk;
    if ((2 * i) % gs == 0) {
        ks[th * ngh + g] = sck;
        vs[th * ngh + g] = scv;
    }
    int a0 = (int)roundf(__fdiv_rn(sk[2 * i], sck)), a1 = (int)roundf(__fdiv_rn(sk[2 * i + 1], sck));
    int b0 = (int)roundf(__fdiv_rn(sv[2 * i], scv)), b1 = (int)roundf(__fdiv_rn(sv[2 * i + 1], scv));
    a0 = a0 > 7 ? 7 : (a0 < -8 ? -8 : a0);
    a1 = a1 > 7 ? 7 : (a1 < -8 ? -8 : a1);
    b0 = b0 > 7 ? 7 : (b0 < -8 ? -8 : b0);
    b1 = b1 > 7 ? 7 : (b1 < -8 ? -8 : b1);
    kc[th * half + i] = (uint8_t)((a0 & 0xF) | ((a1 & 0xF) << 4));
    vc[th * half + i] = (uint8_t)((b0 & 0xF) | ((b1 & 0xF) << 4));
}

// ttok[b] = feed[b][1], d_1 .. d_gamma; vtok[b] = d_1 .. d_gamma (dtok [gamma][B])
__global__ void k_spec_tokens(const int* __restrict__ feed, const int* __restrict__ dtok, int B,
                              int gamma, int* __restrict__ ttok, int* __restrict__ vtok) {
    const int b = blockIdx.x, i = threadIdx.x;
    if (i == 0) ttok[(size_t)b * (gamma + 1)] = feed[2 * b + 1];
    for (int k = i; k < gamma; k += blockDim.x) {
        const int t = dtok[(size_t)k * B + b];
        ttok[(size_t)b * (gamma + 1) + 1 + k] = t;
        vtok[(size_t)b * gamma + k] = t;
    }
}

__device__ __forceinline__ uint32_t lowbias32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

__global__ void k_fill_normal(float* __restrict__ out, size_t n, uint32_t key, float scale) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        uint32_t a = lowbias32(key + 2u * (uint32_t)i);
        uint32_t b = lowbias32(key + 2u * (uint32_t)i + 1u);
        int s = (int)(a & 0xFFFF) + (int)(a >> 16) + (int)(b & 0xFFFF) + (int)(b >> 16);
        out[i] = (float)(s - 131070) * scale;
    }
}

}  // namespace

extern "C" int cgk_embed(const float* table, const int* tokens, int M, int d, int V,
                         float* x) {
    if (M <= 0) return 0;
    int bx = (d + 255) / 256;
    hipLaunchKernelGGL(k_embed, dim3(bx > 16 ? 16 : bx, M), dim3(256), 0, stream(), table,
                       tokens, M, d, V, x);
    return launch_check("k_embed");
}

extern "C" int cgk_rope_table(int rows, int D, int pos0, float theta, float* cs) {
    const int n = rows * (D / 2);
    hipLaunchKernelGGL(k_rope_table, dim3((n + 255) / 256), dim3(256), 0, stream(), rows, D,
                       pos0, theta, (float2*)cs);
    return launch_check("k_rope_table");
}

extern "C" int cgk_embed_rope(const float* table, const int* tokens, int B, int M, int d, int V,
                              float* x, const int* pos0, const int* rel, int D, float theta,
                              float* cs) {
    if (M <= 0) return 0;
    if (B < 1 || B > kMaxBatch || (rel && M > kMaxTreeRows) || D < 2 || (D & 1)) {
        cgx_set_error("embed_rope: batch %d, %d rows, head_dim %d", B, M, D);
        return -1;
    }
    RopeBatch rb;
    rb.has_rel = rel != nullptr;
    for (int r = 0; r < kMaxTreeRows; r++) rb.rel[r] = rel && r < M ? rel[r] : 0;
    rb.M = M;
    for (int b = 0; b < kMaxBatch; b++) rb.pos0[b] = b < B ? pos0[b] : 0;
    rb.seq_kbytes = rb.seq_groups = 0;
    int bx = (d + 255) / 256;
    hipLaunchKernelGGL(k_embed_rope, dim3(bx > 16 ? 16 : bx, B * M), dim3(256), 0, stream(),
                       table, tokens, d, V, x, rb, D, theta, (float2*)cs);
    return launch_check("k_embed_rope");
}

extern "C" int cgk_rope_append_batch(const float* qkv, int ld, int B, int M, int H, int Hk,
                                     int D, int gs, const int* pos0, const int* rel, float theta,
                                     const float* cs, float* q_out, uint8_t* kc, uint8_t* vc,
                                     float* ks, float* vs, size_t seq_kbytes,
                                     size_t seq_groups) {
    if (M <= 0) return 0;
    if (D < 2 || D > 256 || (D & 1) || gs <= 0 || (gs & 1) || D % gs) {
        cgx_set_error("rope_append: unsupported head_dim %d / group %d", D, gs);
        return -1;
    }
    if (B < 1 || B > kMaxBatch) {
        cgx_set_error("rope_append: batch %d outside [1, %d]", B, kMaxBatch);
        return -1;
    }
    if (rel && M > kMaxTreeRows) {
        cgx_set_error("rope_append: %d tree rows above %d", M, kMaxTreeRows);
        return -1;
    }
    RopeBatch rb;
    rb.has_rel = rel != nullptr;
    for (int r = 0; r < kMaxTreeRows; r++) rb.rel[r] = rel && r < M ? rel[r] : 0;
    rb.M = M;
    for (int b = 0; b < kMaxBatch; b++) rb.pos0[b] = b < B ? pos0[b] : 0;
    rb.seq_kbytes = seq_kbytes;
    rb.seq_groups = seq_groups;
    hipLaunchKernelGGL(k_rope_append, dim3(B * M, H + Hk), dim3(D / 2), 0, stream(), qkv, ld, H,
                       Hk, D, gs, rb, theta, (const float2*)cs, q_out, kc, vc, ks, vs);
    return launch_check("k_rope_append");
}

extern "C" int cgk_rope_append(const float* qkv, int ld, int M, int H, int Hk, int D, int gs,
                               int pos0, float theta, float* q_out, uint8_t* kc, uint8_t* vc,
                               float* ks, float* vs) {
    return cgk_rope_append_batch(qkv, ld, 1, M, H, Hk, D, gs, &pos0, nullptr, theta, nullptr,
                                 q_out, kc, vc, ks, vs, 0, 0);
}

extern "C" int cgk_spec_tokens(const int* feed, const int* dtok, int B, int gamma, int* ttok,
                               int* vtok) {
    if (B < 1 || gamma < 1) {
        cgx_set_error("spec_tokens: batch %d, gamma %d", B, gamma);
        return -1;
    }
    hipLaunchKernelGGL(k_spec_tokens, dim3(B), dim3(64), 0, stream(), feed, dtok, B, gamma, ttok,
                       vtok);
    return launch_check("k_spec_tokens");
}

// Per-matrix key: mixes the seed and the matrix id.
extern "C" uint32_t cgx_fill_key(uint64_t seed, uint32_t stream_id) {
    uint32_t k = (uint32_t)seed ^ (uint32_t)(seed >> 32) * 0x9E3779B9u;
    k = k * 0x85EBCA6Bu + stream_id * 0xC2B2AE35u;
    k ^= k >> 15;
    k *= 0x2C1B3C6Du;
    k ^= k >> 12;
    return k;
}

extern "C" int cgk_fill_normal(float* out, size_t n, uint64_t seed, uint32_t stream_id,
                               float stddev) {
    if (!n) return 0;
    // unit variance: 4 uniforms on [0, 65535] have variance 4 * (65536^2 - 1) / 12
    float scale = (float)((double)stddev * sqrt(3.0) / 65536.0);
    hipLaunchKernelGGL(k_fill_normal, dim3(4096), dim3(256), 0, stream(), out, n,
                       cgx_fill_key(seed, stream_id), scale);
    return launch_check("k_fill_normal");
}
