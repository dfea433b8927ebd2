// tree.hip -- tree verification on gfx950: the per-path acceptance walk over
// a verified draft tree, and the KV-cache compaction of the accepted path.
//
// Reference: cogito declares tree verification (include/cg_speculative.h:
// 15-25 cg_token_tree, :123-130 cg_tree_attention_mask) but its EAGLE tree
// builder is a stub (src/inference/speculative.c:244-262), so the walk
// below is this library's definition (recorded with the design decisions):
// drafted children are deterministic (the draft's top-c tokens), so the draft
// distribution at a node is a point mass on each candidate, and the lossless
// multi-candidate rule is recursive rejection against the target: at the
// current node, with target distribution p (its row's top-k list, T and
// top-p as in cg_sample_top_k / the filtered verify), candidate x is accepted
// with probability w[x] / W; a rejected candidate's mass is removed
// (w[x] = 0, W -= w[x]); the first accepted candidate becomes the current
// node.  When every candidate is rejected, or the node is a leaf, the next
// token is drawn from w / W by the reference's scan (r = u * W, first entry
// whose running sum exceeds r).
//
// One workgroup per sequence runs the walk on one lane: it touches at most
// depth + 1 lists of top_k entries, and one lane keeps the fp32 operation
// order identical to the oracle's (bit-exact decisions).
#include <hip/hip_runtime.h>

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

constexpr int kTreeMax = 64;       // nodes per tree (root included)
constexpr int kKidsMax = 4;        // children per node
constexpr int kListMax = 64;       // top-k entries per list
constexpr int kDepthMax = 15;
constexpr int kBatchMax = 16;

struct TreeArgs {
    int R;                         // nodes per tree (rows per sequence)
    int K;                         // entries per list
    int depth;                     // deepest node
    int nkids[kTreeMax];
    int kids[kTreeMax][kKidsMax];  // children in rank order
    int len0[kBatchMax];           // compaction: verified prefix length per sequence
};

// Walk of sequence blockIdx.x.  lidx/lp [B*R][K] lists; tok [B][R] node
// tokens (node 0: the verified root); u [B][depth + 1][kKidsMax + 1];
// outputs: out [B][depth + 2] accepted tokens then the drawn one, nacc [B],
// path [B][depth] node index of each accepted node.
__global__ void k_tree_accept(TreeArgs a, const int* __restrict__ lidx,
                              const float* __restrict__ lp, const int* __restrict__ tok,
                              const float* __restrict__ u, int* __restrict__ out,
                              int* __restrict__ nacc, int* __restrict__ path) {
    if (threadIdx.x != 0) return;
    const int b = blockIdx.x;
    const int K = a.K;
    const float* ub = u + (size_t)b * (a.depth + 1) * (kKidsMax + 1);
    int* ob = out + (size_t)b * (a.depth + 2);
    float w[kListMax];
    int node = 0, n = 0;
    for (int s = 0; s <= a.depth; s++) {
        const size_t row = (size_t)b * a.R + node;
        const int* li = lidx + row * K;
        const float* pl = lp + row * K;
        float W = 0.0f;
        for (int j = 0; j < K; j++) {
            w[j] = pl[j];
            W = __fadd_rn(W, w[j]);
        }
        int next = -1;
        for (int r = 0; r < a.nkids[node]; r++) {
            const int c = a.kids[node][r];
            const int x = tok[(size_t)b * a.R + c];
            int jx = -1;
            for (int j = 0; j < K; j++)
                if (w[j] > 0.0f && li[j] == x) {
                    jx = j;
                    break;
                }
            const float acc = jx >= 0 ? __fdiv_rn(w[jx], W) : 0.0f;
            if (ub[s * (kKidsMax + 1) + r] < acc) {
                next = c;
                break;
            }
            if (jx >= 0) {
                W = __fsub_rn(W, w[jx]);
                w[jx] = 0.0f;
            }
        }
        if (next >= 0) {
            path[(size_t)b * a.depth + n] = next;
            ob[n++] = tok[(size_t)b * a.R + next];
            node = next;
            continue;
        }
        // draw from w / W (all mass removed: from the list itself)
        if (!(W > 0.0f)) {
            W = 0.0f;
            for (int j = 0; j < K; j++) {
                w[j] = pl[j];
                W = __fadd_rn(W, w[j]);
            }
        }
        const float rr = __fmul_rn(ub[s * (kKidsMax + 1) + kKidsMax], W);
        float cum = 0.0f;
        int t = li[0];
        for (int j = 0; j < K; j++) {
            if (!(w[j] > 0.0f)) continue;
            cum = __fadd_rn(cum, w[j]);
            t = li[j];
            if (rr < cum) break;
        }
        ob[n] = t;
        break;
    }
    nacc[b] = n;
}

// Compaction of the accepted path in every layer's cache: for sequence b,
// the rows of nodes path[b][0..n) (cache slots len0 + node) move to slots
// len0 + 1 .. len0 + n.  The node at depth d has index >= d, so reading
// every source before writing any destination is enough.
__global__ __launch_bounds__(256) void k_kv_compact(TreeArgs a, const int* __restrict__ nacc,
                                                    const int* __restrict__ path, int B, int nb,
                                                    uint8_t* kc, uint8_t* vc, float* ks,
                                                    float* vs, int row_bytes, int row_groups,
                                                    size_t layer_bytes, size_t layer_groups) {
    __shared__ uint32_t sk[kDepthMax][256], sv[kDepthMax][256];
    __shared__ float gk[kDepthMax][64], gv[kDepthMax][64];
    const int l = blockIdx.x / B, b = blockIdx.x % B;
    const int n = nacc[b];
    const size_t slot = (size_t)l * nb + b;
    uint8_t* kb = kc + layer_bytes * slot;
    uint8_t* vb = vc + layer_bytes * slot;
    float* ksb = ks + layer_groups * slot;
    float* vsb = vs + layer_groups * slot;
    const int words = row_bytes / 4;
    for (int d = 0; d < n; d++) {
        const size_t src = (size_t)a.len0[b] + path[(size_t)b * a.depth + d];
        for (int i = threadIdx.x; i < words; i += blockDim.x) {
            sk[d][i] = ((const uint32_t*)(kb + src * row_bytes))[i];
            sv[d][i] = ((const uint32_t*)(vb + src * row_bytes))[i];
        }
        for (int i = threadIdx.x; i < row_groups; i += blockDim.x) {
            gk[d][i] = ksb[src * row_groups + i];
            gv[d][i] = vsb[src * row_groups + i];
        }
    }
    __syncthreads();
    for (int d = 0; d < n; d++) {
        const size_t dst = (size_t)a.len0[b] + 1 + d;
        for (int i = threadIdx.x; i < words; i += blockDim.x) {
            ((uint32_t*)(kb + dst * row_bytes))[i] = sk[d][i];
            ((uint32_t*)(vb + dst * row_bytes))[i] = sv[d][i];
        }
        for (int i = threadIdx.x; i < row_groups; i += blockDim.x) {
            ksb[dst * row_groups + i] = gk[d][i];
            vsb[dst * row_groups + i] = gv[d][i];
        }
    }
}

int fill_args(TreeArgs& a, const cgx_tree_shape* t, int K, int B, const int* len0) {
    if (!t || t->nodes < 1 || t->nodes > kTreeMax || t->depth < 0 || t->depth > kDepthMax ||
        K < 1 || K > kListMax || B < 1 || B > kBatchMax) {
        cgx_set_error("tree: unsupported tree (%d nodes, depth %d), list %d or batch %d",
                      t ? t->nodes : 0, t ? t->depth : 0, K, B);
        return -1;
    }
    a.R = t->nodes;
    a.K = K;
    a.depth = t->depth;
    for (int i = 0; i < kTreeMax; i++) {
        a.nkids[i] = i < t->nodes ? t->nkids[i] : 0;
        for (int r = 0; r < kKidsMax; r++) a.kids[i][r] = i < t->nodes ? t->kids[i][r] : 0;
        if (i < t->nodes && (a.nkids[i] < 0 || a.nkids[i] > kKidsMax)) {
            cgx_set_error("tree: node %d has %d children", i, a.nkids[i]);
            return -1;
        }
    }
    for (int b = 0; b < kBatchMax; b++) a.len0[b] = len0 && b < B ? len0[b] : 0;
    return 0;
}

// Tokens of the nodes first .. first + count - 1 (one tree level) of every
// sequence from their parents' top lists: the parents are the previous
// level's nodes pfirst .. pfirst + pcount - 1, whose lists (K entries) are
// rows b * pcount + (parent - pfirst) of lidx; a node of rank r takes entry r.
__global__ void k_tree_children(TreeArgs a, int first, int count, int pfirst, int pcount,
                                const int* __restrict__ parent, const int* __restrict__ rank,
                                const int* __restrict__ lidx, int* __restrict__ tok) {
    const int b = blockIdx.x, j = threadIdx.x;
    if (j >= count) return;
    const int node = first + j;
    const int pr = parent[node] - pfirst;
    tok[(size_t)b * a.R + node] = lidx[((size_t)b * pcount + pr) * a.K + rank[node]];
}

// out [B][count] = tok[b][first .. first + count) (the rows of one level).
__global__ void k_tree_gather(int R, int first, int count, const int* __restrict__ tok,
                              int* __restrict__ out) {
    const int b = blockIdx.x, j = threadIdx.x;
    if (j < count) out[(size_t)b * count + j] = tok[(size_t)b * R + first + j];
}

}  // namespace

extern "C" int cgk_tree_gather(int B, int R, int first, int count, const int* tok, int* out) {
    if (B < 1 || count < 1 || count > 64 || first < 0 || first + count > R) {
        cgx_set_error("tree_gather: invalid level (%d + %d of %d)", first, count, R);
        return -1;
    }
    hipLaunchKernelGGL(k_tree_gather, dim3(B), dim3(64), 0, stream(), R, first, count, tok, out);
    return launch_check("k_tree_gather");
}

extern "C" int cgk_tree_children(const cgx_tree_shape* t, int B, int K, int first, int count,
                                 int pfirst, int pcount, const int* parent_dev,
                                 const int* rank_dev, const int* lidx, int* tok) {
    TreeArgs a;
    if (fill_args(a, t, K, B, nullptr)) return -1;
    if (count < 1 || count > 64 || first + count > t->nodes || pfirst < 0 ||
        pfirst + pcount > first) {
        cgx_set_error("tree_children: invalid level (%d + %d, parents %d + %d)", first, count,
                      pfirst, pcount);
        return -1;
    }
    hipLaunchKernelGGL(k_tree_children, dim3(B), dim3(64), 0, stream(), a, first, count, pfirst,
                       pcount, parent_dev, rank_dev, lidx, tok);
    return launch_check("k_tree_children");
}

extern "C" int cgk_tree_accept(const cgx_tree_shape* t, int B, int K, const int* lidx,
                               const float* lp, const int* tok, const float* u, int* out,
                               int* nacc, int* path) {
    TreeArgs a;
    if (fill_args(a, t, K, B, nullptr)) return -1;
    hipLaunchKernelGGL(k_tree_accept, dim3(B), dim3(64), 0, stream(), a, lidx, lp, tok, u, out,
                       nacc, path);
    return launch_check("k_tree_accept");
}

extern "C" int cgk_kv_compact(const cgx_tree_shape* t, int B, const int* len0, const int* nacc,
                              const int* path, int layers, int nb, uint8_t* kc, uint8_t* vc,
                              float* ks, float* vs, int row_bytes, int row_groups,
                              size_t layer_bytes, size_t layer_groups) {
    TreeArgs a;
    if (fill_args(a, t, 1, B, len0)) return -1;
    if (row_bytes % 4 || row_bytes / 4 > 256 || row_groups > 64 || B > nb) {
        cgx_set_error("kv_compact: rows of %d bytes / %d groups not supported", row_bytes,
                      row_groups);
        return -1;
    }
    hipLaunchKernelGGL(k_kv_compact, dim3(layers * B), dim3(256), 0, stream(), a, nacc, path,
                       B, nb, kc, vc, ks, vs, row_bytes, row_groups, layer_bytes, layer_groups);
    return launch_check("k_kv_compact");
}
