"""CPU restatement of the synthetic decoder stack (test infrastructure only),
composed from the oracle's pinned primitives:

  orc_fill_normal + orc_quantize_int4   seeded INT4 weights (the library's
                                        documented stream ids)
  orc_rmsnorm                           src/cuda/tensor_kernels.c:888-909
  orc_matmul_int4                       src/quantize/int4.c:90-114
  orc_apply_rope                        src/attention/flash_attn.c:335-360
  orc_kv_append / orc_kv_get            src/quantize/int4.c:147-289
  orc_flash_fwd (aligned causal)        src/cuda/flash_attn_kernels.c:261-396
  orc_swiglu                            src/layers/transformer.c:116-129

Block order: src/layers/transformer.c:26-149 (pre-norm, residuals, no bias).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle_lib import ptr

W_QKV, W_O, W_GU, W_DOWN, W_LM = range(5)


@dataclass
class Cfg:
    n_layers: int
    d_model: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    d_ff: int
    vocab: int
    group_size: int = 128
    kv_group_size: int = 64
    max_seq: int = 256
    max_tokens: int = 8
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    init_std: float = 0.02
    max_batch: int = 0

    def ctype(self):
        from cogito_amd.capi import CgxModelConfig
        return CgxModelConfig(**{k: getattr(self, k) for k in self.__dataclass_fields__})

    def shape(self, which):
        d, hq = self.d_model, self.n_heads * self.head_dim
        nqkv = (self.n_heads + 2 * self.n_kv_heads) * self.head_dim
        return {W_QKV: (d, nqkv), W_O: (hq, d), W_GU: (d, 2 * self.d_ff),
                W_DOWN: (self.d_ff, d), W_LM: (d, self.vocab)}[which]


def sid(layer, which):
    return 2 if which == W_LM else 16 * layer + 3 + which


def fill(orc, n, seed, stream_id, std):
    out = np.zeros(n, np.float32)
    orc.orc_fill_normal(ptr(out), n, seed, stream_id, std)
    return out


class OracleModel:
    """weights: None (the library's seeded weights) or a dict of fp32 arrays
    {"embed": [V, d], (layer, which): [K, N], W_LM: [d, V]} quantized here by
    orc_quantize_int4; norms: None (all 1) or 2 n_layers + 1 vectors (each
    layer's attention and MLP RMSNorm weights, then the final one)."""

    def __init__(self, orc, cfg: Cfg, seed: int, share_from: "OracleModel | None" = None,
                 weights=None, norms=None):
        self.orc, self.c, self.seed = orc, cfg, seed
        self.weights = weights
        d = cfg.d_model
        self.norms = ([np.ones(d, np.float32)] * (2 * cfg.n_layers + 1) if norms is None
                      else [np.ascontiguousarray(w, np.float32) for w in norms])
        if share_from is None:
            if weights is None:
                self.embed = fill(orc, cfg.vocab * cfg.d_model, seed, 1, cfg.init_std).reshape(
                    cfg.vocab, cfg.d_model)
            else:
                self.embed = np.ascontiguousarray(weights["embed"], np.float32)
            self.lm = self._lin(0, W_LM)
        else:
            self.embed, self.lm = share_from.embed, share_from.lm
        self.layers = [[self._lin(l, w) for w in range(4)] for l in range(cfg.n_layers)]
        kvb = cfg.max_seq * cfg.n_kv_heads * cfg.head_dim // 2
        kvg = cfg.max_seq * cfg.n_kv_heads * cfg.head_dim // cfg.kv_group_size
        self.kc = [np.zeros(kvb, np.uint8) for _ in range(cfg.n_layers)]
        self.vc = [np.zeros(kvb, np.uint8) for _ in range(cfg.n_layers)]
        self.ks = [np.zeros(kvg, np.float32) for _ in range(cfg.n_layers)]
        self.vs = [np.zeros(kvg, np.float32) for _ in range(cfg.n_layers)]
        self.len = 0

    def _lin(self, layer, which):
        K, N = self.c.shape(which)
        if self.weights is None:
            w = fill(self.orc, K * N, self.seed, sid(layer, which), self.c.init_std)
        else:
            key = W_LM if which == W_LM else (layer, which)
            w = np.ascontiguousarray(self.weights[key], np.float32).ravel()
            assert w.size == K * N
        data = np.zeros(K * N // 2, np.uint8)
        scales = np.zeros(K * N // self.c.group_size, np.float32)
        self.orc.orc_quantize_int4(ptr(w), K * N, self.c.group_size, ptr(data), ptr(scales))
        return data, scales, K, N

    def matmul(self, x, lin):
        data, scales, K, N = lin
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros((x.shape[0], N), np.float32)
        self.orc.orc_matmul_int4(ptr(x), x.shape[0], K, ptr(data), ptr(scales), N,
                                 self.c.group_size, ptr(y))
        return y

    def rmsnorm(self, x, i):
        """RMSNorm with weights i: 2 l / 2 l + 1 (layer l's attention / MLP
        norm), 2 n_layers (the final one)."""
        x = np.ascontiguousarray(x, np.float32)
        w = self.norms[i]
        y = np.zeros_like(x)
        self.orc.orc_rmsnorm(ptr(x), ptr(w), ptr(y), x.shape[0], x.shape[1], self.c.norm_eps)
        return y

    def forward_tree(self, tokens, rel, anc, tw):
        """Tree rows (host/tree.c, cgx_model_forward_tree): row i at cache slot
        len + i and rotary position len + rel[i]; of the keys, the last tw are
        visible to row i only where bit (key - (n - tw)) of anc[i] is set."""
        return self.forward(tokens, None, (rel, anc, tw))

    def forward(self, tokens, n_logits=None, tree=None):
        c, orc = self.c, self.orc
        M = len(tokens)
        pos0 = self.len
        H, Hk, hd, ff = c.n_heads, c.n_kv_heads, c.head_dim, c.d_ff
        x = self.embed[np.asarray(tokens)].astype(np.float32)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        for l in range(c.n_layers):
            wq, wo, wgu, wd = self.layers[l]
            qkv = self.matmul(self.rmsnorm(x, 2 * l), wq)
            q = np.ascontiguousarray(qkv[:, :H * hd]).reshape(M, H, hd)
            k = np.ascontiguousarray(qkv[:, H * hd:(H + Hk) * hd]).reshape(M, Hk, hd)
            v = np.ascontiguousarray(qkv[:, (H + Hk) * hd:]).reshape(M, Hk, hd)
            if tree is None:
                orc.orc_apply_rope(ptr(q), M, H, hd, pos0, c.rope_theta)
                orc.orc_apply_rope(ptr(k), M, Hk, hd, pos0, c.rope_theta)
            else:
                for m in range(M):
                    qm, km = np.ascontiguousarray(q[m]), np.ascontiguousarray(k[m])
                    orc.orc_apply_rope(ptr(qm), 1, H, hd, pos0 + int(tree[0][m]), c.rope_theta)
                    orc.orc_apply_rope(ptr(km), 1, Hk, hd, pos0 + int(tree[0][m]), c.rope_theta)
                    q[m], k[m] = qm, km
            for m in range(M):
                kt, vt = np.ascontiguousarray(k[m]), np.ascontiguousarray(v[m])
                orc.orc_kv_append(ptr(self.kc[l]), ptr(self.vc[l]), ptr(self.ks[l]),
                                  ptr(self.vs[l]), pos0 + m, Hk, hd, c.kv_group_size, ptr(kt),
                                  ptr(vt))
            n = pos0 + M
            K = np.zeros((n, Hk, hd), np.float32)
            V = np.zeros((n, Hk, hd), np.float32)
            orc.orc_kv_get(ptr(self.kc[l]), ptr(self.vc[l]), ptr(self.ks[l]), ptr(self.vs[l]),
                           n, Hk, hd, c.kv_group_size, ptr(K), ptr(V))
            O = np.zeros((1, M, H, hd), np.float32)
            if tree is None:
                orc.orc_flash_fwd(ptr(q), ptr(K), ptr(V), ptr(O), None, 1, M, n, H, Hk, hd,
                                  scale, 4, 0, None)
            else:
                _, anc, tw = tree
                mask = np.zeros((M, n), np.float32)
                for m in range(M):
                    for j in range(tw):
                        if not (int(anc[m]) >> j) & 1:
                            mask[m, n - tw + j] = -np.finfo(np.float32).max
                orc.orc_flash_fwd(ptr(q), ptr(K), ptr(V), ptr(O), None, 1, M, n, H, Hk, hd,
                                  scale, 3, 0, ptr(mask))
            x = x + self.matmul(O.reshape(M, H * hd), wo)
            gu = self.matmul(self.rmsnorm(x, 2 * l + 1), wgu)
            g = np.ascontiguousarray(gu[:, :ff])
            u = np.ascontiguousarray(gu[:, ff:])
            a = np.zeros_like(g)
            orc.orc_swiglu(ptr(g), ptr(u), ptr(a), g.size)
            x = x + self.matmul(a, wd)
        self.len = pos0 + M
        n_logits = M if n_logits is None else n_logits
        if n_logits == 0:
            return None
        return self.matmul(self.rmsnorm(x[M - n_logits:], 2 * c.n_layers), self.lm)

    def truncate(self, n):
        assert 0 <= n <= self.len
        self.len = n
