"""Pins the oracle's KV-cache, flash-attention, RoPE and ALiBi restatements
(CPU only).

* against cogito's own sources compiled from the reference tree
  (oracle/_ref): bit-exact, same inputs;
* against closed forms: float64 softmax attention computed directly (no
  tiling, no online rescaling), the ALiBi slope formula, RoPE's rotation
  invariants.

Reference: src/quantize/int4.c:116-289 (KV cache),
src/cuda/flash_attn_kernels.c:261-396 (forward simulation),
src/attention/flash_attn.c:17-149 (CPU forward), :318-388 (RoPE, ALiBi).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cogito_amd.capi import CgFlashAttnParams
import oracle_lib
from oracle_lib import RefKv, ptr, ref_tensor  # noqa: F401

FLT_MAX = np.finfo(np.float32).max


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ----------------------------------------------------------------- KV cache

def oracle_kv_fill(oracle, ks_tok, vs_tok, H, D, gs, max_len):
    """Appends tokens [T][H][D] one by one into a one-layer oracle cache."""
    T = ks_tok.shape[0]
    kc = np.zeros(max_len * H * D // 2, np.uint8)
    vc = np.zeros_like(kc)
    ksc = np.zeros(max_len * H * D // gs, np.float32)
    vsc = np.zeros_like(ksc)
    for t in range(T):
        kt = np.ascontiguousarray(ks_tok[t], np.float32)
        vt = np.ascontiguousarray(vs_tok[t], np.float32)
        oracle.orc_kv_append(ptr(kc), ptr(vc), ptr(ksc), ptr(vsc), t, H, D, gs, ptr(kt), ptr(vt))
    return kc, vc, ksc, vsc


def oracle_kv_get(oracle, kc, vc, ksc, vsc, T, H, D, gs):
    ko = np.zeros((T, H, D), np.float32)
    vo = np.zeros_like(ko)
    oracle.orc_kv_get(ptr(kc), ptr(vc), ptr(ksc), ptr(vsc), T, H, D, gs, ptr(ko), ptr(vo))
    return ko, vo


def kv_inputs(rng, T, H, D, gs):
    k = rng.normal(0, 1.0, (T, H, D)).astype(np.float32)
    v = rng.normal(0, 2.0, (T, H, D)).astype(np.float32)
    k[0, 0, :gs] = 0.0                                   # all-zero group: scale 1.0
    if T > 1:
        # exact half steps: x / s = +-(n + 0.5), rounded away from zero
        k[1, 0, :gs] = np.array([7.0, -3.5, 2.5, -0.5] * (gs // 4), np.float32)
    v[-1, -1, :gs] = 1e-9                                 # scale below the 1e-8 floor
    return k, v


@pytest.mark.parametrize("T,H,D,gs", [(9, 4, 64, 32), (5, 2, 128, 128), (3, 3, 80, 16)])
def test_kv_append_get_vs_reference(ref, oracle, rng, T, H, D, gs):
    k, v = kv_inputs(rng, T, H, D, gs)
    max_len = T + 3
    kc, vc, ksc, vsc = oracle_kv_fill(oracle, k, v, H, D, gs, max_len)
    c = ref.cg_kv_cache_int4_new(1, max_len, H, D, gs)
    keep = []
    for t in range(T):
        kt, vt = ref_tensor(ref, k[t][None, None]), ref_tensor(ref, v[t][None, None])
        keep += [kt, vt]
        ref.cg_kv_cache_int4_append(c, 0, kt, vt)
    assert c.contents.current_len == T
    nb = max_len * H * D // 2
    ng = max_len * H * D // gs
    rk = np.ctypeslib.as_array(c.contents.k_cache, shape=(nb,)).copy()
    rv = np.ctypeslib.as_array(c.contents.v_cache, shape=(nb,)).copy()
    rks = np.ctypeslib.as_array(c.contents.k_scales, shape=(ng,)).copy()
    rvs = np.ctypeslib.as_array(c.contents.v_scales, shape=(ng,)).copy()
    np.testing.assert_array_equal(kc, rk)
    np.testing.assert_array_equal(vc, rv)
    np.testing.assert_array_equal(_bits(ksc), _bits(rks))
    np.testing.assert_array_equal(_bits(vsc), _bits(rvs))
    # get: dequantised history
    ko, vo = oracle_kv_get(oracle, kc, vc, ksc, vsc, T, H, D, gs)
    rko = ref_tensor(ref, np.zeros((T, H, D), np.float32))
    rvo = ref_tensor(ref, np.zeros((T, H, D), np.float32))
    ref.cg_kv_cache_int4_get(c, 0, rko, rvo)
    got_k = np.ctypeslib.as_array(rko.contents.data, shape=(T * H * D,)).copy()
    got_v = np.ctypeslib.as_array(rvo.contents.data, shape=(T * H * D,)).copy()
    np.testing.assert_array_equal(_bits(ko.ravel()), _bits(got_k))
    np.testing.assert_array_equal(_bits(vo.ravel()), _bits(got_v))
    ref.cg_kv_cache_int4_free(c)
    for t in keep + [rko, rvo]:
        ref.cg_tensor_free(t)


def test_kv_closed_forms(oracle, rng):
    # scale = absmax / 7; codes round(x / scale) clamped to [-8, 7]; the
    # absmax element dequantises to itself (7 * absmax / 7, up to one rounding)
    H, D, gs = 2, 32, 16
    k, v = kv_inputs(rng, 4, H, D, gs)
    kc, vc, ksc, vsc = oracle_kv_fill(oracle, k, v, H, D, gs, 4)
    ko, vo = oracle_kv_get(oracle, kc, vc, ksc, vsc, 4, H, D, gs)
    g = k.reshape(4, H, D // gs, gs)
    amax = np.abs(g).max(-1)
    exp_scale = np.where(amax / np.float32(7.0) < 1e-8, 1.0, amax / np.float32(7.0))
    np.testing.assert_array_equal(ksc.reshape(4, H, D // gs), exp_scale.astype(np.float32))
    step = np.repeat(exp_scale, gs, -1).reshape(4, H, D)
    assert np.all(np.abs(ko - k) <= 0.5 * step * (1 + 1e-6))
    # the zero group and the sub-floor group decode to exact zeros / tiny
    assert np.all(ko[0, 0, :gs] == 0.0)
    # half steps round away from zero: 7.0/1.0 -> 7, -3.5 -> -4, 2.5 -> 3, -0.5 -> -1
    assert list(ko[1, 0, :4]) == [7.0, -4.0, 3.0, -1.0]


# ------------------------------------------------------------ attention

def np_attention(Q, K, V, H, Hk, mask_fn, scale):
    """Direct float64 softmax attention: O[b,q,h] = softmax(QK^T*s + mask) V.
    mask_fn(q, k) -> additive float (0, -inf or a custom value)."""
    B, Nq, _, D = Q.shape
    Nk = K.shape[1]
    O = np.zeros(Q.shape, np.float64)
    lse = np.zeros((B, H, Nq), np.float64)
    M = np.array([[mask_fn(q, k) for k in range(Nk)] for q in range(Nq)], np.float64)
    for b in range(B):
        for h in range(H):
            hk = h * Hk // H
            s = Q[b, :, h, :].astype(np.float64) @ K[b, :, hk, :].astype(np.float64).T
            s = s * scale + M
            mx = s.max(-1, keepdims=True)
            p = np.exp(s - mx)
            lse[b, h] = mx[:, 0] + np.log(p.sum(-1))
            O[b, :, h, :] = (p / p.sum(-1, keepdims=True)) @ V[b, :, hk, :].astype(np.float64)
    return O, lse


def orc_attention(oracle, Q, K, V, H, Hk, scale, mask_type, window=0, mask=None):
    B, Nq, _, D = Q.shape
    Nk = K.shape[1]
    O = np.zeros(Q.shape, np.float32)
    lse = np.zeros((B, H, Nq), np.float32)
    m = np.ascontiguousarray(mask, np.float32) if mask is not None else None
    oracle.orc_flash_fwd(ptr(Q), ptr(K), ptr(V), ptr(O), ptr(lse), B, Nq, Nk, H, Hk, D,
                         scale, mask_type, window, ptr(m) if m is not None else None)
    return O, lse


def attn_inputs(rng, B, Nq, Nk, H, Hk, D):
    Q = rng.normal(0, 1, (B, Nq, H, D)).astype(np.float32)
    K = rng.normal(0, 1, (B, Nk, Hk, D)).astype(np.float32)
    V = rng.normal(0, 1, (B, Nk, Hk, D)).astype(np.float32)
    return Q, K, V


@pytest.mark.parametrize("mask_type,Nq,Nk", [(0, 70, 70), (1, 70, 70), (1, 5, 130), (2, 40, 90)])
def test_flash_sim_vs_reference(ref, oracle, rng, mask_type, Nq, Nk):
    B, H, Hk, D = 2, 4, 2, 32
    Q, K, V = attn_inputs(rng, B, Nq, Nk, H, Hk, D)
    scale = 1.0 / np.sqrt(D)
    O, lse = orc_attention(oracle, Q, K, V, H, Hk, scale, mask_type, window=7)
    rO = np.zeros_like(Q)
    rlse = np.zeros((B, H, Nq), np.float32)
    p = CgFlashAttnParams(Q=Q.ctypes.data, K=K.ctypes.data, V=V.ctypes.data, O=rO.ctypes.data,
                          batch_size=B, seqlen_q=Nq, seqlen_k=Nk, n_heads=H, n_heads_k=Hk,
                          d_head=D, scale=scale, mask_type=mask_type, window_size=7,
                          softmax_lse=rlse.ctypes.data)
    ref.cg_flash_attention_forward_cuda(C.byref(p))
    np.testing.assert_array_equal(_bits(O), _bits(rO))
    np.testing.assert_array_equal(_bits(lse), _bits(rlse))


def test_flash_cpu_forward_vs_reference(ref, oracle, rng):
    # the reference CPU forward: K/V have n_heads heads, causal k > q masked
    B, Nq, Nk, H, D = 1, 66, 66, 3, 16
    Q, K, V = attn_inputs(rng, B, Nq, Nk, H, H, D)
    scale = 0.3
    O, lse = orc_attention(oracle, Q, K, V, H, H, scale, 1)
    rO = np.zeros_like(Q)
    rlse = np.zeros((B, H, Nq), np.float32)
    p = CgFlashAttnParams(Q=Q.ctypes.data, K=K.ctypes.data, V=V.ctypes.data, O=rO.ctypes.data,
                          batch_size=B, seqlen_q=Nq, seqlen_k=Nk, n_heads=H, n_heads_k=H,
                          d_head=D, scale=scale, mask_type=1, softmax_lse=rlse.ctypes.data)
    ref.cg_flash_attention_forward_cpu(C.byref(p))
    # same algorithm, different loop nest: the CPU forward keeps per-row
    # state across query tiles identically, so results agree bit for bit
    np.testing.assert_array_equal(_bits(O), _bits(rO))
    np.testing.assert_array_equal(_bits(lse), _bits(rlse))


@pytest.mark.parametrize("mask_type", [0, 1, 2, 3, 4])
def test_flash_oracle_vs_direct_softmax(oracle, rng, mask_type):
    # pins the tiled online softmax (and each mask rule) against float64
    # attention computed in one pass
    B, Nq, Nk, H, Hk, D = 1, 20, 150, 4, 1, 24
    if mask_type == 1:
        Nq = Nk = 100
    Q, K, V = attn_inputs(rng, B, Nq, Nk, H, Hk, D)
    scale = 0.2
    W = 9
    add = rng.normal(0, 1, (Nq, Nk)).astype(np.float32)
    rules = {
        0: lambda q, k: 0.0,
        1: lambda q, k: 0.0 if k <= q else -np.inf,
        2: lambda q, k: 0.0 if abs(k - q) <= W else -np.inf,
        3: lambda q, k: float(add[q, k]),
        4: lambda q, k: 0.0 if k <= Nk - Nq + q else -np.inf,
    }
    O, lse = orc_attention(oracle, Q, K, V, H, Hk, scale, mask_type, W,
                           add if mask_type == 3 else None)
    eO, else_ = np_attention(Q, K, V, H, Hk, rules[mask_type], scale)
    np.testing.assert_allclose(O, eO, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(lse, else_, rtol=1e-5, atol=1e-5)


def test_flash_oracle_fully_masked_rows(oracle, rng):
    # rows with no visible key (window, q > Nk - 1 + W): every score is
    # -FLT_MAX, so the reference averages V uniformly (and lse is
    # -FLT_MAX + log(Nk))
    B, Nq, Nk, H, D, W = 1, 12, 4, 1, 8, 2
    Q, K, V = attn_inputs(rng, B, Nq, Nk, H, H, D)
    O, lse = orc_attention(oracle, Q, K, V, H, H, 0.5, 2, W)
    for q in range(Nk + W, Nq):
        np.testing.assert_allclose(O[0, q, 0], V[0, :, 0].mean(0), rtol=1e-5, atol=1e-6)
        assert lse[0, 0, q] == np.float32(-FLT_MAX)


# ------------------------------------------------------------ RoPE, ALiBi

@pytest.mark.parametrize("S,H,D,off,theta", [(7, 3, 64, 0, 10000.0), (5, 2, 128, 4091, 500000.0),
                                             (3, 1, 10, 17, 10000.0)])
def test_rope_vs_reference(ref, oracle, rng, S, H, D, off, theta):
    q = rng.normal(0, 1, (S, H, D)).astype(np.float32)
    k = rng.normal(0, 1, (S, H, D)).astype(np.float32)
    oq, ok = q.copy(), k.copy()
    oracle.orc_apply_rope(ptr(oq), S, H, D, off, theta)
    oracle.orc_apply_rope(ptr(ok), S, H, D, off, theta)
    rq, rk = q.copy(), k.copy()
    ref.cg_apply_rope(ptr(rq), ptr(rk), S, H, D, off, theta)
    np.testing.assert_array_equal(_bits(oq), _bits(rq))
    np.testing.assert_array_equal(_bits(ok), _bits(rk))
    cs = np.zeros((S + off) * (D // 2), np.float32)
    sn = np.zeros_like(cs)
    rcs, rsn = cs.copy(), sn.copy()
    oracle.orc_rope_freqs(ptr(cs), ptr(sn), S + off, D, theta)
    ref.cg_rope_precompute_freqs(ptr(rcs), ptr(rsn), S + off, D, theta)
    np.testing.assert_array_equal(_bits(cs), _bits(rcs))
    np.testing.assert_array_equal(_bits(sn), _bits(rsn))


def test_rope_invariants(oracle, rng):
    # position 0 is the identity; each (i, i + D/2) pair keeps its norm; the
    # score of rotated q (pos m) and k (pos n) depends only on m - n
    D, H = 64, 1
    x = rng.normal(0, 1, (1, H, D)).astype(np.float32)
    y = x.copy()
    oracle.orc_apply_rope(ptr(y), 1, H, D, 0, 10000.0)
    np.testing.assert_array_equal(x, y)
    z = x.copy()
    oracle.orc_apply_rope(ptr(z), 1, H, D, 37, 10000.0)
    n0 = x[0, 0, :32] ** 2 + x[0, 0, 32:] ** 2
    n1 = z[0, 0, :32] ** 2 + z[0, 0, 32:] ** 2
    np.testing.assert_allclose(n0, n1, rtol=1e-5)
    q = rng.normal(0, 1, (1, 1, D)).astype(np.float32)
    k = rng.normal(0, 1, (1, 1, D)).astype(np.float32)

    def score(m, n):
        a, b = q.copy(), k.copy()
        oracle.orc_apply_rope(ptr(a), 1, 1, D, m, 10000.0)
        oracle.orc_apply_rope(ptr(b), 1, 1, D, n, 10000.0)
        return float(a.astype(np.float64).ravel() @ b.astype(np.float64).ravel())

    assert abs(score(10, 3) - score(107, 100)) < 1e-4
    # angle of pair 0 at position p is exactly p radians (freq_0 = 1)
    e = np.zeros((1, 1, D), np.float32)
    e[0, 0, 0] = 1.0
    oracle.orc_apply_rope(ptr(e), 1, 1, D, 5, 10000.0)
    np.testing.assert_allclose([e[0, 0, 0], e[0, 0, 32]], [np.cos(5.0), np.sin(5.0)], atol=1e-6)


@pytest.mark.parametrize("H", [1, 8, 12, 32])
def test_alibi_vs_reference_and_closed_form(ref, oracle, H):
    s = np.zeros(H, np.float32)
    r = np.zeros(H, np.float32)
    oracle.orc_alibi_slopes(ptr(s), H)
    ref.cg_alibi_slopes(ptr(r), H)
    np.testing.assert_array_equal(_bits(s), _bits(r))
    np.testing.assert_allclose(s, 2.0 ** (-8.0 * np.arange(1, H + 1) / H), rtol=2e-6)
    Sq, Sk = 5, 9
    b = np.zeros(H * Sq * Sk, np.float32)
    rb = np.zeros_like(b)
    oracle.orc_alibi_bias(ptr(b), Sq, Sk, H, ptr(s))
    ref.cg_alibi_bias(ptr(rb), Sq, Sk, H, ptr(s))
    np.testing.assert_array_equal(_bits(b), _bits(rb))
    exp = s[:, None, None] * (np.arange(Sk)[None, None, :] - np.arange(Sq)[None, :, None])
    np.testing.assert_array_equal(b.reshape(H, Sq, Sk), exp.astype(np.float32))


# ------------------------------------------------------------ seeded fill

def test_fill_normal_moments_and_determinism(oracle):
    # the synthetic weights' rule: unit variance (Irwin-Hall n = 4 scaled by
    # sqrt(3)), mean 0, bounded by 2*sqrt(3); same seed/stream -> same bits,
    # another stream -> independent values
    from oracle_model import fill
    n = 400000
    a = fill(oracle, n, 123, 7, 1.0).astype(np.float64)
    assert abs(a.mean()) < 0.01
    assert abs(a.std() - 1.0) < 0.01
    assert np.abs(a).max() <= 2 * np.sqrt(3) + 1e-6
    # excess kurtosis of Irwin-Hall(4) is -0.3
    kurt = ((a - a.mean()) ** 4).mean() / a.var() ** 2 - 3
    assert abs(kurt + 0.3) < 0.05
    b = fill(oracle, n, 123, 7, 1.0)
    np.testing.assert_array_equal(a.astype(np.float32), b)
    c = fill(oracle, n, 123, 8, 1.0).astype(np.float64)
    assert abs(np.corrcoef(a, c)[0, 1]) < 0.01
    s = fill(oracle, 1000, 123, 7, 0.02)
    np.testing.assert_allclose(s, (a[:1000] * 0.02).astype(np.float32), rtol=1e-6)


# ----------------------------------------------------- RMSNorm and SwiGLU

@pytest.mark.parametrize("rows,d,eps", [(1, 768, 1e-5), (5, 4096, 1e-5), (3, 70, 1e-6)])
def test_rmsnorm_vs_reference_and_fp64(ref, oracle, rng, rows, d, eps):
    # orc_rmsnorm restates tensor_kernels.c:888-909; the compiled reference
    # pins it bitwise, fp64 pins the formula (a dropped eps or a sum over the
    # wrong axis fails the second check)
    x = rng.normal(0, 2, (rows, d)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, d).astype(np.float32)
    y = np.zeros_like(x)
    oracle.orc_rmsnorm(ptr(x), ptr(w), ptr(y), rows, d, eps)
    tx, tw, ty = (oracle_lib.ref_tensor(ref, a) for a in (x, w, np.zeros_like(x)))
    ref.cg_cuda_rmsnorm_forward(tx, tw, ty, eps)
    yr = oracle_lib.ref_tensor_np(ty)
    for t in (tx, tw, ty):
        ref.cg_tensor_free(t)
    np.testing.assert_array_equal(y.view(np.uint32), yr.view(np.uint32))
    xd = x.astype(np.float64)
    exp = w * xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + eps)
    np.testing.assert_allclose(y, exp, rtol=2e-6, atol=1e-7)


def test_swiglu_closed_form(oracle, rng):
    # transformer.c:116-129: g / (1 + exp(-g)) * u
    g = np.concatenate([rng.normal(0, 3, 5000), [0.0, -0.0, 30.0, -30.0, -100.0, 88.0]])
    g = g.astype(np.float32)
    u = rng.normal(0, 1, g.size).astype(np.float32)
    out = np.zeros_like(g)
    oracle.orc_swiglu(ptr(g), ptr(u), ptr(out), g.size)
    gd = g.astype(np.float64)
    exp = gd / (1.0 + np.exp(-gd)) * u
    np.testing.assert_allclose(out, exp, rtol=1e-6, atol=1e-30)
    # g = 0 gives 0; g = -100 overflows exp(100) to inf and gives (signed) 0
    assert out[-6] == 0.0 and out[-2] == 0.0


@pytest.mark.parametrize("rows,dim", [(1, 6), (3, 4096), (5, 11008)])
def test_swiglu_vs_reference(ref, oracle, rng, rows, dim):
    # orc_swiglu restates transformer.c:122-127; the reference's split form
    # (activations.c:34-54, gate | value halves of one row) is the same
    # expression, so the compiled reference pins it bit for bit, including
    # gates whose exp(-g) overflows or underflows
    g = rng.normal(0, 3, (rows, dim)).astype(np.float32)
    g[0, :6] = [0.0, -0.0, 30.0, -30.0, -100.0, 88.0]
    u = rng.normal(0, 1, (rows, dim)).astype(np.float32)
    out = np.zeros_like(g)
    oracle.orc_swiglu(ptr(g), ptr(u), ptr(out), g.size)
    t = oracle_lib.ref_tensor(ref, np.concatenate([g, u], axis=1))
    r = ref.cg_swiglu_forward_split(t)
    yr = oracle_lib.ref_tensor_np(r)
    ref.cg_tensor_free(t)
    ref.cg_tensor_free(r)
    assert yr.shape == (rows, dim)
    np.testing.assert_array_equal(out.view(np.uint32), yr.view(np.uint32))


@pytest.mark.parametrize("rows,V", [(1, 1), (4, 1000), (2, 32000)])
def test_softmax_rows_vs_reference(ref, oracle, rng, rows, V):
    # orc_softmax_rows restates tensor_kernels.c:699-740 over axis 1 of a
    # [rows][V] tensor: the compiled reference pins it bit for bit (ties at
    # the maximum, a -inf logit), fp64 pins the formula
    x = rng.normal(0, 3, (rows, V)).astype(np.float32)
    if V >= 8:
        x[0, :3] = x[0].max()
        x[-1, 5] = -np.inf
    y = np.zeros_like(x)
    oracle.orc_softmax_rows(ptr(x), ptr(y), rows, V)
    tx, ty = oracle_lib.ref_tensor(ref, x), oracle_lib.ref_tensor(ref, np.zeros_like(x))
    ref.cg_cuda_softmax_forward(tx, ty, 1)
    yr = oracle_lib.ref_tensor_np(ty)
    ref.cg_tensor_free(tx)
    ref.cg_tensor_free(ty)
    np.testing.assert_array_equal(y.view(np.uint32), yr.view(np.uint32))
    # the sequential fp32 sum of V terms is within V 2^-24 (1 + 2^-7) of the
    # real sum; expf and the division add a few ulps
    xd = x.astype(np.float64)
    e = np.exp(xd - xd.max(axis=1, keepdims=True))
    rtol = V * 2.0**-24 * (1 + 2.0**-7) + 4 * 2.0**-24
    np.testing.assert_allclose(y, e / e.sum(axis=1, keepdims=True), rtol=rtol, atol=1e-30)
