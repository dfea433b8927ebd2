"""GPU parity of the INT4 KV cache, attention over it (chain and tree masks),
the fp32 flash-attention API, RoPE and ALiBi against the oracle.

Bars: KV append / get bit-exact (same fp32 division, roundf, clamp);
attention within 1e-3 of max|O| per output row (fp32 products, different
summation order and a hardware exp); RoPE / ALiBi within 1e-3 relative
(GPU powf / sinf / cosf are not glibc's).
Reference: src/quantize/int4.c:116-289, src/cuda/flash_attn_kernels.c:261-396,
src/attention/flash_attn.c:17-149, 318-388.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cogito_amd.capi import CgFlashAttnParams, DeviceArray, last_error
from gpu_util import host_tensor, rel_err_rows
from oracle_lib import ptr
from test_attn_oracle import attn_inputs, oracle_kv_fill, oracle_kv_get, orc_attention

pytestmark = pytest.mark.gpu
TOL = 1e-3
FLT_MAX = np.finfo(np.float32).max


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def cache_arrays(lib, c, layer):
    """Host copies of one layer's K/V bytes and scales."""
    cc = c.contents
    nb = cc.max_seq_len * cc.n_heads * cc.head_dim // 2
    ng = cc.max_seq_len * cc.n_heads * cc.head_dim // cc.group_size
    out = []
    for arr, n, dt, esz in ((cc.k_cache, nb, np.uint8, 1), (cc.v_cache, nb, np.uint8, 1),
                            (cc.k_scales, ng, np.float32, 4), (cc.v_scales, ng, np.float32, 4)):
        h = np.empty(n, dt)
        base = C.cast(arr, C.c_void_p).value + layer * n * esz
        assert lib.cgx_memcpy_d2h(h.ctypes.data, base, n * esz) == 0, last_error(lib)
        out.append(h)
    return out


# ----------------------------------------------------------------- KV cache

def test_kv_append_bitexact_and_length_rule(gpu, oracle, rng):
    L, T, H, D, gs, S = 3, 6, 4, 64, 32, 10
    ks = [rng.normal(0, 1, (T, H, D)).astype(np.float32) for _ in range(L)]
    vs = [rng.normal(0, 2, (T, H, D)).astype(np.float32) for _ in range(L)]
    ks[1][2, 1, :gs] = 0.0                       # zero group -> scale 1.0
    ks[2][0, 0, :8] = [7.0, -3.5, 2.5, -0.5, 0.5, 1.5, -7.0, 0.0]
    c = gpu.cg_kv_cache_int4_new(L, S, H, D, gs)
    assert c, last_error(gpu)
    for t in range(T):
        for layer in range(L):
            kt = host_tensor(gpu, ks[layer][t][None, None])
            vt = host_tensor(gpu, vs[layer][t][None, None])
            gpu.cg_kv_cache_int4_append(c, layer, kt, vt)
            assert last_error(gpu) in ("", None), last_error(gpu)
            # current_len advances once per position, on the last layer
            assert c.contents.current_len == t + (layer == L - 1)
            gpu.cg_tensor_free(kt)
            gpu.cg_tensor_free(vt)
    for layer in range(L):
        exp = oracle_kv_fill(oracle, ks[layer], vs[layer], H, D, gs, S)
        got = cache_arrays(gpu, c, layer)
        for e, g in zip(exp, got):
            if e.dtype == np.float32:
                np.testing.assert_array_equal(_bits(e), _bits(g))
            else:
                np.testing.assert_array_equal(e, g)
        # get: host outputs
        ko, vo = oracle_kv_get(oracle, *exp, T, H, D, gs)
        hk = host_tensor(gpu, np.zeros((T, H, D), np.float32))
        hv = host_tensor(gpu, np.zeros((T, H, D), np.float32))
        gpu.cg_kv_cache_int4_get(c, layer, hk, hv)
        gk = np.ctypeslib.as_array(hk.contents.data, shape=(T * H * D,))
        gv = np.ctypeslib.as_array(hv.contents.data, shape=(T * H * D,))
        np.testing.assert_array_equal(_bits(gk), _bits(ko.ravel()))
        np.testing.assert_array_equal(_bits(gv), _bits(vo.ravel()))
        gpu.cg_tensor_free(hk)
        gpu.cg_tensor_free(hv)
    gpu.cg_kv_cache_int4_free(c)


def test_kv_write_block_and_device_get(gpu, oracle, rng):
    H, D, gs, S, T = 8, 128, 128, 300, 257
    k = rng.normal(0, 1, (T, H, D)).astype(np.float32)
    v = rng.normal(0, 1, (T, H, D)).astype(np.float32)
    c = gpu.cg_kv_cache_int4_new(2, S, H, D, gs)
    assert c, last_error(gpu)
    dk, dv = DeviceArray.from_numpy(gpu, k), DeviceArray.from_numpy(gpu, v)
    # layer 1, device inputs, one call for all T tokens
    assert gpu.cgx_kv_cache_int4_write(c, 1, 0, dk.ptr, dv.ptr, T) == 0, last_error(gpu)
    assert c.contents.current_len == 0
    assert gpu.cgx_kv_cache_int4_set_len(c, T) == 0
    exp = oracle_kv_fill(oracle, k, v, H, D, gs, S)
    got = cache_arrays(gpu, c, 1)
    np.testing.assert_array_equal(exp[0], got[0])
    np.testing.assert_array_equal(exp[1], got[1])
    np.testing.assert_array_equal(_bits(exp[2]), _bits(got[2]))
    np.testing.assert_array_equal(_bits(exp[3]), _bits(got[3]))
    ko, vo = oracle_kv_get(oracle, *exp, T, H, D, gs)
    shape = (C.c_int * 3)(T, H, D)
    tk, tv = gpu.cgx_tensor_device_new(shape, 3), gpu.cgx_tensor_device_new(shape, 3)
    gpu.cg_kv_cache_int4_get(c, 1, tk, tv)
    for t, e in ((tk, ko), (tv, vo)):
        h = np.empty(T * H * D, np.float32)
        assert gpu.cgx_tensor_to_host(t, h.ctypes.data_as(C.POINTER(C.c_float))) == 0
        np.testing.assert_array_equal(_bits(h), _bits(e.ravel()))
        gpu.cg_tensor_free(t)
    # layer 0 untouched
    assert not cache_arrays(gpu, c, 0)[0].any()
    dk.free()
    dv.free()
    gpu.cg_kv_cache_int4_free(c)


def test_kv_cache_errors(gpu):
    gpu.cgx_clear_error()
    assert not gpu.cg_kv_cache_int4_new(1, 4, 2, 7, 7)          # odd head_dim
    assert "invalid" in last_error(gpu)
    c = gpu.cg_kv_cache_int4_new(1, 2, 1, 8, 4)
    assert c, last_error(gpu)
    x = host_tensor(gpu, np.ones((1, 1, 1, 8), np.float32))
    for _ in range(2):
        gpu.cg_kv_cache_int4_append(c, 0, x, x)
    assert c.contents.current_len == 2
    gpu.cgx_clear_error()
    gpu.cg_kv_cache_int4_append(c, 0, x, x)                      # full
    assert "full" in last_error(gpu) and c.contents.current_len == 2
    assert gpu.cgx_kv_cache_int4_truncate(c, 3) != 0
    assert gpu.cgx_kv_cache_int4_truncate(c, 1) == 0 and c.contents.current_len == 1
    assert gpu.cgx_kv_cache_int4_set_len(c, 5) != 0
    gpu.cg_kv_cache_int4_reset(c)
    assert c.contents.current_len == 0
    gpu.cg_tensor_free(x)
    gpu.cg_kv_cache_int4_free(c)


# ------------------------------------------------------- INT4-KV attention

def build_cache(gpu, oracle, rng, H, Hk, D, gs, n_tok, S=None):
    """A one-layer cache holding n_tok random tokens, plus the oracle's
    dequantised K/V [1][n_tok][Hk][D]."""
    S = S or n_tok
    k = rng.normal(0, 1, (n_tok, Hk, D)).astype(np.float32)
    v = rng.normal(0, 1, (n_tok, Hk, D)).astype(np.float32)
    c = gpu.cg_kv_cache_int4_new(1, S, Hk, D, gs)
    assert c, last_error(gpu)
    assert gpu.cgx_kv_cache_int4_write(c, 0, 0, k.ctypes.data, v.ctypes.data, n_tok) == 0, \
        last_error(gpu)
    assert gpu.cgx_kv_cache_int4_set_len(c, n_tok) == 0
    arrs = oracle_kv_fill(oracle, k, v, Hk, D, gs, S)
    ko, vo = oracle_kv_get(oracle, *arrs, n_tok, Hk, D, gs)
    return c, ko[None], vo[None]


CHAIN_CASES = [
    # H, Hk, D, gs, ctx, Nq
    (32, 8, 128, 32, 1000, 1),
    (32, 8, 128, 128, 1000, 5),
    (32, 32, 128, 64, 513, 8),
    (16, 2, 64, 32, 3000, 33),
    (8, 8, 80, 16, 200, 3),        # head_dim not a multiple of 32
    (4, 4, 32, 32, 77, 1),
    (12, 4, 96, 32, 300, 4),
    (32, 8, 128, 32, 16000, 5),    # many key splits
    (2, 1, 64, 64, 0, 6),          # no context: pure causal block
    # one scale per head row (the decoder's cache): the MFMA decode kernel
    (32, 8, 128, 128, 4096, 5),    # 7B-shape verify step
    (12, 12, 64, 64, 1024, 5),     # tiny-decoder verify step
    (32, 8, 128, 128, 16000, 5),   # more than one key round per split
    (8, 2, 32, 32, 300, 7),
    (32, 8, 128, 128, 255, 1),     # fewer keys than one block round
    (4, 1, 64, 64, 70, 16),        # 64 query rows per KV head
]


@pytest.mark.parametrize("H,Hk,D,gs,ctx,Nq", CHAIN_CASES)
def test_attention_int4_chain(gpu, oracle, rng, H, Hk, D, gs, ctx, Nq):
    print(f"chain H={H} Hk={Hk} D={D} gs={gs} ctx={ctx} Nq={Nq}", flush=True)
    n = ctx + Nq
    c, K, V = build_cache(gpu, oracle, rng, H, Hk, D, gs, n)
    Q = rng.normal(0, 1, (1, Nq, H, D)).astype(np.float32)
    exp, _ = orc_attention(oracle, Q, K, V, H, Hk, float(np.float32(1.0 / np.sqrt(D))), 4)
    dq = DeviceArray.from_numpy(gpu, Q)
    do = DeviceArray.from_numpy(gpu, np.zeros_like(Q))
    assert gpu.cgx_attention_int4_kv_dev(dq.ptr, Nq, H, c, 0, 0, None, do.ptr) == 0, \
        last_error(gpu)
    got = do.numpy(np.float32, Q.shape)
    err = rel_err_rows(got.reshape(-1, D), exp.reshape(-1, D))
    assert err <= TOL, err
    dq.free()
    do.free()
    gpu.cg_kv_cache_int4_free(c)


def test_attention_int4_api_host_tensors(gpu, oracle, rng):
    H, Hk, D, gs, n, Nq = 8, 2, 64, 32, 150, 4
    c, K, V = build_cache(gpu, oracle, rng, H, Hk, D, gs, n, S=200)
    Q = rng.normal(0, 1, (Nq, H, D)).astype(np.float32)
    exp, _ = orc_attention(oracle, Q[None], K, V, H, Hk, float(np.float32(1.0 / np.sqrt(D))), 4)
    tq = host_tensor(gpu, Q)
    to = host_tensor(gpu, np.zeros_like(Q))
    gpu.cgx_clear_error()
    gpu.cg_attention_int4_kv(tq, c, 0, to)
    assert last_error(gpu) in ("", None), last_error(gpu)
    got = np.ctypeslib.as_array(to.contents.data, shape=(Q.size,)).reshape(-1, D)
    assert rel_err_rows(got, exp.reshape(-1, D)) <= TOL
    gpu.cg_tensor_free(tq)
    gpu.cg_tensor_free(to)
    gpu.cg_kv_cache_int4_free(c)


def random_tree(rng, n):
    parents = [-1]
    for i in range(1, n):
        parents.append(int(rng.integers(0, i)))
    return np.array(parents, np.int32)


@pytest.mark.parametrize("H,Hk,D,ctx,Nq,gs", [(32, 8, 128, 700, 16, 32), (8, 8, 64, 40, 64, 32),
                                              (4, 2, 80, 0, 9, 16), (16, 4, 128, 5000, 31, 32),
                                              (32, 8, 128, 2048, 64, 128),
                                              (8, 8, 64, 40, 64, 64),
                                              (16, 4, 128, 5000, 31, 128)])
def test_attention_int4_tree(gpu, oracle, rng, H, Hk, D, ctx, Nq, gs):
    print(f"tree H={H} Hk={Hk} D={D} ctx={ctx} Nq={Nq} gs={gs}", flush=True)
    n = ctx + Nq
    c, K, V = build_cache(gpu, oracle, rng, H, Hk, D, gs, n)
    parents = random_tree(rng, Nq)
    anc = []
    for i in range(Nq):
        s, j = {i}, parents[i]
        while j >= 0:
            s.add(int(j))
            j = parents[j]
        anc.append(s)
    mask = np.zeros((Nq, n), np.float32)
    for i in range(Nq):
        for j in range(Nq):
            if j not in anc[i]:
                mask[i, ctx + j] = -np.inf
    Q = rng.normal(0, 1, (1, Nq, H, D)).astype(np.float32)
    exp, _ = orc_attention(oracle, Q, K, V, H, Hk, float(np.float32(1.0 / np.sqrt(D))), 3,
                           mask=mask)
    dq = DeviceArray.from_numpy(gpu, Q)
    do = DeviceArray.from_numpy(gpu, np.zeros_like(Q))
    assert gpu.cgx_attention_int4_kv_dev(dq.ptr, Nq, H, c, 0, 1, parents.ctypes.data,
                                         do.ptr) == 0, last_error(gpu)
    got = do.numpy(np.float32, Q.shape).reshape(-1, D)
    assert rel_err_rows(got, exp.reshape(-1, D)) <= TOL
    # a chain-shaped tree equals the chain mask
    chain = np.arange(-1, Nq - 1, dtype=np.int32)
    do2 = DeviceArray.from_numpy(gpu, np.zeros_like(Q))
    assert gpu.cgx_attention_int4_kv_dev(dq.ptr, Nq, H, c, 0, 1, chain.ctypes.data,
                                         do2.ptr) == 0
    do3 = DeviceArray.from_numpy(gpu, np.zeros_like(Q))
    assert gpu.cgx_attention_int4_kv_dev(dq.ptr, Nq, H, c, 0, 0, None, do3.ptr) == 0
    np.testing.assert_array_equal(do2.numpy(np.float32, Q.shape), do3.numpy(np.float32, Q.shape))
    for d in (dq, do, do2, do3):
        d.free()
    gpu.cg_kv_cache_int4_free(c)


BATCH_CASES = [
    # B, Nq, tree, keys per sequence: uneven lengths, empty trailing splits
    (8, 5, False, [4101, 3000, 4096, 17, 2048, 4101, 5, 3333]),     # 4 key splits
    (8, 64, True, [1200, 64, 700, 1500, 90, 1024, 333, 1100]),      # one split
    (4, 64, True, [2112, 2112, 2112, 2112]),                        # config 5 shape
    (2, 5, False, [4101, 1000]),
]


@pytest.mark.parametrize("B,Nq,tree,nks", BATCH_CASES)
def test_attention_int4_batch(gpu, oracle, rng, B, Nq, tree, nks):
    # the decoder's batched kernel (sequence b in cache slot b, nk[b] keys)
    # against the oracle on each sequence, 7B head shape
    print(f"batch attention B={B} Nq={Nq} tree={tree} nk={nks}", flush=True)
    H, Hk, D, gs = 32, 8, 128, 128
    S = max(nks)
    c = gpu.cg_kv_cache_int4_new(B, S, Hk, D, gs)
    assert c, last_error(gpu)
    refs = []
    for b, n in enumerate(nks):
        k = rng.normal(0, 1, (n, Hk, D)).astype(np.float32)
        v = rng.normal(0, 1, (n, Hk, D)).astype(np.float32)
        assert gpu.cgx_kv_cache_int4_write(c, b, 0, k.ctypes.data, v.ctypes.data, n) == 0, \
            last_error(gpu)
        ko, vo = oracle_kv_get(oracle, *oracle_kv_fill(oracle, k, v, Hk, D, gs, n), n, Hk, D,
                               gs)
        refs.append((ko[None], vo[None]))
    anc = np.zeros(Nq, np.uint64)
    if tree:
        parents = random_tree(rng, Nq)
        for i in range(Nq):
            anc[i] = (1 << i) | (int(anc[parents[i]]) if parents[i] >= 0 else 0)
    Q = rng.normal(0, 1, (B, Nq, H, D)).astype(np.float32)
    dq = DeviceArray.from_numpy(gpu, Q)
    do = DeviceArray.from_numpy(gpu, np.zeros_like(Q))
    nk = np.array(nks, np.int32)
    assert gpu.cgx_attention_int4_kv_batch_dev(dq.ptr, B, Nq, H, c, 0, nk.ctypes.data,
                                               1 if tree else 0,
                                               anc.ctypes.data if tree else None, Nq,
                                               do.ptr) == 0, last_error(gpu)
    got = do.numpy(np.float32, Q.shape)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    for b, n in enumerate(nks):
        K, V = refs[b]
        if tree:
            mask = np.zeros((Nq, n), np.float32)
            for i in range(Nq):
                for j in range(Nq):
                    if not (int(anc[i]) >> j) & 1:
                        mask[i, n - Nq + j] = -np.inf
            exp, _ = orc_attention(oracle, Q[b:b + 1], K, V, H, Hk, scale, 3, mask=mask)
        else:
            exp, _ = orc_attention(oracle, Q[b:b + 1], K, V, H, Hk, scale, 4)
        err = rel_err_rows(got[b].reshape(-1, D), exp.reshape(-1, D))
        assert err <= TOL, (b, n, err)
    dq.free()
    do.free()
    gpu.cg_kv_cache_int4_free(c)


def test_attention_int4_errors(gpu, rng):
    c = gpu.cg_kv_cache_int4_new(1, 8, 2, 32, 32)
    Q = DeviceArray.from_numpy(gpu, np.zeros((3, 2, 32), np.float32))
    gpu.cgx_kv_cache_int4_set_len(c, 2)
    gpu.cgx_clear_error()
    assert gpu.cgx_attention_int4_kv_dev(Q.ptr, 3, 2, c, 0, 0, None, Q.ptr) != 0   # Nq > len
    gpu.cgx_kv_cache_int4_set_len(c, 3)
    bad = np.array([-1, 2, 0], np.int32)                                          # not a tree
    assert gpu.cgx_attention_int4_kv_dev(Q.ptr, 3, 2, c, 0, 1, bad.ctypes.data, Q.ptr) != 0
    assert "parents" in last_error(gpu)
    Q.free()
    gpu.cg_kv_cache_int4_free(c)


# ------------------------------------------------------- fp32 flash API

def run_flash(gpu, fn, Q, K, V, mask_type, window=0, mask=None, n_heads_k=None, extra=None):
    B, Nq, H, D = Q.shape
    O = np.zeros_like(Q)
    lse = np.zeros((B, H, Nq), np.float32)
    p = CgFlashAttnParams(Q=Q.ctypes.data, K=K.ctypes.data, V=V.ctypes.data, O=O.ctypes.data,
                          mask=mask.ctypes.data if mask is not None else None,
                          batch_size=B, seqlen_q=Nq, seqlen_k=K.shape[1], n_heads=H,
                          n_heads_k=K.shape[2] if n_heads_k is None else n_heads_k, d_head=D,
                          scale=float(np.float32(1.0 / np.sqrt(D))), mask_type=mask_type,
                          window_size=window, softmax_lse=lse.ctypes.data)
    gpu.cgx_clear_error()
    if extra is None:
        getattr(gpu, fn)(C.byref(p))
    else:
        getattr(gpu, fn)(C.byref(p), extra)
    assert last_error(gpu) in ("", None), last_error(gpu)
    return O, lse, p


FLASH_CASES = [
    # B, Nq, Nk, H, Hk, D, mask_type
    (2, 77, 77, 8, 2, 64, 0),
    (2, 77, 77, 8, 2, 64, 1),
    (1, 5, 300, 8, 8, 128, 1),       # reference rule (k > q masked) with Nq < Nk
    (1, 130, 200, 4, 1, 100, 2),
    (1, 40, 12, 2, 2, 33, 2),        # rows with no visible key; odd head_dim
    (3, 9, 2048, 16, 4, 128, 0),     # key splits
    (1, 64, 64, 4, 4, 32, 3),
]


@pytest.mark.parametrize("B,Nq,Nk,H,Hk,D,mt", FLASH_CASES)
def test_flash_forward(gpu, oracle, rng, B, Nq, Nk, H, Hk, D, mt):
    print(f"flash B={B} Nq={Nq} Nk={Nk} H={H} Hk={Hk} D={D} mask={mt}", flush=True)
    Q, K, V = attn_inputs(rng, B, Nq, Nk, H, Hk, D)
    W = 5
    mask = rng.normal(0, 2, (Nq, Nk)).astype(np.float32) if mt == 3 else None
    O, lse, p = run_flash(gpu, "cg_flash_attention_forward", Q, K, V, mt, W, mask)
    eO, else_ = orc_attention(oracle, Q, K, V, H, Hk, p.scale, mt, W, mask)
    assert rel_err_rows(O.reshape(-1, D), eO.reshape(-1, D)) <= TOL
    fin = else_ > -1e30
    np.testing.assert_allclose(lse[fin], else_[fin], rtol=1e-4, atol=1e-4)
    assert np.all(lse[~fin] == else_[~fin])


def test_flash_forward_device_pointers(gpu, oracle, rng):
    B, Nq, Nk, H, Hk, D = 1, 50, 50, 4, 2, 64
    Q, K, V = attn_inputs(rng, B, Nq, Nk, H, Hk, D)
    dQ, dK, dV = (DeviceArray.from_numpy(gpu, a) for a in (Q, K, V))
    dO = DeviceArray.from_numpy(gpu, np.zeros_like(Q))
    p = CgFlashAttnParams(Q=dQ.ptr, K=dK.ptr, V=dV.ptr, O=dO.ptr, batch_size=B, seqlen_q=Nq,
                          seqlen_k=Nk, n_heads=H, n_heads_k=Hk, d_head=D, scale=0.125,
                          mask_type=1)
    gpu.cg_flash_attention_forward(C.byref(p))
    eO, _ = orc_attention(oracle, Q, K, V, H, Hk, 0.125, 1)
    assert rel_err_rows(dO.numpy(np.float32, Q.shape).reshape(-1, D), eO.reshape(-1, D)) <= TOL
    for d in (dQ, dK, dV, dO):
        d.free()


def test_flash_cpu_named_forward_and_variants(gpu, oracle, rng):
    B, Nq, Nk, H, D = 1, 33, 33, 4, 64
    Q, K, V = attn_inputs(rng, B, Nq, Nk, H, H, D)
    # _cpu: K/V with n_heads heads whatever n_heads_k says; window ignored
    O, _, p = run_flash(gpu, "cg_flash_attention_forward_cpu", Q, K, V, 2, 3, n_heads_k=1)
    eO, _ = orc_attention(oracle, Q, K, V, H, H, p.scale, 0)
    assert rel_err_rows(O.reshape(-1, D), eO.reshape(-1, D)) <= TOL
    # MQA: n_heads_k forced to 1
    K1, V1 = K[:, :, :1].copy(), V[:, :, :1].copy()
    O, _, p = run_flash(gpu, "cg_flash_attention_mqa", Q, K1, V1, 1, n_heads_k=H)
    assert p.n_heads_k == 1
    eO, _ = orc_attention(oracle, Q, K1, V1, H, 1, p.scale, 1)
    assert rel_err_rows(O.reshape(-1, D), eO.reshape(-1, D)) <= TOL
    # GQA with 2 KV heads
    K2, V2 = K[:, :, :2].copy(), V[:, :, :2].copy()
    O, _, p = run_flash(gpu, "cg_flash_attention_gqa", Q, K2, V2, 0, n_heads_k=H, extra=2)
    eO, _ = orc_attention(oracle, Q, K2, V2, H, 2, p.scale, 0)
    assert rel_err_rows(O.reshape(-1, D), eO.reshape(-1, D)) <= TOL


def test_flash_params_new_and_helpers(gpu, oracle, rng):
    Q, K, V = attn_inputs(rng, 1, 16, 16, 2, 2, 32)
    tq, tk, tv = (host_tensor(gpu, a) for a in (Q, K, V))
    p = gpu.cg_flash_attn_params_new(tq, tk, tv, 1, 0.0)
    assert p, last_error(gpu)
    assert (p.contents.batch_size, p.contents.seqlen_q, p.contents.n_heads,
            p.contents.d_head, p.contents.n_heads_k) == (1, 16, 2, 32, 2)
    gpu.cg_flash_attention_forward(p)
    O = np.ctypeslib.as_array(C.cast(p.contents.O, C.POINTER(C.c_float)), shape=(Q.size,))
    eO, _ = orc_attention(oracle, Q, K, V, 2, 2, p.contents.scale, 1)
    assert rel_err_rows(O.reshape(-1, 32).copy(), eO.reshape(-1, 32)) <= TOL
    gpu.cg_flash_attn_params_free(p)
    gpu.cgx_clear_error()
    gpu.cg_flash_attention_backward(None)
    assert "not implemented" in last_error(gpu)
    gpu.cgx_clear_error()
    cfg = gpu.cg_flash_attn_autotune(1, 4096, 128, 0)
    assert cfg.block_m == 32 and cfg.block_n == 128 and cfg.split_k >= 1
    assert gpu.cg_flash_attn_shared_mem(32, 128, 128) == (32 * 129 + 128 * 129 + 128 * 33
                                                            + 3 * 128) * 4
    for t in (tq, tk, tv):
        gpu.cg_tensor_free(t)


# ------------------------------------------------------------- RoPE, ALiBi

@pytest.mark.parametrize("S,H,D,off,theta", [(7, 3, 64, 0, 10000.0), (5, 8, 128, 4091, 500000.0),
                                             (3, 1, 10, 17, 10000.0)])
def test_rope(gpu, oracle, rng, S, H, D, off, theta):
    q = rng.normal(0, 1, (S, H, D)).astype(np.float32)
    k = rng.normal(0, 1, (S, H, D)).astype(np.float32)
    eq, ek = q.copy(), k.copy()
    oracle.orc_apply_rope(ptr(eq), S, H, D, off, theta)
    oracle.orc_apply_rope(ptr(ek), S, H, D, off, theta)
    gq, gk = q.copy(), k.copy()
    gpu.cg_apply_rope(gq.ctypes.data, gk.ctypes.data, S, H, D, off, theta)
    assert rel_err_rows(gq.reshape(-1, D), eq.reshape(-1, D)) <= TOL
    assert rel_err_rows(gk.reshape(-1, D), ek.reshape(-1, D)) <= TOL
    # device pointer form
    dq = DeviceArray.from_numpy(gpu, q)
    gpu.cg_apply_rope(dq.ptr, None, S, H, D, off, theta)
    np.testing.assert_array_equal(dq.numpy(np.float32, q.shape), gq)
    dq.free()
    n = (S + off) * (D // 2)
    cs, sn = np.zeros(n, np.float32), np.zeros(n, np.float32)
    ecs, esn = cs.copy(), sn.copy()
    oracle.orc_rope_freqs(ptr(ecs), ptr(esn), S + off, D, theta)
    gpu.cg_rope_precompute_freqs(cs.ctypes.data, sn.ctypes.data, S + off, D, theta)
    np.testing.assert_allclose(cs, ecs, atol=1e-3)
    np.testing.assert_allclose(sn, esn, atol=1e-3)


@pytest.mark.parametrize("H", [1, 8, 12, 32])
def test_alibi(gpu, oracle, H):
    s, es = np.zeros(H, np.float32), np.zeros(H, np.float32)
    gpu.cg_alibi_slopes(s.ctypes.data, H)
    oracle.orc_alibi_slopes(ptr(es), H)
    np.testing.assert_allclose(s, es, rtol=1e-6)
    Sq, Sk = 7, 19
    b, eb = np.zeros(H * Sq * Sk, np.float32), np.zeros(H * Sq * Sk, np.float32)
    gpu.cg_alibi_bias(b.ctypes.data, Sq, Sk, H, es.ctypes.data)
    oracle.orc_alibi_bias(ptr(eb), Sq, Sk, H, ptr(es))
    np.testing.assert_array_equal(_bits(b), _bits(eb))


FUSED_CASES = [
    # H, Hk, D, ctx, Nq: RoPE + INT4 append + attention in one call
    (32, 8, 128, 4096, 5),         # 7B-shape verify step
    (12, 12, 64, 1024, 5),         # tiny-decoder verify step
    (16, 2, 64, 300, 33),          # new keys over two tiles
    (8, 2, 32, 77, 7),
    (4, 1, 64, 0, 16),             # no context: the new keys only
    (32, 8, 128, 255, 64),         # 64 new keys, fewer cached than a block round
]


@pytest.mark.parametrize("H,Hk,D,ctx,Nq", FUSED_CASES)
def test_attention_rope_append_vs_oracle(gpu, oracle, rng, H, Hk, D, ctx, Nq):
    """cgx_attention_rope_append_dev against the oracle: RoPE of the new q and
    k rows (src/attention/flash_attn.c:335-360), their INT4 append
    (src/quantize/int4.c:155-231) and attention over the whole cache under the
    chain mask.  The new V rows are bit-exact; K goes through RoPE, whose
    device powf / cos / sin are within tolerance of glibc's, so its scales
    agree to 1e-3 and its values to one quantisation step.  (The decoder test
    test_fused_attention_step_matches_separate_launches pins the fused
    append bit for bit against the separate RoPE / append launches.)"""
    print(f"fused rope+append+attention H={H} Hk={Hk} D={D} ctx={ctx} Nq={Nq}", flush=True)
    theta, S, gs = 10000.0, ctx + Nq, D
    ldq = (H + 2 * Hk) * D
    kc_ = rng.normal(0, 1, (ctx, Hk, D)).astype(np.float32)
    vc_ = rng.normal(0, 1, (ctx, Hk, D)).astype(np.float32)
    qkv = rng.normal(0, 1, (Nq, ldq)).astype(np.float32)
    c = gpu.cg_kv_cache_int4_new(1, S, Hk, D, gs)
    assert c, last_error(gpu)
    if ctx:
        assert gpu.cgx_kv_cache_int4_write(c, 0, 0, kc_.ctypes.data, vc_.ctypes.data, ctx) == 0
    # oracle: rotate, append everything, attend
    q = np.ascontiguousarray(qkv[:, :H * D]).reshape(Nq, H, D)
    k = np.ascontiguousarray(qkv[:, H * D:(H + Hk) * D]).reshape(Nq, Hk, D)
    v = np.ascontiguousarray(qkv[:, (H + Hk) * D:]).reshape(Nq, Hk, D)
    oracle.orc_apply_rope(ptr(q), Nq, H, D, ctx, theta)
    oracle.orc_apply_rope(ptr(k), Nq, Hk, D, ctx, theta)
    arrs = oracle_kv_fill(oracle, np.concatenate([kc_, k]), np.concatenate([vc_, v]), Hk, D, gs,
                          S)
    K, V = oracle_kv_get(oracle, *arrs, S, Hk, D, gs)
    exp, _ = orc_attention(oracle, q[None], K[None], V[None], H, Hk,
                           float(np.float32(1.0 / np.sqrt(D))), 4)
    dqkv = DeviceArray.from_numpy(gpu, qkv)
    dcs = DeviceArray(gpu, Nq * D * 4)
    do = DeviceArray(gpu, Nq * H * D * 4)
    assert gpu.cgx_rope_table_dev(Nq, D, ctx, theta, dcs.ptr) == 0, last_error(gpu)
    assert gpu.cgx_attention_rope_append_dev(dqkv.ptr, ldq, dcs.ptr, Nq, H, c, 0, ctx,
                                             do.ptr) == 0, last_error(gpu)
    got = do.numpy(np.float32, (Nq, H, D))
    assert rel_err_rows(got.reshape(-1, D), exp.reshape(-1, D)) <= TOL
    kb, vb, ks, vs = cache_arrays(gpu, c, 0)
    okc, ovc, oks, ovs = arrs
    nb, ng = ctx * Hk * D // 2, ctx * Hk
    np.testing.assert_array_equal(vb[nb:S * Hk * D // 2], ovc[nb:S * Hk * D // 2])
    np.testing.assert_array_equal(_bits(vs[ng:S * Hk]), _bits(ovs[ng:S * Hk]))
    # the rotary angle is position * frequency: an ulp of a frequency (device
    # powf against glibc's) grows with the position, ~2e-4 of |k| near 4096
    assert np.allclose(ks[ng:S * Hk], oks[ng:S * Hk], rtol=1e-3, atol=0)
    gk = np.zeros((S, Hk, D), np.float32)
    gv = np.zeros_like(gk)
    oracle.orc_kv_get(ptr(kb), ptr(vb), ptr(ks), ptr(vs), S, Hk, D, gs, ptr(gk), ptr(gv))
    step = np.repeat(oks[:S * Hk].reshape(S, Hk, 1), D, axis=2)
    assert np.all(np.abs(gk[ctx:] - K[ctx:]) <= step[ctx:] * 1.01)
    for a in (dqkv, dcs, do):
        a.free()
    gpu.cg_kv_cache_int4_free(c)
