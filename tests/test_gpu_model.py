"""GPU parity of the synthetic decoder stack and the speculative loop.

* seeded weights: the GPU fill and the oracle's restatement agree bit for
  bit, and so do the exported INT4 weights;
* forward: logits within 1e-3 of max|logits| per row of the oracle stack
  (tests/oracle_model.py) across prefill, decode, verify-sized steps and a
  KV rollback;
* speculative loop: a draft identical to the target (same seed, separate
  caches) must accept every drafted token (p == q exactly); with a
  different draft, the loop keeps both caches at the accepted prefix.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error
from gpu_util import rel_err_rows
from oracle_lib import ptr
from oracle_model import W_GU, W_LM, W_QKV, Cfg, OracleModel, fill

pytestmark = pytest.mark.gpu
TOL = 1e-3

TINY = Cfg(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
           vocab=1024, group_size=128, kv_group_size=64, max_seq=64, max_tokens=8,
           init_std=0.05)


def new_model(gpu, cfg, seed, share=None):
    cc = cfg.ctype()
    m = gpu.cgx_model_new(C.byref(cc), seed, share)
    assert m, last_error(gpu)
    return m


def logits_np(gpu, m, rows, V):
    out = np.empty((rows, V), np.float32)
    assert gpu.cgx_memcpy_d2h(out.ctypes.data, gpu.cgx_model_logits(m), out.nbytes) == 0
    return out


@pytest.mark.parametrize("seed,sid,n", [(1, 1, 100000), (2**40 + 7, 35, 4097), (0, 2, 33)])
def test_fill_normal_bitexact(gpu, oracle, seed, sid, n):
    d = DeviceArray(gpu, n * 4)
    assert gpu.cgx_fill_normal_dev(d.ptr, n, seed, sid, 0.02) == 0, last_error(gpu)
    got = d.numpy(np.float32, (n,))
    exp = fill(oracle, n, seed, sid, 0.02)
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))
    d.free()


def test_model_export_matches_oracle(gpu, oracle):
    m = new_model(gpu, TINY, 11)
    om = OracleModel(oracle, TINY, 11)
    for layer, which, lin in ((0, W_QKV, om.layers[0][0]), (1, W_GU, om.layers[1][2]),
                              (0, W_LM, om.lm)):
        data, scales, K, N = lin
        gd = np.zeros_like(data)
        gs = np.zeros_like(scales)
        assert gpu.cgx_model_export(m, layer, which, gd.ctypes.data, gs.ctypes.data) == 0, \
            last_error(gpu)
        np.testing.assert_array_equal(gd, data)
        np.testing.assert_array_equal(gs.view(np.uint32), scales.view(np.uint32))
    gpu.cgx_model_free(m)


def test_model_forward_vs_oracle(gpu, oracle, rng):
    m = new_model(gpu, TINY, 5)
    om = OracleModel(oracle, TINY, 5)
    V = TINY.vocab
    steps = [5, 1, 3, 8, 2]
    for M in steps:
        toks = rng.integers(0, V, M).astype(np.int32)
        assert gpu.cgx_model_forward(m, toks.ctypes.data, M, M, None) == 0, last_error(gpu)
        got = logits_np(gpu, m, M, V)
        exp = om.forward(toks)
        err = rel_err_rows(got, exp)
        assert err <= TOL, (M, err)
        assert gpu.cgx_model_len(m) == om.len
    # rollback: drop the last 4 positions and continue
    assert gpu.cgx_model_truncate(m, om.len - 4) == 0
    om.truncate(om.len - 4)
    toks = rng.integers(0, V, 3).astype(np.int32)
    assert gpu.cgx_model_forward(m, toks.ctypes.data, 3, 1, None) == 0
    got = logits_np(gpu, m, 1, V)
    assert rel_err_rows(got, om.forward(toks, n_logits=1)) <= TOL
    gpu.cgx_model_free(m)


def test_model_forward_k_split_vs_oracle(gpu, oracle, rng):
    # K above 4096 splits the GEMV over blocks (at most two 256-row rounds per
    # wave): d_model 4608 splits wqkv, gate|up and lm_head (RMSNorm prologue,
    # SwiGLU) and wo (accumulate) in two, d_ff 8448 the down projection in three
    cfg = Cfg(n_layers=1, d_model=4608, n_heads=36, n_kv_heads=4, head_dim=128, d_ff=8448,
              vocab=2048, group_size=128, kv_group_size=128, max_seq=64, max_tokens=8,
              init_std=0.02)
    m = new_model(gpu, cfg, 9)
    om = OracleModel(oracle, cfg, 9)
    for M in (5, 1, 8):
        toks = rng.integers(0, cfg.vocab, M).astype(np.int32)
        assert gpu.cgx_model_forward(m, toks.ctypes.data, M, M, None) == 0, last_error(gpu)
        err = rel_err_rows(logits_np(gpu, m, M, cfg.vocab), om.forward(toks))
        assert err <= TOL, (M, err)
    gpu.cgx_model_free(m)


def test_model_forward_stream_gemv_vs_oracle(gpu, oracle, rng):
    # d_model 4096 with the streaming GEMV taking every product it supports
    # (cgx_gemv_stream_min_units(1)): wqkv and lm_head with the RMSNorm
    # prologue, wo accumulating into the residual
    cfg = Cfg(n_layers=1, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128, d_ff=1024,
              vocab=4096, group_size=128, kv_group_size=128, max_seq=64, max_tokens=8,
              init_std=0.02)
    m = new_model(gpu, cfg, 13)
    om = OracleModel(oracle, cfg, 13)
    old = gpu.cgx_gemv_stream_min_units(1)
    try:
        for M in (5, 1, 3):
            toks = rng.integers(0, cfg.vocab, M).astype(np.int32)
            assert gpu.cgx_model_forward(m, toks.ctypes.data, M, M, None) == 0, last_error(gpu)
            err = rel_err_rows(logits_np(gpu, m, M, cfg.vocab), om.forward(toks))
            assert err <= TOL, (M, err)
    finally:
        gpu.cgx_gemv_stream_min_units(old)
    gpu.cgx_model_free(m)


@pytest.mark.parametrize("cfg", [TINY, Cfg(n_layers=1, d_model=512, n_heads=8, n_kv_heads=2,
                                            head_dim=128, d_ff=768, vocab=2048, group_size=128,
                                            kv_group_size=128, max_seq=300, max_tokens=5,
                                            init_std=0.05)])
@pytest.mark.parametrize("B,reduce4", [(3, 512), (8, 512), (8, 0)])
def test_model_forward_batch_vs_oracle(gpu, oracle, rng, cfg, B, reduce4):
    # B sequences with their own caches in one forward: each matches its own
    # oracle stack, also after rollbacks to different lengths per sequence
    # (B = 8: 40 rows per forward, the GEMM path of every linear layer; with
    # reduce4 = 0 its K splits are summed four outputs a thread, with the
    # accumulate and SwiGLU epilogues and the row statistics by DPP)
    from dataclasses import replace
    old = gpu.cgx_gemm_reduce4_min_blocks(reduce4)
    try:
        _forward_batch_case(gpu, oracle, rng, cfg, B, replace)
    finally:
        gpu.cgx_gemm_reduce4_min_blocks(old)


def _forward_batch_case(gpu, oracle, rng, cfg, B, replace):
    m = new_model(gpu, replace(cfg, max_batch=B), 5)
    assert gpu.cgx_model_batch(m) == B
    oms = [OracleModel(oracle, cfg, 5) for _ in range(B)]
    V = cfg.vocab
    for step, M in enumerate([5, 1, 3, 2, 5]):
        M = min(M, cfg.max_tokens)
        toks = rng.integers(0, V, (B, M)).astype(np.int32)
        assert gpu.cgx_model_forward_batch(m, toks.ctypes.data, M, M, None) == 0, \
            last_error(gpu)
        got = logits_np(gpu, m, B * M, V).reshape(B, M, V)
        for b in range(B):
            err = rel_err_rows(got[b], oms[b].forward(toks[b]))
            assert err <= TOL, (step, b, err)
            assert gpu.cgx_model_len_seq(m, b) == oms[b].len
        if step == 1:
            for b in range(B):
                n = oms[b].len - b % 3
                assert gpu.cgx_model_truncate_seq(m, b, n) == 0
                oms[b].truncate(n)
    # the last token's logits of each sequence
    toks = rng.integers(0, V, (B, 2)).astype(np.int32)
    assert gpu.cgx_model_forward_batch(m, toks.ctypes.data, 2, 1, None) == 0
    got = logits_np(gpu, m, B, V)
    for b in range(B):
        assert rel_err_rows(got[b:b + 1], oms[b].forward(toks[b], n_logits=1)) <= TOL
    gpu.cgx_model_free(m)


@pytest.mark.parametrize("M", [2, 5, 8])
def test_gemm_swiglu_in_kernel_matches_reduction(gpu, rng, M):
    # d_model 256 leaves every GEMM one K split: the gate|up product applies
    # SwiGLU in its own epilogue (default) or stores partial sums for the
    # reduction pass (hook off); the logits of 8 sequences x M rows (16, 40
    # and 64 rows: blocks of 16, 48 and 32 rows) must be the same bits either
    # way (the consumer's row factor depends only on the row maxima, which do
    # not depend on the order of reduction)
    from dataclasses import replace
    cfg = replace(TINY, max_batch=8)
    toks = rng.integers(0, cfg.vocab, (8, M)).astype(np.int32)
    outs = []
    old = gpu.cgx_gemm_swiglu_here(-1)
    try:
        for on in (1, 0):
            gpu.cgx_gemm_swiglu_here(on)
            m = new_model(gpu, cfg, 17)
            assert gpu.cgx_model_forward_batch(m, toks.ctypes.data, M, M, None) == 0, \
                last_error(gpu)
            outs.append(logits_np(gpu, m, 8 * M, cfg.vocab))
            gpu.cgx_model_free(m)
    finally:
        gpu.cgx_gemm_swiglu_here(old)
    assert np.isfinite(outs[0]).all()
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("fused", [1, 0])
def test_attention_row_statistics_match_gemm_pass(gpu, rng, fused):
    # head_dim 128 and 8 sequences x 5 rows (the GEMM path): the attention
    # (with RoPE and the cache append inside, or after a launch of their own)
    # writes the O projection's row statistics, or the GEMM computes them
    # from the rows; the row factors come from the row maxima either way, so
    # the logits must be the same bits
    cfg = Cfg(n_layers=2, d_model=512, n_heads=8, n_kv_heads=2, head_dim=128, d_ff=768,
              vocab=2048, group_size=128, kv_group_size=128, max_seq=300, max_tokens=5,
              init_std=0.05, max_batch=8)
    toks = rng.integers(0, cfg.vocab, (2, 8, 5)).astype(np.int32)
    outs = []
    old = gpu.cgx_decoder_attention_stats(-1)
    old_f = gpu.cgx_decoder_fused_attention(fused)
    try:
        for on in (1, 0):
            gpu.cgx_decoder_attention_stats(on)
            m = new_model(gpu, cfg, 23)
            got = []
            for step in range(2):        # the second step attends to the first's keys
                assert gpu.cgx_model_forward_batch(m, toks[step].ctypes.data, 5, 5, None) == 0, \
                    last_error(gpu)
                got.append(logits_np(gpu, m, 40, cfg.vocab))
            outs.append(np.stack(got))
            gpu.cgx_model_free(m)
    finally:
        gpu.cgx_decoder_attention_stats(old)
        gpu.cgx_decoder_fused_attention(old_f)
    assert np.isfinite(outs[0]).all()
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_model_forward_head_dim_128_gqa(gpu, oracle, rng):
    cfg = Cfg(n_layers=1, d_model=512, n_heads=8, n_kv_heads=2, head_dim=128, d_ff=768,
              vocab=2048, group_size=128, kv_group_size=128, max_seq=300, max_tokens=5,
              init_std=0.05)
    m = new_model(gpu, cfg, 9)
    om = OracleModel(oracle, cfg, 9)
    # a longer context through several forwards, then verify-sized steps
    for M in [5] * 40 + [1, 5, 5]:
        toks = rng.integers(0, cfg.vocab, M).astype(np.int32)
        assert gpu.cgx_model_forward(m, toks.ctypes.data, M, M, None) == 0, last_error(gpu)
        exp = om.forward(toks)
    got = logits_np(gpu, m, 5, cfg.vocab)
    assert rel_err_rows(got, exp) <= TOL
    gpu.cgx_model_free(m)


def test_model_rejects_bad_config(gpu):
    bad = Cfg(n_layers=1, d_model=200, n_heads=4, n_kv_heads=2, head_dim=50, d_ff=512,
              vocab=1000)
    cc = bad.ctype()
    gpu.cgx_clear_error()
    assert not gpu.cgx_model_new(C.byref(cc), 1, None)
    assert last_error(gpu)


def run_spec(gpu, draft, target, gamma, T, k, p, prompt, steps, rng):
    s = gpu.cgx_spec_new(draft, target, gamma, T, k, p)
    assert s, last_error(gpu)
    pr = np.asarray(prompt, np.int32)
    assert gpu.cgx_spec_prefill(s, pr.ctypes.data, len(pr)) == 0, last_error(gpu)
    ns, emitted = [], []
    for _ in range(steps):
        ud = rng.uniform(0, 1, gamma).astype(np.float32)
        uv = rng.uniform(0, 1, gamma + 1).astype(np.float32)
        out = np.zeros(gamma + 1, np.int32)
        L = gpu.cgx_model_len(target)
        n = gpu.cgx_spec_step(s, ud.ctypes.data, uv.ctypes.data, out.ctypes.data)
        assert 0 <= n <= gamma, last_error(gpu)
        assert gpu.cgx_model_len(target) == L + n + 1
        assert gpu.cgx_model_len(draft) == L + min(n, gamma - 1) + 1
        assert np.all((out[:n + 1] >= 0) & (out[:n + 1] < 1024 * 64))
        ns.append(n)
        emitted.extend(out[:n + 1].tolist())
    st = [C.c_longlong() for _ in range(3)]
    gpu.cgx_spec_stats(s, *[C.byref(x) for x in st])
    assert st[0].value == steps and st[1].value == steps * gamma and st[2].value == sum(ns)
    gpu.cgx_spec_free(s)
    return ns, emitted


@pytest.mark.parametrize("T,k,p", [(1.0, 0, 1.0), (0.8, 0, 0.9), (0.7, 50, 1.0)])
def test_spec_identical_draft_accepts_everything(gpu, rng, T, k, p):
    cfg = Cfg(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
              vocab=1024, max_seq=128, max_tokens=8, init_std=0.05)
    target = new_model(gpu, cfg, 21)
    draft = new_model(gpu, cfg, 21)
    ns, emitted = run_spec(gpu, draft, target, 4, T, k, p, [1, 2, 3, 4, 5], 10, rng)
    assert ns == [4] * 10
    assert len(emitted) == 50
    gpu.cgx_model_free(draft)
    gpu.cgx_model_free(target)


def test_spec_with_draft_head_rolls_back(gpu, rng):
    cfg = Cfg(n_layers=3, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
              vocab=1024, max_seq=200, max_tokens=8, init_std=0.05)
    dcfg = Cfg(**{**cfg.__dict__, "n_layers": 1})
    target = new_model(gpu, cfg, 31)
    draft = new_model(gpu, dcfg, 32, target)        # shares embedding and lm_head
    ns, _ = run_spec(gpu, draft, target, 4, 1.0, 0, 1.0, list(range(1, 12)), 25, rng)
    assert 0 < sum(ns) < 4 * 25          # some accepted, some rejected
    gpu.cgx_model_free(draft)
    gpu.cgx_model_free(target)


def test_spec_from_filled_context(gpu, rng):
    cfg = Cfg(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
              vocab=1024, max_seq=600, max_tokens=8, init_std=0.05)
    target = new_model(gpu, cfg, 41)
    draft = new_model(gpu, cfg, 41)
    for mdl in (target, draft):
        assert gpu.cgx_model_fill_context(mdl, 512, 7) == 0, last_error(gpu)
        assert gpu.cgx_model_len(mdl) == 512
    s = gpu.cgx_spec_new(draft, target, 4, 1.0, 0, 1.0)
    assert gpu.cgx_spec_set_last(s, 3) == 0
    out = np.zeros(5, np.int32)
    u = rng.uniform(0, 1, 5).astype(np.float32)
    assert gpu.cgx_spec_step(s, u.ctypes.data, u.ctypes.data, out.ctypes.data) == 4
    gpu.cgx_spec_free(s)
    gpu.cgx_model_free(draft)
    gpu.cgx_model_free(target)


def run_spec_batch(gpu, draft, target, gamma, T, B, prompt_len, steps, rng):
    """Prefill B prompts into both models, then batched loop steps; checks the
    per-sequence bookkeeping and returns the accepted counts."""
    V = 1024
    prompts = rng.integers(0, V, (B, prompt_len)).astype(np.int32)
    for mdl in (target, draft):
        assert gpu.cgx_model_forward_batch(mdl, prompts.ctypes.data, prompt_len, 0,
                                           None) == 0, last_error(gpu)
    s = gpu.cgx_spec_batch_new(draft, target, gamma, T)
    assert s, last_error(gpu)
    prev = np.ascontiguousarray(prompts[:, -1])
    last = rng.integers(0, V, B).astype(np.int32)
    assert gpu.cgx_spec_batch_set_last(s, prev.ctypes.data, last.ctypes.data) == 0, \
        last_error(gpu)
    out = np.zeros((B, gamma + 1), np.int32)
    n = np.zeros(B, np.int32)
    lens = np.full(B, prompt_len)
    all_n = []
    for _ in range(steps):
        ud = rng.uniform(0, 1, (B, gamma)).astype(np.float32)
        uv = rng.uniform(0, 1, (B, gamma + 1)).astype(np.float32)
        tot = gpu.cgx_spec_batch_step(s, ud.ctypes.data, uv.ctypes.data, out.ctypes.data,
                                      n.ctypes.data)
        assert tot == n.sum() >= 0, last_error(gpu)
        for b in range(B):
            assert 0 <= n[b] <= gamma
            assert ((out[b, :n[b] + 1] >= 0) & (out[b, :n[b] + 1] < V)).all()
            assert (out[b, n[b] + 1:] == -1).all()
            lens[b] += n[b] + 1
            assert gpu.cgx_model_len_seq(target, b) == lens[b]
        all_n.append(n.copy())
    gpu.cgx_spec_batch_free(s)
    return np.array(all_n)


def test_spec_batch_identical_draft(gpu, rng):
    # same weights and the same prefill: the draft's distributions equal the
    # target's up to the rounding of a recomputed position, so (nearly) every
    # drafted token is accepted
    cfg = Cfg(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
              vocab=1024, max_seq=128, max_tokens=8, init_std=0.05, max_batch=4)
    target = new_model(gpu, cfg, 21)
    draft = new_model(gpu, cfg, 21)
    ns = run_spec_batch(gpu, draft, target, 4, 1.0, 4, 6, 8, rng)
    assert ns.mean() >= 0.9 * 4, ns
    gpu.cgx_model_free(draft)
    gpu.cgx_model_free(target)


def test_spec_batch_with_draft_head(gpu, rng):
    cfg = Cfg(n_layers=3, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
              vocab=1024, max_seq=200, max_tokens=8, init_std=0.05, max_batch=3)
    dcfg = Cfg(**{**cfg.__dict__, "n_layers": 1})
    target = new_model(gpu, cfg, 31)
    draft = new_model(gpu, dcfg, 32, target)
    ns = run_spec_batch(gpu, draft, target, 4, 1.0, 3, 5, 20, rng)
    assert 0 < ns.sum() < 4 * ns.size
    gpu.cgx_model_free(draft)
    gpu.cgx_model_free(target)


def test_spec_batch_rejects_mismatched_models(gpu):
    cfg = Cfg(n_layers=1, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
              vocab=1024, max_seq=64, max_tokens=8, init_std=0.05, max_batch=2)
    a = new_model(gpu, cfg, 1)
    b = new_model(gpu, Cfg(**{**cfg.__dict__, "max_batch": 3}), 2)
    assert not gpu.cgx_spec_batch_new(a, b, 4, 1.0)
    assert "batch" in last_error(gpu)
    gpu.cgx_model_free(a)
    gpu.cgx_model_free(b)


def _cache_arrays(gpu, m, length):
    """Host copies of the written part (positions < length) of each layer
    slot of a model's KV cache: {(kind, slot): array}, kind k / v (nibble
    bytes) or ks / vs (scales)."""
    cc = gpu.cgx_model_kv(m).contents
    row_b = cc.n_heads * cc.head_dim // 2
    row_g = cc.n_heads * cc.head_dim // cc.group_size
    out = {}
    for kind, arr, per, dt in (("k", cc.k_cache, row_b, np.uint8), ("v", cc.v_cache, row_b, np.uint8),
                               ("ks", cc.k_scales, row_g, np.float32),
                               ("vs", cc.v_scales, row_g, np.float32)):
        esz = np.dtype(dt).itemsize
        for slot in range(cc.num_layers):
            h = np.empty(length * per, dt)
            base = C.cast(arr, C.c_void_p).value + slot * cc.max_seq_len * per * esz
            assert gpu.cgx_memcpy_d2h(h.ctypes.data, base, h.nbytes) == 0, last_error(gpu)
            out[(kind, slot)] = h
    return out


def _dequant(c, kind, slot, length, Hk, D):
    nib = c[(kind, slot)].reshape(length, Hk, D // 2)
    lo = (nib & 0xF).astype(np.int8)
    hi = (nib >> 4).astype(np.int8)
    vals = np.stack([np.where(lo > 7, lo - 16, lo), np.where(hi > 7, hi - 16, hi)], -1)
    vals = vals.reshape(length, Hk, D).astype(np.float32)
    return vals * c[(kind + "s", slot)].reshape(length, Hk, 1)


@pytest.mark.parametrize("batch", [0, 3])
def test_fused_attention_step_matches_separate_launches(gpu, rng, batch):
    """RoPE and the INT4 cache append inside the attention launch (the
    default) and as launches of their own (cgx_decoder_fused_attention(0)).
    Layer 0's cache is a function of the tokens and weights alone: the same
    bytes.  Later layers see attention outputs that differ at the last bits
    (the fused launch attends over the new keys in a key split of their own),
    so their caches agree within a quantisation step (a value next to a
    rounding boundary may flip a nibble) and the logits within 1e-4 of
    max|logits| per row."""
    cfg = Cfg(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
              vocab=1024, max_seq=96, max_tokens=8, init_std=0.05, max_batch=batch)
    B, V = max(batch, 1), cfg.vocab
    steps = [rng.integers(0, V, (B, M)).astype(np.int32) for M in (7, 5, 1, 5, 8)]
    models = [new_model(gpu, cfg, 77), new_model(gpu, cfg, 77)]
    outs = [[], []]
    old = gpu.cgx_decoder_fused_attention(-1)
    try:
        for k, m in enumerate(models):
            gpu.cgx_decoder_fused_attention(1 - k)
            for t in steps:
                M = t.shape[1]
                fwd = gpu.cgx_model_forward_batch if batch else gpu.cgx_model_forward
                assert fwd(m, t.ctypes.data, M, M, None) == 0, last_error(gpu)
                outs[k].append(logits_np(gpu, m, B * M, V))
    finally:
        gpu.cgx_decoder_fused_attention(old)
    for a, b in zip(*outs):
        assert rel_err_rows(a, b) < 1e-4
    n = sum(t.shape[1] for t in steps)
    ca, cb = (_cache_arrays(gpu, m, n) for m in models)
    for (kind, slot), a in ca.items():
        if slot < B:                                  # layer 0 of every sequence
            np.testing.assert_array_equal(a.view(np.uint8), cb[(kind, slot)].view(np.uint8),
                                          err_msg=f"{kind} slot {slot}")
        elif kind in ("k", "v"):
            da = _dequant(ca, kind, slot, n, cfg.n_kv_heads, cfg.head_dim)
            db = _dequant(cb, kind, slot, n, cfg.n_kv_heads, cfg.head_dim)
            step = ca[(kind + "s", slot)].reshape(n, cfg.n_kv_heads, 1)
            assert np.all(np.abs(da - db) <= 1.01 * step), f"{kind} slot {slot}"
    for m in models:
        gpu.cgx_model_free(m)
