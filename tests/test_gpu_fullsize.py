"""GPU: the verify loops at the full shapes of configs 3, 4 and 5 (config 3:
12 layers, d = 768, 12 heads of 64, FFN 3072, V = 32000, context 1024; configs
4 and 5: 32 layers,
d = 4096, 32 heads over 8 KV heads, FFN 11008, INT4 weights and KV cache),
checked through properties that hold at any size, so no CPU oracle has to
run the 7B-shape stack:

* a draft with the target's weights and context (separate caches) gives
  p == q exactly, so every drafted token is accepted, at batch 1 (config 4,
  context 4096); at batch 8 (each sequence's 128 MiB cache in one
  allocation) the batched draft recomputes the last cached position with
  another row count, so nearly every one (>= 90 %) is;
* with a different draft, each sequence's cache keeps exactly its accepted
  tokens plus the emitted one after every step (rollback);
* the tree loop of config 5 (V = 128256, batch 4, 64-node trees, context
  2048, top-k 50) emits 1 + n tokens per sequence, n <= depth, keeps the
  caches at the same lengths and writes -1 past the emitted tokens;
* config 3's tiny stack: 5 rows at once against one at a time, and a draft
  with the target's weights accepting every token under T = 0.8 / top-p 0.9
  (p == q exactly through the filtered distributions).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cogito_amd.capi import CgxModelConfig, last_error

pytestmark = pytest.mark.gpu

SHAPE = dict(n_layers=32, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128, d_ff=11008,
             group_size=128, kv_group_size=128, rope_theta=10000.0, norm_eps=1e-5,
             init_std=0.02)


def model(gpu, vocab, max_seq, max_tokens, seed, batch=0, layers=32, share=None):
    cfg = CgxModelConfig(**{**SHAPE, "n_layers": layers}, vocab=vocab, max_seq=max_seq,
                         max_tokens=max_tokens, max_batch=batch)
    m = gpu.cgx_model_new(C.byref(cfg), seed, share)
    assert m, last_error(gpu)
    return m


def test_c4_stack_logits_finite_and_row_count_independent(gpu):
    """The 32-layer stack after a 4096-token context: the logits of 5 tokens
    forwarded at once are finite, spread out, and equal (to the fp32
    accumulation tolerance) to those of the same tokens forwarded one at a
    time -- the M = 5 kernels (GEMV rows, 5-row attention) against the M = 1
    ones at the full shape.  (Acceptance-only checks pass on NaN logits: the
    acceptance ratio of NaN probabilities is 1.)"""
    print("C4 stack logits, 5 rows at once vs one at a time", flush=True)
    V, ctx = 32000, 4096
    m = model(gpu, V, ctx + 16, 5, 7)
    assert gpu.cgx_model_fill_context(m, ctx, 99) == 0, last_error(gpu)
    toks = np.array([11, 222, 3333, 4444, 31999], np.int32)
    assert gpu.cgx_model_forward(m, toks.ctypes.data, 5, 5, None) == 0, last_error(gpu)
    all5 = np.zeros((5, V), np.float32)
    assert gpu.cgx_memcpy_d2h(all5.ctypes.data, gpu.cgx_model_logits(m), all5.nbytes) == 0
    assert np.isfinite(all5).all()
    assert all5.std(axis=1).min() > 1e-3, all5.std(axis=1)
    assert gpu.cgx_model_truncate(m, ctx) == 0
    one = np.zeros((5, V), np.float32)
    for i in range(5):
        assert gpu.cgx_model_forward(m, toks[i:i + 1].ctypes.data, 1, 1, None) == 0, \
            last_error(gpu)
        assert gpu.cgx_memcpy_d2h(one[i].ctypes.data, gpu.cgx_model_logits(m), V * 4) == 0
    scale = float(np.abs(all5).max())
    err = float(np.abs(one - all5).max())
    assert err <= 2e-3 * scale, (err, scale)
    gpu.cgx_model_free(m)


def test_c4_batch1_identical_draft_accepts_everything(gpu):
    print("C4 batch 1, identical draft", flush=True)
    g, ctx, steps = 4, 4096, 3
    ms = ctx + (g + 1) * (steps + 2)
    mt = model(gpu, 32000, ms, g + 1, 7)
    md = model(gpu, 32000, ms, 2, 7)
    assert gpu.cgx_model_fill_context(mt, ctx, 99) == 0 and \
        gpu.cgx_model_fill_context(md, ctx, 99) == 0, last_error(gpu)
    sp = gpu.cgx_spec_new(md, mt, g, 1.0, 0, 1.0)
    assert sp and gpu.cgx_spec_set_last(sp, 5) == 0, last_error(gpu)
    rng = np.random.default_rng(1)
    out = np.zeros(g + 1, np.int32)
    for s in range(steps):
        ud = rng.random(g, dtype=np.float32)
        uv = rng.random(g + 1, dtype=np.float32)
        n = gpu.cgx_spec_step(sp, ud.ctypes.data, uv.ctypes.data, out.ctypes.data)
        assert n == g, (s, n, last_error(gpu))
        assert ((out >= 0) & (out < 32000)).all()
        assert gpu.cgx_model_len(mt) == ctx + (s + 1) * (g + 1)
    gpu.cgx_spec_free(sp)
    gpu.cgx_model_free(md)
    gpu.cgx_model_free(mt)


def test_c4_batch8_identical_draft_and_rollback(gpu):
    print("C4 batch 8, identical then 1-layer draft", flush=True)
    g, ctx, B, steps = 4, 4096, 8, 3
    ms = ctx + (g + 1) * (2 * steps + 2)
    mt = model(gpu, 32000, ms, g + 1, 7, batch=B)
    md = model(gpu, 32000, ms, 2, 7, batch=B)
    rng = np.random.default_rng(2)
    prev = rng.integers(0, 32000, B).astype(np.int32)
    last = rng.integers(0, 32000, B).astype(np.int32)
    # the batched loop recomputes the last cached position from `prev` in the
    # draft: that position must come from a forward of prev, not the fill
    for m in (mt, md):
        assert gpu.cgx_model_fill_context(m, ctx - 1, 99) == 0, last_error(gpu)
        assert gpu.cgx_model_forward_batch(m, prev.ctypes.data, 1, 0, None) == 0, \
            last_error(gpu)
    out = np.zeros((B, g + 1), np.int32)
    n = np.zeros(B, np.int32)
    sp = gpu.cgx_spec_batch_new(md, mt, g, 1.0)
    assert sp and gpu.cgx_spec_batch_set_last(sp, prev.ctypes.data, last.ctypes.data) == 0, \
        last_error(gpu)
    lens = np.full(B, ctx)
    accepted = 0
    for s in range(steps):
        ud = rng.random((B, g), dtype=np.float32)
        uv = rng.random((B, g + 1), dtype=np.float32)
        tot = gpu.cgx_spec_batch_step(sp, ud.ctypes.data, uv.ctypes.data, out.ctypes.data,
                                      n.ctypes.data)
        assert tot == n.sum() >= 0, last_error(gpu)
        accepted += tot
        lens += n + 1
        assert [gpu.cgx_model_len_seq(mt, b) for b in range(B)] == lens.tolist()
    # the recomputed position differs from the target's by rounding only, so
    # (nearly) every drafted token is accepted
    assert accepted >= 0.9 * steps * B * g, accepted
    gpu.cgx_spec_batch_free(sp)
    gpu.cgx_model_free(md)
    # a 1-layer draft over the target's head: rejections, per-sequence rollback
    md1 = model(gpu, 32000, ms, 2, 8, batch=B, layers=1, share=mt)
    assert gpu.cgx_model_fill_context(md1, ctx, 5) == 0
    # the draft's context is shorter than the target's: bring both to ctx
    for b in range(B):
        assert gpu.cgx_model_truncate_seq(mt, b, ctx) == 0
    lens[:] = ctx
    sp = gpu.cgx_spec_batch_new(md1, mt, g, 1.0)
    assert sp and gpu.cgx_spec_batch_set_last(sp, prev.ctypes.data, last.ctypes.data) == 0, \
        last_error(gpu)
    seen = set()
    for s in range(steps):
        ud = rng.random((B, g), dtype=np.float32)
        uv = rng.random((B, g + 1), dtype=np.float32)
        tot = gpu.cgx_spec_batch_step(sp, ud.ctypes.data, uv.ctypes.data, out.ctypes.data,
                                      n.ctypes.data)
        assert tot == n.sum() >= 0, last_error(gpu)
        seen.update(n.tolist())
        for b in range(B):
            assert (out[b, :n[b] + 1] >= 0).all() and (out[b, n[b] + 1:] == -1).all()
        lens += n + 1
        assert [gpu.cgx_model_len_seq(mt, b) for b in range(B)] == lens.tolist()
    gpu.cgx_spec_batch_free(sp)
    gpu.cgx_model_free(md1)
    gpu.cgx_model_free(mt)


def test_c5_tree_loop_invariants(gpu):
    print("C5 tree loop, batch 4", flush=True)
    nodes, depth, ctx, B, V, steps = 64, 6, 2048, 4, 128256, 3
    ms = ctx + (depth + 2) * (steps + 2) + nodes + 8
    mt = model(gpu, V, ms, nodes, 11, batch=B)
    md = model(gpu, V, ms, nodes, 12, batch=B, layers=1, share=mt)
    assert gpu.cgx_model_fill_context(mt, ctx, 3) == 0 and \
        gpu.cgx_model_fill_context(md, ctx, 4) == 0, last_error(gpu)
    sp = gpu.cgx_tree_spec_new(md, mt, nodes, depth, 0.7, 50, 1.0)
    assert sp, last_error(gpu)
    D = gpu.cgx_tree_spec_depth(sp)
    assert D == depth and gpu.cgx_tree_spec_nodes(sp) == nodes
    root = np.array([2, 3, 5, 7], np.int32)
    assert gpu.cgx_tree_spec_set_root(sp, root.ctypes.data) == 0, last_error(gpu)
    rng = np.random.default_rng(3)
    out = np.zeros((B, D + 2), np.int32)
    n = np.zeros(B, np.int32)
    lens = np.array([gpu.cgx_model_len_seq(mt, b) for b in range(B)])
    for s in range(steps):
        u = rng.random((B, D + 1, 5), dtype=np.float32)
        tot = gpu.cgx_tree_spec_step(sp, u.ctypes.data, out.ctypes.data, n.ctypes.data)
        assert tot == n.sum() >= 0, last_error(gpu)
        assert ((n >= 0) & (n <= D)).all()
        for b in range(B):
            assert ((out[b, :n[b] + 1] >= 0) & (out[b, :n[b] + 1] < V)).all()
            assert (out[b, n[b] + 1:] == -1).all()
        lens += n + 1
        assert [gpu.cgx_model_len_seq(mt, b) for b in range(B)] == lens.tolist()
        assert [gpu.cgx_model_len_seq(md, b) for b in range(B)] == lens.tolist()
    gpu.cgx_tree_spec_free(sp)
    gpu.cgx_model_free(md)
    gpu.cgx_model_free(mt)


C3 = dict(n_layers=12, d_model=768, n_heads=12, n_kv_heads=12, head_dim=64, d_ff=3072,
          group_size=128, kv_group_size=64, rope_theta=10000.0, norm_eps=1e-5, init_std=0.02)


def c3_model(gpu, max_seq, max_tokens, seed, layers=12):
    cfg = CgxModelConfig(**{**C3, "n_layers": layers}, vocab=32000, max_seq=max_seq,
                         max_tokens=max_tokens, max_batch=0)
    m = gpu.cgx_model_new(C.byref(cfg), seed, None)
    assert m, last_error(gpu)
    return m


def test_c3_stack_rows_and_identical_draft(gpu):
    """Config 3's stack after a 1024-token context: the logits of 5 tokens at
    once equal those of the same tokens one at a time (fp32 accumulation
    tolerance), and a draft with the target's weights accepts every drafted
    token with T = 0.8 and top-p 0.9 (the 768 x 6144 fused gate|up and the
    768 x 32000 head at their real shapes)."""
    print("C3 stack: 5 rows vs one at a time; identical draft, top-p 0.9", flush=True)
    V, ctx, g, steps = 32000, 1024, 4, 4
    ms = ctx + (g + 1) * (steps + 2)
    m = c3_model(gpu, ms, g + 1, 3)
    assert gpu.cgx_model_fill_context(m, ctx, 5) == 0, last_error(gpu)
    toks = np.array([7, 700, 7000, 17000, 31999], np.int32)
    assert gpu.cgx_model_forward(m, toks.ctypes.data, 5, 5, None) == 0, last_error(gpu)
    all5 = np.zeros((5, V), np.float32)
    assert gpu.cgx_memcpy_d2h(all5.ctypes.data, gpu.cgx_model_logits(m), all5.nbytes) == 0
    assert np.isfinite(all5).all() and all5.std(axis=1).min() > 1e-3
    assert gpu.cgx_model_truncate(m, ctx) == 0
    one = np.zeros((5, V), np.float32)
    for i in range(5):
        assert gpu.cgx_model_forward(m, toks[i:i + 1].ctypes.data, 1, 1, None) == 0, \
            last_error(gpu)
        assert gpu.cgx_memcpy_d2h(one[i].ctypes.data, gpu.cgx_model_logits(m), V * 4) == 0
    scale = float(np.abs(all5).max())
    assert float(np.abs(one - all5).max()) <= 2e-3 * scale
    assert gpu.cgx_model_truncate(m, ctx) == 0
    d = c3_model(gpu, ms, 2, 3)
    assert gpu.cgx_model_fill_context(d, ctx, 5) == 0, last_error(gpu)
    sp = gpu.cgx_spec_new(d, m, g, 0.8, 0, 0.9)
    assert sp and gpu.cgx_spec_set_last(sp, 5) == 0, last_error(gpu)
    rng = np.random.default_rng(3)
    out = np.zeros(g + 1, np.int32)
    for s in range(steps):
        ud = rng.random(g, dtype=np.float32)
        uv = rng.random(g + 1, dtype=np.float32)
        n = gpu.cgx_spec_step(sp, ud.ctypes.data, uv.ctypes.data, out.ctypes.data)
        assert n == g, (s, n, last_error(gpu))
        assert ((out >= 0) & (out < V)).all()
        assert gpu.cgx_model_len(m) == ctx + (s + 1) * (g + 1)
    gpu.cgx_spec_free(sp)
    gpu.cgx_model_free(d)
    gpu.cgx_model_free(m)
