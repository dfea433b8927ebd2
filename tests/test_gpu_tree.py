"""GPU parity of the tree verify path (tree.hip, host/tree.c):

* top-k lists (index and probability per entry) bit-exact with the oracle's
  list form of the filtered distribution, at V up to 128256;
* the acceptance walk: accepted count, path and emitted tokens identical to
  the oracle's walk on the same lists, node tokens and draws;
* the tree forward of the model: logits within 1e-3 of the oracle stack with
  per-row rotary positions and the tree mask;
* the tree loop: after a step the caches hold exactly the committed tokens
  (a follow-up forward matches a model that took them as a chain).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import replace

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error
from gpu_util import rel_err_rows
from oracle_lib import ptr
from oracle_model import Cfg, OracleModel

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _shape(gpu, nodes=64, depth=6):
    par = np.zeros(nodes, np.int32)
    dep = np.zeros(nodes, np.int32)
    rank = np.zeros(nodes, np.int32)
    n = gpu.cgx_tree_shape_get(nodes, depth, par.ctypes.data, dep.ctypes.data,
                               rank.ctypes.data)
    assert n == nodes, last_error(gpu)
    return par, dep, rank


def _anc(par):
    anc = np.zeros(len(par), np.uint64)
    for i in range(len(par)):
        anc[i] = np.uint64(1 << i) | (anc[par[i]] if par[i] >= 0 else np.uint64(0))
    return anc


@pytest.mark.parametrize("V,K,top_p", [(5000, 50, 1.0), (128256, 50, 1.0), (128256, 4, 1.0),
                                       (32000, 50, 0.9), (300, 64, 1.0)])
def test_topk_lists_vs_oracle(gpu, oracle, rng, V, K, top_p):
    rows, T = 6, 0.7
    logits = rng.normal(0, 2, (rows, V)).astype(np.float32)
    logits[1, rng.integers(0, V, 20)] = 5.0                 # ties in the list
    logits[2, 7:] = -np.inf                                  # fewer than K finite entries
    z = (logits / np.float32(T)).astype(np.float32)
    dz = DeviceArray.from_numpy(gpu, z)
    di = DeviceArray(gpu, rows * K * 4)
    dp = DeviceArray(gpu, rows * K * 4)
    assert gpu.cgx_topk_lists_dev(dz.ptr, rows, V, K, top_p, di.ptr, dp.ptr) == 0, \
        last_error(gpu)
    gpu.cgx_synchronize()
    gi = di.numpy(np.int32, (rows, K))
    gp = dp.numpy(np.float32, (rows, K))
    for r in range(rows):
        ei = np.zeros(K, np.int32)
        ep = np.zeros(K, np.float32)
        oracle.orc_topk_lists(ptr(z[r]), V, K, top_p, ptr(ei), ptr(ep))
        live = ep > 0
        np.testing.assert_array_equal(gi[r][live], ei[live])
        np.testing.assert_array_equal(gp[r].view(np.uint32), ep.view(np.uint32))
    for d in (dz, di, dp):
        d.free()


@pytest.mark.parametrize("mode", ["random", "accepting", "rejecting"])
def test_tree_accept_vs_oracle(gpu, oracle, rng, mode):
    par, dep, rank = _shape(gpu)
    R, D, B, K, V = 64, 6, 4, 50, 3000
    z = (rng.normal(0, 1.5, (B, R, V)) / np.float32(0.7)).astype(np.float32)
    lidx = np.zeros((B, R, K), np.int32)
    lp = np.zeros((B, R, K), np.float32)
    for b in range(B):
        for i in range(R):
            oracle.orc_topk_lists(ptr(z[b, i]), V, K, 1.0, ptr(lidx[b, i]), ptr(lp[b, i]))
    # node tokens: mostly high entries of the parent's list (accepts happen),
    # some outside it
    tok = np.zeros((B, R), np.int32)
    for b in range(B):
        tok[b, 0] = rng.integers(0, V)
        for i in range(1, R):
            j = min(int(rng.integers(0, 4)) + rank[i], K - 1)
            tok[b, i] = lidx[b, par[i], j] if rng.uniform() < 0.85 else rng.integers(0, V)
    u = rng.uniform(0, 1, (B, D + 1, 5)).astype(np.float32)
    if mode == "accepting":
        u[:, :, :4] *= 0.02
    elif mode == "rejecting":
        u[:, :, :4] = 0.999999
    dl = DeviceArray.from_numpy(gpu, lidx)
    dp = DeviceArray.from_numpy(gpu, lp)
    dt = DeviceArray.from_numpy(gpu, tok)
    du = DeviceArray.from_numpy(gpu, u)
    dout = DeviceArray(gpu, B * (D + 2) * 4)
    dn = DeviceArray(gpu, B * 4)
    dpath = DeviceArray(gpu, B * D * 4)
    assert gpu.cgx_tree_accept_dev(par.ctypes.data, R, B, K, dl.ptr, dp.ptr, dt.ptr, du.ptr,
                                   dout.ptr, dn.ptr, dpath.ptr) == 0, last_error(gpu)
    gpu.cgx_synchronize()
    out = dout.numpy(np.int32, (B, D + 2))
    n = dn.numpy(np.int32, (B,))
    path = dpath.numpy(np.int32, (B, D))
    for b in range(B):
        eo = np.zeros(D + 2, np.int32)
        ep = np.zeros(D, np.int32)
        en = oracle.orc_tree_accept(ptr(par), R, K, ptr(lidx[b]), ptr(lp[b]), ptr(tok[b]),
                                    ptr(u[b]), ptr(eo), ptr(ep))
        assert n[b] == en, (b, n[b], en)
        np.testing.assert_array_equal(out[b, :en + 1], eo[:en + 1])
        np.testing.assert_array_equal(path[b, :en], ep[:en])
    if mode == "accepting":
        assert n.sum() > 0
    if mode == "rejecting":
        assert (n == 0).all()
    for d in (dl, dp, dt, du, dout, dn, dpath):
        d.free()


def _tiny(**kw):
    return Cfg(**{**dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64,
                         d_ff=512, vocab=1024, group_size=128, kv_group_size=64, max_seq=160,
                         max_tokens=64, init_std=0.05), **kw})


def new_model(gpu, cfg, seed, share=None):
    cc = cfg.ctype()
    m = gpu.cgx_model_new(C.byref(cc), seed, share)
    assert m, last_error(gpu)
    return m


@pytest.mark.parametrize("B", [1, 3])
def test_model_forward_tree_vs_oracle(gpu, oracle, rng, B):
    # a prefix, then a 16-node tree in one forward, then its first 2 levels
    # again as two separate calls with windows over the nodes so far (the
    # draft's level-by-level pattern)
    cfg = _tiny(max_batch=B)
    m = new_model(gpu, cfg, 9)
    oms = [OracleModel(oracle, replace(cfg, max_batch=0), 9) for _ in range(B)]
    V = cfg.vocab
    par, dep, _ = _shape(gpu, 16, 4)
    anc = _anc(par)
    prompts = rng.integers(0, V, (B, 7)).astype(np.int32)
    assert gpu.cgx_model_forward_batch(m, prompts.ctypes.data, 7, 0, None) == 0, last_error(gpu)
    for b in range(B):
        oms[b].forward(prompts[b], n_logits=0)
    toks = rng.integers(0, V, (B, 16)).astype(np.int32)
    rel = dep.astype(np.int32)
    assert gpu.cgx_model_forward_tree_rows(m, toks.ctypes.data, 16, rel.ctypes.data,
                                           anc.ctypes.data, 16, None) == 0, last_error(gpu)
    got = np.empty((B * 16, V), np.float32)
    assert gpu.cgx_memcpy_d2h(got.ctypes.data, gpu.cgx_model_logits(m), got.nbytes) == 0
    got = got.reshape(B, 16, V)
    for b in range(B):
        exp = oms[b].forward_tree(toks[b], rel, anc, 16)
        assert rel_err_rows(got[b], exp) <= TOL, b
    # level pattern: drop the tree, re-add the root then level 1 (window 1 + 4)
    for b in range(B):
        assert gpu.cgx_model_truncate_seq(m, b, 7) == 0
        oms[b].truncate(7)
    levels = [(0, 1), (1, 4)]
    for f, c in levels:
        lt = np.ascontiguousarray(toks[:, f:f + c])
        lrel = (dep[f:f + c] - f).astype(np.int32)
        lanc = np.ascontiguousarray(anc[f:f + c])
        assert gpu.cgx_model_forward_tree_rows(m, lt.ctypes.data, c, lrel.ctypes.data,
                                               lanc.ctypes.data, f + c, None) == 0, \
            last_error(gpu)
        got = np.empty((B * c, V), np.float32)
        assert gpu.cgx_memcpy_d2h(got.ctypes.data, gpu.cgx_model_logits(m), got.nbytes) == 0
        got = got.reshape(B, c, V)
        for b in range(B):
            exp = oms[b].forward_tree(lt[b], lrel, lanc, f + c)
            assert rel_err_rows(got[b], exp) <= TOL, (f, b)
    gpu.cgx_model_free(m)


def test_tree_spec_keeps_the_committed_tokens(gpu, rng):
    # after each tree step, a forward of both caches continues exactly like a
    # model that took the committed tokens as a plain chain
    B, T, K = 2, 0.7, 50
    cfg = _tiny(max_batch=B, max_seq=400)
    dcfg = replace(cfg, n_layers=1)
    target = new_model(gpu, cfg, 41)
    draft = new_model(gpu, dcfg, 42, target)
    chain = new_model(gpu, cfg, 41)                # same weights as the target
    V = cfg.vocab
    prompts = rng.integers(0, V, (B, 9)).astype(np.int32)
    for mdl in (target, draft, chain):
        assert gpu.cgx_model_forward_batch(mdl, prompts.ctypes.data, 9, 0, None) == 0
    s = gpu.cgx_tree_spec_new(draft, target, 64, 6, T, K, 1.0)
    assert s, last_error(gpu)
    D = gpu.cgx_tree_spec_depth(s)
    root = rng.integers(0, V, B).astype(np.int32)
    assert gpu.cgx_tree_spec_set_root(s, root.ctypes.data) == 0, last_error(gpu)
    out = np.zeros((B, D + 2), np.int32)
    n = np.zeros(B, np.int32)
    lens = np.full(B, 9)
    for step in range(4):
        u = rng.uniform(0, 1, (B, D + 1, 5)).astype(np.float32)
        if step % 2:
            u[:, :, :4] *= 0.05                      # accept-heavy steps
        tot = gpu.cgx_tree_spec_step(s, u.ctypes.data, out.ctypes.data, n.ctypes.data)
        assert tot == n.sum() >= 0, last_error(gpu)
        # the chain model takes the root and the accepted tokens
        for b in range(B):
            assert 0 <= n[b] <= D
            assert ((out[b, :n[b] + 1] >= 0) & (out[b, :n[b] + 1] < V)).all()
            assert (out[b, n[b] + 1:] == -1).all()
            lens[b] += n[b] + 1
            assert gpu.cgx_model_len_seq(target, b) == lens[b]
            assert gpu.cgx_model_len_seq(draft, b) == lens[b]
        committed = [np.concatenate([[root[b]], out[b, :n[b]]]).astype(np.int32)
                     for b in range(B)]
        # the chain model: one row per call for sequence b, the other
        # sequences' extra row dropped again
        for b in range(B):
            for t in committed[b]:
                row = np.zeros(B, np.int32)
                row[b] = t
                # advance only sequence b: the others are truncated back after
                keep = [gpu.cgx_model_len_seq(chain, bb) for bb in range(B)]
                assert gpu.cgx_model_forward_batch(chain, row.ctypes.data, 1, 0, None) == 0
                for bb in range(B):
                    if bb != b:
                        assert gpu.cgx_model_truncate_seq(chain, bb, keep[bb]) == 0
        for b in range(B):
            assert gpu.cgx_model_len_seq(chain, b) == lens[b]
        root = np.array([out[b, n[b]] for b in range(B)], np.int32)
    # a probe token after the last step: logits of the target and of the chain
    probe = rng.integers(0, V, B).astype(np.int32)
    assert gpu.cgx_model_forward_batch(target, probe.ctypes.data, 1, 1, None) == 0
    got = np.empty((B, V), np.float32)
    assert gpu.cgx_memcpy_d2h(got.ctypes.data, gpu.cgx_model_logits(target), got.nbytes) == 0
    assert gpu.cgx_model_forward_batch(chain, probe.ctypes.data, 1, 1, None) == 0
    exp = np.empty((B, V), np.float32)
    assert gpu.cgx_memcpy_d2h(exp.ctypes.data, gpu.cgx_model_logits(chain), exp.nbytes) == 0
    # the cached K/V were computed by different kernels (tree GEMM vs chain
    # GEMV) before INT4 quantisation, so allow a few flipped nibbles
    assert rel_err_rows(got, exp) <= 2e-2
    gpu.cgx_tree_spec_free(s)
    for mdl in (chain, draft, target):
        gpu.cgx_model_free(mdl)


def test_tree_spec_rejects_bad_arguments(gpu):
    cfg = _tiny(max_batch=2)
    a = new_model(gpu, cfg, 1)
    b = new_model(gpu, replace(cfg, n_layers=1), 2, a)
    assert not gpu.cgx_tree_spec_new(a, b, 64, 6, 0.7, 0, 1.0)          # top_k 0
    assert "top_k" in last_error(gpu)
    small = new_model(gpu, replace(cfg, max_tokens=8), 3)
    assert not gpu.cgx_tree_spec_new(small, a, 64, 6, 0.7, 50, 1.0)     # 8 rows < 64 nodes
    for mdl in (small, b, a):
        gpu.cgx_model_free(mdl)
