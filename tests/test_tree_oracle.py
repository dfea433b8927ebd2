"""The tree walk's oracle (oracle/cg_oracle.c orc_tree_accept) and the
default draft tree, on the CPU.

The walk has no reference counterpart (cogito's EAGLE builder is a stub,
src/inference/speculative.c:244-262), so it is pinned by what the
mathematics fixes: recursive rejection with point-mass drafts is lossless --
the first emitted token follows the root's target distribution exactly, and
given that child c was accepted, the next emitted token follows c's.  A
walk that kept a rejected candidate's mass, or renormalised with the wrong
total, biases the first token and fails these checks.
"""
from __future__ import annotations

import numpy as np

from oracle_lib import ptr


def _lists(oracle, rng, nodes, V, K, T=0.7, spread=1.5):
    z = (rng.normal(0, spread, (nodes, V)) / np.float32(T)).astype(np.float32)
    lidx = np.zeros((nodes, K), np.int32)
    lp = np.zeros((nodes, K), np.float32)
    for i in range(nodes):
        oracle.orc_topk_lists(ptr(z[i]), V, K, 1.0, ptr(lidx[i]), ptr(lp[i]))
    return lidx, lp


def _walk(oracle, parent, lidx, lp, tok, u):
    nodes, K = lidx.shape
    depth = int(u.shape[0] - 1)
    out = np.zeros(depth + 2, np.int32)
    path = np.zeros(max(depth, 1), np.int32)
    n = oracle.orc_tree_accept(ptr(parent), nodes, K, ptr(lidx), ptr(lp), ptr(tok), ptr(u),
                               ptr(out), ptr(path))
    return n, out, path


def test_topk_lists_are_the_filtered_distribution(oracle, rng):
    # the list form equals the dense filtered distribution of the chain verify
    V, K, T = 300, 20, 0.7
    logits = rng.normal(0, 2, V).astype(np.float32)
    z = (logits / np.float32(T)).astype(np.float32)
    lidx = np.zeros(K, np.int32)
    lp = np.zeros(K, np.float32)
    oracle.orc_topk_lists(ptr(z), V, K, 1.0, ptr(lidx), ptr(lp))
    dense = np.zeros(V, np.float32)
    oracle.orc_filtered_dist(ptr(logits), V, T, K, 1.0, ptr(dense))
    np.testing.assert_array_equal(dense[lidx], lp)
    assert np.count_nonzero(dense) == K
    assert (np.diff(z[lidx]) <= 0).all()


def test_walk_is_lossless(oracle, rng):
    # a root with 3 candidates (one outside the root's list), the first child
    # with 2; empirical first-token and conditional second-token laws
    V, K = 12, 12
    parent = np.array([-1, 0, 0, 0, 1, 1], np.int32)
    lidx, lp = _lists(oracle, rng, 6, V, K)
    tok = np.zeros(6, np.int32)
    tok[1], tok[2] = lidx[0, 1], lidx[0, 0]
    tok[3] = 11 if 11 not in lidx[0, :0] else 10
    tok[4], tok[5] = lidx[1, 2], lidx[1, 5]
    p_root = np.zeros(V)
    p_root[lidx[0]] = lp[0]
    p_c1 = np.zeros(V)
    p_c1[lidx[1]] = lp[1]
    N = 40000
    first = np.zeros(V)
    second = np.zeros(V)
    for _ in range(N):
        u = rng.uniform(0, 1, (3, 5)).astype(np.float32)
        n, out, path = _walk(oracle, parent, lidx, lp, tok, u)
        first[out[0]] += 1
        # the walk from child 1 on: its first test always passes
        u[0, 0] = 0.0
        n, out, path = _walk(oracle, parent, lidx, lp, tok, u)
        assert n >= 1 and path[0] == 1
        second[out[1]] += 1
    _chi2_ok(first, p_root)
    _chi2_ok(second, p_c1)


def _chi2_ok(counts, p, alpha=1e-6):
    """Counts follow p: no mass outside p's support, and a chi-square test
    over the bins with an expected count of at least 5 does not reject."""
    from scipy.stats import chi2
    n = counts.sum()
    assert counts[p == 0].sum() == 0
    e = n * p
    big = e >= 5
    obs = np.append(counts[big], counts[~big].sum())
    exp = np.append(e[big], e[~big].sum())
    keep = exp > 0
    stat = (((obs - exp) ** 2)[keep] / exp[keep]).sum()
    assert chi2.sf(stat, keep.sum() - 1) > alpha, (stat, obs, exp)


def test_walk_fixed_draws(oracle, rng):
    V, K = 40, 8
    parent = np.array([-1, 0, 0, 1, 3], np.int32)        # root -> {1, 2}, 1 -> 3 -> 4
    lidx, lp = _lists(oracle, rng, 5, V, K)
    tok = np.array([0, lidx[0, 0], lidx[0, 1], lidx[1, 0], lidx[3, 0]], np.int32)
    # every test passes: the deepest path is accepted, the bonus from node 4
    u = np.zeros((4, 5), np.float32)
    n, out, path = _walk(oracle, parent, lidx, lp, tok, u)
    assert n == 3 and list(path[:3]) == [1, 3, 4]
    assert list(out[:3]) == [tok[1], tok[3], tok[4]] and out[3] == lidx[4, 0]
    # every test fails: the draw from the root's residual, which excludes the
    # two rejected candidates
    u = np.full((4, 5), 0.99999, np.float32)
    for draw in (0.0, 0.5, 0.99999):
        u[0, 4] = draw
        n, out, _ = _walk(oracle, parent, lidx, lp, tok, u)
        assert n == 0 and out[0] not in (tok[1], tok[2]) and out[0] in lidx[0]


def test_default_shape(lib):
    # pure host code of the product library (no device needed)
    par = np.zeros(64, np.int32)
    dep = np.zeros(64, np.int32)
    rank = np.zeros(64, np.int32)
    n = lib.cgx_tree_shape_get(64, 6, par.ctypes.data, dep.ctypes.data, rank.ctypes.data)
    assert n == 64
    assert par[0] == -1 and (par[1:] < np.arange(1, 64)).all()
    assert (np.diff(dep) >= 0).all() and dep.max() == 6
    assert list(np.bincount(dep)) == [1, 4, 13, 14, 14, 11, 7]
    for i in range(64):
        kids = np.flatnonzero(par == i)
        assert len(kids) <= 4 and list(rank[kids]) == list(range(len(kids)))
    # best-first: a node's path score is at least that of any non-member child
    w = np.array([0.6, 0.2, 0.12, 0.08])
    score = np.ones(64)
    for i in range(1, 64):
        score[i] = score[par[i]] * w[rank[i]]
    frontier = [score[i] * w[len(np.flatnonzero(par == i))]
                for i in range(64) if dep[i] < 6 and len(np.flatnonzero(par == i)) < 4]
    assert score[1:].min() >= max(frontier) - 1e-12
