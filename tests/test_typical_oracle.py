"""CPU: pins the oracle's typical sampling (orc_typ_log, orc_typical_sorted,
orc_sample_typical, orc_typical_dist; decision D16 of this build).

The reference declares cg_sample_typical (include/cg_speculative.h:186) and
never defines it, so nothing of the reference pins it.  What the
mathematics fixes does:
* orc_typ_log is log(x) to within 2 ulp of binary64 over random and special
  floats (log 1 = 0 exactly, log 2^k = k ln 2);
* the entropy is -sum p log p: uniform logits over V give H = log V;
* the kept set is the locally typical set of Meister et al. (2023), from a
  float64 brute force: tokens ordered by |-log p - H| (ties: lower index),
  the shortest prefix with mass >= typical_p;
* the distribution is p / kept mass on that set and 0 elsewhere;
* the draw over a dense grid of u reproduces that distribution, and u -> 0
  gives the most typical token.
A planted error of the kind a restatement could make (ordering by -log p
instead of its distance to H) changes the kept set on these cases.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

from oracle_lib import ptr


def _sorted(oracle, x, tp):
    V = x.size
    probs = np.zeros(V, np.float32)
    order = np.zeros(V, np.int32)
    mass = C.c_float(0)
    cut = oracle.orc_typical_sorted(ptr(x), V, tp, ptr(probs), ptr(order), C.byref(mass))
    return cut, probs, order, mass.value


def _brute(x, tp):
    """float64 definition: returns (kept index set, kept mass, H)."""
    z = x.astype(np.float64) - x.max()
    p = np.exp(z) / np.exp(z).sum()
    nz = p > 0
    H = -np.sum(p[nz] * np.log(p[nz]))
    score = np.where(nz, np.abs(-np.log(np.where(nz, p, 1.0)) - H), np.inf)
    order = np.lexsort((np.arange(p.size), score))
    c = np.cumsum(p[order])
    hit = np.flatnonzero(c >= tp)
    cut = int(hit[0]) + 1 if hit.size else p.size
    return set(order[:cut].tolist()), float(c[cut - 1]), H, c, order


def test_typ_log_against_float64(oracle, rng):
    xs = np.concatenate([rng.random(20000, dtype=np.float32),
                         np.exp(rng.uniform(-100, 80, 20000)).astype(np.float32),
                         np.array([1.0, 2.0, 0.5, 1e-45, 3.4e38, 0.70710677, 1.4142135],
                                  np.float32)])
    xs = xs[xs > 0]
    worst = 0.0
    for x in xs:
        got = oracle.orc_typ_log(float(x))
        exp = math.log(float(x))
        ulp = math.ulp(exp) if exp != 0 else 0.0
        if exp == 0:
            assert got == 0.0
            continue
        worst = max(worst, abs(got - exp) / ulp)
    assert worst <= 2.0, worst
    for k in range(-140, 128, 7):
        got = oracle.orc_typ_log(float(np.float32(2.0) ** k))
        assert abs(got - k * math.log(2)) <= 2 * math.ulp(k * math.log(2) or 1.0), k


@pytest.mark.parametrize("V", [1, 7, 1000, 32000])
def test_uniform_logits_entropy_and_order(oracle, V):
    # all scores equal: the order is the index order, and H = log V
    x = np.zeros(V, np.float32)
    cut, probs, order, mass = _sorted(oracle, x, 0.5)
    assert list(order[:min(V, 50)]) == list(range(min(V, 50)))
    p = np.float32(1.0) / np.float32(V)
    c = np.add.accumulate(np.full(V, p, np.float32), dtype=np.float32)
    assert cut == int(np.flatnonzero(c >= np.float32(0.5))[0]) + 1
    assert mass == c[cut - 1]
    # entropy of the uniform distribution through the score of any token:
    # score = |-log p - H| = 0 up to fp32 rounding
    L = np.float32(oracle.orc_typ_log(float(p)))
    H = np.float32(0)
    for _ in range(min(V, 2000)):
        H = np.float32(H + np.float32(p * -L))
    if V <= 2000:
        assert abs(float(H) - math.log(V)) <= 1e-6 * max(1.0, math.log(V)) + V * 2e-7


@pytest.mark.parametrize("V,tp,spread", [(12, 0.9, 1.5), (40, 0.5, 2.0), (300, 0.95, 1.0),
                                         (300, 0.2, 3.0), (2000, 0.9, 2.0), (60, 1.0, 1.0)])
def test_typical_set_from_definition(oracle, rng, V, tp, spread):
    checked = 0
    for trial in range(6):
        x = rng.normal(0, spread, V).astype(np.float32)
        kept, mass64, H, c, order64 = _brute(x, tp)
        # keep the case away from rounding boundaries of the cutoff and order
        if tp < 1.0 and np.min(np.abs(c - tp)) < 1e-5:
            continue
        cut, probs, order, mass = _sorted(oracle, x, tp)
        assert set(order[:cut].tolist()) == kept, trial
        assert abs(mass - mass64) <= 1e-5 * mass64
        dist = np.zeros(V, np.float32)
        oracle.orc_typical_dist(ptr(x), V, tp, ptr(dist))
        nz = np.flatnonzero(dist)
        assert set(nz.tolist()) == kept
        p64 = np.exp(x.astype(np.float64) - x.max())
        p64 /= p64.sum()
        np.testing.assert_allclose(dist[nz], p64[nz] / mass64, rtol=1e-5)
        assert abs(float(dist.sum(dtype=np.float64)) - 1.0) <= V * 2.0 ** -23
        checked += 1
    assert checked >= 4


def test_typical_draws_follow_the_kept_distribution(oracle, rng):
    V, tp = 20, 0.8
    x = rng.normal(0, 1.5, V).astype(np.float32)
    dist = np.zeros(V, np.float32)
    oracle.orc_typical_dist(ptr(x), V, tp, ptr(dist))
    n = 20000
    counts = np.zeros(V)
    for u in (np.arange(n) + 0.5) / n:
        counts[oracle.orc_sample_typical(ptr(x), V, tp, float(u))] += 1
    assert np.all(counts[dist == 0] == 0)
    np.testing.assert_allclose(counts / n, dist, atol=2.0 / n + 1e-6)
    # u = 0: the first token of the typical order, the one closest to H
    _, _, order, _ = _sorted(oracle, x, tp)
    assert oracle.orc_sample_typical(ptr(x), V, tp, 0.0) == order[0]


def test_typical_differs_from_most_likely_first(oracle, rng):
    # a peaked distribution: the most likely token is not the most typical
    # one (its -log p is far below H), so ordering by -log p would keep a
    # different set than the typical order does
    x = np.array([4.0] + [2.0] * 20 + [0.0] * 100, np.float32)
    kept, *_ = _brute(x, 0.5)
    cut, probs, order, mass = _sorted(oracle, x, 0.5)
    assert set(order[:cut].tolist()) == kept
    assert 0 not in kept
    by_logp = set(np.argsort(-probs, kind="stable")[:cut].tolist())
    assert by_logp != kept
