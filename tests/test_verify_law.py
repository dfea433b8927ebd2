"""CPU: pins the oracle's chain-verify composition (orc_verify_chain) and the
filtered distribution it runs on (orc_filtered_dist) by what the mathematics
fixes, not by restating them.

* The filtered distribution (top-k list -> softmax -> top-p inclusive cutoff
  -> renormalise; the reference's rules of src/inference/speculative.c:77-146)
  is recomputed independently in float64 from its definition: same support,
  values within fp32 rounding, total 1 within fp32 rounding.
* Speculative sampling is lossless (Leviathan et al. 2023, Chen et al. 2023):
  with the draft token x ~ q, acceptance with probability min(1, p(x)/q(x))
  (speculative.c:49-52) and, on a reject, a fresh draw from
  max(0, p - q) / sum (speculative.c:148-172), the emitted token follows p.
  Over 2*10^5 seeded draw sets of a gamma = 2 chain the first emitted token
  must follow the filtered target row 0; given the first draft was accepted,
  the second emitted token must follow row 1; given both were, the bonus
  must follow row 2.  A chi-square test at alpha = 1e-6 decides each.
* The checks have power: the oracle rebuilt with each planted mistake
  (oracle/cg_oracle.c ORC_MUTANT: the correction reusing the accept draw, p
  and q swapped in the ratio, top-p not renormalised, the bonus reusing the
  last accept draw) fails at least one of them.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle_lib
from oracle_lib import ptr

GAMMA = 2
CASES = [  # (V, T, top_k, top_p)
    (8, 1.0, 0, 1.0),
    (8, 0.7, 0, 1.0),
    (8, 1.0, 4, 1.0),
    (8, 0.8, 0, 0.8),
    (8, 0.7, 5, 0.9),
]


def filtered64(logits: np.ndarray, T: float, top_k: int, top_p: float) -> np.ndarray:
    """The filtered distribution from its definition, in float64.  The one
    fp32 step kept is z = logits / T, the input both sides see."""
    V = logits.size
    z = (logits.astype(np.float32) / np.float32(T)).astype(np.float64)
    if 0 < top_k < V:
        keep = np.argsort(-z, kind="stable")[:top_k]      # ties: lower index first
    else:
        keep = np.arange(V)
    w = np.exp(z[keep] - z[keep].max())
    p = np.zeros(V)
    p[keep] = w / w.sum()
    if top_p < 1.0:
        order = np.argsort(-p, kind="stable")
        c = np.cumsum(p[order])
        # keep the inputs away from the cutoff's rounding boundary
        assert np.min(np.abs(c - top_p)) > 1e-5, "cutoff within rounding of top_p"
        cut = int(np.argmax(c >= top_p)) + 1 if (c >= top_p).any() else V
        kept = order[:cut]
        p2 = np.zeros(V)
        p2[kept] = p[kept] / c[cut - 1]
        p = p2
    return p


def _dist(orc, logits, T, top_k, top_p):
    out = np.zeros(logits.size, np.float32)
    row = np.ascontiguousarray(logits, np.float32)
    orc.orc_filtered_dist(ptr(row), row.size, T, top_k, top_p, ptr(out))
    return out


def _dist_ok(orc, logits, T, top_k, top_p) -> bool:
    got = _dist(orc, logits, T, top_k, top_p).astype(np.float64)
    exp = filtered64(logits, T, top_k, top_p)
    V = logits.size
    if not np.array_equal(got != 0, exp != 0):
        return False
    if abs(got.sum() - 1.0) > V * 2.0 ** -23:
        return False
    nz = exp != 0
    return bool(np.all(np.abs(got[nz] - exp[nz]) <= 1e-5 * exp[nz] + 1e-12))


def _chi2_pvalue(counts: np.ndarray, p: np.ndarray) -> float:
    """p-value of counts ~ Multinomial(n, p); 0 when any count falls where p is 0."""
    from scipy.stats import chi2
    n = counts.sum()
    if n == 0:
        return 1.0
    if counts[p == 0].sum() > 0:
        return 0.0
    e = n * p
    big = e >= 5
    obs = np.append(counts[big], counts[~big].sum())
    ex = np.append(e[big], e[~big].sum())
    keep = ex > 0
    stat = float((((obs - ex) ** 2)[keep] / ex[keep]).sum())
    return float(chi2.sf(stat, max(int(keep.sum()) - 1, 1)))


def _make_case(seed: int, V: int):
    rng = np.random.default_rng(seed)
    t = rng.normal(0, 1.5, (GAMMA + 1, V)).astype(np.float32)
    d = rng.normal(0, 1.5, (GAMMA, V)).astype(np.float32)
    return t, d


def _law_pvalues(orc, case, N: int, seed: int) -> list[float]:
    """p-values of: first token ~ p0; second | first accepted ~ p1; bonus |
    both accepted ~ p2."""
    V, T, k, tp = case
    t, d = _make_case(seed, V)
    p = [filtered64(t[i], T, k, tp) for i in range(GAMMA + 1)]
    q = [filtered64(d[i], T, k, tp) for i in range(GAMMA)]
    rng = np.random.default_rng(seed + 1)
    x = np.stack([rng.choice(V, size=N, p=q[i]) for i in range(GAMMA)], axis=1)
    x = np.ascontiguousarray(x, np.int32)
    u = rng.random((N, GAMMA + 1), dtype=np.float32)
    out = np.zeros((N, GAMMA + 1), np.int32)
    n = np.zeros(N, np.int32)
    orc.orc_verify_chain_many(ptr(t), ptr(d), ptr(x), ptr(u), N, GAMMA, V, T, k, tp,
                              ptr(out), ptr(n))
    pv = [_chi2_pvalue(np.bincount(out[:, 0], minlength=V), p[0])]
    sel = n >= 1
    pv.append(_chi2_pvalue(np.bincount(out[sel, 1], minlength=V), p[1]))
    sel = n == GAMMA
    pv.append(_chi2_pvalue(np.bincount(out[sel, GAMMA], minlength=V), p[GAMMA]))
    return pv


@pytest.mark.parametrize("V,T,top_k,top_p", [(300, 1.0, 0, 1.0), (300, 0.7, 0, 1.0),
                                             (300, 1.0, 50, 1.0), (300, 0.8, 0, 0.9),
                                             (300, 0.7, 50, 0.9), (300, 1.3, 7, 0.5)])
def test_filtered_dist_from_definition(oracle, V, T, top_k, top_p):
    rng = np.random.default_rng(7)
    for _ in range(5):
        logits = rng.normal(0, 2, V).astype(np.float32)
        assert _dist_ok(oracle, logits, T, top_k, top_p)


@pytest.mark.parametrize("case", CASES, ids=[f"V{c[0]}-T{c[1]}-k{c[2]}-p{c[3]}" for c in CASES])
def test_chain_verify_is_lossless(oracle, case):
    pv = _law_pvalues(oracle, case, 200_000, seed=11)
    assert min(pv) > 1e-6, pv
    t, d = _make_case(11, case[0])
    for row in (*t, *d):
        assert _dist_ok(oracle, row, *case[1:])


@pytest.mark.parametrize("mutant", [1, 2, 3, 4])
def test_law_checks_catch_planted_mistakes(mutant):
    orc = oracle_lib.load_oracle_mutant(mutant)
    caught = []
    for case in CASES:
        t, d = _make_case(11, case[0])
        dist_ok = all(_dist_ok(orc, row, *case[1:]) for row in (*t, *d))
        pv = _law_pvalues(orc, case, 100_000, seed=11)
        caught.append(not dist_ok or min(pv) < 1e-6)
    assert any(caught), f"planted mistake {mutant} passed every check"
