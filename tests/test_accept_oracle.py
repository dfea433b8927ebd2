"""CPU: pins the sampling part of the oracle.

* closed forms: the LCG stream, the acceptance ratio, tiny-V CDFs;
* the compiled reference (oracle/_ref): every sampler on identical inputs,
  with the reference's global LCG mirrored draw for draw;
* the glibc-identical expf formula the GPU kernel uses, checked against this
  host's libm (the same formula is then checked on the GPU).
Reference: src/inference/speculative.c:11-172, 197-238.
"""
from __future__ import annotations

import ctypes as C
import math
import subprocess
import textwrap
from pathlib import Path

import numpy as np
import pytest

from oracle_lib import LCG, ptr, ref_tensor_np

ROOT = Path(__file__).resolve().parents[1]


def test_lcg_first_draws(oracle):
    lcg = LCG(42)
    draws = [round(lcg.draw(oracle), 4) for _ in range(6)]
    assert draws == [0.9675, 0.5912, 0.0401, 0.8454, 0.9383, 0.0180]


def test_lcg_closed_form(oracle):
    s = 42
    lcg = LCG(42)
    for _ in range(1000):
        s = (s * 1103515245 + 12345) & 0xFFFFFFFF
        assert lcg.draw(oracle) == np.float32(s % 10000) / np.float32(10000.0)


@pytest.mark.parametrize("q,p,exp", [(0.0, 0.3, 1.0), (1e-11, 0.5, 1.0), (0.5, 0.25, 0.5),
                                     (0.2, 0.9, 1.0), (0.4, 0.1, 0.25)])
def test_acceptance_prob_closed_form(oracle, q, p, exp):
    assert oracle.orc_acceptance_prob(q, p) == pytest.approx(exp, rel=1e-7)


def test_temperature_tiny_v_brute_force(oracle):
    # p proportional to 1:2:3 -> CDF steps at 1/6, 1/2, 1
    logits = np.log(np.array([1.0, 2.0, 3.0])).astype(np.float32)
    for u, tok in [(0.0, 0), (0.1, 0), (0.2, 1), (0.49, 1), (0.51, 2), (0.999, 2)]:
        assert oracle.orc_sample_temperature(ptr(logits), 3, 1.0, u) == tok
    # u beyond the rounded total -> default V-1 (speculative.c:68)
    assert oracle.orc_sample_temperature(ptr(logits), 3, 1.0, 1.5) == 2


def test_temperature_probs_vs_fp64(oracle, rng):
    for T in (1.0, 0.7, 2.0):
        x = rng.normal(0, 2, 5000).astype(np.float32)
        p = np.zeros_like(x)
        oracle.orc_temperature_probs(ptr(x), x.size, T, ptr(p))
        z = (x.astype(np.float64) - x.max()) / T
        e = np.exp(z)
        np.testing.assert_allclose(p, e / e.sum(), rtol=2e-5, atol=1e-12)


def _ref_sampler_check(oracle, ref, fn_ref, fn_orc, make_args, n_cases, lcg):
    for case in range(n_cases):
        args_ref, args_orc = make_args(case)   # make_args.keep holds the arrays
        u = lcg.draw(oracle)              # the draw the reference makes
        got = fn_ref(*args_ref)
        exp = fn_orc(*args_orc, u)
        assert got == exp, (case, got, exp)


@pytest.fixture()
def ref_lcg(ref, oracle):
    """Mirror of the reference library's global LCG.  Its state lives in the
    loaded .so for the whole session; every sampler call makes exactly one
    draw, so one session-wide mirror stays in lock-step."""
    return _REF_LCG_STATE


class _RefLcgState:
    def __init__(self):
        self.lcg = LCG(42)

    def draw(self, oracle):
        return self.lcg.draw(oracle)


_REF_LCG_STATE = _RefLcgState()


@pytest.mark.parametrize("V,T", [(64, 1.0), (1000, 0.7), (32000, 1.0), (32000, 1.3)])
def test_temperature_matches_reference(oracle, ref, ref_lcg, rng, V, T):
    def make(case):
        x = rng.normal(0, 2, V).astype(np.float32)
        if case % 3 == 1:
            x[rng.integers(0, V, 5)] = x.max()      # exact ties at the max
        make.keep = x
        return (x.ctypes.data, V, T), (x.ctypes.data, V, T)
    _ref_sampler_check(oracle, ref, ref.cg_sample_temperature,
                       oracle.orc_sample_temperature, make, 20, ref_lcg)


@pytest.mark.parametrize("V,k", [(64, 5), (1000, 50), (1000, 1), (32000, 50)])
def test_top_k_matches_reference(oracle, ref, ref_lcg, rng, V, k):
    def make(case):
        x = rng.normal(0, 2, V).astype(np.float32)
        if case % 2:
            x = np.round(x * 2) / 2               # many exact ties
        make.keep = x
        return (x.ctypes.data, V, k), (x.ctypes.data, V, k)
    _ref_sampler_check(oracle, ref, ref.cg_sample_top_k, oracle.orc_sample_top_k, make,
                       20, ref_lcg)


@pytest.mark.parametrize("V,p", [(64, 0.9), (300, 0.5), (1000, 0.9)])
def test_top_p_matches_reference(oracle, ref, ref_lcg, rng, V, p):
    def make(case):
        x = rng.normal(0, 2, V).astype(np.float32)
        if case % 2:
            x = np.round(x)                       # ties -> unstable-sort order
        make.keep = x
        return (x.ctypes.data, V, p), (x.ctypes.data, V, p)
    _ref_sampler_check(oracle, ref, ref.cg_sample_top_p, oracle.orc_sample_top_p, make,
                       12, ref_lcg)


@pytest.mark.parametrize("V", [64, 1000, 32000])
def test_corrected_matches_reference(oracle, ref, ref_lcg, rng, V):
    def make(case):
        lt = rng.normal(0, 2, V).astype(np.float32)
        ld = (lt + rng.normal(0, 0.5, V)).astype(np.float32)
        p = np.zeros(V, np.float32)
        q = np.zeros(V, np.float32)
        oracle.orc_temperature_probs(ptr(lt), V, 1.0, ptr(p))
        oracle.orc_temperature_probs(ptr(ld), V, 1.0, ptr(q))
        if case % 4 == 3:
            q = p.copy()                          # residual mass 0 -> fallback branch
        make.keep = (p, q)
        return (q.ctypes.data, p.ctypes.data, V), (q.ctypes.data, p.ctypes.data, V)
    _ref_sampler_check(oracle, ref, ref.cg_sample_corrected, oracle.orc_sample_corrected,
                       make, 16, ref_lcg)


def test_tree_mask_matches_reference(oracle, ref):
    seqlen, depth = 7, 4
    tree = ref.cg_token_tree_new(depth)
    m = ref.cg_tree_attention_mask(tree, seqlen)
    got = ref_tensor_np(m).reshape(seqlen + depth, seqlen + depth)
    exp = np.zeros((seqlen + depth) ** 2, np.float32)
    oracle.orc_tree_mask_chain(ptr(exp), seqlen, depth)
    np.testing.assert_array_equal(got, exp.reshape(got.shape))
    ref.cg_tensor_free(m)
    ref.cg_token_tree_free(tree)


def test_verify_chain_composition(oracle, rng):
    # accept/reject walk and draw order of the composition (decisions D4/D6)
    V, g = 50, 4
    t = rng.normal(0, 2, (g + 1, V)).astype(np.float32)
    d = rng.normal(0, 2, (g, V)).astype(np.float32)
    x = rng.integers(0, V, g).astype(np.int32)
    for u0 in ([0.0] * (g + 1), [0.999] * (g + 1)):
        u = np.array(u0, np.float32)
        out = np.zeros(g + 1, np.int32)
        ap = np.zeros(g, np.float32)
        n = oracle.orc_verify_chain(ptr(t), ptr(d), ptr(x), ptr(u), g, V, 1.0, 0, 1.0,
                                    ptr(out), ptr(ap))
        # recompute the walk from the oracle's own primitives
        n_exp = g
        for i in range(g):
            if not (u[i] < ap[i]):
                n_exp = i
                break
        assert n == n_exp
        assert list(out[:n]) == list(x[:n])
        if n == g:
            row = t[g].copy()
            assert out[g] == oracle.orc_sample_temperature(ptr(row), V, 1.0, u[g])
        else:
            p = np.zeros(V, np.float32)
            q = np.zeros(V, np.float32)
            trow, drow = t[n].copy(), d[n].copy()
            oracle.orc_temperature_probs(ptr(trow), V, 1.0, ptr(p))
            oracle.orc_temperature_probs(ptr(drow), V, 1.0, ptr(q))
            assert out[n] == oracle.orc_sample_corrected(ptr(q), ptr(p), V, u[n + 1])


# ------------------------------------------------------------ expf formula

_EXPF_CHECK = textwrap.dedent(r"""
    #include <math.h>
    #include <stdint.h>
    #include <stdio.h>
    #include <string.h>
    /* table-driven exp (ARM optimized-routines / glibc >= 2.28 method),
       identical to exp_glibc() in cogito_amd/csrc/accept.hip */
    static const uint64_t T[32] = {
    0x3ff0000000000000ull,0x3fefd9b0d3158574ull,0x3fefb5586cf9890full,0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull,0x3fef54873168b9aaull,0x3fef387a6e756238ull,0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull,0x3feef1a7373aa9cbull,0x3feedea64c123422ull,0x3feece086061892dull,
    0x3feebfdad5362a27ull,0x3feeb42b569d4f82ull,0x3feeab07dd485429ull,0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull,0x3fee9f75e8ec5f74ull,0x3feea11473eb0187ull,0x3feea589994cce13ull,
    0x3feeace5422aa0dbull,0x3feeb737b0cdc5e5ull,0x3feec49182a3f090ull,0x3feed503b23e255dull,
    0x3feee89f995ad3adull,0x3feeff76f2fb5e47ull,0x3fef199bdd85529cull,0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull,0x3fef7c97337b9b5full,0x3fefa4afa2a490daull,0x3fefd0765b6e4540ull};
    static float ex(float x) {
      if (!(x <= 0x1.62e42ep6f)) return x != x ? x + x : INFINITY;
      if (x < -0x1.9fe368p6f) return 0.0f;
      double N = 0x1.71547652b82fep+0 * 32.0, S = 0x1.8p+52, xd = x, kd, r, s, y, z;
      uint64_t ki, t;
      kd = fma(N, xd, S); memcpy(&ki, &kd, 8); kd -= S; r = fma(N, xd, -kd);
      t = T[ki & 31] + (ki << 47); memcpy(&s, &t, 8);
      z = fma(0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0, r, 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0);
      y = fma(0x1.62e42ff0c52d6p-1 / 32.0, r, 1.0);
      y = fma(z, r * r, y); y = y * s;
      return (float)y;
    }
    int main(void) {
      long bad = 0, n = 0;
      /* every 13th binary32 in [-104, 0], plus both ends */
      for (uint32_t b = 0x80000000u; b <= 0xC2D00000u; b += 13) {
        float x, a, g; memcpy(&x, &b, 4); a = ex(x); g = expf(x); n++;
        if (memcmp(&a, &g, 4)) bad++;
      }
      printf("%ld %ld\n", n, bad);
      return 0;
    }
""")


def test_expf_formula_matches_host_libm(tmp_path):
    src = tmp_path / "expf_check.c"
    src.write_text(_EXPF_CHECK)
    exe = tmp_path / "expf_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", str(src), "-o", str(exe), "-lm"],
                   check=True)
    n, bad = map(int, subprocess.run([str(exe)], capture_output=True, text=True,
                                     check=True).stdout.split())
    assert n > 80_000_000 and bad == 0


def _tie_rule_order(p):
    """Order in which the reference's selection sort (speculative.c:93-100)
    emits equal values, from counts only: members i_1 < ... < i_n of the
    group of value v, g_t = number of elements > v between i_t and i_(t+1)
    (g_n after i_n); for t = 1..n append i_t to R and rotate R left by g_t.
    The GPU top-p kernel (filter.hip) uses this rule."""
    out = []
    for v in sorted(set(p.tolist()), reverse=True):
        mem = [i for i in range(len(p)) if p[i] == v]
        gt = np.concatenate([[0], np.cumsum(p > v)])
        cnt = [int(gt[i]) for i in mem]
        R = []
        for t, i in enumerate(mem):
            R.append(i)
            g = (cnt[t + 1] if t + 1 < len(mem) else int(gt[-1])) - cnt[t]
            g %= len(R)
            R = R[g:] + R[:g]
        out.extend(R)
    return out


@pytest.mark.parametrize("V,levels", [(12, 3), (40, 4), (200, 6), (1000, 40)])
def test_top_p_tie_rule_matches_selection_sort(oracle, rng, V, levels):
    for _ in range(30):
        x = rng.integers(0, levels, V).astype(np.float32)
        probs = np.zeros(V, np.float32)
        idx = np.zeros(V, np.int32)
        cum = C.c_float()
        oracle.orc_top_p_sorted(ptr(x), V, 2.0, ptr(probs), ptr(idx), C.byref(cum))
        # the rule applied to the (index-order) probabilities
        pi = np.zeros(V, np.float32)
        pi[idx] = probs
        assert _tie_rule_order(pi) == idx.tolist()


def test_ulp_count_identities_of_the_exact_sum_walk():
    """The exact ordered sum's walk works on binary32 bit patterns (eos.hpp:
    binade_bits, parity_bits, add_ulps): inside binade b (ulp u_b) the bits
    of a non-negative value are its ulp count plus a constant, so s + q u_b
    is the bit pattern plus q, the count's parity is the low bit, and the
    binade is the exponent field minus 127 (-127: zero and subnormals).
    Checked here against real fp32 additions (numpy) over every binade:
    running sums of values that keep s inside one binade, each addition's
    ulp increment rounded as the hardware does (ties to even), land exactly
    on bits(s0) + sum of increments."""
    rng = np.random.default_rng(5)
    for b in range(-127, 128):
        ub = 2.0 ** (b - 23) if b > -127 else 2.0 ** -149
        lo = 2.0 ** b if b > -127 else 0.0
        hi = 2.0 ** (b + 1) if b > -127 else 2.0 ** -126
        for _ in range(20):
            start = int(rng.integers(0, 1 << 22))
            bits0 = ((b + 127) << 23 | start) if b > -127 else start
            s = np.array([bits0], np.uint32).view(np.float32)[0]
            assert lo <= float(s) < hi
            # binade from the exponent field; parity = low bit of the count
            assert (int(bits0) >> 23) - 127 == b
            n0 = float(s) / ub
            assert n0 == int(n0) and int(n0) & 1 == bits0 & 1
            # a run of additions that stays in the binade: values on the
            # half-ulp grid (ties included) below 4 ulps each; binary32 has no
            # half ulp below 2^-149, so binades -127 and -126 take whole ulps
            cnt = bits0
            cur = s
            halves = rng.integers(0, 8, 40)
            if b <= -126:
                halves &= ~1
            for h in halves:
                x = np.float32(h * ub / 2)
                nxt = np.float32(cur + x)
                if float(nxt) >= hi:
                    break
                f, half = divmod(int(h), 2)
                n = int(float(cur) / ub)
                inc = f + ((n + f) & 1) if half else f
                cnt += inc
                cur = nxt
                assert np.array([cnt], np.uint32).view(np.float32)[0] == cur
                assert float(cur) == float(s) + (cnt - bits0) * ub
    # +inf and NaN lie in no binade (exponent field 255)
    assert (int(np.array([np.inf], np.float32).view(np.uint32)[0]) >> 23) == 255
