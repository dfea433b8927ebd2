"""GPU parity of the chunk-parallel verify pipeline (verify.hip) against the
oracle: accept ratios bit-exact, accepted counts and emitted tokens equal.
The draws are placed on and next to the CDF steps of the row that is
searched (bonus: softmax of target row gamma; correction: residual
max(0, p - q) of the first rejected pair), where a one-ulp error in any
running sum changes the token.  Reference: src/inference/speculative.c:49-172.
"""
from __future__ import annotations

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error
from oracle_lib import ptr

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _certified_at_every_size(gpu):
    """Calls without accept_prob take the certified decisions at every size
    (by default only large calls do)."""
    old = gpu.cgx_verify_lean_min_blocks(0)
    yield
    gpu.cgx_verify_lean_min_blocks(old)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _probs(oracle, x, T):
    x = np.ascontiguousarray(x, np.float32)
    p = np.zeros_like(x)
    oracle.orc_temperature_probs(ptr(x), x.size, T, ptr(p))
    return p


def _run(gpu, oracle, target, draft, toks, u, gamma, V, T):
    out_g = np.zeros(gamma + 1, np.int32)
    ap_g = np.zeros(gamma, np.float32)
    n_g = gpu.cgx_verify_chain(target.ctypes.data, draft.ctypes.data, toks.ctypes.data,
                               u.ctypes.data, gamma, V, T, 0, 1.0, out_g.ctypes.data,
                               ap_g.ctypes.data)
    assert n_g >= 0, last_error(gpu)
    out_o = np.zeros(gamma + 1, np.int32)
    ap_o = np.zeros(gamma, np.float32)
    n_o = oracle.orc_verify_chain(ptr(target), ptr(draft), ptr(toks), ptr(u), gamma, V, T, 0,
                                  1.0, ptr(out_o), ptr(ap_o))
    np.testing.assert_array_equal(_bits(ap_g), _bits(ap_o))
    assert n_g == n_o, (n_g, n_o)
    np.testing.assert_array_equal(out_g[:n_g + 1], out_o[:n_o + 1])
    # without the ratios: certified decisions, the same tokens
    out_l = np.zeros(gamma + 1, np.int32)
    n_l = gpu.cgx_verify_chain(target.ctypes.data, draft.ctypes.data, toks.ctypes.data,
                               u.ctypes.data, gamma, V, T, 0, 1.0, out_l.ctypes.data, None)
    assert n_l == n_o, (n_l, n_o)
    np.testing.assert_array_equal(out_l[:n_l + 1], out_o[:n_o + 1])
    return n_g, out_g


def _step_draws(cdf, total, rng, n=6, scale=None):
    """Draws u whose threshold (u, or fl(u * total) when scale) sits on, just
    below and just above CDF steps."""
    us = []
    idx = rng.integers(0, cdf.size, n)
    for i in idx:
        c = np.float32(cdf[i])
        for v in (c, np.nextafter(c, np.float32(0)), np.nextafter(c, np.float32(np.inf))):
            if scale:
                v = np.float32(v / total)
            us.append(np.float32(min(max(v, 0.0), 0.99999)))
    return us


def _inputs(rng, V, gamma, spread=2.0):
    target = rng.normal(0, spread, (gamma + 1, V)).astype(np.float32)
    draft = rng.normal(0, spread, (gamma, V)).astype(np.float32)
    toks = rng.integers(0, V, gamma).astype(np.int32)
    return target, draft, toks


@pytest.mark.parametrize("V", [1, 7, 4095, 4096, 4097, 12289, 32000, 128256])
def test_bonus_draws_on_cdf_steps(gpu, oracle, V):
    # every draft token accepted (u = 0 < a), the bonus drawn from target row gamma
    rng = np.random.default_rng(V)
    gamma, T = 3, 1.0
    target, draft, toks = _inputs(rng, V, gamma)
    draft[:] = target[:gamma]
    p = _probs(oracle, target[gamma], T)
    cdf = np.add.accumulate(p, dtype=np.float32)
    for uu in _step_draws(cdf, None, rng) + [np.float32(0.0), np.float32(0.5)]:
        u = np.zeros(gamma + 1, np.float32)
        u[gamma] = uu
        n, _ = _run(gpu, oracle, target, draft, toks, u, gamma, V, T)
        assert n == gamma


@pytest.mark.parametrize("V,T", [(50, 1.0), (4096, 1.0), (32000, 1.0), (32000, 0.7),
                                 (70001, 1.3), (128256, 1.0)])
def test_correction_draws_on_residual_steps(gpu, oracle, V, T):
    # reject at position 0 (u[0] just below 1), correction from the residual
    # of pair 0 with draws on its CDF steps
    rng = np.random.default_rng(V + int(T * 10))
    gamma = 4
    target, draft, toks = _inputs(rng, V, gamma)
    p = _probs(oracle, target[0], T)
    q = _probs(oracle, draft[0], T)
    toks[0] = int(np.argmax(q - p))               # p/q < 1: u[0] near 1 rejects
    r = np.maximum(np.float32(0), p - q)
    cdf = np.add.accumulate(r, dtype=np.float32)
    R = cdf[-1]
    draws = _step_draws(cdf, R, rng, scale=True) + [np.float32(0.0), np.float32(0.75)]
    for uu in draws:
        u = rng.uniform(0, 1, gamma + 1).astype(np.float32)
        u[0] = np.float32(0.999999)
        u[1] = uu
        _run(gpu, oracle, target, draft, toks, u, gamma, V, T)


@pytest.mark.parametrize("V", [33, 5000, 32000])
def test_masked_and_out_of_range_tokens(gpu, oracle, V):
    rng = np.random.default_rng(3 * V)
    gamma, T = 5, 1.0
    for rep in range(4):
        target, draft, toks = _inputs(rng, V, gamma)
        # masked vocabulary entries (-inf logits), some drafted tokens masked
        mask = rng.uniform(0, 1, V) < 0.3
        target[:, mask] = -np.inf
        draft[:, mask[::-1]] = -np.inf
        toks[2] = int(np.flatnonzero(mask)[0]) if mask.any() else 0
        u = rng.uniform(0, 1, gamma + 1).astype(np.float32)
        u[:rep] = 0.0
        _run(gpu, oracle, target, draft, toks, u, gamma, V, T)


def test_out_of_range_tokens_are_rejected(gpu, oracle):
    # the reference reads outside the row for such a token (undefined); here
    # its acceptance ratio is 0, so it is rejected and never emitted
    rng = np.random.default_rng(8)
    V, gamma, T = 5000, 4, 1.0
    for bad, pos in ((-1, 0), (V, 2), (2**31 - 1, 3)):
        target, draft, toks = _inputs(rng, V, gamma)
        draft[:] = target[:gamma]                  # in-range tokens: ratio 1
        toks[pos] = bad
        u = np.zeros(gamma + 1, np.float32)
        out = np.zeros(gamma + 1, np.int32)
        ap = np.zeros(gamma, np.float32)
        n = gpu.cgx_verify_chain(target.ctypes.data, draft.ctypes.data, toks.ctypes.data,
                                 u.ctypes.data, gamma, V, T, 0, 1.0, out.ctypes.data,
                                 ap.ctypes.data)
        assert n == pos, (bad, pos, n)
        assert ap[pos] == 0.0
        assert (out[:pos] == toks[:pos]).all() and 0 <= out[pos] < V


def test_spiky_and_tied_rows(gpu, oracle):
    # one dominant logit (the row sum jumps through many binades in a chunk),
    # ties at the maximum, and a grid of repeated values
    rng = np.random.default_rng(11)
    V, gamma, T = 20000, 4, 1.0
    for rep in range(5):
        target, draft, toks = _inputs(rng, V, gamma, spread=[0.1, 2.0, 8.0, 20.0, 2.0][rep])
        target[:, rng.integers(0, V, 3)] = 40.0
        if rep == 4:
            target = (rng.integers(-30, 1, target.shape) / 2.0).astype(np.float32)
            draft = (rng.integers(-30, 1, draft.shape) / 2.0).astype(np.float32)
        u = rng.uniform(0, 1, gamma + 1).astype(np.float32)
        _run(gpu, oracle, target, draft, toks, u, gamma, V, T)


@pytest.mark.parametrize("shift", [1e-6, 1e-3, 0.5])
def test_near_identical_rows_small_residual(gpu, oracle, shift):
    # draft == target except a raised logit at the drafted token: the token is
    # rejected and the residual mass is tiny (below 1e-10 for the smallest
    # shift: cg_sample_corrected then samples softmax(p))
    rng = np.random.default_rng(5)
    V, gamma, T = 3000, 2, 1.0
    target, draft, toks = _inputs(rng, V, gamma)
    draft[:] = target[:gamma]
    draft[0, toks[0]] += np.float32(shift)
    for u1 in (0.3, 0.7, 0.0):
        u = np.array([0.999999, u1, 0.5], np.float32)
        _run(gpu, oracle, target, draft, toks, u, gamma, V, T)


def test_batch_matches_single_chains(gpu, oracle):
    rng = np.random.default_rng(21)
    B, V, gamma, T = 9, 9000, 4, 1.0
    tg = rng.normal(0, 2, (B, gamma + 1, V)).astype(np.float32)
    df = (tg[:, :gamma] + rng.normal(0, 0.5, (B, gamma, V))).astype(np.float32)
    tk = rng.integers(0, V, (B, gamma)).astype(np.int32)
    uu = rng.uniform(0, 1, (B, gamma + 1)).astype(np.float32)
    uu[::3, :gamma] = 0.0
    dt, dd, dk, du = (DeviceArray.from_numpy(gpu, a) for a in (tg, df, tk, uu))
    dout = DeviceArray(gpu, B * (gamma + 1) * 4)
    dn = DeviceArray(gpu, B * 4)
    dap = DeviceArray(gpu, B * gamma * 4)
    assert gpu.cgx_verify_chain_batch_dev(dt.ptr, dd.ptr, dk.ptr, du.ptr, B, gamma, V, T, 0,
                                          1.0, dout.ptr, dn.ptr, dap.ptr) == 0, last_error(gpu)
    gpu.cgx_synchronize()
    out = dout.numpy(np.int32, (B, gamma + 1))
    n = dn.numpy(np.int32, (B,))
    ap = dap.numpy(np.float32, (B, gamma))
    for c in range(B):
        out_o = np.zeros(gamma + 1, np.int32)
        ap_o = np.zeros(gamma, np.float32)
        n_o = oracle.orc_verify_chain(ptr(tg[c]), ptr(df[c]), ptr(tk[c]), ptr(uu[c]), gamma, V,
                                      T, 0, 1.0, ptr(out_o), ptr(ap_o))
        assert n[c] == n_o
        np.testing.assert_array_equal(out[c, :n_o + 1], out_o[:n_o + 1])
        assert (out[c, n_o + 1:] == -1).all()
        np.testing.assert_array_equal(_bits(ap[c]), _bits(ap_o))


def _batch(gpu, tg, df, tk, uu, T, with_ap):
    B, g1, V = tg.shape
    gamma = g1 - 1
    args = [DeviceArray.from_numpy(gpu, a) for a in (tg, df, tk, uu)]
    dout = DeviceArray(gpu, B * (gamma + 1) * 4)
    dn = DeviceArray(gpu, B * 4)
    dap = DeviceArray(gpu, B * gamma * 4) if with_ap else None
    assert gpu.cgx_verify_chain_batch_dev(*(a.ptr for a in args), B, gamma, V, T, 0, 1.0,
                                          dout.ptr, dn.ptr, dap.ptr if dap else None) == 0, \
        last_error(gpu)
    assert gpu.cgx_synchronize() == 0, last_error(gpu)
    res = (dout.numpy(np.int32, (B, gamma + 1)), dn.numpy(np.int32, (B,)),
           dap.numpy(np.float32, (B, gamma)) if dap else None)
    for a in args + [dout, dn] + ([dap] if dap else []):
        a.free()
    return res


@pytest.mark.parametrize("V", [4097, 32000, 128256])
def test_certified_decisions_on_ratio_boundaries(gpu, oracle, V):
    """Without accept_prob the pipeline settles accept tests from bounds of
    the row sums and sums exactly only the rows the outcome still needs.
    Draws on, one ulp either side of, and at small relative offsets from
    each chain's exact ratio at one position (earlier positions accepted)
    leave that test open; the tokens and counts must equal those taken with
    every ratio exact, and the oracle's."""
    rng = np.random.default_rng(V + 1)
    B, gamma, T = 12, 4, 1.0
    tg = rng.normal(0, 2, (B, gamma + 1, V)).astype(np.float32)
    df = (tg[:, :gamma] + rng.normal(0, 0.3, (B, gamma, V))).astype(np.float32)
    tk = rng.integers(0, V, (B, gamma)).astype(np.int32)
    uu = rng.uniform(0, 1, (B, gamma + 1)).astype(np.float32)
    _, _, ap = _batch(gpu, tg, df, tk, uu, T, True)
    f32 = np.float32
    offsets = [lambda a: a, lambda a: np.nextafter(a, f32(0)), lambda a: np.nextafter(a, f32(2)),
               lambda a: f32(a * f32(1 - 1e-4)), lambda a: f32(a * f32(1 + 1e-4)),
               lambda a: f32(a * f32(1 - 3e-3)), lambda a: f32(a * f32(1 + 3e-3))]
    for rep in range(3):
        u = rng.uniform(0, 1, (B, gamma + 1)).astype(np.float32)
        for c in range(B):
            pos = (c + rep) % gamma
            u[c, :pos] = 0.0
            u[c, pos] = min(offsets[(c + 5 * rep) % len(offsets)](ap[c, pos]), f32(1.0))
        out_e, n_e, _ = _batch(gpu, tg, df, tk, u, T, True)
        out_l, n_l, _ = _batch(gpu, tg, df, tk, u, T, False)
        np.testing.assert_array_equal(n_l, n_e)
        np.testing.assert_array_equal(out_l, out_e)
        for c in range(B):
            out_o = np.zeros(gamma + 1, np.int32)
            ap_o = np.zeros(gamma, np.float32)
            n_o = oracle.orc_verify_chain(ptr(tg[c]), ptr(df[c]), ptr(tk[c]), ptr(u[c]), gamma,
                                          V, T, 0, 1.0, ptr(out_o), ptr(ap_o))
            assert n_l[c] == n_o, (rep, c, n_l[c], n_o)
            np.testing.assert_array_equal(out_l[c, :n_o + 1], out_o[:n_o + 1])
