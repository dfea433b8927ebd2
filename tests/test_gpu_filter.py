"""GPU parity of the top-k / top-p samplers, the filtered distributions and
the filtered chain verification against the oracle: bit-exact tokens,
accept probabilities and distributions (the oracle's top-p runs the
reference's literal O(V^2) selection sort, so tie order is checked too).
Reference: src/inference/speculative.c:54-172.
"""
from __future__ import annotations

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error
from oracle_lib import LCG, ptr

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def logits_case(rng, V, kind):
    if kind == "normal":
        return rng.normal(0, 2, V).astype(np.float32)
    if kind == "ties":                      # a handful of distinct values
        return rng.integers(-3, 3, V).astype(np.float32)
    if kind == "flat":                      # near-uniform, fp32 probability ties
        return rng.normal(0, 0.01, V).astype(np.float32)
    if kind == "peaked":                    # a few tokens hold almost all the mass
        return rng.normal(0, 8, V).astype(np.float32)
    if kind == "spread":                    # the cutoff falls deep in the sorted row
        return rng.normal(0, 1, V).astype(np.float32)
    if kind == "halves":
        return (np.round(rng.normal(0, 2, V) * 2) / 2).astype(np.float32)
    if kind == "floor":                     # most values at/below -1e30
        x = np.full(V, -1e30, np.float32)
        x[rng.integers(0, V, 7)] = rng.normal(0, 1, 7).astype(np.float32)
        x[3] = -np.inf
        x[5] = -0.0
        x[6] = 0.0
        return x
    raise ValueError(kind)


TOPK_CASES = [(32000, 50, "normal"), (128256, 50, "normal"), (1000, 1, "ties"),
              (5000, 4096, "halves"), (2000, 300, "ties"), (64, 20, "floor"),
              (32000, 50, "flat"), (100, 99, "normal"),
              # rows of 16384 values and more gather their candidates over many
              # workgroups: a k-th largest bin too large for the list (ties) falls
              # back to the single-workgroup select; a large k; a floor-heavy row
              (40000, 3000, "ties"), (70000, 4096, "normal"), (20000, 7, "floor"),
              (16384, 1000, "halves")]


@pytest.mark.parametrize("V,k,kind", TOPK_CASES)
def test_sample_top_k_bitexact(gpu, oracle, rng, V, k, kind):
    print(f"top-k V={V} k={k} {kind}", flush=True)
    for trial in range(6):
        x = logits_case(rng, V, kind)
        for u in (float(rng.uniform()), 0.0, 0.9999):
            got = gpu.cgx_sample_top_k_u(x.ctypes.data, V, k, u)
            assert got >= 0, last_error(gpu)
            exp = oracle.orc_sample_top_k(ptr(x), V, k, u)
            assert got == exp, (trial, u, got, exp)


TOPP_CASES = [(1000, 0.9, "ties"), (1000, 0.5, "halves"), (3000, 0.9, "flat"),
              (2000, 1.0, "normal"), (2000, 0.0, "normal"), (500, 0.95, "ties"),
              (32000, 0.9, "normal"), (32000, 0.9, "flat"),
              # the summed prefix of the sorted row: cut after a few tokens, deep in
              # the row, and top_p close to 1 (the running sum near the binade at 1)
              (8000, 0.9, "peaked"), (8000, 0.3, "peaked"), (8000, 0.9, "spread"),
              (8000, 0.999, "normal"), (8000, 0.99999, "peaked"),
              # full-size rows: long runs of ties, the largest row the
              # probabilities hold in registers (32768), a cut deep in a wide row
              (32000, 0.9, "ties"), (32768, 0.5, "halves"), (32768, 0.9, "normal"),
              (32000, 0.99, "spread")]


@pytest.mark.parametrize("V,p,kind", TOPP_CASES)
def test_sample_top_p_bitexact(gpu, oracle, rng, V, p, kind):
    print(f"top-p V={V} p={p} {kind}", flush=True)
    trials = 2 if V > 10000 else 8
    for trial in range(trials):
        x = logits_case(rng, V, kind)
        for u in (float(rng.uniform()), float(rng.uniform()), 0.0):
            got = gpu.cgx_sample_top_p_u(x.ctypes.data, V, p, u)
            assert got >= 0, last_error(gpu)
            exp = oracle.orc_sample_top_p(ptr(x), V, p, u)
            assert got == exp, (trial, u, got, exp)


SORT_CASES = [(1, 1, "full"), (3, 100, "dups"), (2, 4096, "full"), (2, 4097, "dups"),
              (5, 32000, "probs"), (2, 32768, "full"), (1, 32767, "dups"),
              (4, 40000, "probs"), (1, 128256, "probs"), (2, 70001, "dups")]


@pytest.mark.parametrize("rows,n,kind", SORT_CASES)
def test_row_sort_matches_numpy(gpu, rng, rows, n, kind):
    # the multi-workgroup radix sort of rows (rowsort.hip): keys and the
    # payload of a stable sort, both directions
    print(f"row sort rows={rows} n={n} {kind}", flush=True)
    if kind == "full":
        keys = rng.integers(0, 2**32, (rows, n), dtype=np.uint64).astype(np.uint32)
    elif kind == "dups":
        keys = rng.integers(0, 40, (rows, n)).astype(np.uint32) * np.uint32(0x01010101)
    else:
        x = rng.normal(0, 2, (rows, n))
        keys = (np.exp(x - x.max()) / np.exp(x - x.max()).sum()).astype(np.float32).view(np.uint32)
    dk = DeviceArray.from_numpy(gpu, keys)
    pay = rng.integers(0, 2**31, (rows, n)).astype(np.uint32)
    dp = DeviceArray.from_numpy(gpu, pay)
    ok_, op_ = DeviceArray(gpu, keys.nbytes), DeviceArray(gpu, keys.nbytes)
    for desc in (1, 0):
        order = np.argsort(-keys.astype(np.int64) if desc else keys, axis=1, kind="stable")
        for payload in (None, dp):
            rc = gpu.cgx_sort_rows_dev(dk.ptr, payload.ptr if payload else None, rows, n, desc,
                                       ok_.ptr, op_.ptr)
            assert rc == 0, last_error(gpu)
            np.testing.assert_array_equal(ok_.numpy(np.uint32, (rows, n)),
                                          np.take_along_axis(keys, order, 1))
            exp_pay = order if payload is None else np.take_along_axis(pay, order, 1)
            np.testing.assert_array_equal(op_.numpy(np.uint32, (rows, n)), exp_pay)
        # keys only
        rc = gpu.cgx_sort_rows_dev(dk.ptr, None, rows, n, desc, ok_.ptr, None)
        assert rc == 0, last_error(gpu)
        np.testing.assert_array_equal(ok_.numpy(np.uint32, (rows, n)),
                                      np.take_along_axis(keys, order, 1))
    for a in (dk, dp, ok_, op_):
        a.free()


@pytest.mark.parametrize("V,p,kind", [(40000, 0.9, "flat"), (40000, 0.7, "ties"),
                                      (40000, 0.95, "normal")])
def test_sample_top_p_beyond_lds_sort(gpu, oracle, rng, V, p, kind):
    # rows longer than the LDS sort's 32768 take the multi-workgroup sort
    print(f"top-p V={V} p={p} {kind}", flush=True)
    x = logits_case(rng, V, kind)
    for u in (float(rng.uniform()), 0.0):
        got = gpu.cgx_sample_top_p_u(x.ctypes.data, V, p, u)
        assert got >= 0, last_error(gpu)
        assert got == oracle.orc_sample_top_p(ptr(x), V, p, u), u


def test_top_p_7b_vocabulary(gpu, oracle, rng):
    # V = 128256 (config 5's vocabulary), near-uniform logits: the cutoff
    # falls deep in the sorted row and fp32 ties are everywhere.  One O(V^2)
    # oracle sort gives the sorted probabilities, indices and cutoff; the
    # draws and the distribution follow from them by the reference's scan
    # (speculative.c:102-115).
    V, p = 128256, 0.9
    x = logits_case(rng, V, "flat")
    sp = np.zeros(V, np.float32)
    si = np.zeros(V, np.int32)
    import ctypes as C
    mass = C.c_float(0)
    cut = oracle.orc_top_p_sorted(ptr(x), V, p, ptr(sp), ptr(si), C.byref(mass))
    assert cut > V // 2
    cum = np.add.accumulate(sp[:cut], dtype=np.float32)
    for u in (0.0, 0.3141, 0.9999):
        r = np.float32(u) * np.float32(mass.value)
        hit = np.flatnonzero(r < cum)
        exp = int(si[hit[0]]) if hit.size else int(si[0])
        got = gpu.cgx_sample_top_p_u(x.ctypes.data, V, p, u)
        assert got == exp, (u, got, exp, last_error(gpu))
    got = np.full(V, 7.0, np.float32)
    assert gpu.cgx_filtered_dist(x.ctypes.data, V, 1.0, 0, p, got.ctypes.data) == 0, \
        last_error(gpu)
    dist = np.zeros(V, np.float32)
    dist[si[:cut]] = sp[:cut] / np.float32(mass.value)
    np.testing.assert_array_equal(_bits(got), _bits(dist))


def test_top_p_tie_order_dense_draws(gpu, oracle, rng):
    # many draws on one row with large tie groups: every rank inside the
    # groups is exercised against the literal sort
    V = 400
    x = rng.integers(0, 4, V).astype(np.float32)
    for u in np.linspace(0.0, 0.999, 200, dtype=np.float32):
        got = gpu.cgx_sample_top_p_u(x.ctypes.data, V, 0.97, float(u))
        exp = oracle.orc_sample_top_p(ptr(x), V, 0.97, float(u))
        assert got == exp, (float(u), got, exp)


FILTER_CASES = [
    # V, T, top_k, top_p, kind
    (32000, 0.8, 0, 0.9, "normal"),
    (4000, 0.8, 0, 0.9, "ties"),
    (4000, 1.0, 0, 0.5, "flat"),
    (40000, 0.8, 0, 0.9, "ties"),
    (128256, 0.7, 50, 1.0, "normal"),
    (128256, 0.7, 50, 0.9, "normal"),
    (2000, 1.3, 300, 0.8, "halves"),
    (64, 1.0, 20, 1.0, "floor"),
    (8000, 1.0, 0, 0.999, "peaked"),
    (8000, 0.8, 0, 0.9, "spread"),
]


@pytest.mark.parametrize("V,T,k,p,kind", FILTER_CASES)
def test_filtered_dist_bitexact(gpu, oracle, rng, V, T, k, p, kind):
    print(f"dist V={V} T={T} k={k} p={p} {kind}", flush=True)
    x = logits_case(rng, V, kind)
    got = np.full(V, 7.0, np.float32)
    assert gpu.cgx_filtered_dist(x.ctypes.data, V, T, k, p, got.ctypes.data) == 0, \
        last_error(gpu)
    exp = np.zeros(V, np.float32)
    oracle.orc_filtered_dist(ptr(x), V, T, k, p, ptr(exp))
    np.testing.assert_array_equal(_bits(got), _bits(exp))


def verify_inputs(oracle, rng, V, gamma, T, k, p, close):
    target = rng.normal(0, 2, (gamma + 1, V)).astype(np.float32)
    draft = rng.normal(0, 2, (gamma, V)).astype(np.float32)
    if close:
        target[:gamma] = draft + rng.normal(0, 0.05, draft.shape).astype(np.float32)
    toks = np.zeros(gamma, np.int32)
    for i in range(gamma):
        row = np.ascontiguousarray(draft[i])
        toks[i] = oracle.orc_sample_filtered(ptr(row), V, T, k, p, float(rng.uniform()))
    u = rng.uniform(0, 1, gamma + 1).astype(np.float32)
    return target, draft, toks, u


@pytest.mark.parametrize("V,gamma,T,k,p,close", [
    (32000, 4, 0.8, 0, 0.9, True),          # config 3's sampler settings
    (4000, 4, 0.8, 0, 0.9, False),
    (128256, 4, 0.7, 50, 1.0, True),        # config 5's sampler settings
    (128256, 4, 0.7, 50, 1.0, False),
    (3000, 3, 1.0, 20, 0.8, True),
])
def test_filtered_verify_bitexact(gpu, oracle, rng, V, gamma, T, k, p, close):
    print(f"verify V={V} g={gamma} T={T} k={k} p={p} close={close}", flush=True)
    for rep in range(2):
        target, draft, toks, u = verify_inputs(oracle, rng, V, gamma, T, k, p, close)
        out_g = np.zeros(gamma + 1, np.int32)
        ap_g = np.zeros(gamma, np.float32)
        n_g = gpu.cgx_verify_chain(target.ctypes.data, draft.ctypes.data, toks.ctypes.data,
                                   u.ctypes.data, gamma, V, T, k, p, out_g.ctypes.data,
                                   ap_g.ctypes.data)
        assert n_g >= 0, last_error(gpu)
        out_o = np.zeros(gamma + 1, np.int32)
        ap_o = np.zeros(gamma, np.float32)
        n_o = oracle.orc_verify_chain(ptr(target), ptr(draft), ptr(toks), ptr(u), gamma, V,
                                      T, k, p, ptr(out_o), ptr(ap_o))
        np.testing.assert_array_equal(_bits(ap_g), _bits(ap_o))
        assert n_g == n_o
        np.testing.assert_array_equal(out_g[:n_g + 1], out_o[:n_o + 1])


def test_filtered_verify_batch_device(gpu, oracle, rng):
    B, V, gamma, T, k, p = 3, 2000, 4, 0.8, 40, 0.9
    ins = [verify_inputs(oracle, rng, V, gamma, T, k, p, b % 2 == 0) for b in range(B)]
    arrs = [np.stack([i[j] for i in ins]) for j in range(4)]
    dt, dd, dk, du = (DeviceArray.from_numpy(gpu, a) for a in arrs)
    dout = DeviceArray(gpu, B * (gamma + 1) * 4)
    dn = DeviceArray(gpu, B * 4)
    assert gpu.cgx_verify_chain_batch_dev(dt.ptr, dd.ptr, dk.ptr, du.ptr, B, gamma, V, T, k,
                                          p, dout.ptr, dn.ptr, None) == 0, last_error(gpu)
    gpu.cgx_synchronize()
    out = dout.numpy(np.int32, (B, gamma + 1))
    n = dn.numpy(np.int32, (B,))
    for b in range(B):
        o = np.zeros(gamma + 1, np.int32)
        tb, db, kb, ub = (np.ascontiguousarray(a[b]) for a in arrs)
        n_o = oracle.orc_verify_chain(ptr(tb), ptr(db), ptr(kb), ptr(ub), gamma, V, T, k, p,
                                      ptr(o), None)
        assert n[b] == n_o
        np.testing.assert_array_equal(out[b, :n_o + 1], o[:n_o + 1])
    for d in (dt, dd, dk, du, dout, dn):
        d.free()


def test_dropin_top_k_top_p_follow_reference_lcg(gpu, oracle, rng):
    gpu.cgx_lcg_seed(42)
    mirror = LCG(42)
    V = 1500
    for i in range(6):
        x = logits_case(rng, V, "ties" if i % 2 else "normal")
        got = gpu.cg_sample_top_k(x.ctypes.data, V, 30)
        assert got == oracle.orc_sample_top_k(ptr(x), V, 30, mirror.draw(oracle))
        got = gpu.cg_sample_top_p(x.ctypes.data, V, 0.9)
        assert got == oracle.orc_sample_top_p(ptr(x), V, 0.9, mirror.draw(oracle))
    # k >= V falls back to temperature sampling at T = 1 (speculative.c:123)
    x = logits_case(rng, V, "normal")
    got = gpu.cg_sample_top_k(x.ctypes.data, V, V)
    assert got == oracle.orc_sample_temperature(ptr(x), V, 1.0, mirror.draw(oracle))
    assert gpu.cgx_lcg_state() == mirror.state.value


def test_filter_limits_report_errors(gpu, rng):
    x = rng.normal(0, 1, 40000).astype(np.float32)
    gpu.cgx_clear_error()
    big = np.zeros(262145, np.float32)
    assert gpu.cgx_sample_top_p_u(big.ctypes.data, big.size, 0.9, 0.5) == -1
    assert "vocabulary size" in last_error(gpu)
    gpu.cgx_clear_error()
    assert gpu.cgx_sample_top_k_u(x.ctypes.data, 40000, 5000, 0.5) == -1
    assert "top-k" in last_error(gpu)
    gpu.cgx_clear_error()
    assert gpu.cgx_sample_top_k_u(x.ctypes.data, 40000, 0, 0.5) == -1
