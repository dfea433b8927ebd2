"""GPU parity of the acceptance-sampling path (accept.hip) against the oracle:
token decisions and probability vectors bit-exact, on identical logits and
uniforms.  Reference: src/inference/speculative.c:49-172."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error
from oracle_lib import LCG, ptr

pytestmark = pytest.mark.gpu

LIBM = C.CDLL("libm.so.6")
LIBM.expf.restype = C.c_float
LIBM.expf.argtypes = [C.c_float]


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _host_expf_vec(x: np.ndarray) -> np.ndarray:
    # the host's glibc expf, value by value (the reference links libm)
    f = LIBM.expf
    return np.array([f(float(v)) for v in x], np.float32)


def test_exact_expf_matches_host_libm(gpu, rng):
    # a strided sweep over every binade of [-104, 0] plus specials
    bits = np.arange(0x80000000, 0xC2D00000, 997, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, -103.97, -104.5, -np.inf, 1.0, 88.7,
                                     88.73, -1e-30], np.float32),
                        rng.uniform(-20, 0, 20000).astype(np.float32)])
    dx = DeviceArray.from_numpy(gpu, x)
    dy = DeviceArray(gpu, x.nbytes)
    assert gpu.cgx_exact_expf_dev(dx.ptr, dy.ptr, x.size) == 0, last_error(gpu)
    y = dy.numpy(np.float32, x.shape)
    sample = np.arange(0, x.size, 7)           # libm via ctypes: check a subset
    ref = _host_expf_vec(x[sample])
    np.testing.assert_array_equal(_bits(y[sample]), _bits(ref))


def test_exp_fast_within_certified_bound(gpu):
    # every fp32 in [-87, 0]: the certified sampler paths fold approximate
    # exponentials and re-evaluate exactly only where 2^-20 relative error
    # could change a rounding, so the bound must hold everywhere
    out = DeviceArray.from_numpy(gpu, np.zeros(1, np.uint32))
    assert gpu.cgx_exp_fast_maxerr_dev(-87.0, 0.0, out.ptr) == 0, last_error(gpu)
    worst = out.numpy(np.uint32, (1,)).view(np.float32)[0]
    assert 0.0 < worst <= 2.0 ** -20, worst
    # and it is tight enough to be worth having: a few fp32 ulps
    assert worst < 2.0 ** -21


def test_exp_stat_within_certified_bound(gpu):
    # every fp32 in [-87, 0]: the acceptance pipeline's segment statistics
    # sum this exponential, and the guide's error bound charges it 2^-16
    # (with the other terms, 2^-15 of the rescaled sum); the measured worst
    # case must leave a factor 2 to that
    out = DeviceArray.from_numpy(gpu, np.zeros(1, np.uint32))
    assert gpu.cgx_exp_stat_maxerr_dev(-87.0, 0.0, out.ptr) == 0, last_error(gpu)
    worst = out.numpy(np.uint32, (1,)).view(np.float32)[0]
    assert 0.0 < worst <= 2.0 ** -17, worst


def _seq_sum(x: np.ndarray) -> np.float32:
    # left-to-right binary32 accumulation (np.add.accumulate is sequential)
    return np.add.accumulate(np.ascontiguousarray(x, np.float32), dtype=np.float32)[-1]


def _sum_cases(rng):
    yield "softmax32000", np.exp(rng.normal(0, 2, 32000) - 8).astype(np.float32)
    yield "uniform", rng.uniform(0, 1, 100000).astype(np.float32)
    yield "powers_of_two", (2.0 ** rng.integers(-30, 2, 50000)).astype(np.float32)
    yield "halves", (rng.integers(0, 8, 40000) / 2.0).astype(np.float32)
    yield "tiny_then_big", np.concatenate([np.full(5000, 1e-30), np.full(5000, 1.0),
                                          rng.uniform(0, 1e-8, 5000)]).astype(np.float32)
    yield "denormals", (rng.integers(0, 50, 40000) * 1e-45).astype(np.float32)
    yield "zeros", np.zeros(70000, np.float32)
    yield "one", np.array([0.3], np.float32)
    yield "chunk_edges", rng.uniform(0, 1, 32769).astype(np.float32)
    yield "vocab128256", np.exp(rng.normal(0, 2, 128256) - 9).astype(np.float32)
    yield "growing", (np.arange(1, 60001) * 1e-3).astype(np.float32)
    big = rng.uniform(0, 1, 64000).astype(np.float32)
    big[::1000] = 1e6
    yield "spikes", big


def test_ordered_sum_exact(gpu, rng):
    out = DeviceArray(gpu, 4)
    for name, x in _sum_cases(rng):
        dx = DeviceArray.from_numpy(gpu, x)
        assert gpu.cgx_ordered_sum_dev(dx.ptr, x.size, out.ptr) == 0, last_error(gpu)
        got = out.numpy(np.float32, (1,))[0]
        exp = _seq_sum(x)
        assert _bits(got) == _bits(exp), (name, got, exp)
        dx.free()


def _oracle_probs(oracle, x, T):
    p = np.zeros(x.size, np.float32)
    oracle.orc_temperature_probs(ptr(x), x.size, T, ptr(p))
    return p


@pytest.mark.parametrize("V", [1, 2, 64, 1000, 32000, 50257, 128256])
@pytest.mark.parametrize("T", [1.0, 0.7, 1.3])
def test_temperature_probs_bitexact(gpu, oracle, rng, V, T):
    x = rng.normal(0, 2, V).astype(np.float32)
    out = np.zeros(V, np.float32)
    assert gpu.cgx_filtered_dist(x.ctypes.data, V, T, 0, 1.0, out.ctypes.data) == 0, \
        last_error(gpu)
    np.testing.assert_array_equal(_bits(out), _bits(_oracle_probs(oracle, x, T)))


@pytest.mark.parametrize("V", [1, 3, 1000, 32000, 128256])
def test_sample_temperature_bitexact(gpu, oracle, rng, V):
    for trial in range(8):
        T = [1.0, 0.8, 0.7, 1.3, 1.0, 2.0, 1.0, 0.5][trial]
        x = rng.normal(0, 2, V).astype(np.float32)
        if trial == 4:
            x[rng.integers(0, V, min(V, 7))] = x.max()
        if trial >= 6:
            # few distinct logits on a coarse grid: repeated exponentials make
            # exact roundings and ties in the running sums common
            x = (rng.integers(-48, 1, V) / 4.0).astype(np.float32)
        p = _oracle_probs(oracle, x, T)
        cdf = np.add.accumulate(p, dtype=np.float32)
        us = list(rng.uniform(0, 1, 6).astype(np.float32))
        # uniforms exactly on and next to CDF steps, the LCG grid, and the ends
        for i in rng.integers(0, V, 4):
            c = cdf[i]
            us += [c, np.nextafter(c, np.float32(0)), np.nextafter(c, np.float32(2))]
        us += [np.float32(0.0), np.float32(0.9999), np.float32(0.5)]
        for u in us:
            u = np.float32(min(max(u, 0.0), 1.5))
            got = gpu.cgx_sample_temperature_u(x.ctypes.data, V, T, float(u))
            exp = oracle.orc_sample_temperature(ptr(x), V, T, float(u))
            assert got == exp, (V, T, float(u), got, exp, last_error(gpu))


@pytest.mark.parametrize("V", [3, 1000, 32000, 32768])
def test_certified_row_draw_matches_exact(gpu, oracle, rng, V):
    """The single-row draw decides from certified approximations first and
    runs the exact sums only where u lies within the bounds of a CDF step:
    the token equals the exact path's and the oracle's on diffuse rows, on
    peaked rows (which the approximations settle) and for uniforms on and
    next to the CDF steps (which they must leave to the exact sums)."""
    assert gpu.cgx_sample_row_certified(-1) == 1
    peaked_draws = peaked_fb = step_draws = step_fb = 0
    try:
        for trial, scale in enumerate([2.0, 20.0, 6.0, 40.0]):
            T = [1.0, 0.8, 1.3, 1.0][trial]
            x = rng.normal(0, scale, V).astype(np.float32)
            p = _oracle_probs(oracle, x, T)
            cdf = np.add.accumulate(p, dtype=np.float32)
            us = list(rng.uniform(0, 1, 12).astype(np.float32)) + [np.float32(0.0)]
            steps = []
            for i in rng.integers(0, V, 4):
                c = cdf[i]
                steps += [c, np.nextafter(c, np.float32(0)), np.nextafter(c, np.float32(2))]
            for j, u in enumerate(us + steps):
                exp = oracle.orc_sample_temperature(ptr(x), V, T, float(u))
                f0 = gpu.cgx_sample_row_fallbacks()
                got = gpu.cgx_sample_temperature_u(x.ctypes.data, V, T, float(u))
                fb = gpu.cgx_sample_row_fallbacks() - f0
                assert f0 >= 0 and fb in (0, 1), (f0, fb, last_error(gpu))
                assert got == exp, (V, T, scale, float(u), got, exp, last_error(gpu))
                gpu.cgx_sample_row_certified(0)
                try:
                    assert gpu.cgx_sample_temperature_u(x.ctypes.data, V, T, float(u)) == exp
                    assert gpu.cgx_sample_row_fallbacks() - f0 == fb   # off: not counted
                finally:
                    gpu.cgx_sample_row_certified(1)
                if scale >= 20.0 and j < len(us):
                    peaked_draws += 1
                    peaked_fb += fb
                if j >= len(us):
                    step_draws += 1
                    step_fb += fb
    finally:
        gpu.cgx_sample_row_certified(1)
    # a peaked row's steps are wide: most random uniforms are settled by the
    # bounds; a uniform within an ulp of a step cannot be (except at the last
    # steps, where V-1 is the token on both sides)
    if V > 3:
        assert peaked_fb < peaked_draws // 2, (peaked_fb, peaked_draws)
    assert step_fb > 0, (step_fb, step_draws)


@pytest.mark.parametrize("V", [1000, 32000, 50257])
def test_sample_temperature_dev_matches_oracle(gpu, oracle, rng, V):
    """The device-row draw (queued, no synchronisation) returns the oracle's
    token on a diffuse and a peaked row (rows above 32768 values: the
    pipeline)."""
    out = DeviceArray(gpu, 4)
    for scale in (2.0, 20.0):
        x = rng.normal(0, scale, V).astype(np.float32)
        dx = DeviceArray.from_numpy(gpu, x)
        for u in rng.uniform(0, 1, 6).astype(np.float32):
            assert gpu.cgx_sample_temperature_dev(dx.ptr, V, 1.0, float(u), out.ptr) == 0, \
                last_error(gpu)
            got = out.numpy(np.int32, (1,))[0]
            exp = oracle.orc_sample_temperature(ptr(x), V, 1.0, float(u))
            assert got == exp, (V, scale, float(u), got, exp)
        dx.free()
    out.free()


@pytest.mark.parametrize("V,ld_pad", [(1000, 0), (32000, 4000), (32768, 0), (50257, 7)])
def test_sample_temperature_rows_dev_matches_oracle(gpu, oracle, rng, V, ld_pad):
    """Draws from several device rows in one call (one workgroup per row up
    to 32768 values, the pipeline above) equal the oracle's row by row:
    diffuse and peaked rows, T = 1 and 0.8, uniforms on and next to a CDF
    step."""
    rows, ld = 6, V + ld_pad
    for T in (1.0, 0.8):
        x = np.zeros((rows, ld), np.float32)
        x[:, :V] = rng.normal(0, 2, (rows, V)) * np.array([2, 2, 10, 10, 1, 30])[:, None]
        u = rng.uniform(0, 1, rows).astype(np.float32)
        for r in (1, 3):
            p = _oracle_probs(oracle, np.ascontiguousarray(x[r, :V]), T)
            cdf = np.add.accumulate(p, dtype=np.float32)
            c = cdf[rng.integers(0, V)]
            u[r] = c if r == 1 else np.nextafter(c, np.float32(0))
        dx, du = DeviceArray.from_numpy(gpu, x), DeviceArray.from_numpy(gpu, u)
        out = DeviceArray(gpu, rows * 4)
        assert gpu.cgx_sample_temperature_rows_dev(dx.ptr, rows, V, T, du.ptr, out.ptr,
                                                   ld) == 0, last_error(gpu)
        got = out.numpy(np.int32, (rows,))
        for r in range(rows):
            row = np.ascontiguousarray(x[r, :V])
            exp = oracle.orc_sample_temperature(ptr(row), V, T, float(u[r]))
            assert got[r] == exp, (V, T, r, float(u[r]), got[r], exp)
        for a in (dx, du, out):
            a.free()


@pytest.mark.parametrize("V", [64, 1000, 32000])
def test_sample_corrected_bitexact(gpu, oracle, rng, V):
    for trial in range(8):
        lt = rng.normal(0, 2, V).astype(np.float32)
        ld = (lt + rng.normal(0, [0.3, 1.0, 2.0, 0.0][trial % 4], V)).astype(np.float32)
        p = _oracle_probs(oracle, lt, 1.0)
        q = _oracle_probs(oracle, ld, 1.0)
        if trial == 7:
            q = p.copy()                       # zero residual -> temperature fallback
        for u in rng.uniform(0, 1, 5).astype(np.float32):
            got = gpu.cgx_sample_corrected_u(q.ctypes.data, p.ctypes.data, V, float(u))
            exp = oracle.orc_sample_corrected(ptr(q), ptr(p), V, float(u))
            assert got == exp, (trial, float(u), got, exp, last_error(gpu))


def _config1_inputs(oracle, rng, V=32000, gamma=4, T=1.0):
    """target [5,V], draft [4,V] ~ N(0, 2^2); draft tokens
    drawn from the draft softmax with pre-drawn uniforms; uniforms U(0,1)."""
    target = rng.normal(0, 2, (gamma + 1, V)).astype(np.float32)
    draft = rng.normal(0, 2, (gamma, V)).astype(np.float32)
    toks = np.zeros(gamma, np.int32)
    for i in range(gamma):
        row = np.ascontiguousarray(draft[i])
        toks[i] = oracle.orc_sample_temperature(ptr(row), V, T, float(rng.uniform()))
    u = rng.uniform(0, 1, gamma + 1).astype(np.float32)
    return target, draft, toks, u


def _verify_both(gpu, oracle, target, draft, toks, u, gamma, V, T):
    out_g = np.zeros(gamma + 1, np.int32)
    ap_g = np.zeros(gamma, np.float32)
    n_g = gpu.cgx_verify_chain(target.ctypes.data, draft.ctypes.data, toks.ctypes.data,
                               u.ctypes.data, gamma, V, T, 0, 1.0, out_g.ctypes.data,
                               ap_g.ctypes.data)
    assert n_g >= 0, last_error(gpu)
    out_o = np.zeros(gamma + 1, np.int32)
    ap_o = np.zeros(gamma, np.float32)
    n_o = oracle.orc_verify_chain(ptr(target), ptr(draft), ptr(toks), ptr(u), gamma, V, T,
                                  0, 1.0, ptr(out_o), ptr(ap_o))
    return n_g, out_g, ap_g, n_o, out_o, ap_o


@pytest.mark.parametrize("seed", range(12))
def test_verify_chain_config1_bitexact(gpu, oracle, seed):
    rng = np.random.default_rng(1000 + seed)
    V, gamma, T = 32000, 4, 1.0
    target, draft, toks, u = _config1_inputs(oracle, rng, V, gamma, T)
    if seed % 3 == 1:
        # make acceptance likely: target close to draft
        target[:gamma] = draft + rng.normal(0, 0.1, draft.shape).astype(np.float32)
    n_g, out_g, ap_g, n_o, out_o, ap_o = _verify_both(gpu, oracle, target, draft, toks, u,
                                                      gamma, V, T)
    np.testing.assert_array_equal(_bits(ap_g), _bits(ap_o))
    assert n_g == n_o
    np.testing.assert_array_equal(out_g[:n_g + 1], out_o[:n_o + 1])


@pytest.mark.parametrize("V,gamma,T", [(1000, 1, 0.8), (5000, 8, 0.7), (128256, 4, 1.0)])
def test_verify_chain_shapes(gpu, oracle, V, gamma, T):
    rng = np.random.default_rng(V + gamma)
    for rep in range(3):
        target, draft, toks, u = _config1_inputs(oracle, rng, V, gamma, T)
        target[:gamma] = draft + rng.normal(0, 0.3 * rep, draft.shape).astype(np.float32)
        n_g, out_g, ap_g, n_o, out_o, ap_o = _verify_both(gpu, oracle, target, draft, toks,
                                                          u, gamma, V, T)
        np.testing.assert_array_equal(_bits(ap_g), _bits(ap_o))
        assert n_g == n_o
        np.testing.assert_array_equal(out_g[:n_g + 1], out_o[:n_o + 1])


@pytest.mark.parametrize("V", [1000, 32000])
def test_verify_chain_grid_logits(gpu, oracle, V):
    # logits on a coarse grid (repeated exponentials, exact roundings and ties
    # in the running sums of the certified single-round path)
    rng = np.random.default_rng(5 * V)
    gamma, T = 4, 1.0
    for rep in range(4):
        target, draft, toks, u = _config1_inputs(oracle, rng, V, gamma, T)
        draft = (rng.integers(-40, 1, draft.shape) / 4.0).astype(np.float32)
        target = (draft[[0, 1, 2, 3, 3]] + rng.integers(-2 * rep, 2 * rep + 1, target.shape)
                  / 4.0).astype(np.float32)
        for i in range(gamma):
            row = np.ascontiguousarray(draft[i])
            toks[i] = oracle.orc_sample_temperature(ptr(row), V, T, float(rng.uniform()))
        n_g, out_g, ap_g, n_o, out_o, ap_o = _verify_both(gpu, oracle, target, draft, toks,
                                                          u, gamma, V, T)
        np.testing.assert_array_equal(_bits(ap_g), _bits(ap_o))
        assert n_g == n_o
        np.testing.assert_array_equal(out_g[:n_g + 1], out_o[:n_o + 1])


def test_verify_chain_batch_device(gpu, oracle):
    rng = np.random.default_rng(77)
    B, V, gamma, T = 6, 4096, 4, 1.0
    ins = [_config1_inputs(oracle, rng, V, gamma, T) for _ in range(B)]
    tgt = np.stack([i[0] for i in ins])
    dft = np.stack([i[1] for i in ins])
    tok = np.stack([i[2] for i in ins])
    uu = np.stack([i[3] for i in ins])
    dt, dd, dk, du = (DeviceArray.from_numpy(gpu, a) for a in (tgt, dft, tok, uu))
    dout = DeviceArray(gpu, B * (gamma + 1) * 4)
    dn = DeviceArray(gpu, B * 4)
    assert gpu.cgx_verify_chain_batch_dev(dt.ptr, dd.ptr, dk.ptr, du.ptr, B, gamma, V, T, 0,
                                          1.0, dout.ptr, dn.ptr, None) == 0, last_error(gpu)
    gpu.cgx_synchronize()
    out = dout.numpy(np.int32, (B, gamma + 1))
    n = dn.numpy(np.int32, (B,))
    for b in range(B):
        o = np.zeros(gamma + 1, np.int32)
        tb, db, kb, ub = (np.ascontiguousarray(a[b]) for a in (tgt, dft, tok, uu))
        n_o = oracle.orc_verify_chain(ptr(tb), ptr(db), ptr(kb), ptr(ub), gamma, V, T,
                                      0, 1.0, ptr(o), None)
        assert n[b] == n_o
        np.testing.assert_array_equal(out[b, :n_o + 1], o[:n_o + 1])


def test_dropin_samplers_follow_reference_lcg(gpu, oracle, rng):
    # cg_sample_* draw from the reference's global LCG: same tokens as the
    # oracle fed with the mirrored stream
    gpu.cgx_lcg_seed(42)
    mirror = LCG(42)
    V = 2000
    for i in range(10):
        x = rng.normal(0, 2, V).astype(np.float32)
        got = gpu.cg_sample_temperature(x.ctypes.data, V, 1.0)
        exp = oracle.orc_sample_temperature(ptr(x), V, 1.0, mirror.draw(oracle))
        assert got == exp
    assert gpu.cgx_lcg_state() == mirror.state.value
