"""GPU parity of typical sampling (cg_sample_typical, decision D16; declared
only in the reference, include/cg_speculative.h:186) against the oracle's
restatement (pinned in tests/test_typical_oracle.py): the binary64 log bit
for bit over every kind of float, tokens and dense distributions bit for bit
at vocabularies up to 128256, and the drop-in sampler's LCG draws.
"""
from __future__ import annotations

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error
from oracle_lib import LCG, ptr
from test_gpu_filter import logits_case

pytestmark = pytest.mark.gpu


def test_typ_log_bitexact(gpu, oracle, rng):
    x = np.concatenate([rng.random(100000, dtype=np.float32),
                        np.exp(rng.uniform(-103, 88, 100000)).astype(np.float32),
                        np.array([1.0, 2.0, 0.5, 1e-45, 1.4e-45, 3.4e38, 0.70710677,
                                  0.70710683, 1.4142135, 1.4142137], np.float32)])
    x = x[x > 0]
    dx = DeviceArray.from_numpy(gpu, x)
    dy = DeviceArray(gpu, x.size * 8)
    assert gpu.cgx_typ_log_dev(dx.ptr, dy.ptr, x.size) == 0, last_error(gpu)
    assert gpu.cgx_synchronize() == 0
    got = dy.numpy(np.float64, (x.size,))
    exp = np.array([oracle.orc_typ_log(float(v)) for v in x])
    np.testing.assert_array_equal(got.view(np.uint64), exp.view(np.uint64))


CASES = [(1000, 0.9, "normal"), (1000, 0.5, "ties"), (3000, 0.95, "flat"),
         (2000, 0.2, "halves"), (32000, 0.9, "normal"), (40000, 0.8, "ties"),
         (128256, 0.9, "normal"), (128256, 0.95, "flat"), (500, 1.0, "normal"),
         (64, 0.9, "floor")]


@pytest.mark.parametrize("V,tp,kind", CASES)
def test_typical_bitexact(gpu, oracle, rng, V, tp, kind):
    print(f"typical V={V} p={tp} {kind}", flush=True)
    x = logits_case(rng, V, kind)
    for u in (float(rng.uniform()), 0.0, 0.9999):
        got = gpu.cgx_sample_typical_u(x.ctypes.data, V, tp, u)
        assert got >= 0, last_error(gpu)
        assert got == oracle.orc_sample_typical(ptr(x), V, tp, u), u
    got = np.full(V, 7.0, np.float32)
    assert gpu.cgx_typical_dist(x.ctypes.data, V, tp, got.ctypes.data) == 0, last_error(gpu)
    exp = np.zeros(V, np.float32)
    oracle.orc_typical_dist(ptr(x), V, tp, ptr(exp))
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_dropin_typical_follows_reference_lcg(gpu, oracle, rng):
    V = 5000
    state = 12345
    gpu.cgx_lcg_seed(state)
    lcg = LCG(state)
    for _ in range(5):
        x = logits_case(rng, V, "normal")
        got = gpu.cg_sample_typical(x.ctypes.data, V, 0.9)
        assert got == oracle.orc_sample_typical(ptr(x), V, 0.9, lcg.draw(oracle))
    assert gpu.cgx_lcg_state() == lcg.state.value
