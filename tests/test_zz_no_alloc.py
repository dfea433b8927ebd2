"""GPU: the allocation-free verify entry point (cgx_verify_chain_batch_dev_noalloc)
against the allocating one (cgx_verify_chain_batch_dev) through the C ABI.

Two calls in a row, the second smaller than the first (the static workspace
keeps the first call's contents), must give the allocating entry point's
tokens, accepted counts and acceptance ratios bit for bit; calls beyond the
static maximum, and filtered calls, are refused with an error.
"""
from __future__ import annotations

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error

pytestmark = pytest.mark.gpu


def _inputs(gpu, rng, batch, gamma, V):
    t = rng.normal(0, 2, (batch, gamma + 1, V)).astype(np.float32)
    d = (t[:, :gamma] + rng.normal(0, 0.5, (batch, gamma, V))).astype(np.float32)
    x = np.argmax(d, axis=2).astype(np.int32)
    x[:, 1] = rng.integers(0, V, batch)                  # some rejects
    u = rng.random((batch, gamma + 1), dtype=np.float32)
    return [DeviceArray.from_numpy(gpu, a) for a in (t, d, x, u)]


def _run(gpu, fn, args, batch, gamma, T, with_ap=True):
    """(tokens, counts, ratios or None); without ratios the pipeline takes
    the certified decisions."""
    out = DeviceArray(gpu, batch * (gamma + 1) * 4)
    n = DeviceArray(gpu, batch * 4)
    ap = DeviceArray(gpu, batch * gamma * 4) if with_ap else None
    t, d, x, u = args
    V = t.nbytes // 4 // (batch * (gamma + 1))
    rc = fn(t.ptr, d.ptr, x.ptr, u.ptr, batch, gamma, V, T, 0, 1.0, out.ptr, n.ptr,
            ap.ptr if ap else None)
    assert rc == 0, last_error(gpu)
    assert gpu.cgx_synchronize() == 0, last_error(gpu)
    res = (out.numpy(np.int32, (batch, gamma + 1)), n.numpy(np.int32, (batch,)),
           ap.numpy(np.float32, (batch, gamma)) if ap else None)
    for a in (out, n, ap):
        if a:
            a.free()
    return res


@pytest.mark.parametrize("T", [1.0, 0.7])
def test_noalloc_matches_allocating_entry(gpu, T):
    rng = np.random.default_rng(17)
    for batch, gamma, V in ((8, 4, 32000), (3, 2, 20011)):   # second call smaller
        args = _inputs(gpu, rng, batch, gamma, V)
        got = _run(gpu, gpu.cgx_verify_chain_batch_dev_noalloc, args, batch, gamma, T)
        exp = _run(gpu, gpu.cgx_verify_chain_batch_dev, args, batch, gamma, T)
        np.testing.assert_array_equal(got[0], exp[0])
        np.testing.assert_array_equal(got[1], exp[1])
        np.testing.assert_array_equal(got[2].view(np.uint32), exp[2].view(np.uint32))
        old = gpu.cgx_verify_lean_min_blocks(0)     # certified decisions at this size
        lean = _run(gpu, gpu.cgx_verify_chain_batch_dev_noalloc, args, batch, gamma, T, False)
        gpu.cgx_verify_lean_min_blocks(old)
        np.testing.assert_array_equal(lean[0], exp[0])
        np.testing.assert_array_equal(lean[1], exp[1])
        assert 0 < got[1].sum() < batch * gamma or batch == 3
        for a in args:
            a.free()


def test_noalloc_refuses_what_it_cannot_hold(gpu):
    tiny = DeviceArray(gpu, 4096)
    p = tiny.ptr
    # 64 chains at V = 128256 need far more than the static 32 MiB
    assert gpu.cgx_verify_chain_batch_dev_noalloc(p, p, p, p, 64, 4, 128256, 1.0, 0, 1.0,
                                                  p, p, p) == -1
    assert "static maximum" in last_error(gpu)
    gpu.cgx_clear_error()
    assert gpu.cgx_verify_chain_batch_dev_noalloc(p, p, p, p, 1, 4, 1000, 1.0, 50, 1.0,
                                                  p, p, p) == -1
    assert "top-k" in last_error(gpu)
    gpu.cgx_clear_error()
    tiny.free()
