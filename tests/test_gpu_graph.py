"""GPU: the verify captured into a HIP graph (cgx_graph_*) and replayed.

The allocation-free verify (cgx_verify_chain_batch_dev_noalloc) is captured
once; each replay reads new logits and draws written to the same device
buffers between replays, with eager calls of the same entry point (the
same static workspace) in between.  Every replay must match, bit for bit,
an eager call on the same inputs: tokens, counts and, when asked for, the
acceptance ratios; once with every ratio and once tokens-only with the
certified decisions forced on.
"""
from __future__ import annotations

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error

pytestmark = pytest.mark.gpu


def _inputs(rng, B, gamma, V):
    t = rng.normal(0, 2, (B, gamma + 1, V)).astype(np.float32)
    d = (t[:, :gamma] + rng.normal(0, 0.5, (B, gamma, V))).astype(np.float32)
    x = np.argmax(d, axis=2).astype(np.int32)
    x[:, 1] = rng.integers(0, V, B)                      # some rejects
    u = rng.random((B, gamma + 1), dtype=np.float32)
    return t, d, x, u


@pytest.mark.parametrize("ratios", [True, False])
def test_graph_replays_match_eager_verify(gpu, ratios):
    print(f"graph replay of the verify, ratios={ratios}", flush=True)
    rng = np.random.default_rng(23 + ratios)
    B, gamma, V, T = 4, 4, 32000, 1.0
    host = _inputs(rng, B, gamma, V)
    dev = [DeviceArray.from_numpy(gpu, a) for a in host]
    outs = [DeviceArray(gpu, B * (gamma + 1) * 4), DeviceArray(gpu, B * 4),
            DeviceArray(gpu, B * gamma * 4)]
    refs = [DeviceArray(gpu, B * (gamma + 1) * 4), DeviceArray(gpu, B * 4),
            DeviceArray(gpu, B * gamma * 4)]
    old = gpu.cgx_verify_lean_min_blocks(-1 if ratios else 0)

    def call(o):
        ap = o[2].ptr if ratios else None
        return gpu.cgx_verify_chain_batch_dev_noalloc(*(a.ptr for a in dev), B, gamma, V, T, 0,
                                                      1.0, o[0].ptr, o[1].ptr, ap)

    def read(o):
        return (o[0].numpy(np.int32, (B, gamma + 1)), o[1].numpy(np.int32, (B,)),
                o[2].numpy(np.float32, (B, gamma)))

    assert call(refs) == 0, last_error(gpu)           # eager, before the capture
    assert gpu.cgx_synchronize() == 0, last_error(gpu)
    assert gpu.cgx_graph_begin() == 0, last_error(gpu)
    rc = call(outs)
    g = gpu.cgx_graph_end()
    assert rc == 0 and g, last_error(gpu)
    try:
        for rep in range(3):
            if rep:
                # new inputs at the same addresses
                for d_, a in zip(dev, _inputs(rng, B, gamma, V)):
                    assert gpu.cgx_memcpy_h2d(d_.ptr, a.ctypes.data, a.nbytes) == 0
            assert call(refs) == 0, last_error(gpu)   # eager work between replays
            assert gpu.cgx_synchronize() == 0, last_error(gpu)
            for o in outs:
                assert gpu.cgx_memset(o.ptr, 0xFF, o.nbytes) == 0
            assert gpu.cgx_graph_launch(g) == 0, last_error(gpu)
            assert gpu.cgx_synchronize() == 0, last_error(gpu)
            got, exp = read(outs), read(refs)
            np.testing.assert_array_equal(got[0], exp[0])
            np.testing.assert_array_equal(got[1], exp[1])
            if ratios:
                np.testing.assert_array_equal(got[2].view(np.uint32), exp[2].view(np.uint32))
    finally:
        gpu.cgx_graph_free(g)
        gpu.cgx_verify_lean_min_blocks(old)
        for a in dev + outs + refs:
            a.free()


def test_capture_refuses_memset_and_allocation(gpu):
    """During a capture, calls that would record a memset node or grow the
    library's device memory refuse with an error naming the capture; the
    capture (which then holds no node) ends and is freed, never replayed."""
    print("capture guard: cgx_memset inside a capture", flush=True)
    buf = DeviceArray(gpu, 4096)
    assert gpu.cgx_graph_begin() == 0, last_error(gpu)
    rc = gpu.cgx_memset(buf.ptr, 0, 4096)
    err = last_error(gpu)
    g = gpu.cgx_graph_end()
    if g:
        assert gpu.cgx_graph_free(g) == 0
    assert rc == -1 and "captured" in err, err
    gpu.cgx_clear_error()
    # outside a capture the same call works
    assert gpu.cgx_memset(buf.ptr, 0, 4096) == 0 and gpu.cgx_synchronize() == 0
    buf.free()
