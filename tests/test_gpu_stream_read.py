"""GPU: cgx_stream_read, the plain-read floor that bench.py's `floor` leg
times next to the headline GEMV.  Each wave's word of `out` must be the XOR
of the 32-bit words of its two 1 KiB runs (16-byte words b*512 + 64w + l and
b*512 + 256 + 64w + l), ragged tails included; bad arguments are refused."""
from __future__ import annotations

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error

pytestmark = pytest.mark.gpu


def fold(words: np.ndarray, blocks: int) -> np.ndarray:
    pad = np.zeros(blocks * 512 * 4, np.uint32)
    pad[:words.size] = words
    return np.bitwise_xor.reduce(pad.reshape(blocks, 2, 4, 64, 4), axis=(1, 3, 4)).ravel()


@pytest.mark.parametrize("nbytes", [16, 1024, 8192, 8208, 100000, 9076736])
def test_stream_read_fold(gpu, rng, nbytes):
    print(f"stream read {nbytes} B", flush=True)
    words = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    d = DeviceArray.from_numpy(gpu, words)
    blocks = -(-(nbytes // 16) // 512)
    out = DeviceArray.from_numpy(gpu, np.full(blocks * 4, 0xDEADBEEF, np.uint32))
    assert gpu.cgx_stream_read(d.ptr, nbytes, out.ptr) == 0, last_error(gpu)
    np.testing.assert_array_equal(out.numpy(np.uint32, (blocks * 4,)), fold(words, blocks))
    d.free()
    out.free()


def test_stream_read_rejects(gpu):
    d = DeviceArray(gpu, 64)
    out = DeviceArray(gpu, 64)
    for ptr, n in ((d.ptr, 15), (d.ptr, 0), (d.ptr + 4, 16), (None, 16)):
        assert gpu.cgx_stream_read(ptr, n, out.ptr) == -1
        gpu.cgx_clear_error()
    d.free()
    out.free()
