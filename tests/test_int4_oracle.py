"""CPU: pins the INT4 part of the oracle (quantize, dequantize, matmul,
unpack) against closed forms, the compiled reference and the golden
fixtures.  Reference: src/quantize/int4.c:10-114, include/cg_quantize.h:155-175.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle_lib import (oracle_matmul, oracle_quantize, ptr, ref_tensor,
                        ref_tensor_np)


def test_unpack_all_bytes_closed_form(oracle):
    # every byte, scale 1: low nibble then high nibble, two's complement
    data = np.arange(256, dtype=np.uint8)
    scales = np.ones(1, np.float32)
    out = np.zeros(512, np.float32)
    oracle.orc_dequantize_int4(ptr(data), ptr(scales), 512, 512, ptr(out))
    lo = (data & 0xF).astype(np.int32)
    hi = (data >> 4).astype(np.int32)
    exp = np.empty(512, np.float32)
    exp[0::2] = np.where(lo >= 8, lo - 16, lo)
    exp[1::2] = np.where(hi >= 8, hi - 16, hi)
    np.testing.assert_array_equal(out, exp)


def test_quantize_hand_cases(oracle):
    # absmax 7 -> scale 1; roundf rounds half away from zero; clamp at -8
    x = np.array([7.0, -7.0, 3.5, -3.5, 2.5, -2.5, 0.49, -0.5], np.float32)
    data, scales = oracle_quantize(oracle, x, 8)
    assert scales[0] == np.float32(1.0)
    vals = []
    for b in data.tolist():
        for nib in (b & 0xF, b >> 4):
            vals.append(nib - 16 if nib >= 8 else nib)
    assert vals == [7, -7, 4, -4, 3, -3, 0, -1]


def test_quantize_scale_floor(oracle):
    # all-zero group: absmax/7 < 1e-10 -> scale 1.0 (int4.c:38)
    x = np.zeros(16, np.float32)
    x[8:] = 1e-12
    data, scales = oracle_quantize(oracle, x, 8)
    assert scales.tolist() == [1.0, 1.0]
    assert not data.any()


def test_quantize_odd_length_pads_high_nibble(oracle):
    x = np.array([7.0, 1.0, -7.0], np.float32)
    data, scales = oracle_quantize(oracle, x, 4)
    assert data.size == 2 and (int(data[1]) >> 4) == 0


def test_matmul_closed_form_fp64(oracle, rng):
    # brute force in float64 from the dequantised weights: within fp32 noise
    K, N, gs = 64, 48, 16
    w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
    x = rng.normal(0, 1, (3, K)).astype(np.float32)
    data, scales = oracle_quantize(oracle, w, gs)
    deq = np.zeros(K * N, np.float32)
    oracle.orc_dequantize_int4(ptr(data), ptr(scales), K * N, gs, ptr(deq))
    y = oracle_matmul(oracle, x, data, scales, K, N, gs)
    y64 = x.astype(np.float64) @ deq.reshape(K, N).astype(np.float64)
    np.testing.assert_allclose(y, y64, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("shape,gs", [((64, 64), 64), ((32, 96), 32), ((10, 7), 6),
                                      ((5, 129), 128)])
def test_quantize_matches_reference(oracle, ref, rng, shape, gs):
    w = rng.normal(0, 0.5, shape).astype(np.float32)
    t = ref_tensor(ref, w)
    q = ref.cg_quantize_int4(t, gs)
    n = w.size
    ref_data = np.ctypeslib.as_array(q.contents.data, shape=((n + 1) // 2,)).copy()
    ng = q.contents.num_groups
    ref_scales = np.ctypeslib.as_array(q.contents.scales, shape=(ng,)).copy()
    data, scales = oracle_quantize(oracle, w, gs)
    np.testing.assert_array_equal(data, ref_data)
    np.testing.assert_array_equal(scales.view(np.uint32), ref_scales.view(np.uint32))
    deq_t = ref.cg_dequantize(q)
    ref_deq = ref_tensor_np(deq_t).ravel()
    deq = np.zeros(n, np.float32)
    oracle.orc_dequantize_int4(ptr(data), ptr(scales), n, gs, ptr(deq))
    np.testing.assert_array_equal(deq.view(np.uint32), ref_deq.view(np.uint32))
    ref.cg_tensor_free(deq_t)
    ref.cg_tensor_quant_free(q)
    ref.cg_tensor_free(t)


@pytest.mark.parametrize("M,K,N,gs", [(1, 64, 64, 64), (5, 128, 96, 32), (3, 17, 10, 4)])
def test_matmul_matches_reference_bitwise(oracle, ref, rng, M, K, N, gs):
    w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    tw = ref_tensor(ref, w)
    q = ref.cg_quantize_int4(tw, gs)
    tx = ref_tensor(ref, x)
    ty = ref_tensor(ref, np.zeros((M, N), np.float32))
    ref.cg_matmul_int4(tx, q, ty)
    y_ref = ref_tensor_np(ty)
    data, scales = oracle_quantize(oracle, w, gs)
    y = oracle_matmul(oracle, x, data, scales, K, N, gs)
    np.testing.assert_array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    for t in (tw, tx, ty):
        ref.cg_tensor_free(t)
    ref.cg_tensor_quant_free(q)
