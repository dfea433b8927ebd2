"""GPU parity of the INT4 path against the oracle (bit-exact for quantize,
unpack/dequantize and the reference-order kernel; 1e-3 of max|y| per row for
the tiled GEMV, whose fp32 summation order differs).
Reference: src/quantize/int4.c:10-114."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cogito_amd.capi import DeviceArray, last_error
from gpu_util import (host_quant_from_arrays, host_tensor, quant_host_arrays,
                      rel_err_rows, tensor_np)
from oracle_lib import oracle_matmul, oracle_quantize, ptr

pytestmark = pytest.mark.gpu
TOL = 1e-3          # north star: GEMV within 1e-3 relative (fp32 accumulate)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("shape,gs", [((64, 128), 64), ((33, 7), 8), ((4096, 64), 128),
                                      ((3, 1000), 100)])
def test_quantize_bitexact(gpu, oracle, rng, shape, gs):
    w = rng.normal(0, 0.3, shape).astype(np.float32)
    w.ravel()[::97] = 0.0
    t = host_tensor(gpu, w)
    q = gpu.cg_quantize_int4(t, gs)
    assert q, last_error(gpu)
    data, scales = quant_host_arrays(q)
    odata, oscales = oracle_quantize(oracle, w, gs)
    np.testing.assert_array_equal(data, odata)
    np.testing.assert_array_equal(_bits(scales), _bits(oscales))
    gpu.cg_tensor_quant_free(q)
    gpu.cg_tensor_free(t)


def test_unpack_all_bytes_on_gpu(gpu, oracle):
    # all 256 bytes, flat and tiled layouts: dequantised values bit-exact
    K, N, gs = 256, 512, 64
    data = np.tile(np.arange(256, dtype=np.uint8), K * N // 2 // 256)
    rng = np.random.default_rng(7)
    scales = rng.uniform(0.005, 0.02, K * N // gs).astype(np.float32)
    exp = np.zeros(K * N, np.float32)
    oracle.orc_dequantize_int4(ptr(data), ptr(scales), K * N, gs, ptr(exp))
    hq, keep = host_quant_from_arrays(data, scales, K, N, gs)
    for layout in (1, 2, 3):
        dq = gpu.cgx_quant_to_device_layout(C.byref(hq), layout)
        assert dq, last_error(gpu)
        assert gpu.cgx_quant_layout(dq) == layout
        t = gpu.cg_dequantize(dq)
        assert t, last_error(gpu)
        got = tensor_np(gpu, t).ravel()
        np.testing.assert_array_equal(_bits(got), _bits(exp))
        gpu.cg_tensor_free(t)
        gpu.cg_tensor_quant_free(dq)
    # host-resident quant through the API
    t = gpu.cg_dequantize(C.byref(hq))
    np.testing.assert_array_equal(_bits(tensor_np(gpu, t).ravel()), _bits(exp))
    gpu.cg_tensor_free(t)


def _make_weight(oracle, rng, K, N, gs, config2=False):
    if config2:
        # nibbles uniform in [-8, 7], fp16-valued scales
        v = rng.integers(-8, 8, size=K * N)
        nib = (v & 0xF).astype(np.uint8)
        data = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
        scales = rng.uniform(0.005, 0.02, K * N // gs).astype(np.float16).astype(np.float32)
        return data, scales
    w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
    return oracle_quantize(oracle, w, gs)


SHAPES = [(4096, 4096, 128), (256, 512, 64), (1024, 2048, 128), (4096, 1024, 128),
          (11008, 4096, 128), (256, 16, 16), (768, 2304, 128), (3072, 768, 128)]


@pytest.mark.parametrize("K,N,gs", SHAPES)
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("layout,kernel", [(2, 1), (3, 3)], ids=["valu", "mfma"])
def test_gemv_tiled_vs_oracle(gpu, oracle, rng, K, N, gs, M, layout, kernel):
    if K * N > 4096 * 4096 and M not in (1, 5):
        pytest.skip("large shape: M=1 and M=5 only")
    _gemv_case(gpu, oracle, rng, K, N, gs, M, layout, kernel)


@pytest.mark.parametrize("K,N,gs,M", [(4096, 4096, 128, 16), (1024, 2048, 128, 12),
                                      (768, 2304, 128, 20), (4096, 22016, 128, 5),
                                      (4096, 32000, 128, 5), (4096, 8192, 64, 7),
                                      (256, 512, 16, 40)])
def test_gemv_mfma_more_rows_and_wide(gpu, oracle, rng, K, N, gs, M):
    # M > 8 (row chunks of 16), and N wide enough for 2 / 4 column tiles per block
    _gemv_case(gpu, oracle, rng, K, N, gs, M, 3, 3)


@pytest.mark.parametrize("K,N,gs,M", [(4096, 4096, 128, 40), (1024, 2048, 128, 32),
                                      (256, 512, 128, 100), (768, 1280, 256, 64),
                                      (1024, 1024, 128, 128), (512, 384, 128, 256),
                                      (4096, 32000, 128, 40), (256, 128, 128, 1)])
def test_gemm_mfma_vs_oracle(gpu, oracle, rng, K, N, gs, M):
    # the shared-A-tile GEMM (row blocks of up to 64 / 128 rows, split K)
    _gemv_case(gpu, oracle, rng, K, N, gs, M, 3, 4)


def _stream_case(gpu, oracle, rng, K, N, gs, M, min_units):
    """The persistent streaming GEMV (taken at K = 4096, up to 5 rows, once
    the output has min_units 32-column units per CU) against the oracle, and
    against the block-per-tile kernel on the same inputs (both carry the rows
    as hi + lo fp16: within 1e-5 of max|y| per row)."""
    # nibble bytes and fp16-valued scales drawn directly (a normal draw of a
    # 4096 x 128256 matrix would take 2 GiB)
    data = rng.integers(0, 256, K * N // 2, dtype=np.uint8)
    scales = rng.uniform(0.005, 0.02, K * N // gs).astype(np.float16).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    y_ref = oracle_matmul(oracle, x, data, scales, K, N, gs)
    hq, keep = host_quant_from_arrays(data, scales, K, N, gs)
    dq = gpu.cgx_quant_to_device_layout(C.byref(hq), 3)
    assert dq, last_error(gpu)
    dx = DeviceArray.from_numpy(gpu, x)
    dy = DeviceArray(gpu, M * N * 4)
    old = gpu.cgx_gemv_stream_min_units(-1)
    ys = []
    try:
        for units in (min_units, 0):
            gpu.cgx_gemv_stream_min_units(units)
            for rep in range(2):         # a second call on the same buffers
                gpu.cgx_memset(dy.ptr, 0xFF, M * N * 4)
                assert gpu.cgx_matmul_int4_dev_kernel(dx.ptr, M, dq, dy.ptr, 3) == 0, \
                    last_error(gpu)
                assert gpu.cgx_synchronize() == 0, last_error(gpu)
                y = dy.numpy(np.float32, (M, N))
                assert np.all(np.isfinite(y))
                assert rel_err_rows(y, y_ref) <= TOL
            ys.append(y)
    finally:
        gpu.cgx_gemv_stream_min_units(old)
    assert rel_err_rows(ys[0], ys[1]) <= 1e-5
    gpu.cg_tensor_quant_free(dq)


@pytest.mark.parametrize("N,M", [(128256, 5), (65536, 1), (65536, 3)])
def test_gemv_stream_wide_vocab(gpu, oracle, rng, N, M):
    # the default dispatch: a 64k / 128k-column lm_head at 1-5 rows
    _stream_case(gpu, oracle, rng, 4096, N, 128, M, 8)


@pytest.mark.parametrize("N,gs,M", [(4096, 128, 5), (22016, 128, 2), (2048, 64, 4),
                                    (6144, 256, 1), (4160, 64, 5)])
def test_gemv_stream_forced(gpu, oracle, rng, N, gs, M):
    # every supported product through the streaming kernel: runs of one to
    # three units (odd runs end with an idle unit), groups of two units
    _stream_case(gpu, oracle, rng, 4096, N, gs, M, 1)


def test_gemv_mfma_wide_dynamic_range(gpu, oracle, rng):
    # activations spanning many binades, a zero row, huge and tiny scales:
    # the per-round power-of-two scaling keeps the fp16 terms in range
    K, N, gs, M = 1024, 512, 128, 4
    data, scales = _make_weight(oracle, rng, K, N, gs)
    scales = scales.copy()
    scales[::7] *= 1e4
    scales[3::11] *= 1e-6
    x = (rng.normal(0, 1, (M, K)) * np.exp(rng.uniform(-20, 20, (M, K)))).astype(np.float32)
    x[2] = 0.0
    y_ref = oracle_matmul(oracle, x, data, scales, K, N, gs)
    hq, keep = host_quant_from_arrays(data, scales, K, N, gs)
    dq = gpu.cgx_quant_to_device_layout(C.byref(hq), 3)
    dx = DeviceArray.from_numpy(gpu, x)
    dy = DeviceArray(gpu, M * N * 4)
    assert gpu.cgx_matmul_int4_dev_kernel(dx.ptr, M, dq, dy.ptr, 3) == 0, last_error(gpu)
    assert gpu.cgx_synchronize() == 0
    y = dy.numpy(np.float32, (M, N))
    assert np.all(y[2] == 0.0)
    keep_rows = [0, 1, 3]
    assert rel_err_rows(y[keep_rows], y_ref[keep_rows]) <= TOL
    gpu.cg_tensor_quant_free(dq)


def _gemv_case(gpu, oracle, rng, K, N, gs, M, layout, kernel):
    data, scales = _make_weight(oracle, rng, K, N, gs, config2=(K == 4096 and N == 4096))
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    y_ref = oracle_matmul(oracle, x, data, scales, K, N, gs)
    hq, keep = host_quant_from_arrays(data, scales, K, N, gs)
    dq = gpu.cgx_quant_to_device_layout(C.byref(hq), layout)
    assert dq and gpu.cgx_quant_layout(dq) == layout, last_error(gpu)
    dx = DeviceArray.from_numpy(gpu, x)
    dy = DeviceArray(gpu, M * N * 4)
    for rep in range(2):         # a second call on the same buffers
        gpu.cgx_memset(dy.ptr, 0xFF, M * N * 4)
        assert gpu.cgx_matmul_int4_dev_kernel(dx.ptr, M, dq, dy.ptr, kernel) == 0, \
            last_error(gpu)
        assert gpu.cgx_synchronize() == 0, last_error(gpu)
        y = dy.numpy(np.float32, (M, N))
        assert np.all(np.isfinite(y))
        assert rel_err_rows(y, y_ref) <= TOL
    gpu.cg_tensor_quant_free(dq)


@pytest.mark.parametrize("M,K,N,gs", [(1, 64, 64, 64), (5, 128, 96, 32), (3, 17, 10, 4),
                                      (2, 300, 130, 26)])
def test_generic_kernel_bitexact(gpu, oracle, rng, M, K, N, gs):
    w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    data, scales = oracle_quantize(oracle, w, gs)
    y_ref = oracle_matmul(oracle, x, data, scales, K, N, gs)
    # host tensors + host quant through cg_matmul_int4 (reference-order kernel)
    hq, keep = host_quant_from_arrays(data, scales, K, N, gs)
    tx = host_tensor(gpu, x)
    ty = host_tensor(gpu, np.full((M, N), 7.0, np.float32))
    gpu.cg_matmul_int4(tx, C.byref(hq), ty)
    assert last_error(gpu) == "", last_error(gpu)
    np.testing.assert_array_equal(_bits(tensor_np(gpu, ty)), _bits(y_ref))
    gpu.cg_tensor_free(tx)
    gpu.cg_tensor_free(ty)


def test_gemv_api_host_io_device_weight(gpu, oracle, rng):
    K, N, gs = 512, 256, 128
    data, scales = _make_weight(oracle, rng, K, N, gs)
    x = rng.normal(0, 1, (1, K)).astype(np.float32)
    y_ref = oracle_matmul(oracle, x, data, scales, K, N, gs)
    hq, keep = host_quant_from_arrays(data, scales, K, N, gs)
    dq = gpu.cgx_quant_to_device(C.byref(hq))
    tx = host_tensor(gpu, x)
    ty = host_tensor(gpu, np.zeros((1, N), np.float32))
    gpu.cgx_clear_error()
    gpu.cg_gemv_int4(tx, dq, ty)
    assert last_error(gpu) == "", last_error(gpu)
    assert rel_err_rows(tensor_np(gpu, ty), y_ref) <= TOL
    gpu.cg_tensor_quant_free(dq)
    gpu.cg_tensor_free(tx)
    gpu.cg_tensor_free(ty)


def test_matmul_shape_mismatch_sets_error(gpu, rng):
    x = host_tensor(gpu, np.ones((2, 10), np.float32))
    w = host_tensor(gpu, np.ones((12, 8), np.float32))
    q = gpu.cg_quantize_int4(w, 8)
    y = host_tensor(gpu, np.zeros((2, 8), np.float32))
    gpu.cgx_clear_error()
    gpu.cg_matmul_int4(x, q, y)
    assert "shape mismatch" in last_error(gpu)
    for t in (x, w, y):
        gpu.cg_tensor_free(t)
    gpu.cg_tensor_quant_free(q)
