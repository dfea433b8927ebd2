#!/usr/bin/env python3
"""Benchmark of the speculative-decoding verify path on one MI355X.

Headline: INT4 dequant GEMV, W 4096x4096 packed
INT4 (nibbles uniform in [-8,7], groups of 128, fp16-valued scales
U(0.005,0.02)), activation fp32 [M,4096] ~ N(0,1), output fp32.  A step is
one GEMV launch; weights rotate over enough copies (>= 2x the 256 MB MALL) so
every launch streams W from HBM.  `value` is the achieved algorithmic HBM
bandwidth of that launch (GB/s): bytes = K*N/2 + (K*N/128)*4 + M*K*4 + M*N*4
(fp32 scales on device) divided by the mean launch time, measured with HIP
events on the library stream around the K timed launches.

Also reported (same JSON line): the GEMV at every M in 1..5, and the CPU
baseline -- cogito's own cg_matmul_int4 compiled from the reference sources
(oracle/_ref) or, when that is absent, the C restatement (oracle/), timed on
this host's cores, single-threaded, on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--rows M]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 * 1024 * 1024
# HBM bytes per GEMV launch measured with rocprofv3 FETCH_SIZE + WRITE_SIZE,
# scaled by a copy kernel of known size (profiles/int4_gemv_4096x4096.md).
# Measured for k_gemv_strip<M, 2, 8>; re-measure when the kernel changes.
GEMV_TRAFFIC_BYTES = {1: 9136128, 2: 9306112, 3: 9474048, 4: 9641984, 5: 9809920}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemv_bytes(M: int, K: int, N: int, gs: int) -> int:
    return K * N // 2 + (K * N // gs) * 4 + M * K * 4 + M * N * 4


def make_config2_weight(rng, K: int, N: int, gs: int):
    v = rng.integers(-8, 8, size=K * N, dtype=np.int64)
    nib = (v & 0xF).astype(np.uint8)
    data = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    scales = rng.uniform(0.005, 0.02, K * N // gs).astype(np.float16).astype(np.float32)
    return data, scales


def bench_gemv(lib, M_list, K, N, gs, steps, warmup, seed=2024):
    from cogito_amd.capi import DeviceArray, host_quant_from_arrays, last_error

    rng = np.random.default_rng(seed)
    data, scales = make_config2_weight(rng, K, N, gs)
    hq, keep = host_quant_from_arrays(data, scales, K, N, gs)
    per_copy = K * N // 2 + (K * N // gs) * 4
    copies = max(4, -(-2 * MALL_BYTES // per_copy) + 1)
    log(f"[bench] gemv K={K} N={N} gs={gs}: {copies} weight copies "
        f"({copies * per_copy / 1e6:.0f} MB) to defeat the MALL")
    dws = []
    for _ in range(copies):
        dq = lib.cgx_quant_to_device(C.byref(hq))
        if not dq or lib.cgx_quant_layout(dq) != 2:
            raise RuntimeError(f"weight upload failed: {last_error(lib)}")
        dws.append(dq)
    results = {}
    for M in M_list:
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        dx = DeviceArray.from_numpy(lib, x)
        dy = DeviceArray(lib, M * N * 4)
        for i in range(warmup):
            if lib.cgx_matmul_int4_dev(dx.ptr, M, dws[i % copies], dy.ptr):
                raise RuntimeError(last_error(lib))
        lib.cgx_synchronize()
        lib.cgx_event_record(0)
        for i in range(steps):
            lib.cgx_matmul_int4_dev(dx.ptr, M, dws[i % copies], dy.ptr)
        lib.cgx_event_record(1)
        if lib.cgx_synchronize():
            raise RuntimeError(last_error(lib))
        ms = lib.cgx_event_elapsed_ms(0, 1) / steps
        nbytes = gemv_bytes(M, K, N, gs)
        results[M] = {"us_per_launch": ms * 1e3, "bytes": nbytes,
                      "gbs": nbytes / (ms * 1e-3) / 1e9}
        log(f"[bench] gemv M={M}: {ms * 1e3:.2f} us/launch, "
            f"{results[M]['gbs']:.0f} GB/s ({results[M]['gbs'] / HBM_PEAK_GBS:.1%} of 8 TB/s)")
        dx.free()
        dy.free()
    for dq in dws:
        lib.cg_tensor_quant_free(dq)
    return results


def cpu_baseline_gemv(M, K, N, gs, budget_s=12.0, seed=2024):
    """cogito's cg_matmul_int4 on the host, 1 thread, bounded sample."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib
    rng = np.random.default_rng(seed)
    data, scales = make_config2_weight(rng, K, N, gs)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    y = np.zeros((M, N), np.float32)
    ref = oracle_lib.load_ref()
    if ref is not None:
        kind = "reference"
        # build a reference cg_tensor_quant around the arrays
        q = oracle_lib.RefQuant()
        shape = (C.c_int * 2)(K, N)
        zeros = np.zeros_like(scales)
        q.data = data.ctypes.data_as(C.POINTER(C.c_uint8))
        q.scales = scales.ctypes.data_as(C.POINTER(C.c_float))
        q.zeros = zeros.ctypes.data_as(C.POINTER(C.c_float))
        q.shape = C.cast(shape, C.POINTER(C.c_int))
        q.ndim, q.size, q.group_size = 2, K * N, gs
        q.num_groups = K * N // gs
        tx = oracle_lib.ref_tensor(ref, x)
        ty = oracle_lib.ref_tensor(ref, y)

        def run():
            ref.cg_matmul_int4(tx, C.byref(q), ty)
    else:
        kind = "port"
        orc = oracle_lib.load_oracle()

        def run():
            orc.orc_matmul_int4(x.ctypes.data, M, K, data.ctypes.data,
                                scales.ctypes.data, N, gs, y.ctypes.data)
    run()  # warm-up
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < 3:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    med = float(np.median(times))
    nbytes = gemv_bytes(M, K, N, gs)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"cg_matmul_int4 M={M} K={K} N={N} gs={gs}, median of "
                      f"{len(times)} runs ({med * 1e3:.1f} ms each), 1 thread",
            "cpu": platform.processor() or platform.machine()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--rows", type=int, default=5,
                    help="activation rows M of the headline line (gamma+1 = 5)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device-to-device copy (a plain copy kernel "
                         "of known size, to scale rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the verify kernels are sized for one MI355X); run with --gpus 1",
              file=sys.stderr)
        return 2

    import cogito_amd
    from cogito_amd.capi import last_error
    lib = cogito_amd.load()
    if lib.cgx_init(0):
        raise RuntimeError(f"cgx_init: {last_error(lib)}")
    log(f"[bench] device: {lib.cgx_device_name().decode()}")
    if args.calibrate_copy:
        n = 256 << 20
        a, b = lib.cgx_malloc(n), lib.cgx_malloc(n)
        lib.cgx_memset(a, 1, n)
        for _ in range(5):
            lib.cgx_memcpy_d2d(b, a, n)
        lib.cgx_synchronize()
        log(f"[bench] copied {n} bytes device-to-device 5 times")
        lib.cgx_free(a)
        lib.cgx_free(b)
        return 0

    K = N = 4096
    gs = 128
    M_list = sorted(set([1, 2, 3, 4, 5, args.rows]))
    res = bench_gemv(lib, M_list, K, N, gs, args.steps, args.warmup)
    head = res[args.rows]

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline (cogito cg_matmul_int4, 1 thread) ...")
        cpu = cpu_baseline_gemv(args.rows, K, N, gs)
        log(f"[bench] CPU: {cpu['value']:.3f} GB/s ({cpu['kind']})")

    line = {
        "metric": "verified tok/s @ γ=4 on 1 GPU; INT4 GEMV achieved HBM GB/s (% of peak)",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["us_per_launch"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xfp32->fp32",
        "data": "synthetic (BASELINE config 2: uniform nibbles, fp16-valued scales, "
                "x~N(0,1)); weights rotated over >2x MALL",
        "config": {"workload": f"int4_gemv K={K} N={N} g={gs} M={args.rows}",
                   "M": args.rows, "K": K, "N": N, "group_size": gs,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": GEMV_TRAFFIC_BYTES.get(args.rows)},
        "cpu_baseline": cpu,
        "per_rows": {str(m): {"us": round(r["us_per_launch"], 3),
                              "GB/s": round(r["gbs"], 1),
                              "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}
                     for m, r in res.items()},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
