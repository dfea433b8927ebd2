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
one pinned core of this host on a bounded sample.  The legs carry CPU
figures of their own: config 1's verify from cogito's softmax and samplers,
and per-step estimates of configs 3-5 composed from timed pieces (see
cpu_verify_step).

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
# Measured for k_gemv_mfma (layout 3); re-measure when the kernel changes.
GEMV_TRAFFIC_BYTES = {1: 9149663, 2: 9287892, 3: 9431241, 4: 9578685, 5: 9735345}


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


def bench_gemv(lib, M_list, K, N, gs, steps, warmup, seed=2024, layout=3, cold_rows=0):
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
        dq = lib.cgx_quant_to_device_layout(C.byref(hq), layout)
        if not dq or lib.cgx_quant_layout(dq) != layout:
            raise RuntimeError(f"weight upload failed: {last_error(lib)}")
        dws.append(dq)
    results = {}
    # one rotation index over every warm-up and timed launch of every M: a
    # launch reads the copy the previous `copies - 1` launches (> 2x the MALL)
    # did not touch, whatever --steps is
    rot = 0
    for M in M_list:
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        dx = DeviceArray.from_numpy(lib, x)
        dy = DeviceArray(lib, M * N * 4)
        for _ in range(warmup):
            if lib.cgx_matmul_int4_dev(dx.ptr, M, dws[rot % copies], dy.ptr):
                raise RuntimeError(last_error(lib))
            rot += 1
        lib.cgx_synchronize()
        lib.cgx_event_record(0)
        for _ in range(steps):
            lib.cgx_matmul_int4_dev(dx.ptr, M, dws[rot % copies], dy.ptr)
            rot += 1
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
        if cold_rows == M:
            # the same launches with the activations rotated too (64 copies,
            # each reused only after 64 weight copies have streamed past), so
            # that no launch finds x or its output in a cache: the state a
            # kernel trace sees, where every dispatch ends with a cache flush
            nx = 64
            dxs = [DeviceArray.from_numpy(lib, rng.normal(0, 1, (M, K)).astype(np.float32))
                   for _ in range(nx)]
            dys = [DeviceArray(lib, M * N * 4) for _ in range(nx)]
            for i in range(warmup + steps):
                if i == warmup:
                    if lib.cgx_synchronize():
                        raise RuntimeError(last_error(lib))
                    lib.cgx_event_record(0)
                lib.cgx_matmul_int4_dev(dxs[i % nx].ptr, M, dws[rot % copies], dys[i % nx].ptr)
                rot += 1
            lib.cgx_event_record(1)
            if lib.cgx_synchronize():
                raise RuntimeError(last_error(lib))
            ms = lib.cgx_event_elapsed_ms(0, 1) / steps
            results[M]["cold_x_us"] = ms * 1e3
            log(f"[bench] gemv M={M}, activations rotated past the caches: {ms * 1e3:.2f} "
                f"us/launch")
            for a in dxs + dys:
                a.free()
    for dq in dws:
        lib.cg_tensor_quant_free(dq)
    return results


def bench_floor(lib, nbytes, steps, warmup, seed=31):
    """A plain streaming read of the headline's algorithmic bytes
    (cgx_stream_read), rotated over copies like the GEMV: the floor of any
    kernel that has to read those bytes on this GPU.  The first copy's XOR
    fold is checked on the host."""
    from cogito_amd.capi import DeviceArray, last_error

    nbytes = (nbytes + 15) // 16 * 16
    copies = max(4, -(-2 * MALL_BYTES // nbytes) + 1)
    rng = np.random.default_rng(seed)
    host = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    bufs = [DeviceArray.from_numpy(lib, host) for _ in range(copies)]
    blocks = -(-(nbytes // 16) // 512)
    out = DeviceArray(lib, blocks * 4 * 4)
    for i in range(warmup):
        if lib.cgx_stream_read(bufs[i % copies].ptr, nbytes, out.ptr):
            raise RuntimeError(last_error(lib))
    got = out.numpy(np.uint32, (blocks * 4,))
    words = np.zeros(blocks * 512 * 4, np.uint32)
    words[:host.size] = host
    exp = np.bitwise_xor.reduce(words.reshape(blocks, 2, 4, 64, 4), axis=(1, 3, 4)).ravel()
    if not np.array_equal(got, exp):
        raise RuntimeError("cgx_stream_read: fold mismatch")
    rot = warmup
    lib.cgx_synchronize()
    lib.cgx_event_record(0)
    for _ in range(steps):
        lib.cgx_stream_read(bufs[rot % copies].ptr, nbytes, out.ptr)
        rot += 1
    lib.cgx_event_record(1)
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    us = lib.cgx_event_elapsed_ms(0, 1) / steps * 1e3
    for b in bufs:
        b.free()
    out.free()
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"[bench] plain read of {nbytes} B: {us:.2f} us, {gbs:.0f} GB/s "
        f"({gbs / HBM_PEAK_GBS:.1%} of 8 TB/s)")
    return {"bytes": nbytes, "us": round(us, 3), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies,
            "what": "cgx_stream_read: 256-thread blocks, two 16-byte loads per thread, "
                    "rotated like the headline GEMV; the floor of a kernel reading these bytes"}


def _rotations(per_copy: int, floor: int = 2) -> int:
    """Copies needed so one pass over them streams >= 2x the MALL."""
    return max(floor, -(-2 * MALL_BYTES // per_copy) + 1)


def bench_gemv_shapes(lib, shapes, M, steps, warmup, gs=128, seed=77):
    """GEMV launches at the linear-layer shapes of the 7B-shape stack (one
    launch streams W[K,N] once), weights rotated past the MALL."""
    from cogito_amd.capi import DeviceArray, host_quant_from_arrays, last_error

    rng = np.random.default_rng(seed)
    out = {}
    for name, K, N in shapes:
        data = rng.integers(0, 256, size=K * N // 2, dtype=np.uint8)
        scales = rng.uniform(0.005, 0.02, K * N // gs).astype(np.float16).astype(np.float32)
        hq, keep = host_quant_from_arrays(data, scales, K, N, gs)
        per_copy = K * N // 2 + (K * N // gs) * 4
        copies = _rotations(per_copy)
        dws = []
        for _ in range(copies):
            dq = lib.cgx_quant_to_device_layout(C.byref(hq), 3)
            if not dq or lib.cgx_quant_layout(dq) != 3:
                raise RuntimeError(f"weight upload failed: {last_error(lib)}")
            dws.append(dq)
        del keep, data, scales
        dx = DeviceArray.from_numpy(lib, rng.normal(0, 1, (M, K)).astype(np.float32))
        dy = DeviceArray(lib, M * N * 4)
        rot = 0
        for _ in range(warmup):
            lib.cgx_matmul_int4_dev(dx.ptr, M, dws[rot % copies], dy.ptr)
            rot += 1
        if lib.cgx_synchronize():
            raise RuntimeError(last_error(lib))
        lib.cgx_event_record(0)
        for _ in range(steps):
            lib.cgx_matmul_int4_dev(dx.ptr, M, dws[rot % copies], dy.ptr)
            rot += 1
        lib.cgx_event_record(1)
        if lib.cgx_synchronize():
            raise RuntimeError(last_error(lib))
        us = lib.cgx_event_elapsed_ms(0, 1) / steps * 1e3
        nbytes = gemv_bytes(M, K, N, gs)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"K": K, "N": N, "M": M, "us": round(us, 3), "bytes": nbytes,
                     "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"[bench] gemv {name} {K}x{N} M={M}: {us:.2f} us, {gbs:.0f} GB/s "
            f"({gbs / HBM_PEAK_GBS:.1%})")
        dx.free()
        dy.free()
        for dq in dws:
            lib.cg_tensor_quant_free(dq)
    return out


def _draft_tokens_from(logits: np.ndarray, u: np.ndarray) -> np.ndarray:
    """Draft ids drawn from softmax(draft row) by inverse CDF (fp64)."""
    z = logits.astype(np.float64)
    z -= z.max(axis=-1, keepdims=True)
    p = np.exp(z)
    cdf = np.cumsum(p, axis=-1)
    cdf /= cdf[..., -1:]
    flat = cdf.reshape(-1, cdf.shape[-1])
    toks = [min(int(np.searchsorted(row, uu, side="right")), row.size - 1)
            for row, uu in zip(flat, u.reshape(-1))]
    return np.asarray(toks, np.int32).reshape(u.shape)


def bench_accept(lib, V, B, gamma, T, steps, warmup, sets=1, seed=5, top_k=0, top_p=1.0,
                 ratios=False):
    """cgx_verify_chain_batch_dev on B independent chains: target logits
    [B][gamma+1][V], draft [B][gamma][V] ~ N(0, 2^2), draft ids drawn from
    the draft softmax, pre-drawn uniforms.  `sets` rotating input sets.
    ratios=False asks for the emitted tokens and counts only, as the
    speculative loops do (certified decisions); True also for every exact
    acceptance ratio."""
    from cogito_amd.capi import DeviceArray, last_error

    rng = np.random.default_rng(seed)
    bufs = []
    for s in range(sets):
        nt, nd = B * (gamma + 1) * V, B * gamma * V
        dt, dd = DeviceArray(lib, nt * 4), DeviceArray(lib, nd * 4)
        if (lib.cgx_fill_normal_dev(dt.ptr, nt, seed, 100 + 2 * s, 2.0) or
                lib.cgx_fill_normal_dev(dd.ptr, nd, seed, 101 + 2 * s, 2.0)):
            raise RuntimeError(last_error(lib))
        ud = rng.random((B, gamma), dtype=np.float32)
        toks = _draft_tokens_from(dd.numpy(np.float32, (B, gamma, V)) / T, ud)
        uv = rng.random((B, gamma + 1), dtype=np.float32)
        bufs.append((dt, dd, DeviceArray.from_numpy(lib, toks),
                     DeviceArray.from_numpy(lib, uv)))
    dout = DeviceArray(lib, B * (gamma + 1) * 4)
    dn = DeviceArray(lib, B * 4)
    dap = DeviceArray(lib, B * gamma * 4) if ratios else None

    def call(i):
        dt, dd, dtok, du = bufs[i % sets]
        return lib.cgx_verify_chain_batch_dev(dt.ptr, dd.ptr, dtok.ptr, du.ptr, B, gamma, V,
                                              T, top_k, top_p, dout.ptr, dn.ptr,
                                              dap.ptr if dap else None)
    for i in range(warmup):
        if call(i):
            raise RuntimeError(last_error(lib))
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    lib.cgx_event_record(0)
    for i in range(steps):
        call(i)
    lib.cgx_event_record(1)
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    us = lib.cgx_event_elapsed_ms(0, 1) / steps * 1e3
    nacc = dn.numpy(np.int32, (B,))
    nbytes = (2 * gamma + 1) * V * 4 * B
    gbs = nbytes / (us * 1e-6) / 1e9
    for b in bufs:
        for d in b:
            d.free()
    for d in (dout, dn) + ((dap,) if dap else ()):
        d.free()
    log(f"[bench] accept V={V} B={B} gamma={gamma} T={T} top_k={top_k} top_p={top_p} "
        f"ratios={ratios}: "
        f"{us:.2f} us/call, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}), "
        f"mean accepted {nacc.mean():.2f}")
    return {"V": V, "batch": B, "gamma": gamma, "temperature": T, "top_k": top_k,
            "top_p": top_p, "ratios": ratios, "us_per_call": round(us, 3), "bytes": nbytes,
            "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "rotating_sets": sets, "mean_accepted_last_call": float(nacc.mean())}


def bench_draws(lib, V, draws, warmup, seed=41):
    """The single-row draft draw (cgx_sample_temperature_dev: the
    single-workgroup sampler the loops use for rows of up to 32768 values) on
    device rows of three shapes, with the certified decision on and off: us
    per draw from events around `draws` queued draws, and how many of them
    the exact sums decided.  The same tokens either way."""
    from cogito_amd.capi import DeviceArray, last_error

    rng = np.random.default_rng(seed)
    out = DeviceArray(lib, 4)
    res = {}
    for name, scale in (("diffuse_N0_2", 2.0), ("N0_6", 6.0), ("peaked_N0_20", 20.0)):
        x = DeviceArray.from_numpy(lib, rng.normal(0, scale, V).astype(np.float32))
        us = rng.random(draws + warmup, dtype=np.float32)
        r = {}
        for cert in (0, 1):
            lib.cgx_sample_row_certified(cert)
            for u in us[:warmup]:
                lib.cgx_sample_temperature_dev(x.ptr, V, 1.0, float(u), out.ptr)
            f0 = lib.cgx_sample_row_fallbacks()
            lib.cgx_event_record(0)
            for u in us[warmup:]:
                if lib.cgx_sample_temperature_dev(x.ptr, V, 1.0, float(u), out.ptr):
                    raise RuntimeError(last_error(lib))
            lib.cgx_event_record(1)
            lib.cgx_synchronize()
            per = lib.cgx_event_elapsed_ms(0, 1) / draws * 1e3
            fb = lib.cgx_sample_row_fallbacks() - f0
            r["certified" if cert else "exact"] = {"us_per_draw": round(per, 2),
                                                   "exact_fallbacks": fb if cert else draws}
        lib.cgx_sample_row_certified(1)
        x.free()
        res[name] = r
        log(f"[bench] row draw V={V} {name}: exact {r['exact']['us_per_draw']} us, certified "
            f"{r['certified']['us_per_draw']} us ({r['certified']['exact_fallbacks']} of "
            f"{draws} left to the exact sums)")
    out.free()
    res["V"] = V
    res["draws"] = draws
    return res


def bench_accept_graph(lib, V, B, gamma, T, steps, warmup, seed=5):
    """The same verify as bench_accept (tokens only), through the
    allocation-free entry point captured once into a HIP graph and replayed:
    the launch cost a serving loop pays per call without the host's seven
    launches."""
    from cogito_amd.capi import DeviceArray, last_error

    rng = np.random.default_rng(seed)
    nt, nd = B * (gamma + 1) * V, B * gamma * V
    dt, dd = DeviceArray(lib, nt * 4), DeviceArray(lib, nd * 4)
    if (lib.cgx_fill_normal_dev(dt.ptr, nt, seed, 100, 2.0) or
            lib.cgx_fill_normal_dev(dd.ptr, nd, seed, 101, 2.0)):
        raise RuntimeError(last_error(lib))
    ud = rng.random((B, gamma), dtype=np.float32)
    toks = _draft_tokens_from(dd.numpy(np.float32, (B, gamma, V)) / T, ud)
    uv = rng.random((B, gamma + 1), dtype=np.float32)
    dtok, du = DeviceArray.from_numpy(lib, toks), DeviceArray.from_numpy(lib, uv)
    dout, dn = DeviceArray(lib, B * (gamma + 1) * 4), DeviceArray(lib, B * 4)
    if lib.cgx_graph_begin():
        raise RuntimeError(last_error(lib))
    rc = lib.cgx_verify_chain_batch_dev_noalloc(dt.ptr, dd.ptr, dtok.ptr, du.ptr, B, gamma, V, T,
                                                0, 1.0, dout.ptr, dn.ptr, None)
    g = lib.cgx_graph_end()
    if rc or not g:
        raise RuntimeError(last_error(lib))
    for _ in range(warmup):
        lib.cgx_graph_launch(g)
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    lib.cgx_event_record(0)
    for _ in range(steps):
        lib.cgx_graph_launch(g)
    lib.cgx_event_record(1)
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    us = lib.cgx_event_elapsed_ms(0, 1) / steps * 1e3
    lib.cgx_graph_free(g)
    for d in (dt, dd, dtok, du, dout, dn):
        d.free()
    log(f"[bench] accept (HIP graph replay) V={V} B={B} gamma={gamma} T={T}: {us:.2f} us/call")
    return {"V": V, "batch": B, "gamma": gamma, "temperature": T, "ratios": False,
            "us_per_call": round(us, 3), "graph": True}


def bench_attention(lib, ctx, Nq, H, Hk, D, kv_gs, steps, warmup, seed=9):
    """INT4-KV verify attention (chain mask) of one layer per launch at the
    7B shape; launches rotate over enough layers to stream past the MALL."""
    from cogito_amd.capi import DeviceArray, last_error

    Nk = ctx + Nq
    per_layer = Nk * Hk * D // 2 * 2 + Nk * Hk * (D // kv_gs) * 4 * 2
    layers = _rotations(per_layer)
    cache = lib.cg_kv_cache_int4_new(layers, Nk, Hk, D, kv_gs)
    if not cache:
        raise RuntimeError(last_error(lib))
    n = Nk * Hk * D
    dk, dv = DeviceArray(lib, n * 4), DeviceArray(lib, n * 4)
    if (lib.cgx_fill_normal_dev(dk.ptr, n, seed, 1, 1.0) or
            lib.cgx_fill_normal_dev(dv.ptr, n, seed, 2, 1.0)):
        raise RuntimeError(last_error(lib))
    for l in range(layers):
        if lib.cgx_kv_cache_int4_write(cache, l, 0, dk.ptr, dv.ptr, Nk):
            raise RuntimeError(last_error(lib))
    lib.cgx_kv_cache_int4_set_len(cache, Nk)
    dk.free()
    dv.free()
    dq = DeviceArray(lib, Nq * H * D * 4)
    lib.cgx_fill_normal_dev(dq.ptr, Nq * H * D, seed, 3, 1.0)
    do = DeviceArray(lib, Nq * H * D * 4)
    for i in range(warmup):
        if lib.cgx_attention_int4_kv_dev(dq.ptr, Nq, H, cache, i % layers, 0, None, do.ptr):
            raise RuntimeError(last_error(lib))
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    lib.cgx_event_record(0)
    for i in range(steps):
        lib.cgx_attention_int4_kv_dev(dq.ptr, Nq, H, cache, i % layers, 0, None, do.ptr)
    lib.cgx_event_record(1)
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    us = lib.cgx_event_elapsed_ms(0, 1) / steps * 1e3
    nbytes = per_layer + 2 * Nq * H * D * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    lib.cg_kv_cache_int4_free(cache)
    dq.free()
    do.free()
    log(f"[bench] attention ctx={ctx} Nq={Nq} H={H} Hk={Hk} D={D}: {us:.2f} us/layer, "
        f"{gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%})")
    return {"ctx": ctx, "Nq": Nq, "H": H, "Hk": Hk, "D": D, "kv_group": kv_gs,
            "us_per_layer": round(us, 3), "bytes": nbytes, "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "layers_rotated": layers}


def bench_attention_step(lib, ctx, Nq, H, Hk, D, steps, warmup, seed=9, theta=10000.0):
    """The decoder's attention step of one layer per launch at the 7B shape:
    RoPE of the new q / k rows, their INT4 append at positions ctx .. ctx+Nq-1,
    attention over the whole cache and the split combine
    (cgx_attention_rope_append_dev); launches rotate over layers as above."""
    from cogito_amd.capi import DeviceArray, last_error

    Nk = ctx + Nq
    per_layer = Nk * Hk * D // 2 * 2 + Nk * Hk * 4 * 2
    layers = _rotations(per_layer)
    cache = lib.cg_kv_cache_int4_new(layers, Nk, Hk, D, D)
    if not cache:
        raise RuntimeError(last_error(lib))
    n = ctx * Hk * D
    dk, dv = DeviceArray(lib, n * 4), DeviceArray(lib, n * 4)
    if (lib.cgx_fill_normal_dev(dk.ptr, n, seed, 1, 1.0) or
            lib.cgx_fill_normal_dev(dv.ptr, n, seed, 2, 1.0)):
        raise RuntimeError(last_error(lib))
    for l in range(layers):
        if lib.cgx_kv_cache_int4_write(cache, l, 0, dk.ptr, dv.ptr, ctx):
            raise RuntimeError(last_error(lib))
    dk.free()
    dv.free()
    ldq = (H + 2 * Hk) * D
    dqkv = DeviceArray(lib, Nq * ldq * 4)
    lib.cgx_fill_normal_dev(dqkv.ptr, Nq * ldq, seed, 3, 1.0)
    dcs = DeviceArray(lib, Nq * D * 4)
    do = DeviceArray(lib, Nq * H * D * 4)
    if lib.cgx_rope_table_dev(Nq, D, ctx, theta, dcs.ptr):
        raise RuntimeError(last_error(lib))

    def call(i):
        return lib.cgx_attention_rope_append_dev(dqkv.ptr, ldq, dcs.ptr, Nq, H, cache,
                                                 i % layers, ctx, do.ptr)
    for i in range(warmup):
        if call(i):
            raise RuntimeError(last_error(lib))
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    lib.cgx_event_record(0)
    for i in range(steps):
        call(i)
    lib.cgx_event_record(1)
    if lib.cgx_synchronize():
        raise RuntimeError(last_error(lib))
    us = lib.cgx_event_elapsed_ms(0, 1) / steps * 1e3
    # cache read, new rows and Q in, O out, new K/V rows written
    nbytes = per_layer + Nq * ldq * 4 + Nq * H * D * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    lib.cg_kv_cache_int4_free(cache)
    for a in (dqkv, dcs, do):
        a.free()
    log(f"[bench] attention step (RoPE + append + attention) ctx={ctx} Nq={Nq}: {us:.2f} "
        f"us/layer, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%})")
    return {"ctx": ctx, "Nq": Nq, "H": H, "Hk": Hk, "D": D, "kv_group": D,
            "us_per_layer": round(us, 3), "bytes": nbytes, "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "layers_rotated": layers,
            "fused": "RoPE + INT4 append + attention + split combine"}


def _model_cfg(n_layers, d, H, Hk, hd, ff, V, max_seq, max_tokens, kv_gs):
    from cogito_amd.capi import CgxModelConfig
    return CgxModelConfig(n_layers=n_layers, d_model=d, n_heads=H, n_kv_heads=Hk,
                          head_dim=hd, d_ff=ff, vocab=V, group_size=128,
                          kv_group_size=kv_gs, max_seq=max_seq, max_tokens=max_tokens,
                          rope_theta=10000.0, norm_eps=1e-5, init_std=0.02)


def bench_e2e(lib, name, tgt, drf, share_head, ctx, gamma, T, top_k, top_p, steps, warmup,
              seed=2025):
    """Chain speculative decoding on the GPU (cgx_spec_step): the draft
    proposes gamma tokens, the target verifies gamma+1 rows in one forward,
    the verify kernels accept a prefix, both KV caches roll back.  Verified
    tok/s = sum(accepted + 1) / wall time over the timed steps (host round
    trip per step included)."""
    from cogito_amd.capi import last_error

    max_seq = ctx + (gamma + 1) * (steps + warmup + 2) + 8
    ct = _model_cfg(*tgt, max_seq=max_seq, max_tokens=gamma + 1, kv_gs=tgt[4])
    cd = _model_cfg(*drf, max_seq=max_seq, max_tokens=2, kv_gs=drf[4])
    t0 = time.perf_counter()
    mt = lib.cgx_model_new(C.byref(ct), seed, None)
    if not mt:
        raise RuntimeError(last_error(lib))
    md = lib.cgx_model_new(C.byref(cd), seed + 1, mt if share_head else None)
    if not md:
        raise RuntimeError(last_error(lib))
    if (lib.cgx_model_fill_context(mt, ctx, seed) or
            lib.cgx_model_fill_context(md, ctx, seed + 7)):
        raise RuntimeError(last_error(lib))
    log(f"[bench] {name}: models built and context {ctx} filled in "
        f"{time.perf_counter() - t0:.1f} s")
    sp = lib.cgx_spec_new(md, mt, gamma, T, top_k, top_p)
    if not sp or lib.cgx_spec_set_last(sp, 1):
        raise RuntimeError(last_error(lib))
    rng = np.random.default_rng(seed)
    out = np.zeros(gamma + 1, np.int32)

    def step():
        ud = rng.random(gamma, dtype=np.float32)
        uv = rng.random(gamma + 1, dtype=np.float32)
        n = lib.cgx_spec_step(sp, ud.ctypes.data, uv.ctypes.data, out.ctypes.data)
        if n < 0:
            raise RuntimeError(last_error(lib))
        return n
    for _ in range(warmup):
        step()
    lib.cgx_synchronize()
    emitted = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        emitted += step() + 1
    lib.cgx_synchronize()
    wall = time.perf_counter() - t0
    lib.cgx_spec_free(sp)
    lib.cgx_model_free(md)
    lib.cgx_model_free(mt)
    tps = emitted / wall
    acc = (emitted - steps) / (steps * gamma)
    log(f"[bench] {name}: {tps:.0f} verified tok/s, {wall / steps * 1e3:.3f} ms/step, "
        f"acceptance {acc:.3f}")
    return {"verified_tok_s": round(tps, 1), "ms_per_step": round(wall / steps * 1e3, 4),
            "acceptance_rate": round(acc, 4), "tokens_per_step": round(emitted / steps, 3),
            "steps": steps, "gamma": gamma, "temperature": T, "top_k": top_k, "top_p": top_p,
            "ctx": ctx, "target": dict(zip(("layers", "d", "H", "Hk", "hd", "ff", "V"), tgt)),
            "draft": dict(zip(("layers", "d", "H", "Hk", "hd", "ff", "V"), drf)),
            "draft_shares_embed_lm_head": bool(share_head), "batch": 1}




def bench_e2e_batch(lib, name, tgt, drf, ctx, gamma, T, B, steps, warmup, seed=2026):
    """The batched chain loop (cgx_spec_batch_step): B sequences in lockstep,
    the target verifying B x (gamma+1) rows per forward.  Verified tok/s =
    sum over sequences of (accepted + 1) / wall time."""
    from cogito_amd.capi import CgxModelConfig, last_error

    max_seq = ctx + (gamma + 1) * (steps + warmup + 2) + 8
    ct = _model_cfg(*tgt, max_seq=max_seq, max_tokens=gamma + 1, kv_gs=tgt[4])
    cd = _model_cfg(*drf, max_seq=max_seq, max_tokens=2, kv_gs=drf[4])
    ct.max_batch = B
    cd.max_batch = B
    t0 = time.perf_counter()
    mt = lib.cgx_model_new(C.byref(ct), seed, None)
    if not mt:
        raise RuntimeError(last_error(lib))
    md = lib.cgx_model_new(C.byref(cd), seed + 1, mt)
    if not md:
        raise RuntimeError(last_error(lib))
    if (lib.cgx_model_fill_context(mt, ctx, seed) or
            lib.cgx_model_fill_context(md, ctx, seed + 7)):
        raise RuntimeError(last_error(lib))
    log(f"[bench] {name}: models built and {B} contexts of {ctx} filled in "
        f"{time.perf_counter() - t0:.1f} s")
    sp = lib.cgx_spec_batch_new(md, mt, gamma, T)
    prev = np.ones(B, np.int32)
    last = np.full(B, 2, np.int32)
    if not sp or lib.cgx_spec_batch_set_last(sp, prev.ctypes.data, last.ctypes.data):
        raise RuntimeError(last_error(lib))
    rng = np.random.default_rng(seed)
    out = np.zeros((B, gamma + 1), np.int32)
    n = np.zeros(B, np.int32)

    def step():
        ud = rng.random((B, gamma), dtype=np.float32)
        uv = rng.random((B, gamma + 1), dtype=np.float32)
        tot = lib.cgx_spec_batch_step(sp, ud.ctypes.data, uv.ctypes.data, out.ctypes.data,
                                      n.ctypes.data)
        if tot < 0:
            raise RuntimeError(last_error(lib))
        return tot
    for _ in range(warmup):
        step()
    lib.cgx_synchronize()
    emitted = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        emitted += step() + B
    lib.cgx_synchronize()
    wall = time.perf_counter() - t0
    lib.cgx_spec_batch_free(sp)
    lib.cgx_model_free(md)
    lib.cgx_model_free(mt)
    tps = emitted / wall
    acc = (emitted - steps * B) / (steps * B * gamma)
    log(f"[bench] {name}: {tps:.0f} verified tok/s, {wall / steps * 1e3:.3f} ms/step, "
        f"acceptance {acc:.3f}")
    return {"verified_tok_s": round(tps, 1), "ms_per_step": round(wall / steps * 1e3, 4),
            "acceptance_rate": round(acc, 4), "tokens_per_step": round(emitted / steps, 3),
            "steps": steps, "gamma": gamma, "temperature": T, "ctx": ctx, "batch": B,
            "target": dict(zip(("layers", "d", "H", "Hk", "hd", "ff", "V"), tgt)),
            "draft": dict(zip(("layers", "d", "H", "Hk", "hd", "ff", "V"), drf)),
            "draft_shares_embed_lm_head": True}


def bench_e2e_tree(lib, name, tgt, drf, ctx, nodes, depth, T, top_k, B, steps, warmup,
                   seed=2027):
    """The tree loop (cgx_tree_spec_step): B sequences in lockstep, each step
    drafting a `nodes`-node tree level by level, verifying B x nodes rows in
    one target forward (the GEMM path) and walking the tree.  Verified tok/s
    = sum over sequences of (accepted + 1) / wall time."""
    from cogito_amd.capi import CgxModelConfig, last_error

    max_seq = ctx + (depth + 1) * (steps + warmup + 2) + nodes + 8
    ct = _model_cfg(*tgt, max_seq=max_seq, max_tokens=nodes, kv_gs=tgt[4])
    cd = _model_cfg(*drf, max_seq=max_seq, max_tokens=nodes, kv_gs=drf[4])
    ct.max_batch = B
    cd.max_batch = B
    t0 = time.perf_counter()
    mt = lib.cgx_model_new(C.byref(ct), seed, None)
    if not mt:
        raise RuntimeError(last_error(lib))
    md = lib.cgx_model_new(C.byref(cd), seed + 1, mt)
    if not md:
        raise RuntimeError(last_error(lib))
    if (lib.cgx_model_fill_context(mt, ctx, seed) or
            lib.cgx_model_fill_context(md, ctx, seed + 7)):
        raise RuntimeError(last_error(lib))
    log(f"[bench] {name}: models built and {B} contexts of {ctx} filled in "
        f"{time.perf_counter() - t0:.1f} s")
    sp = lib.cgx_tree_spec_new(md, mt, nodes, depth, T, top_k, 1.0)
    if not sp:
        raise RuntimeError(last_error(lib))
    D = lib.cgx_tree_spec_depth(sp)
    root = np.full(B, 2, np.int32)
    if lib.cgx_tree_spec_set_root(sp, root.ctypes.data):
        raise RuntimeError(last_error(lib))
    rng = np.random.default_rng(seed)
    out = np.zeros((B, D + 2), np.int32)
    n = np.zeros(B, np.int32)

    def step():
        u = rng.random((B, D + 1, 5), dtype=np.float32)
        tot = lib.cgx_tree_spec_step(sp, u.ctypes.data, out.ctypes.data, n.ctypes.data)
        if tot < 0:
            raise RuntimeError(last_error(lib))
        return tot
    for _ in range(warmup):
        step()
    lib.cgx_synchronize()
    emitted = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        emitted += step() + B
    lib.cgx_synchronize()
    wall = time.perf_counter() - t0
    lib.cgx_tree_spec_free(sp)
    lib.cgx_model_free(md)
    lib.cgx_model_free(mt)
    tps = emitted / wall
    acc = (emitted - steps * B) / (steps * B)
    L, d, H, Hk, hd, ff, V = tgt
    params = L * (d * (H + 2 * Hk) * hd + H * hd * d + 2 * d * ff + ff * d) + d * V
    flops = 2.0 * B * nodes * params
    log(f"[bench] {name}: {tps:.0f} verified tok/s, {wall / steps * 1e3:.3f} ms/step, "
        f"{acc:.3f} accepted per sequence-step; target {flops / 1e12:.2f} TFLOP per verify")
    return {"verified_tok_s": round(tps, 1), "ms_per_step": round(wall / steps * 1e3, 4),
            "accepted_per_seq_step": round(acc, 4), "tokens_per_step": round(emitted / steps, 3),
            "steps": steps, "tree_nodes": nodes, "tree_depth": D, "temperature": T,
            "top_k": top_k, "ctx": ctx, "batch": B,
            "target_flop_per_verify": flops,
            "target_tflops_over_step": round(flops / (wall / steps) / 1e12, 2),
            "target": dict(zip(("layers", "d", "H", "Hk", "hd", "ff", "V"), tgt)),
            "draft": dict(zip(("layers", "d", "H", "Hk", "hd", "ff", "V"), drf)),
            "draft_shares_embed_lm_head": True}


# ------------------------------------------------------------ CPU side

def cpu_info() -> dict:
    """The host's CPU model (lscpu's "Model name", from /proc/cpuinfo), the
    logical CPUs it has and the ones this process may use."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model or platform.processor() or platform.machine(),
            "nproc": os.cpu_count(), "usable": len(os.sched_getaffinity(0))}


class one_core:
    """Pins the calling thread (the one timing the CPU baseline) to one core
    of those it may use, and restores its affinity afterwards."""

    def __enter__(self):
        self.saved = os.sched_getaffinity(0)
        self.core = max(self.saved)
        os.sched_setaffinity(0, {self.core})
        return self.core

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.saved)
        return False


def _median_time(run, budget_s, max_runs=50, min_runs=3, warm=True):
    if warm:
        run()
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < min_runs:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if len(times) >= max_runs:
            break
    return float(np.median(times)), len(times)


def _oracle_libs():
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib
    return oracle_lib, oracle_lib.load_ref(), oracle_lib.load_oracle()


class _RefMatmul:
    """cogito's cg_matmul_int4 (oracle/_ref) on a random INT4 weight
    [K, N] with rows x [M, K]; the C restatement when the reference build is
    absent."""

    def __init__(self, K, N, gs, M, seed=11):
        self.olib, self.ref, self.orc = _oracle_libs()
        rng = np.random.default_rng(seed)
        self.data = rng.integers(0, 256, K * N // 2, dtype=np.uint8)
        self.scales = rng.uniform(0.005, 0.02, K * N // gs).astype(np.float32)
        self.x = rng.normal(0, 1, (M, K)).astype(np.float32)
        self.y = np.zeros((M, N), np.float32)
        self.K, self.N, self.gs, self.M = K, N, gs, M
        self.kind = "reference" if self.ref is not None else "port"
        if self.ref is not None:
            q = self.olib.RefQuant()
            self.shape = (C.c_int * 2)(K, N)
            self.zeros = np.zeros_like(self.scales)
            q.data = self.data.ctypes.data_as(C.POINTER(C.c_uint8))
            q.scales = self.scales.ctypes.data_as(C.POINTER(C.c_float))
            q.zeros = self.zeros.ctypes.data_as(C.POINTER(C.c_float))
            q.shape = C.cast(self.shape, C.POINTER(C.c_int))
            q.ndim, q.size, q.group_size = 2, K * N, gs
            q.num_groups = K * N // gs
            self.q = q
            self.tx = self.olib.ref_tensor(self.ref, self.x)
            self.ty = self.olib.ref_tensor(self.ref, self.y)

    def __call__(self):
        if self.ref is not None:
            self.ref.cg_matmul_int4(self.tx, C.byref(self.q), self.ty)
        else:
            self.orc.orc_matmul_int4(self.x.ctypes.data, self.M, self.K, self.data.ctypes.data,
                                     self.scales.ctypes.data, self.N, self.gs,
                                     self.y.ctypes.data)

    def close(self):
        if self.ref is not None:
            self.ref.cg_tensor_free(self.tx)
            self.ref.cg_tensor_free(self.ty)


def cpu_baseline_gemv(M, K, N, gs, budget_s=6.0):
    """cogito's cg_matmul_int4 on the host, one pinned core, bounded sample."""
    mm = _RefMatmul(K, N, gs, M, seed=2024)
    with one_core() as core:
        med, runs = _median_time(mm, budget_s)
    mm.close()
    nbytes = gemv_bytes(M, K, N, gs)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": 1, "kind": mm.kind,
            "sample": f"cg_matmul_int4 M={M} K={K} N={N} gs={gs}, median of {runs} runs "
                      f"({med * 1e3:.1f} ms each), 1 thread pinned to core {core}",
            "cpu": cpu_info()}


def cpu_baseline_accept(V=32000, gamma=4, budget_s=3.0, seed=5):
    """Config 1's verify on the host from cogito's own compiled functions
    (oracle/_ref): cg_cuda_softmax_forward for the gamma + 1 target and gamma
    draft rows (src/cuda/tensor_kernels.c:699-740), cg_acceptance_prob per
    drafted token, then cg_sample_corrected at the first reject or
    cg_sample_temperature of target row gamma (src/inference/speculative.c:
    49-75,148-172).  Accept draws are pre-drawn; the samplers draw from the
    reference's own LCG."""
    olib, ref, orc = _oracle_libs()
    rng = np.random.default_rng(seed)
    t = rng.normal(0, 2, (gamma + 1, V)).astype(np.float32)
    d = rng.normal(0, 2, (gamma, V)).astype(np.float32)
    x = _draft_tokens_from(d, rng.random(gamma, dtype=np.float32)).astype(np.int32)
    u = rng.random(gamma, dtype=np.float32)
    if ref is None:
        uu = rng.random(gamma + 1, dtype=np.float32)
        out = np.zeros(gamma + 1, np.int32)

        def run():
            orc.orc_verify_chain(t.ctypes.data, d.ctypes.data, x.ctypes.data, uu.ctypes.data,
                                 gamma, V, 1.0, 0, 1.0, out.ctypes.data, None)
        kind = "port"
    else:
        kind = "reference"
        tt, td = olib.ref_tensor(ref, t), olib.ref_tensor(ref, d)
        tp = olib.ref_tensor(ref, np.zeros_like(t))
        tq = olib.ref_tensor(ref, np.zeros_like(d))
        P = np.ctypeslib.as_array(tp.contents.data, shape=(gamma + 1, V))
        Q = np.ctypeslib.as_array(tq.contents.data, shape=(gamma, V))

        def run():
            ref.cg_cuda_softmax_forward(tt, tp, 1)
            ref.cg_cuda_softmax_forward(td, tq, 1)
            for i in range(gamma):
                a = ref.cg_acceptance_prob(float(Q[i, x[i]]), float(P[i, x[i]]))
                if not u[i] < a:
                    ref.cg_sample_corrected(Q[i:].ctypes.data, P[i:].ctypes.data, V)
                    return
            ref.cg_sample_temperature(t[gamma:].ctypes.data, V, 1.0)
    with one_core() as core:
        med, runs = _median_time(run, budget_s, max_runs=400)
    if kind == "reference":
        for tt_ in (tt, td, tp, tq):
            ref.cg_tensor_free(tt_)
    nbytes = (2 * gamma + 1) * V * 4
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
            "us_per_call": round(med * 1e6, 2),
            "sample": f"config 1 verify (V={V}, gamma={gamma}, T=1) from cogito's softmax, "
                      f"acceptance ratio and samplers, median of {runs} runs, 1 thread pinned "
                      f"to core {core}"}


_ROW_TIMES: dict = {}   # cg_matmul_int4 seconds per row, by weight shape


def cpu_verify_step(tgt, drf, ctx, target_rows, draft_rows, batch, T, top_k, top_p,
                    tokens_per_step, sampler_rows, budget_s=0.6):
    """Host time of one speculative step of a synthetic stack, composed from
    timed pieces (the full step is minutes of single-core work at these
    shapes; the pieces are timed once and scaled):
      - every linear shape of the target and the draft through cogito's
        cg_matmul_int4 at one row, scaled by the rows of the step (the
        reference loop is O(M K N): each row re-reads and dequantises W) and
        by the layer count;
      - one layer of attention (the C restatement of cogito's GQA flash
        forward, src/cuda/flash_attn_kernels.c:261-396) at the step's query
        rows and context, scaled by the layer count;
      - the samplers the step runs, as cogito's own (cg_sample_temperature,
        or cg_sample_top_p with its O(V^2) sort when top-p is on), one call
        timed and scaled by the number of rows sampled.
    RMSNorm, SwiGLU, RoPE and the KV writes (O(rows * d)) are left out.
    Returns the estimate and its parts; "verified tok/s" uses the GPU leg's
    tokens per step, so both sides are compared at the same acceptance."""
    olib, ref, orc = _oracle_libs()
    parts = {}
    M_t = target_rows * batch           # target rows per step (one forward)
    M_d = draft_rows * batch            # draft rows per step

    def linears(cfg):
        L, d, H, Hk, hd, ff, V = cfg
        return [("qkv", d, (H + 2 * Hk) * hd), ("o", H * hd, d), ("gate_up", d, 2 * ff),
                ("down", ff, d)], ("lm_head", d, V)

    total = 0.0
    with one_core() as core:
        for who, cfg, M in (("target", tgt, M_t), ("draft", drf, M_d)):
            lin, head = linears(cfg)
            L = cfg[0]
            for name, K, N in lin + [head]:
                if (K, N) not in _ROW_TIMES:
                    mm = _RefMatmul(K, N, 128, 1)
                    _ROW_TIMES[(K, N)] = _median_time(mm, budget_s, max_runs=5, min_runs=1,
                                                      warm=K * N < 1 << 26)[0]
                    mm.close()
                t1 = _ROW_TIMES[(K, N)]
                reps = M * (L if name != "lm_head" else 1)
                parts[f"{who}.{name} {K}x{N}"] = {"s_one_row": round(t1, 6), "rows": reps}
                total += t1 * reps
            L, d, H, Hk, hd, ff, V = cfg
            Nq = target_rows if who == "target" else 1
            Nk = ctx + Nq
            rng = np.random.default_rng(3)
            Q = rng.normal(0, 1, (Nq, H, hd)).astype(np.float32)
            Kc = rng.normal(0, 1, (Nk, Hk, hd)).astype(np.float32)
            Vc = rng.normal(0, 1, (Nk, Hk, hd)).astype(np.float32)
            O = np.zeros_like(Q)
            sc = 1.0 / np.sqrt(hd)

            def attn():
                orc.orc_flash_fwd(Q.ctypes.data, Kc.ctypes.data, Vc.ctypes.data, O.ctypes.data,
                                  None, 1, Nq, Nk, H, Hk, hd, sc, 4, 0, None)
            big = Nq * Nk * H * hd > 1 << 26
            ta, _ = _median_time(attn, 0.0 if big else budget_s, max_runs=5, min_runs=1,
                                 warm=not big)
            reps = L * (batch if who == "target" else M_d)
            parts[f"{who}.attention Nq={Nq} Nk={Nk}"] = {"s_one": round(ta, 6), "count": reps}
            total += ta * reps
        V = tgt[6]
        rng = np.random.default_rng(4)
        row = rng.normal(0, 2, V).astype(np.float32)
        f32p = row.ctypes.data
        if top_p < 1.0 and (top_k <= 0 or top_k >= V):
            fn, name = (lambda: ref.cg_sample_top_p(f32p, V, top_p)), "cg_sample_top_p"
        elif 0 < top_k < V:
            fn, name = (lambda: ref.cg_sample_top_k(f32p, V, top_k)), "cg_sample_top_k"
        else:
            fn, name = (lambda: ref.cg_sample_temperature(f32p, V, T)), "cg_sample_temperature"
        if ref is None:
            fn, name = (lambda: orc.orc_sample_filtered(f32p, V, T, top_k, top_p, 0.5)), \
                "orc_sample_filtered"
        ts, _ = _median_time(fn, 0.0, max_runs=1, min_runs=1, warm=False)
        parts[f"sampler {name} V={V}"] = {"s_one": round(ts, 6), "rows": sampler_rows}
        total += ts * sampler_rows
    # "port": the attention pieces are the oracle's restatement, so the step
    # as a whole is not the reference's code even where its matmul and
    # sampler are
    return {"value": round(tokens_per_step / total, 4), "unit": "verified tok/s", "cores": 1,
            "kind": "port",
            "composition": ("cg_matmul_int4 and the sampler from the reference's sources "
                            "(oracle/_ref)" if ref is not None else
                            "the oracle's matmul and sampler") +
                           ", attention from the oracle's restatement",
            "s_per_step": round(total, 3), "parts": parts,
            "sample": f"one step composed from pieces timed once on 1 thread pinned to core "
                      f"{core} and scaled by their counts (cg_matmul_int4 per row and layer, "
                      f"attention per layer, the sampler per sampled row); RMSNorm, SwiGLU, "
                      f"RoPE and KV writes left out; the GPU leg's {tokens_per_step} tokens "
                      f"per step"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--rows", type=int, default=5,
                    help="activation rows M of the headline line (gamma+1 = 5)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--legs", default="floor,valu,shapes,accept,draws,attn,e2e,tree",
                    help="comma list of legs beside the headline GEMV: floor (a plain read "
                         "of the headline's bytes, rotated the same way), valu (the VALU "
                         "GEMV on the headline workload), shapes (7B-stack "
                         "GEMV shapes), accept (acceptance sampling C1 + V=128256 x 64 "
                         "chains), draws (the single-row draft draw, V=32000, certified "
                         "decision on and off), attn (INT4-KV verify attention, 7B shape), e2e "
                         "(verified tok/s, tiny and 7B-shape stacks), c3 (C3 alone; part of e2e), "
                         "c4 (C4 at batch 1 alone; "
                         "part of e2e), batch (C4 at batch 8 alone; part of e2e), tree (C5: the "
                         "EAGLE-style tree loop, 7B shape at V=128256, batch 4)")
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
    legs = set(x for x in args.legs.split(",") if x)
    M_list = sorted(set([1, 2, 3, 4, 5, args.rows]))
    res = bench_gemv(lib, M_list, K, N, gs, args.steps, args.warmup, layout=3,
                     cold_rows=args.rows)
    head = res[args.rows]
    extra = {}
    if "floor" in legs:
        extra["read_floor"] = bench_floor(lib, gemv_bytes(args.rows, K, N, gs), args.steps,
                                          args.warmup)
    if "valu" in legs:
        # the VALU GEMV (weight layout 2) on the same workload, for comparison
        rv = bench_gemv(lib, M_list, K, N, gs, args.steps, args.warmup, layout=2)
        extra["gemv_valu_per_rows"] = {str(m): {"us": round(r["us_per_launch"], 3),
                                                "GB/s": round(r["gbs"], 1)}
                                       for m, r in rv.items()}
    if "shapes" in legs:
        d, ff, hd = 4096, 11008, 128
        extra["gemv_7b_shapes"] = bench_gemv_shapes(
            lib, [("qkv", d, (32 + 2 * 8) * hd), ("o", d, d), ("gate_up", d, 2 * ff),
                  ("down", ff, d), ("lm_head", d, 32000), ("lm_head_128k", d, 128256)],
            args.rows, max(50, args.steps // 4), 10)
    cpu_on = not args.no_cpu
    if "accept" in legs:
        extra["accept_c1"] = bench_accept(lib, 32000, 1, 4, 1.0, args.steps, args.warmup)
        extra["accept_c1_graph"] = bench_accept_graph(lib, 32000, 1, 4, 1.0, args.steps,
                                                       args.warmup)
        extra["accept_roofline"] = bench_accept(lib, 128256, 64, 4, 1.0, 50, 5, sets=2)
        extra["accept_roofline_ratios"] = bench_accept(lib, 128256, 64, 4, 1.0, 50, 5, sets=2,
                                                       ratios=True)
        if cpu_on:
            extra["accept_c1"]["cpu_baseline"] = cpu_baseline_accept()
            log(f"[bench] CPU C1 verify: {extra['accept_c1']['cpu_baseline']['us_per_call']} "
                f"us/call")
    if "draws" in legs:
        extra["row_draws"] = bench_draws(lib, 32000, 200, 20)
    if "attn" in legs:
        extra["attention_7b"] = bench_attention(lib, 4096, 5, 32, 8, 128, 128, args.steps,
                                                args.warmup)
        extra["attention_7b_step"] = bench_attention_step(lib, 4096, 5, 32, 8, 128, args.steps,
                                                          args.warmup)
    if "e2e" in legs or "c3" in legs:
        c3t, c3d = (12, 768, 12, 12, 64, 3072, 32000), (2, 768, 12, 12, 64, 3072, 32000)
        extra["e2e_tiny_c3"] = bench_e2e(lib, "C3 tiny", c3t, c3d, False, 1024, 4, 0.8, 0,
                                         0.9, 100, 10)
        if cpu_on:
            # top-p sorts: the 4 draft draws and the 9 verified rows
            extra["e2e_tiny_c3"]["cpu_baseline"] = cpu_verify_step(
                c3t, c3d, 1024, 5, 4, 1, 0.8, 0, 0.9,
                extra["e2e_tiny_c3"]["tokens_per_step"], 13)
    if "e2e" in legs or "c4" in legs:
        c4t, c4d = (32, 4096, 32, 8, 128, 11008, 32000), (1, 4096, 32, 8, 128, 11008, 32000)
        extra["e2e_7b_c4"] = bench_e2e(lib, "C4 7B-shape", c4t, c4d, True, 4096, 4, 1.0, 0,
                                       1.0, 40, 5)
        if cpu_on:
            # softmax-sized passes: 4 draft draws, 9 verified rows, the last draw
            extra["e2e_7b_c4"]["cpu_baseline"] = cpu_verify_step(
                c4t, c4d, 4096, 5, 4, 1, 1.0, 0, 1.0,
                extra["e2e_7b_c4"]["tokens_per_step"], 14)
    if "e2e" in legs or "batch" in legs:
        c4t, c4d = (32, 4096, 32, 8, 128, 11008, 32000), (1, 4096, 32, 8, 128, 11008, 32000)
        extra["e2e_7b_c4_b8"] = bench_e2e_batch(lib, "C4 7B-shape batch 8", c4t, c4d, 4096,
                                                4, 1.0, 8, 20, 3)
        if cpu_on:
            extra["e2e_7b_c4_b8"]["cpu_baseline"] = cpu_verify_step(
                c4t, c4d, 4096, 5, 4, 8, 1.0, 0, 1.0,
                extra["e2e_7b_c4_b8"]["tokens_per_step"], 14 * 8)
    if "tree" in legs:
        c5t, c5d = (32, 4096, 32, 8, 128, 11008, 128256), (1, 4096, 32, 8, 128, 11008, 128256)
        extra["e2e_7b_c5_tree"] = bench_e2e_tree(lib, "C5 7B-shape tree", c5t, c5d, 2048, 64,
                                                 6, 0.7, 50, 4, 10, 2)
        if cpu_on:
            # every node drafted and verified; top-k lists of 64 draft and 64
            # target rows per sequence
            extra["e2e_7b_c5_tree"]["cpu_baseline"] = cpu_verify_step(
                c5t, c5d, 2048, 64, 64, 4, 0.7, 50, 1.0,
                extra["e2e_7b_c5_tree"]["tokens_per_step"], 128 * 4)

    cpu = None
    if cpu_on:
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
        # INT4 weights (exact in fp16) times the fp32 activation*scale carried
        # as hi + lo fp16 (22 significant bits) on the matrix cores, fp32 sums
        "dtype": "int4 x fp32(as fp16 hi+lo, 22 bits) -> fp32",
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
                              "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                              **({"cold_x_us": round(r["cold_x_us"], 3)}
                                 if "cold_x_us" in r else {})}
                     for m, r in res.items()},
        "legs": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
