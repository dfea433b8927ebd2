"""GPU: decoders built from "COG1" model files (cgx_model_load /
cgx_model_save; the reference reads the layout in
src/core/serialization.c:46-77 and quantizes with src/quantize/int4.c:10-59).

* A seeded model saved with INT4 entries and loaded again gives logits equal
  to the original's bit for bit over a prefill, a verify-sized step and a
  decode step, and every exported matrix is the same.
* Saved as fp32 (the values before quantization) and quantized at load: the
  same bits.
* A file written independently (tests/cog_file.py) with q/k/v and gate/up as
  separate fp32 blocks, non-unit RMSNorm weights and an INT4 lm_head loads
  and matches the oracle stack built from the same weights within 1e-3 of
  max|logits| per row.
* cg_speculative_generate on a loaded target / draft pair emits exactly the
  tokens it emits on the seeded pair they were saved from.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import cog_file
from cogito_amd.capi import last_error
from gpu_util import host_tensor, rel_err_rows, tensor_np
from oracle_lib import ptr
from oracle_model import W_DOWN, W_GU, W_LM, W_O, W_QKV, Cfg, OracleModel

pytestmark = pytest.mark.gpu
TOL = 1e-3

TINY = Cfg(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
           vocab=1024, group_size=128, kv_group_size=64, max_seq=64, max_tokens=8,
           init_std=0.05)


def new_model(gpu, cfg, seed):
    cc = cfg.ctype()
    m = gpu.cgx_model_new(C.byref(cc), seed, None)
    assert m, last_error(gpu)
    return m


def load_model(gpu, cfg, path, share=None):
    cc = cfg.ctype()
    m = gpu.cgx_model_load(C.byref(cc), str(path).encode(), share)
    assert m, last_error(gpu)
    return m


def logits(gpu, m, rows, V):
    out = np.empty((rows, V), np.float32)
    assert gpu.cgx_memcpy_d2h(out.ctypes.data, gpu.cgx_model_logits(m), out.nbytes) == 0
    return out


def run_steps(gpu, m, steps, V):
    outs = []
    for toks in steps:
        M = len(toks)
        assert gpu.cgx_model_forward(m, toks.ctypes.data, M, M, None) == 0, last_error(gpu)
        outs.append(logits(gpu, m, M, V))
    return outs


def exports(gpu, m, cfg):
    out = []
    for layer, which in [(l, w) for l in range(cfg.n_layers) for w in range(4)] + [(0, W_LM)]:
        K, N = cfg.shape(which)
        d = np.zeros(K * N // 2, np.uint8)
        s = np.zeros(K * N // cfg.group_size, np.float32)
        assert gpu.cgx_model_export(m, layer, which, d.ctypes.data, s.ctypes.data) == 0, \
            last_error(gpu)
        out.append((d, s.view(np.uint32)))
    return out


@pytest.mark.parametrize("fp32", [0, 1])
def test_save_load_bit_identical(gpu, rng, tmp_path, fp32):
    m = new_model(gpu, TINY, 17)
    path = tmp_path / f"m{fp32}.cog"
    assert gpu.cgx_model_save(m, str(path).encode(), fp32) == 0, last_error(gpu)
    _, _, ents = cog_file.parse(path)
    names = {e["name"]: e for e in ents}
    assert names["layers.1.mlp_gate_up"]["shape"][:2] == [256, 1024]
    assert names["lm_head"]["dtype"] == (0 if fp32 else 2)
    m2 = load_model(gpu, TINY, path)
    for (d1, s1), (d2, s2) in zip(exports(gpu, m, TINY), exports(gpu, m2, TINY)):
        np.testing.assert_array_equal(d1, d2)
        np.testing.assert_array_equal(s1, s2)
    steps = [rng.integers(0, TINY.vocab, M).astype(np.int32) for M in (7, 5, 1)]
    for a, b in zip(run_steps(gpu, m, steps, TINY.vocab), run_steps(gpu, m2, steps, TINY.vocab)):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    # a loaded model has no seeded fp32 values to save
    assert gpu.cgx_model_save(m2, str(tmp_path / "x.cog").encode(), 1) == -1
    gpu.cgx_clear_error()
    gpu.cgx_model_free(m2)
    gpu.cgx_model_free(m)


def test_reference_style_file_vs_oracle(gpu, oracle, rng, tmp_path):
    c = TINY
    d, hq, hk, ff, V = c.d_model, c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim, c.d_ff, \
        c.vocab
    weights = {"embed": rng.normal(0, 1, (V, d)).astype(np.float32)}
    for l in range(c.n_layers):
        for w in range(4):
            weights[(l, w)] = rng.normal(0, 0.05, c.shape(w)).astype(np.float32)
    weights[W_LM] = rng.normal(0, 0.05, (d, V)).astype(np.float32)
    norms = [rng.uniform(0.5, 1.5, d).astype(np.float32) for _ in range(2 * c.n_layers + 1)]
    ents = [cog_file.fp32_entry("embed", weights["embed"]),
            cog_file.fp32_entry("norm", norms[-1])]
    for l in range(c.n_layers):
        p = f"layers.{l}."
        qkv, gu = weights[(l, W_QKV)], weights[(l, W_GU)]
        ents += [cog_file.fp32_entry(p + "norm1", norms[2 * l]),
                 cog_file.fp32_entry(p + "norm2", norms[2 * l + 1]),
                 # the reference block's separate projections (column blocks)
                 cog_file.fp32_entry(p + "attn_q_proj", qkv[:, :hq]),
                 cog_file.fp32_entry(p + "attn_k_proj", qkv[:, hq:hq + hk]),
                 cog_file.fp32_entry(p + "attn_v_proj", qkv[:, hq + hk:]),
                 cog_file.fp32_entry(p + "attn_o_proj", weights[(l, W_O)]),
                 cog_file.fp32_entry(p + "mlp_gate", gu[:, :ff]),
                 cog_file.fp32_entry(p + "mlp_up", gu[:, ff:]),
                 cog_file.fp32_entry(p + "mlp_down", weights[(l, W_DOWN)])]
    # the lm_head as INT4 entries, quantized by the oracle's cg_quantize_int4
    lm = np.ascontiguousarray(weights[W_LM]).ravel()
    data = np.zeros(lm.size // 2, np.uint8)
    scales = np.zeros(lm.size // c.group_size, np.float32)
    oracle.orc_quantize_int4(ptr(lm), lm.size, c.group_size, ptr(data), ptr(scales))
    ents += cog_file.int4_entries("lm_head", data, scales, d, V, c.group_size)
    path = tmp_path / "ref_style.cog"
    cog_file.write(path, ents)

    m = load_model(gpu, c, path)
    om = OracleModel(oracle, c, 0, weights=weights, norms=norms)
    for M in (6, 5, 1, 3):
        toks = rng.integers(0, V, M).astype(np.int32)
        assert gpu.cgx_model_forward(m, toks.ctypes.data, M, M, None) == 0, last_error(gpu)
        err = rel_err_rows(logits(gpu, m, M, V), om.forward(toks))
        assert err < TOL, (M, err)
    gpu.cgx_model_free(m)


def test_speculative_generate_on_loaded_models(gpu, rng, tmp_path):
    target = Cfg(**{**TINY.__dict__, "max_seq": 96})
    draft = Cfg(**{**target.__dict__, "n_layers": 1})
    tm, dm = new_model(gpu, target, 20), new_model(gpu, draft, 21)
    tp, dp = tmp_path / "t.cog", tmp_path / "d.cog"
    assert gpu.cgx_model_save(tm, str(tp).encode(), 0) == 0, last_error(gpu)
    assert gpu.cgx_model_save(dm, str(dp).encode(), 1) == 0, last_error(gpu)
    tm2, dm2 = load_model(gpu, target, tp), load_model(gpu, draft, dp)
    prompt = np.asarray(rng.integers(0, target.vocab, 7), np.float32).reshape(1, -1)
    gens = []
    for d_, t_ in ((dm, tm), (dm2, tm2)):
        dec = gpu.cg_speculative_decoder_new(d_, t_, 3)
        ids = host_tensor(gpu, prompt)
        gpu.cgx_lcg_seed(99)
        res = gpu.cg_speculative_generate(dec, ids, 20, 0.8, 0.95)
        assert res, last_error(gpu)
        gens.append(tensor_np(gpu, res).ravel().astype(int).tolist())
        gpu.cg_tensor_free(res)
        gpu.cg_tensor_free(ids)
        gpu.cg_speculative_decoder_free(dec)
    assert len(gens[0]) == 7 + 20 and gens[0] == gens[1]
    for m in (tm, dm, tm2, dm2):
        gpu.cgx_model_free(m)
