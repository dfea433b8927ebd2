"""CPU: "COG1" tensor files (include/cg_serialization.h; reference
src/core/serialization.c:9-77) and the INT4 entries of this library.

The reference's serialization.c does not compile as shipped (its header uses
uint32_t without <stdint.h>, and the file is outside the reference's own
build), so the format is pinned by an independent reader and writer here,
written from the struct layout of the reference header
(include/cg_serialization.h:13-27 in the reference: a 24-byte header, then
120-byte directory entries, then the data at the entries' offsets):
* cg_save_model's file parses as the reference writes it, data included;
* a file written the reference's way loads through cg_load_model;
* INT4 tensors round-trip through cgx_save_quantized / cgx_load_quantized bit
  for bit, as an INT4 entry (dtype 2, group size in shape[7]) plus an fp32
  ".scales" entry, which a reference reader sees as two plain entries;
* cg_load_model skips INT4 entries (and says so) and refuses fp32 entries
  whose byte count is not their shape's; cgx_load_quantized refuses shapes
  whose element count overflows;
* cgx_model_load checks a model file's directory before it touches the
  device: a missing, misshapen or wrongly grouped entry is named.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from cog_file import ENT, HDR, MAGIC, fp32_entry, int4_entries, parse, write
from cogito_amd.capi import PQ, CgTensor, host_quant_from_arrays, last_error
from gpu_util import host_tensor


def free_names(ns, n):
    """free() the loader's name strings and array (raw pointers: indexing a
    c_char_p array yields Python copies)."""
    libc = C.CDLL(None)
    raw = C.cast(ns, C.POINTER(C.c_void_p))
    for i in range(n):
        libc.free(C.c_void_p(raw[i]))
    libc.free(C.cast(ns, C.c_void_p))


def test_layout_sizes():
    assert HDR.size == 24 and ENT.size == 120


def test_save_model_matches_reference_layout(lib, tmp_path, rng):
    arrs = [rng.normal(0, 1, (3, 5)).astype(np.float32), np.arange(7, dtype=np.float32),
            rng.normal(0, 1, (2, 2, 2)).astype(np.float32)]
    names = [b"w0", b"bias", b"cube"]
    ts = [host_tensor(lib, a) for a in arrs]
    tarr = (C.POINTER(CgTensor) * 3)(*ts)
    narr = (C.c_char_p * 3)(*names)
    path = tmp_path / "m.cog"
    lib.cg_save_model(str(path).encode(), tarr, narr, 3)
    magic, version, ents = parse(path)
    assert magic == MAGIC and version == 1 and len(ents) == 3
    for e, a, nm in zip(ents, arrs, names):
        assert e["name"] == nm.decode() and e["dtype"] == 0 and e["ndim"] == a.ndim
        assert e["shape"][:a.ndim] == list(a.shape) and e["shape"][a.ndim:] == [0] * (8 - a.ndim)
        np.testing.assert_array_equal(np.frombuffer(e["data"], np.float32), a.ravel())
    for t in ts:
        lib.cg_tensor_free(t)


def test_load_model_reads_reference_files(lib, tmp_path, rng):
    # written exactly as src/core/serialization.c:9-43 does
    arrs = {"a": rng.normal(0, 1, (4, 6)).astype(np.float32),
            "b": rng.normal(0, 1, (5,)).astype(np.float32)}
    off = HDR.size + len(arrs) * ENT.size
    blob = HDR.pack(MAGIC, 1, len(arrs), 0)
    for name, a in arrs.items():
        shape = list(a.shape) + [0] * (8 - a.ndim)
        blob += ENT.pack(name.encode(), a.ndim, *shape, 0, off, a.nbytes)
        off += a.nbytes
    for a in arrs.values():
        blob += a.tobytes()
    path = tmp_path / "ref.cog"
    path.write_bytes(blob)
    ts = C.POINTER(C.POINTER(CgTensor))()
    ns = C.POINTER(C.c_char_p)()
    n = C.c_int(0)
    lib.cg_load_model(str(path).encode(), C.byref(ts), C.byref(ns), C.byref(n))
    assert n.value == 2
    for i, (name, a) in enumerate(arrs.items()):
        assert ns[i].decode() == name
        t = ts[i].contents
        assert [t.shape[d] for d in range(t.ndim)] == list(a.shape)
        np.testing.assert_array_equal(np.ctypeslib.as_array(t.data, shape=(t.size,)), a.ravel())
        lib.cg_tensor_free(ts[i])
    free_names(ns, 2)
    C.CDLL(None).free(C.cast(ts, C.c_void_p))


def test_int4_round_trip(lib, oracle, tmp_path, rng):
    import oracle_lib
    specs = [("wqkv", 256, 384, 128), ("odd", 3, 5, 4), ("wo", 128, 256, 32)]
    qs, keep, ref = [], [], []
    for name, K, N, gs in specs:
        w = rng.normal(0, 0.05, (K, N)).astype(np.float32)
        data, scales = oracle_lib.oracle_quantize(oracle, w, gs)
        q, k = host_quant_from_arrays(data, scales, K, N, gs)
        qs.append(q)
        keep.append(k)
        ref.append((data, scales, K, N, gs))
    qarr = (PQ * 3)(*[C.pointer(q) for q in qs])
    narr = (C.c_char_p * 3)(*[s[0].encode() for s in specs])
    path = tmp_path / "q.cog"
    assert lib.cgx_save_quantized(str(path).encode(), qarr, narr, 3) == 0
    magic, version, ents = parse(path)
    assert magic == MAGIC and len(ents) == 6
    for (name, K, N, gs), (data, scales, *_), e, s in zip(specs, ref, ents[0::2], ents[1::2]):
        assert e["name"] == name and e["dtype"] == 2 and e["ndim"] == 2
        assert e["shape"][:2] == [K, N] and e["shape"][7] == gs
        assert e["data"] == data.tobytes()
        assert s["name"] == name + ".scales" and s["dtype"] == 0 and s["shape"][0] == scales.size
        np.testing.assert_array_equal(np.frombuffer(s["data"], np.float32), scales)
    out = C.POINTER(PQ)()
    ns = C.POINTER(C.c_char_p)()
    n = C.c_int(0)
    assert lib.cgx_load_quantized(str(path).encode(), C.byref(out), C.byref(ns),
                                  C.byref(n)) == 0
    assert n.value == 3
    for i, (name, K, N, gs) in enumerate(specs):
        q = out[i].contents
        data, scales = ref[i][0], ref[i][1]
        assert ns[i].decode() == name and q.group_size == gs and q.size == K * N
        assert [q.shape[0], q.shape[1]] == [K, N] and q.num_groups == scales.size
        np.testing.assert_array_equal(np.ctypeslib.as_array(q.data, shape=(data.size,)), data)
        np.testing.assert_array_equal(np.ctypeslib.as_array(q.scales, shape=(scales.size,)),
                                      scales)
        lib.cg_tensor_quant_free(out[i])
    free_names(ns, 3)
    C.CDLL(None).free(C.cast(out, C.c_void_p))


def test_load_rejects_other_files(lib, tmp_path):
    bad = tmp_path / "bad.cog"
    bad.write_bytes(b"NOPE" + b"\0" * 40)
    out = C.POINTER(PQ)()
    ns = C.POINTER(C.c_char_p)()
    n = C.c_int(0)
    assert lib.cgx_load_quantized(str(bad).encode(), C.byref(out), C.byref(ns),
                                  C.byref(n)) == -1
    lib.cgx_clear_error()


def load_fp32(lib, path):
    ts = C.POINTER(C.POINTER(CgTensor))()
    ns = C.POINTER(C.c_char_p)()
    n = C.c_int(-1)
    lib.cgx_clear_error()
    lib.cg_load_model(str(path).encode(), C.byref(ts), C.byref(ns), C.byref(n))
    return ts, ns, n.value


def test_load_model_skips_int4_entries(lib, oracle, tmp_path, rng):
    import oracle_lib
    w = rng.normal(0, 0.05, (64, 256)).astype(np.float32)
    data, scales = oracle_lib.oracle_quantize(oracle, w, 128)
    q, keep = host_quant_from_arrays(data, scales, 64, 256, 128)
    path = tmp_path / "q.cog"
    assert lib.cgx_save_quantized(str(path).encode(), (PQ * 1)(C.pointer(q)),
                                  (C.c_char_p * 1)(b"w"), 1) == 0
    ts, ns, n = load_fp32(lib, path)
    # only the fp32 ".scales" entry is a tensor; the nibbles are not read as floats
    assert n == 1 and ns[0].decode() == "w.scales"
    t = ts[0].contents
    np.testing.assert_array_equal(np.ctypeslib.as_array(t.data, shape=(t.size,)), scales)
    assert "skipped 1" in last_error(lib)
    lib.cg_tensor_free(ts[0])
    free_names(ns, 1)
    C.CDLL(None).free(C.cast(ts, C.c_void_p))


def test_load_model_refuses_short_fp32_entry(lib, tmp_path):
    e = fp32_entry("a", np.arange(12, dtype=np.float32).reshape(3, 4))
    e["data"] = e["data"][:40]                # 10 of the 12 values
    path = tmp_path / "short.cog"
    write(path, [e])
    _, _, n = load_fp32(lib, path)
    assert n == -1 and "malformed" in last_error(lib)


def test_load_quantized_refuses_overflowing_shape(lib, tmp_path):
    big = 2**31 - 1
    ent = dict(name="w", shape=[big] * 7, gs=128, dtype=2, data=b"\0" * 16)
    path = tmp_path / "big.cog"
    write(path, [ent, fp32_entry("w.scales", np.ones(1, np.float32))])
    out = C.POINTER(PQ)()
    ns = C.POINTER(C.c_char_p)()
    n = C.c_int(0)
    assert lib.cgx_load_quantized(str(path).encode(), C.byref(out), C.byref(ns),
                                  C.byref(n)) == -1
    lib.cgx_clear_error()


# ------------------------------------------------ model files (directory)

SMALL = dict(n_layers=1, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
             vocab=512, group_size=128, kv_group_size=64, max_seq=32, max_tokens=8,
             rope_theta=10000.0, norm_eps=1e-5, init_std=0.02, max_batch=0)


def small_model_entries(rng, drop=(), split=False, gs_file=128):
    c = SMALL
    d, hq, hk, ff, V = (c["d_model"], c["n_heads"] * c["head_dim"],
                        c["n_kv_heads"] * c["head_dim"], c["d_ff"], c["vocab"])
    ents = [fp32_entry("embed", rng.normal(0, 1, (V, d))), fp32_entry("norm", np.ones(d))]
    mats = {"layers.0.attn_o_proj": (hq, d), "layers.0.mlp_down": (ff, d),
            "lm_head": (d, V)}
    if split:
        mats.update({"layers.0.attn_q_proj": (d, hq), "layers.0.attn_k_proj": (d, hk),
                     "layers.0.attn_v_proj": (d, hk), "layers.0.mlp_gate": (d, ff),
                     "layers.0.mlp_up": (d, ff)})
    else:
        mats.update({"layers.0.attn_qkv_proj": (d, hq + 2 * hk),
                     "layers.0.mlp_gate_up": (d, 2 * ff)})
    for name, (K, N) in mats.items():
        if name in drop:
            continue
        if name == "lm_head":   # one INT4 entry, with the file's group size
            data = rng.integers(0, 256, K * N // 2, dtype=np.uint8)
            ents += int4_entries(name, data, np.full(K * N // gs_file, 0.01), K, N, gs_file)
        else:
            ents.append(fp32_entry(name, rng.normal(0, 0.02, (K, N))))
    return [e for e in ents if e["name"] not in drop]


def model_load_error(lib, path):
    from cogito_amd.capi import CgxModelConfig
    cc = CgxModelConfig(**SMALL)
    lib.cgx_clear_error()
    m = lib.cgx_model_load(C.byref(cc), str(path).encode(), None)
    assert not m
    return last_error(lib)


def test_model_load_names_missing_entries(lib, tmp_path, rng):
    path = tmp_path / "m.cog"
    write(path, small_model_entries(rng, drop=("layers.0.mlp_down",)))
    assert "no entry layers.0.mlp_down" in model_load_error(lib, path)
    write(path, small_model_entries(rng, drop=("embed",)))
    assert "no entry embed" in model_load_error(lib, path)
    # split q/k/v with one block missing
    write(path, small_model_entries(rng, split=True, drop=("layers.0.attn_k_proj",)))
    err = model_load_error(lib, path)
    assert "layers.0.attn_qkv_proj" in err and "attn_k_proj" in err


def test_model_load_checks_shapes_and_groups(lib, tmp_path, rng):
    path = tmp_path / "m.cog"
    ents = small_model_entries(rng)
    for e in ents:
        if e["name"] == "layers.0.mlp_down":
            e["shape"] = [256, 512]          # transposed
    write(path, ents)
    assert "layers.0.mlp_down has shape [256, 512]" in model_load_error(lib, path)
    write(path, small_model_entries(rng, gs_file=64))
    assert "lm_head: group size 64" in model_load_error(lib, path)
    ents = small_model_entries(rng)
    for e in ents:
        if e["name"] == "norm":
            e["shape"], e["data"] = [255], e["data"][:1020]
    write(path, ents)
    assert "entry norm must be fp32 of shape [256]" in model_load_error(lib, path)
    (tmp_path / "x.cog").write_bytes(b"NOPE" + b"\0" * 40)
    assert "not a COG1 file" in model_load_error(lib, tmp_path / "x.cog")
