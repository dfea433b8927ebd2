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
  ".scales" entry, which a reference reader sees as two plain entries.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

from cogito_amd.capi import PQ, CgTensor, host_quant_from_arrays
from gpu_util import host_tensor

HDR = struct.Struct("<III4xQ")                 # magic, version, num_tensors, total_size
ENT = struct.Struct("<64si8iiQQ")              # name, ndim, shape[8], dtype, offset, size
MAGIC = 0x434F4731


def parse(path):
    raw = open(path, "rb").read()
    magic, version, n, _ = HDR.unpack_from(raw, 0)
    ents = []
    for i in range(n):
        name, ndim, *rest = ENT.unpack_from(raw, HDR.size + i * ENT.size)
        shape, dtype, off, size = rest[:8], rest[8], rest[9], rest[10]
        ents.append(dict(name=name.rstrip(b"\0").decode(), ndim=ndim, shape=list(shape),
                         dtype=dtype, data=raw[off:off + size]))
    return magic, version, ents


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
