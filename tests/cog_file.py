"""An independent reader and writer of the "COG1" tensor file layout (test
infrastructure), written from the struct layout of the reference header
(include/cg_serialization.h:13-27 in the reference: a 24-byte header, then
120-byte directory entries, then the data at the entries' offsets; the
writer follows src/core/serialization.c:9-43's order).

INT4 entries are this library's extension: dtype 2 with the group size in
shape[7] and the reference's packed nibbles as data, followed by an fp32
entry "<name>.scales".
"""
from __future__ import annotations

import struct

import numpy as np

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


def fp32_entry(name, a):
    a = np.ascontiguousarray(a, np.float32)
    return dict(name=name, shape=list(a.shape), dtype=0, data=a.tobytes())


def int4_entries(name, data, scales, K, N, gs):
    """The two entries of an INT4 matrix [K, N] (flat nibbles, flat scales)."""
    return [dict(name=name, shape=[K, N], gs=gs, dtype=2,
                 data=np.ascontiguousarray(data, np.uint8).tobytes()),
            fp32_entry(name + ".scales", np.ascontiguousarray(scales, np.float32).ravel())]


def write(path, entries):
    """entries: dicts with name, shape, dtype, data (bytes) and, for INT4, gs."""
    off = HDR.size + len(entries) * ENT.size
    head = HDR.pack(MAGIC, 1, len(entries), 0)
    body = b""
    for e in entries:
        shape = list(e["shape"]) + [0] * (8 - len(e["shape"]))
        if e["dtype"] == 2:
            shape[7] = e["gs"]
        head += ENT.pack(e["name"].encode(), len(e["shape"]), *shape, e["dtype"], off,
                         len(e["data"]))
        off += len(e["data"])
        body += e["data"]
    with open(path, "wb") as f:
        f.write(head + body)
