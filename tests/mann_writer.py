"""Writes MANN v3 index files as IndexSerializer.saveMmapCompatible does
(IndexSerializer.swift:74-140): the 28-byte little-endian header ("MANN",
version 3, node count, degree, dim, metric code, storage type), page padding,
the vector section, padding, adjacency (node count x degree u32), padding,
distances (node count x degree f32), padding, then the IDMap byte count, the
IDMap payload and the entry point.  Test infrastructure: the files feed the
loader's parity and corruption tests."""
from __future__ import annotations

import json
import struct

import numpy as np


def idmap_json(n: int, numeric: int = 0) -> bytes:
    """An IDMap as JSONEncoder writes it (IDMap.swift:113-120): external ids
    "e0".."e{n-1}" for the first n - numeric rows, numeric keys for the rest;
    dictionaries with integer keys are flat arrays of alternating key and
    value."""
    named = n - numeric
    e2i = {f"e{i}": i for i in range(named)}
    i2e = [x for i in range(named) for x in (i, f"e{i}")]
    n2i = [x for i in range(named, n) for x in (1000 + i, i)]
    i2n = [x for i in range(named, n) for x in (i, 1000 + i)]
    return json.dumps({"externalToInternal": e2i, "internalToExternal": i2e, "nextID": n,
                       "numericToInternal": n2i, "internalToNumeric": i2n},
                      separators=(",", ":")).encode()


def _pad(buf: bytearray, page: int) -> None:
    buf.extend(b"\0" * ((page - len(buf) % page) % page))


def mann_v3_bytes(vectors: np.ndarray, degree: int = 4, metric: int = 0, page: int = 4096,
                  storage: int | None = None, dim: int | None = None, idmap: bytes | None = None,
                  entry_point: int = 0, version: int = 3, magic: bytes = b"MANN") -> bytes:
    n = vectors.shape[0]
    if storage is None:
        storage = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.uint8): 2}[vectors.dtype]
    if dim is None:
        dim = vectors.shape[1] * (8 if storage == 2 else 1)
    if idmap is None:
        idmap = idmap_json(n)
    buf = bytearray(magic)
    buf += struct.pack("<6I", version, n, degree, dim, metric, storage)
    _pad(buf, page)
    buf += np.ascontiguousarray(vectors).tobytes()
    _pad(buf, page)
    rng = np.random.default_rng(n)
    buf += rng.integers(0, max(n, 1), (n, degree), dtype=np.uint32).tobytes()
    _pad(buf, page)
    buf += rng.random((n, degree), dtype=np.float32).tobytes()
    _pad(buf, page)
    buf += struct.pack("<I", len(idmap)) + idmap + struct.pack("<I", entry_point)
    return bytes(buf)


def write_mann_v3(path, vectors: np.ndarray, **kw) -> None:
    with open(path, "wb") as f:
        f.write(mann_v3_bytes(vectors, **kw))
