"""MANN v3 file validation (mans_mann_inspect), no device needed.

The rules follow MmapIndexLoader.load (MmapIndexLoader.swift:38-196): magic,
version 3 only, metric and storage codes, non-zero node count and degree,
binary dims divisible by 8, page-aligned sections within the file, the
trailer's IDMap within the file, an IDMap payload that decodes with as
many entries as nodes (MmapIndexLoader.swift:174-182) and the entry point
below the node count; every failure is ANNSError.corruptFile with the
reference's reason.
"""
import struct

import numpy as np
import pytest

import meltan_amd as M
from mann_writer import idmap_json, mann_v3_bytes


def _inspect(tmp_path, data: bytes, page=4096):
    p = tmp_path / "index.mann"
    p.write_bytes(data)
    return M.mann_inspect(p, page)


@pytest.mark.parametrize("page", [4096, 16384])
def test_layout_of_a_valid_file(tmp_path, page):
    vec = np.arange(50 * 12, dtype=np.float32).reshape(50, 12)
    info = _inspect(tmp_path, mann_v3_bytes(vec, degree=3, metric=2, page=page, entry_point=7), page)
    assert (info.version, info.node_count, info.degree, info.dim) == (3, 50, 3, 12)
    assert (info.metric, info.storage_type, info.entry_point) == (2, 0, 7)
    assert info.page_size == page
    assert info.vector_offset == page and info.vector_bytes == 50 * 12 * 4
    # Each section starts on the next page boundary after the previous one.
    assert info.adjacency_offset == page * 2
    assert info.distance_offset == page * 3
    assert info.trailer_offset == page * 4
    assert info.idmap_bytes == len(idmap_json(50))


def test_f16_and_binary_storage_are_described(tmp_path):
    info = _inspect(tmp_path, mann_v3_bytes(np.zeros((10, 8), np.float16)))
    assert info.storage_type == 1 and info.vector_bytes == 10 * 8 * 2
    info = _inspect(tmp_path, mann_v3_bytes(np.zeros((10, 4), np.uint8)))
    assert info.storage_type == 2 and info.dim == 32 and info.vector_bytes == 40


def _corrupt(tmp_path, data, reason):
    with pytest.raises(M.ANNSError) as ei:
        _inspect(tmp_path, data)
    assert ei.value.code == M.CORRUPT_FILE and not ei.value.is_tier_degradeable
    assert reason in str(ei.value), str(ei.value)


def test_corrupt_files(tmp_path):
    vec = np.ones((20, 8), np.float32)
    good = mann_v3_bytes(vec)
    _corrupt(tmp_path, b"MANX" + good[4:], "Invalid file magic")
    _corrupt(tmp_path, mann_v3_bytes(vec, version=2), "requires version 3, found 2")
    _corrupt(tmp_path, good[:20], "Unexpected EOF")
    _corrupt(tmp_path, mann_v3_bytes(vec, metric=9), "Unsupported metric code")
    _corrupt(tmp_path, mann_v3_bytes(vec, storage=5), "Unsupported storage type 5")
    _corrupt(tmp_path, mann_v3_bytes(vec, degree=0), "Degree must be greater than zero")
    zero = bytearray(good)
    zero[8:12] = struct.pack("<I", 0)
    _corrupt(tmp_path, bytes(zero), "Node count must be greater than zero")
    _corrupt(tmp_path, mann_v3_bytes(np.zeros((4, 2), np.uint8), dim=12), "not divisible by 8")
    # Sections past the end of the file.
    _corrupt(tmp_path, good[:4096 + 100], "truncated")
    # The trailer's IDMap runs past the end.
    _corrupt(tmp_path, good[:-3], "Truncated IDMap payload")
    _corrupt(tmp_path, mann_v3_bytes(vec, entry_point=20), "Entry point is out of bounds")
    # Counts whose section sizes overflow 64 bits (checkedMultiply).
    huge = bytearray(good)
    huge[8:12] = struct.pack("<I", 0xFFFFFFFF)
    huge[16:20] = struct.pack("<I", 0xFFFFFFFF)
    _corrupt(tmp_path, bytes(huge), "Integer overflow")


def test_idmap_payload_is_decoded_and_counted(tmp_path):
    vec = np.ones((6, 4), np.float32)
    ok = [
        idmap_json(6),
        idmap_json(6, numeric=2),  # IDMap.count adds the numeric keys
        # Optional numeric maps absent or null; unknown keys ignored; the
        # object form of an integer-keyed dictionary.
        b'{"externalToInternal":{"a":0,"b":1,"c":2,"d":3,"e":4,"f":5},'
        b'"internalToExternal":{"0":"a","1":"b"},"nextID":6,"extra":[1,{"x":null}]}',
        b' {"nextID":6,"internalToExternal":[],"numericToInternal":null,'
        b'"externalToInternal":{"a\\u0062":0,"b":1,"c":2,"d":3,"e":4,"\\n":5}} ',
    ]
    for payload in ok:
        assert _inspect(tmp_path, mann_v3_bytes(vec, idmap=payload)).node_count == 6
    corrupt = [
        b"{}",  # required keys missing
        b"",
        b"[]",
        b'{"externalToInternal":{"a":0},"internalToExternal":[0],"nextID":1}',  # odd array
        b'{"externalToInternal":{"a":-1},"internalToExternal":[],"nextID":1}',
        b'{"externalToInternal":{"a":4294967296},"internalToExternal":[],"nextID":1}',
        b'{"externalToInternal":{"a":1.5},"internalToExternal":[],"nextID":1}',
        b'{"externalToInternal":{"a":0},"internalToExternal":[],"nextID":1} x',
        idmap_json(6)[:-1],
    ]
    for payload in corrupt:
        _corrupt(tmp_path, mann_v3_bytes(vec, idmap=payload), "IDMap payload is corrupt")
    # Decodes, but with fewer (or duplicate) entries than nodes.
    _corrupt(tmp_path, mann_v3_bytes(vec, idmap=idmap_json(5)), "ID map size does not match node count")
    dup = b'{"externalToInternal":{"a":0,"a":1,"b":2,"c":3,"d":4,"e":5},"internalToExternal":[],"nextID":6}'
    _corrupt(tmp_path, mann_v3_bytes(vec, idmap=dup), "ID map size does not match node count")


def test_missing_file_is_reported(tmp_path):
    with pytest.raises(M.ANNSError) as ei:
        M.mann_inspect(tmp_path / "absent.mann")
    assert ei.value.code == M.CORRUPT_FILE
