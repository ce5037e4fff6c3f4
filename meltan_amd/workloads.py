"""Seeded synthetic workloads for the four scans (generator in datagen.c).

Sizes follow the benchmark configurations of the exact, int8, IVF-flat and
IVF-PQ scans.  Generation is split across threads by row range; every row
has its own random stream, so the bytes do not depend on the split.
"""
from __future__ import annotations

import concurrent.futures as cf
import ctypes as C
import hashlib
import os
from pathlib import Path

import numpy as np

from . import DATAGEN_PATH

_dg = None


def datagen() -> C.CDLL:
    global _dg
    if _dg is None:
        if not Path(DATAGEN_PATH).exists():
            raise ImportError(f"{DATAGEN_PATH} is missing: build the package first")
        L = C.CDLL(str(DATAGEN_PATH))
        L.mans_gen_gauss_rows.argtypes = [C.c_uint64, C.c_int64, C.c_int64, C.c_int64, C.c_int,
                                          C.c_void_p]
        L.mans_gen_centers.argtypes = [C.c_uint64, C.c_int64, C.c_int64, C.c_void_p]
        L.mans_gen_mixture_rows.argtypes = [C.c_uint64, C.c_void_p, C.c_int64, C.c_int64,
                                            C.c_double, C.c_int64, C.c_int64, C.c_int, C.c_void_p,
                                            C.c_void_p]
        L.mans_gen_noisy_queries.argtypes = [C.c_uint64, C.c_void_p, C.c_int64, C.c_int64,
                                             C.c_double, C.c_int64, C.c_int64, C.c_void_p,
                                             C.c_void_p]
        L.mans_gen_lcg.argtypes = [C.c_int, C.c_uint64, C.c_int64, C.c_void_p]
        L.mans_gen_lcg.restype = None
        _dg = L
    return _dg


def _threads(threads: int | None) -> int:
    if threads:
        return threads
    return max(1, min(16, os.cpu_count() or 1))


def _split(n: int, parts: int):
    step = max(1, (n + parts - 1) // parts)
    return [(s, min(n, s + step)) for s in range(0, n, step)]


def gauss_rows(seed: int, n: int, dim: int, normalize: bool = True,
               threads: int | None = None) -> np.ndarray:
    out = np.empty((n, dim), dtype=np.float32)
    L = datagen()

    def work(r):
        s, e = r
        rc = L.mans_gen_gauss_rows(seed, s, e - s, dim, 1 if normalize else 0,
                                   out[s:e].ctypes.data)
        if rc != 0:
            raise ValueError("gauss_rows: bad shape")

    with cf.ThreadPoolExecutor(_threads(threads)) as ex:
        list(ex.map(work, _split(n, 4 * _threads(threads))))
    return out


def centers(seed: int, ncenters: int, dim: int) -> np.ndarray:
    out = np.empty((ncenters, dim), dtype=np.float64)
    if datagen().mans_gen_centers(seed, ncenters, dim, out.ctypes.data) != 0:
        raise ValueError("centers: bad shape")
    return out


def mixture_rows(seed: int, ctr: np.ndarray, sigma: float, n: int, normalize: bool,
                 row0: int = 0, threads: int | None = None):
    ncenters, dim = ctr.shape
    out = np.empty((n, dim), dtype=np.float32)
    which = np.empty(n, dtype=np.uint32)
    L = datagen()

    def work(r):
        s, e = r
        rc = L.mans_gen_mixture_rows(seed, ctr.ctypes.data, ncenters, dim, sigma, row0 + s, e - s,
                                     1 if normalize else 0, out[s:e].ctypes.data,
                                     which[s:e].ctypes.data)
        if rc != 0:
            raise ValueError("mixture_rows: bad shape")

    with cf.ThreadPoolExecutor(_threads(threads)) as ex:
        list(ex.map(work, _split(n, 4 * _threads(threads))))
    return out, which


def noisy_queries(seed: int, db: np.ndarray, nq: int, noise: float = 0.1):
    n, dim = db.shape
    out = np.empty((nq, dim), dtype=np.float32)
    src = np.empty(nq, dtype=np.uint32)
    if datagen().mans_gen_noisy_queries(seed, db.ctypes.data, n, dim, noise, 0, nq,
                                        out.ctypes.data, src.ctypes.data) != 0:
        raise ValueError("noisy_queries: bad shape")
    return out, src


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# --- the benchmark workloads ----------------------------------------------------

def flat_10k(nq: int = 1000):
    """Exact cosine, 10,000 x 384 N(0,1) normalised (seed 1001), queries seed 1002."""
    db = gauss_rows(1001, 10_000, 384, True)
    q = gauss_rows(1002, nq, 384, True)
    return db, q


def flat_100k(nq: int = 1024):
    """Exact cosine, 100,000 x 384 normalised (seed 2001); queries (seed 2002):
    even indices noisy copies row + 0.1 N(0,1), odd indices random."""
    db = gauss_rows(2001, 100_000, 384, True)
    q, _ = noisy_queries(2002, db, nq, 0.1)
    return db, q


def mixture_1m_384(nq: int = 1024, n: int = 1_000_000):
    """1,000,000 x 384 from 1,000 centres, sigma 0.3, normalised (seed 3001);
    queries from the same mixture (seed 3002)."""
    ctr = centers(3001, 1000, 384)
    db, _ = mixture_rows(3001, ctr, 0.3, n, True)
    q, _ = mixture_rows(3002, ctr, 0.3, nq, True)
    return db, q


def mixture_1m_128(nq: int = 1024, n: int = 1_000_000):
    """IVF-flat L2 workload: 1,000,000 x 128 from 4,096 centres, sigma 0.25,
    not normalised (seed 4001); queries seed 4002."""
    ctr = centers(4001, 4096, 128)
    db, _ = mixture_rows(4001, ctr, 0.25, n, False)
    q, _ = mixture_rows(4002, ctr, 0.25, nq, False)
    return db, q


def mixture_10m_96(nq: int = 1024, n: int = 10_000_000):
    """IVF-PQ inner-product workload: 10,000,000 x 96 from 8,192 centres,
    sigma 0.25 (seed 5001); queries seed 5002."""
    ctr = centers(5001, 8192, 96)
    db, _ = mixture_rows(5001, ctr, 0.25, n, False)
    q, _ = mixture_rows(5002, ctr, 0.25, nq, False)
    return db, q, ctr


def mixture_10m_96_train(n: int = 262_144):
    """The IVF-PQ training sample: 262,144 rows of the same 8,192-centre
    mixture (seed 5003)."""
    ctr = centers(5001, 8192, 96)
    rows, _ = mixture_rows(5003, ctr, 0.25, n, False)
    return rows


# Test-suite generators of the reference, restated (reproducible in C):
# FlatSearchTests.swift:15-22 and BoundedExactScanTests.swift:23-34.

def lcg_vectors(kind: int, count: int, dim: int, seed: int) -> np.ndarray:
    """kind 0: FlatSearchTests.seededVectors; kind 1: BoundedExactScanTests.SeededGenerator."""
    out = np.empty((count, dim), dtype=np.float32)
    datagen().mans_gen_lcg(kind, seed & ((1 << 64) - 1), count * dim, out.ctypes.data)
    return out
