"""ctypes binding of ``libmans_hip.so`` (the C ABI in ``include/mans_hip.h``).

This module is the thin Python face of the library used by the tests and the
benchmark.  It never computes a search result itself: every search runs the
HIP kernels through the C ABI, and loading fails loudly when the native
library has not been built.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libmans_hip.so"
DATAGEN_PATH = PKG / "libmans_datagen.so"

METRIC_COSINE = 0
METRIC_L2 = 1
METRIC_INNER_PRODUCT = 2
METRIC_HAMMING = 3
METRICS = {"cosine": 0, "l2": 1, "innerProduct": 2, "ip": 2, "hamming": 3}

MAX_TOP_K = 256
EMPTY_ID = 0xFFFFFFFF

OK = 0
DEVICE_NOT_SUPPORTED = -1
DIMENSION_MISMATCH = -2
PIPELINE_UNAVAILABLE = -3
RESOURCE_EXHAUSTED = -4
EXECUTION_FAILED = -5
SEARCH_FAILED = -6
CORRUPT_FILE = -7
ERROR_NAMES = {
    -1: "deviceNotSupported",
    -2: "dimensionMismatch",
    -3: "gpuPipelineUnavailable",
    -4: "gpuResourceExhausted",
    -5: "gpuExecutionFailed",
    -6: "searchFailed",
    -7: "corruptFile",
}
DEGRADEABLE = {-3, -4, -5, -6}  # Errors.swift:21-31

# Every symbol the header declares, in declaration order.
EXPORTS = [
    "mans_last_error", "mans_ctx_create", "mans_ctx_destroy", "mans_corpus_upload_f32",
    "mans_mann_inspect", "mans_corpus_upload_mann", "mans_corpus_write_rows", "mans_corpus_invalidate", "mans_corpus_release",
    "mans_corpus_count", "mans_corpus_dim", "mans_flat_search", "mans_flat_search_device",
    "mans_flat_search_device_noalloc",
    "mans_int8_search", "mans_int8_search_device", "mans_int8_codes_download",
    "mans_ivf_flat_build", "mans_kmeans", "mans_ivf_flat_train", "mans_ivf_flat_search",
    "mans_ivf_flat_search_device", "mans_ivf_download_lists", "mans_ivf_release",
    "mans_ivfpq_train", "mans_ivfpq_build", "mans_ivfpq_search",
    "mans_ivfpq_search_device", "mans_ivfpq_download_codes", "mans_ivfpq_save", "mans_ivfpq_load",
    "mans_ivfpq_release",
    "mans_timing_enable", "mans_timing_read", "mans_timing_reset",
]

NOALLOC_SCRATCH_BYTES = 16 * 1024 * 1024  # MANS_NOALLOC_SCRATCH_BYTES


class ANNSError(RuntimeError):
    """Mirror of ANNSError (Errors.swift:6-19) for the C ABI return codes."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.kind = ERROR_NAMES.get(code, f"error{code}")
        super().__init__(f"{self.kind}: {message}")

    @property
    def is_tier_degradeable(self) -> bool:
        return self.code in DEGRADEABLE


class MannInfo(C.Structure):
    """mans_mann_info: the validated layout of a MANN v3 file."""
    _fields_ = [(name, C.c_uint32) for name in
                ("version", "node_count", "degree", "dim", "metric", "storage_type", "entry_point")] + \
               [(name, C.c_int64) for name in
                ("page_size", "vector_offset", "vector_bytes", "adjacency_offset", "distance_offset",
                 "trailer_offset", "idmap_bytes")]


_lib = None
_datagen = None

_vp = C.c_void_p
_i64 = C.c_int64
_u32 = C.c_uint32
_i32 = C.c_int32
_fp = C.POINTER(C.c_float)


def lib() -> C.CDLL:
    """Loads libmans_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: run `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        L = C.CDLL(str(LIB_PATH))
        L.mans_last_error.restype = C.c_char_p
        L.mans_ctx_create.argtypes = [C.c_int, C.POINTER(_vp)]
        L.mans_ctx_destroy.argtypes = [_vp]
        L.mans_ctx_destroy.restype = None
        L.mans_corpus_upload_f32.argtypes = [_vp, _vp, _i64, _i64, C.POINTER(_vp)]
        L.mans_mann_inspect.argtypes = [C.c_char_p, _i64, C.POINTER(MannInfo)]
        L.mans_corpus_upload_mann.argtypes = [_vp, C.c_char_p, _i64, C.POINTER(_vp),
                                              C.POINTER(_u32)]
        L.mans_corpus_write_rows.argtypes = [_vp, _i64, _vp, _i64]
        L.mans_corpus_invalidate.argtypes = [_vp]
        L.mans_corpus_release.argtypes = [_vp]
        L.mans_corpus_release.restype = None
        L.mans_corpus_count.argtypes = [_vp]
        L.mans_corpus_count.restype = _i64
        L.mans_corpus_dim.argtypes = [_vp]
        L.mans_corpus_dim.restype = _i64
        L.mans_flat_search.argtypes = [_vp, _vp, _vp, _i64, _i64, _u32, _vp, _vp]
        L.mans_flat_search_device.argtypes = [_vp, _vp, _vp, _i64, _i64, _u32, _vp, _vp, _vp]
        L.mans_flat_search_device_noalloc.argtypes = [_vp, _vp, _vp, _i64, _i64, _u32, _vp, _vp,
                                                      _vp]
        L.mans_int8_search.argtypes = [_vp, _vp, _vp, _i64, _i64, _u32, _i32, _i64, _vp, _vp, _vp]
        L.mans_int8_search_device.argtypes = [_vp, _vp, _vp, _i64, _i64, _u32, _i32, _i64, _vp,
                                              _vp, _vp]
        L.mans_int8_codes_download.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp]
        L.mans_ivf_flat_build.argtypes = [_vp, _vp, _vp, _i64, _u32, C.POINTER(_vp)]
        L.mans_kmeans.argtypes = [_vp, _vp, _i64, _i64, _u32, _vp]
        L.mans_ivf_flat_train.argtypes = [_vp, _vp, _i64, _u32, _vp, C.POINTER(_i64)]
        L.mans_ivfpq_train.argtypes = [_vp, _vp, _i64, _i64, _i64, _u32, _vp, _vp]
        L.mans_ivfpq_save.argtypes = [_vp, C.c_char_p]
        L.mans_ivfpq_load.argtypes = [_vp, _vp, C.c_char_p, C.POINTER(_vp)]
        L.mans_ivf_flat_search.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp]
        L.mans_ivf_flat_search_device.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp]
        L.mans_ivf_download_lists.argtypes = [_vp, _vp, _vp]
        L.mans_ivf_release.argtypes = [_vp]
        L.mans_ivf_release.restype = None
        L.mans_ivfpq_build.argtypes = [_vp, _vp, _vp, _i64, _vp, _i64, _u32, C.POINTER(_vp)]
        L.mans_ivfpq_search.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp]
        L.mans_ivfpq_search_device.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp,
                                               _vp]
        L.mans_ivfpq_download_codes.argtypes = [_vp, _vp, _vp]
        L.mans_ivfpq_release.argtypes = [_vp]
        L.mans_ivfpq_release.restype = None
        L.mans_timing_enable.argtypes = [_vp, C.c_int]
        L.mans_timing_read.argtypes = [_vp, C.c_char_p, C.POINTER(C.c_double), C.POINTER(_i64)]
        L.mans_timing_reset.argtypes = [_vp]
        _lib = L
    return _lib


def mann_inspect(path, page_size: int = 0) -> MannInfo:
    """Validates a MANN v3 file (no device needed); raises ANNSError."""
    info = MannInfo()
    _check(lib().mans_mann_inspect(str(path).encode(), page_size, C.byref(info)))
    return info


def _check(rc: int) -> None:
    if rc != OK:
        msg = lib().mans_last_error().decode(errors="replace")
        raise ANNSError(rc, msg)


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def _f32(a, dim: int | None = None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dim is not None:
        a = a.reshape(-1, dim)
    return a


def metric_code(metric) -> int:
    if isinstance(metric, str):
        return METRICS[metric]
    return int(metric)


class Context:
    """A HIP device context (mans_ctx): stream pool, workspaces, timing."""

    def __init__(self, device: int = 0):
        h = _vp()
        _check(lib().mans_ctx_create(device, C.byref(h)))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            lib().mans_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, rows: np.ndarray) -> "Corpus":
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        if rows.ndim != 2:
            raise ValueError("rows must be a 2-D array")
        h = _vp()
        _check(lib().mans_corpus_upload_f32(self.handle, _ptr(rows), rows.shape[0], rows.shape[1],
                                            C.byref(h)))
        return Corpus(self, h, rows.shape[0], rows.shape[1])

    def upload_mann(self, path, page_size: int = 0) -> tuple["Corpus", int]:
        """loadReadOnly(.mmap): the vector section of a MANN v3 file into a
        new corpus; returns (corpus, metric code of the file)."""
        h = _vp()
        metric = _u32()
        _check(lib().mans_corpus_upload_mann(self.handle, str(path).encode(), page_size, C.byref(h),
                                             C.byref(metric)))
        n = lib().mans_corpus_count(h)
        dim = lib().mans_corpus_dim(h)
        return Corpus(self, h, n, dim), metric.value

    # timing ---------------------------------------------------------------
    def timing(self, enable: bool) -> None:
        _check(lib().mans_timing_enable(self.handle, 1 if enable else 0))

    def timing_reset(self) -> None:
        _check(lib().mans_timing_reset(self.handle))

    def timing_read(self, kernel: str) -> tuple[float, int]:
        ms = C.c_double()
        cnt = _i64()
        _check(lib().mans_timing_read(self.handle, kernel.encode(), C.byref(ms), C.byref(cnt)))
        return ms.value, cnt.value


class Corpus:
    """Device-resident corpus (mans_corpus)."""

    def __init__(self, ctx: Context, handle, n: int, dim: int):
        self.ctx = ctx
        self.handle = handle
        self.n = n
        self.dim = dim

    def release(self) -> None:
        if self.handle:
            lib().mans_corpus_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def write_rows(self, first_row: int, rows: np.ndarray) -> None:
        rows = _f32(rows, self.dim)
        _check(lib().mans_corpus_write_rows(self.handle, first_row, _ptr(rows), rows.shape[0]))

    def invalidate(self) -> None:
        _check(lib().mans_corpus_invalidate(self.handle))

    def flat_search(self, queries, k: int, metric="cosine"):
        """Exact flat top-k: (distances, ids), each nq x k."""
        q = _f32(queries, self.dim)
        nq = q.shape[0]
        dist = np.empty((nq, k), dtype=np.float32)
        ids = np.empty((nq, k), dtype=np.uint32)
        _check(lib().mans_flat_search(self.ctx.handle, self.handle, _ptr(q), nq, k,
                                      metric_code(metric), _ptr(dist), _ptr(ids)))
        return dist, ids

    def flat_search_device(self, d_queries: int, nq: int, k: int, metric, d_dist: int,
                           d_ids: int, stream: int | None = None) -> None:
        _check(lib().mans_flat_search_device(self.ctx.handle, self.handle, d_queries, nq, k,
                                             metric_code(metric), d_dist, d_ids, stream))

    def flat_search_device_noalloc(self, d_queries: int, nq: int, k: int, metric, d_dist: int,
                                   d_ids: int, stream: int | None = None) -> None:
        """mans_flat_search_device_noalloc: the same results with no device
        allocation (workspace in the library's fixed scratch array)."""
        _check(lib().mans_flat_search_device_noalloc(self.ctx.handle, self.handle, d_queries, nq,
                                                     k, metric_code(metric), d_dist, d_ids,
                                                     stream))

    def int8_search(self, queries, k: int, metric="cosine", mode: int = 0, budget: int = 0):
        q = _f32(queries, self.dim)
        nq = q.shape[0]
        dist = np.empty((nq, k), dtype=np.float32)
        ids = np.empty((nq, k), dtype=np.uint32)
        rounds = np.empty(nq, dtype=np.int32)
        _check(lib().mans_int8_search(self.ctx.handle, self.handle, _ptr(q), nq, k,
                                      metric_code(metric), mode, budget, _ptr(dist), _ptr(ids),
                                      _ptr(rounds)))
        return dist, ids, rounds

    def int8_search_device(self, d_queries: int, nq: int, k: int, metric, mode: int,
                           budget: int, d_dist: int, d_ids: int,
                           stream: int | None = None) -> None:
        _check(lib().mans_int8_search_device(self.ctx.handle, self.handle, d_queries, nq, k,
                                             metric_code(metric), mode, budget, d_dist, d_ids,
                                             stream))

    def int8_codes(self):
        n, d = self.n, self.dim
        codes = np.empty((n, d), dtype=np.int8)
        planes = [np.empty(n, dtype=np.float32) for _ in range(4)]
        _check(lib().mans_int8_codes_download(self.ctx.handle, self.handle, _ptr(codes),
                                              *[_ptr(p) for p in planes]))
        return (codes, *planes)

    def kmeans(self, k: int, iters: int, metric="l2") -> np.ndarray:
        out = np.empty((k, self.dim), dtype=np.float32)
        _check(lib().mans_kmeans(self.ctx.handle, self.handle, k, iters, metric_code(metric),
                                 _ptr(out)))
        return out

    def ivf_flat_train(self, nlist: int, metric="l2") -> np.ndarray:
        """IVFFlatSearch.buildPartition's sampled 8-iteration k-means:
        min(nlist, n) x dim centroids."""
        out = np.empty((max(1, nlist), self.dim), dtype=np.float32)
        lists = _i64()
        _check(lib().mans_ivf_flat_train(self.ctx.handle, self.handle, nlist, metric_code(metric),
                                         _ptr(out), C.byref(lists)))
        return out[:lists.value]

    def ivfpq_train(self, nlist: int, m: int, iters: int, metric="innerProduct"):
        """_IVFPQIndex.train on these rows: (coarse nlist x dim, codebooks
        m x 256 x dim/m)."""
        coarse = np.empty((nlist, self.dim), dtype=np.float32)
        books = np.empty((m, 256, self.dim // m), dtype=np.float32)
        _check(lib().mans_ivfpq_train(self.ctx.handle, self.handle, nlist, m, iters,
                                      metric_code(metric), _ptr(coarse), _ptr(books)))
        return coarse, books

    def ivf_flat_build(self, centroids, metric="l2") -> "IVFFlat":
        c = _f32(centroids, self.dim)
        h = _vp()
        _check(lib().mans_ivf_flat_build(self.ctx.handle, self.handle, _ptr(c), c.shape[0],
                                         metric_code(metric), C.byref(h)))
        return IVFFlat(self, h, c.shape[0])

    def ivfpq_build(self, coarse, codebooks, metric="innerProduct") -> "IVFPQ":
        c = _f32(coarse, self.dim)
        cb = np.ascontiguousarray(codebooks, dtype=np.float32)
        m = cb.shape[0]
        h = _vp()
        _check(lib().mans_ivfpq_build(self.ctx.handle, self.handle, _ptr(c), c.shape[0], _ptr(cb),
                                      m, metric_code(metric), C.byref(h)))
        return IVFPQ(self.ctx, self, h, c.shape[0], m, self.n, self.dim)


class IVFFlat:
    def __init__(self, corpus: Corpus, handle, nlist: int):
        self.corpus = corpus
        self.handle = handle
        self.nlist = nlist

    def release(self) -> None:
        if self.handle:
            lib().mans_ivf_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def search(self, queries, k: int, nprobe: int, want_probes: bool = False):
        q = _f32(queries, self.corpus.dim)
        nq = q.shape[0]
        dist = np.empty((nq, k), dtype=np.float32)
        ids = np.empty((nq, k), dtype=np.uint32)
        probes = np.empty((nq, min(nprobe, self.nlist)), dtype=np.int32) if want_probes else None
        _check(lib().mans_ivf_flat_search(self.corpus.ctx.handle, self.handle, _ptr(q), nq, k,
                                          nprobe, _ptr(dist), _ptr(ids), _ptr(probes)))
        return (dist, ids, probes) if want_probes else (dist, ids)

    def search_device(self, d_queries: int, nq: int, k: int, nprobe: int, d_dist: int,
                      d_ids: int, stream: int | None = None) -> None:
        _check(lib().mans_ivf_flat_search_device(self.corpus.ctx.handle, self.handle, d_queries,
                                                 nq, k, nprobe, d_dist, d_ids, stream))

    def lists(self):
        offsets = np.empty(self.nlist + 1, dtype=np.int64)
        ids = np.empty(self.corpus.n, dtype=np.uint32)
        _check(lib().mans_ivf_download_lists(self.handle, _ptr(offsets), _ptr(ids)))
        return offsets, ids


class IVFPQ:
    def __init__(self, ctx: Context, corpus: "Corpus | None", handle, nlist: int, m: int, n: int,
                 dim: int):
        self.ctx = ctx
        self.corpus = corpus  # rows of the exact rerank (None after a load without them)
        self.handle = handle
        self.nlist = nlist
        self.m = m
        self.n = n
        self.dim = dim

    def release(self) -> None:
        if self.handle:
            lib().mans_ivfpq_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def search(self, queries, k_adc: int, nprobe: int, rerank_k: int = 0):
        q = _f32(queries, self.dim)
        nq = q.shape[0]
        kout = rerank_k if rerank_k > 0 else k_adc
        score = np.empty((nq, kout), dtype=np.float32)
        ids = np.empty((nq, kout), dtype=np.uint32)
        _check(lib().mans_ivfpq_search(self.ctx.handle, self.handle, _ptr(q), nq, k_adc,
                                       nprobe, rerank_k, _ptr(score), _ptr(ids)))
        return score, ids

    def search_device(self, d_queries: int, nq: int, k_adc: int, nprobe: int, rerank_k: int,
                      d_score: int, d_ids: int, stream: int | None = None) -> None:
        _check(lib().mans_ivfpq_search_device(self.ctx.handle, self.handle, d_queries, nq,
                                              k_adc, nprobe, rerank_k, d_score, d_ids, stream))

    def codes(self):
        codes = np.empty((self.n, self.m), dtype=np.uint8)
        assign = np.empty(self.n, dtype=np.int32)
        _check(lib().mans_ivfpq_download_codes(self.handle, _ptr(codes), _ptr(assign)))
        return codes, assign

    def save(self, path) -> None:
        """Binary persistence (mans_ivfpq_save)."""
        _check(lib().mans_ivfpq_save(self.handle, str(path).encode()))


IVPB_HEADER = struct.Struct("<4s3I2Q2IQ")  # magic, version, dim, metric, n, nlist, m, dsub, reserved


def ivfpq_load(ctx: Context, path, corpus: "Corpus | None" = None) -> IVFPQ:
    """mans_ivfpq_load: a saved index onto the device; `corpus` serves the
    exact rerank."""
    h = _vp()
    _check(lib().mans_ivfpq_load(ctx.handle, corpus.handle if corpus else None,
                                 str(path).encode(), C.byref(h)))
    with open(path, "rb") as f:
        _, _, dim, _, n, nlist, m, _, _ = IVPB_HEADER.unpack(f.read(IVPB_HEADER.size))
    return IVFPQ(ctx, corpus, h, nlist, m, n, dim)
