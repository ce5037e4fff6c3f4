"""ctypes binding of liboracle.so -- the CPU restatement of the reference's
exact-search path (see oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's CPU-baseline leg, always as the checker or the timed baseline,
never as a search path of the library.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libdots_ref.so"

_vp, _i64, _i32, _f = C.c_void_p, C.c_int64, C.c_int, C.c_float
_L = None


def lib() -> C.CDLL:
    global _L
    if _L is None:
        if not LIB.exists():
            raise ImportError(f"{LIB} missing: run `make -C oracle`")
        L = C.CDLL(str(LIB))
        L.orc_f32_dot_rows.argtypes = [_vp, _vp, _i64, _i64, _vp]
        L.orc_i8_dot_rows_f32.argtypes = [_vp, _vp, _i64, _i64, _vp]
        L.orc_f32_dot_rows_gather.argtypes = [_vp, _vp, _vp, _i64, _i64, _vp]
        L.orc_row_norms.argtypes = [_vp, _i64, _i64, _vp]
        L.orc_query_norm.argtypes = [_vp, _i64]
        L.orc_query_norm.restype = _f
        L.orc_host_distance.argtypes = [_f, _f, _f, _i32]
        L.orc_host_distance.restype = _f
        L.orc_slice_count.argtypes = [_i64, _i64]
        L.orc_slice_count.restype = _i64
        L.orc_flat_search.argtypes = [_vp, _vp, _i64, _i64, _vp, _i64, _i32, _i64, _i32, _vp, _vp]
        L.orc_flat_search.restype = _i64
        L.orc_flat_search_batch.argtypes = [_vp, _vp, _i64, _i64, _vp, _i64, _i64, _i32, _i64,
                                            _i32, _vp, _vp, _vp]
        L.orc_flat_search_batch.restype = None
        L.orc_int8_build.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp]
        L.orc_int8_quantize_query.argtypes = [_vp, _i64, _f, _vp, _vp]
        L.orc_int8_search.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64,
                                      _i32, _i64, _i32, _i64, _i32, _vp, _vp, _vp]
        L.orc_int8_search.restype = _i64
        L.orc_host_batch_search.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp,
                                            _i64, _i64, _i32, _i64, _i32, _vp, _vp, _vp, _vp]
        L.orc_host_batch_search.restype = None
        L.orc_ivf_assign.argtypes = [_vp, _vp, _i64, _i64, _vp, _vp, _i64, _i32, _vp]
        L.orc_ivf_lists.argtypes = [_vp, _i64, _i64, _vp, _vp]
        L.orc_ivf_probe.argtypes = [_vp, _vp, _i64, _i64, _vp, _i64, _i32, _vp]
        L.orc_ivf_probe.restype = _i64
        L.orc_ivf_search.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64,
                                     _i64, _i32, _vp, _vp, _vp]
        L.orc_ivf_search.restype = _i64
        L.orc_kmeans.argtypes = [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp]
        L.orc_ivf_flat_train.argtypes = [_vp, _i64, _i64, _i64, _i32, _vp]
        L.orc_ivf_flat_train.restype = _i64
        L.orc_ivfpq_train.argtypes = [_vp, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _vp]
        L.orc_ivfpq_train.restype = None
        L.orc_simd_distance.argtypes = [_vp, _vp, _i64, _i32]
        L.orc_simd_distance.restype = _f
        L.orc_nearest_coarse.argtypes = [_vp, _vp, _i64, _i64, _i32]
        L.orc_nearest_coarse.restype = C.c_int32
        L.orc_pq_encode.argtypes = [_vp, _vp, _vp, _i64, _i64, _vp]
        L.orc_ivfpq_encode_rows.argtypes = [_vp, _i64, _i64, _vp, _i64, _vp, _i64, _i32, _vp, _vp]
        L.orc_pq_lut.argtypes = [_vp, _vp, _i64, _i64, _i32, _vp]
        L.orc_sorted_list_run.argtypes = [_vp, _vp, _i64, _i64, _vp, _vp]
        L.orc_sorted_list_run.restype = _i64
        L.orc_ivfpq_probe.argtypes = [_vp, _i64, _i64, _vp, _i64, _i32, _vp, _vp]
        L.orc_ivfpq_probe.restype = _i64
        L.orc_ivfpq_search.argtypes = [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i32, _vp,
                                       _i64, _i64, _vp, _i64, _vp, _vp]
        L.orc_ivfpq_search.restype = _i64
        L.orc_distances_for_ids.argtypes = [_vp, _vp, _i64, _vp, _vp, _i64, _i32, _vp]
        L.orc_distances_for_ids.restype = None
        _L = L
    return _L


def ref_lib() -> C.CDLL | None:
    """The reference's own dots.c built by `make -C oracle ref` (None if absent)."""
    if not REF_LIB.exists():
        return None
    L = C.CDLL(str(REF_LIB))
    L.mans_f32_dot_rows.argtypes = [_vp, _vp, _i64, _i64, _vp]
    L.mans_i8_dot_rows_f32.argtypes = [_vp, _vp, _i64, _i64, _vp]
    L.mans_f32_dot_rows_gather.argtypes = [_vp, _vp, _vp, _i64, _i64, _vp]
    return L


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a):
    return None if a is None else a.ctypes.data


def f32_dot_rows(corpus, q):
    corpus, q = _c(corpus, np.float32), _c(q, np.float32)
    out = np.empty(corpus.shape[0], np.float32)
    lib().orc_f32_dot_rows(_p(corpus), _p(q), corpus.shape[0], corpus.shape[1], _p(out))
    return out


def i8_dot_rows(codes, qcodes):
    codes, qcodes = _c(codes, np.int8), _c(qcodes, np.int8)
    out = np.empty(codes.shape[0], np.float32)
    lib().orc_i8_dot_rows_f32(_p(codes), _p(qcodes), codes.shape[0], codes.shape[1], _p(out))
    return out


def f32_dot_rows_gather(corpus, q, idx):
    corpus, q, idx = _c(corpus, np.float32), _c(q, np.float32), _c(idx, np.uint32)
    out = np.empty(idx.shape[0], np.float32)
    lib().orc_f32_dot_rows_gather(_p(corpus), _p(q), _p(idx), idx.shape[0], corpus.shape[1],
                                  _p(out))
    return out


def row_norms(corpus):
    corpus = _c(corpus, np.float32)
    out = np.empty(corpus.shape[0], np.float32)
    lib().orc_row_norms(_p(corpus), corpus.shape[0], corpus.shape[1], _p(out))
    return out


def host_distance(dot, qn, vn, metric: int) -> float:
    return lib().orc_host_distance(dot, qn, vn, metric)


def flat_search(corpus, norms, q, k, metric, cores=None, threads=1):
    corpus, q = _c(corpus, np.float32), _c(q, np.float32)
    norms = _c(norms, np.float32) if norms is not None else None
    cores = cores or os.cpu_count() or 1
    kk = min(k, 256)
    dist = np.empty(kk, np.float32)
    ids = np.empty(kk, np.uint32)
    m = lib().orc_flat_search(_p(corpus), _p(norms), corpus.shape[0], corpus.shape[1], _p(q), k,
                              metric, cores, threads, _p(dist), _p(ids))
    return dist[:m], ids[:m]


def flat_search_batch(corpus, norms, queries, k, metric, cores=None, threads=None):
    corpus, queries = _c(corpus, np.float32), _c(queries, np.float32)
    norms = _c(norms, np.float32) if norms is not None else None
    cores = cores or os.cpu_count() or 1
    threads = threads or os.cpu_count() or 1
    nq = queries.shape[0]
    kk = min(k, 256)
    dist = np.full((nq, kk), np.finfo(np.float32).max, np.float32)
    ids = np.full((nq, kk), 0xFFFFFFFF, np.uint32)
    counts = np.empty(nq, np.int64)
    lib().orc_flat_search_batch(_p(corpus), _p(norms), corpus.shape[0], corpus.shape[1],
                                _p(queries), nq, k, metric, cores, threads, _p(dist), _p(ids),
                                _p(counts))
    return dist, ids, counts


def int8_build(corpus):
    corpus = _c(corpus, np.float32)
    n, d = corpus.shape
    codes = np.empty((n, d), np.int8)
    planes = [np.empty(n, np.float32) for _ in range(4)]
    lib().orc_int8_build(_p(corpus), n, d, _p(codes), *[_p(p) for p in planes])
    return (codes, *planes)


def int8_search(corpus, norms, planes, q, k, metric, cores=None, mode=0, budget=0,
                enforce_min_count=True):
    corpus, q = _c(corpus, np.float32), _c(q, np.float32)
    norms = _c(norms, np.float32) if norms is not None else None
    codes, u, w, ns, inv = planes
    cores = cores or os.cpu_count() or 1
    kk = min(k, 256)
    dist = np.empty(kk, np.float32)
    ids = np.empty(kk, np.uint32)
    fb = _i64()
    m = lib().orc_int8_search(_p(corpus), _p(norms), _p(codes), _p(u), _p(w), _p(ns), _p(inv),
                              corpus.shape[0], corpus.shape[1], _p(q), k, metric, cores, mode,
                              budget, 1 if enforce_min_count else 0, _p(dist), _p(ids),
                              C.byref(fb))
    if m < 0:
        return None
    return dist[:m], ids[:m], fb.value


def host_batch_search(corpus, norms, planes, queries, k, metric, cores=None, threads=None):
    """HostBatchWork.run over a batch: int8 bounded scan per query when
    planes are given and n >= 16384, else the fp32 host scan.  Returns
    (dist, ids, counts, route) with route 1 for the int8 scan."""
    corpus, queries = _c(corpus, np.float32), _c(queries, np.float32)
    norms = _c(norms, np.float32) if norms is not None else None
    codes, u, w, ns, inv = planes if planes is not None else (None,) * 5
    cores = cores or os.cpu_count() or 1
    threads = threads or os.cpu_count() or 1
    nq = queries.shape[0]
    kk = min(k, 256)
    dist = np.full((nq, kk), np.finfo(np.float32).max, np.float32)
    ids = np.full((nq, kk), 0xFFFFFFFF, np.uint32)
    counts = np.empty(nq, np.int64)
    route = np.empty(nq, np.int32)
    lib().orc_host_batch_search(_p(corpus), _p(norms), _p(codes), _p(u), _p(w), _p(ns), _p(inv),
                                corpus.shape[0], corpus.shape[1], _p(queries), nq, k, metric,
                                cores, threads, _p(dist), _p(ids), _p(counts), _p(route))
    return dist, ids, counts, route


def ivf_assign(rows, centroids, metric):
    rows, centroids = _c(rows, np.float32), _c(centroids, np.float32)
    rn, cn = row_norms(rows), row_norms(centroids)
    out = np.empty(rows.shape[0], np.int32)
    lib().orc_ivf_assign(_p(rows), _p(rn), rows.shape[0], rows.shape[1], _p(centroids), _p(cn),
                         centroids.shape[0], metric, _p(out))
    return out


def ivf_lists(assign, nlist):
    assign = _c(assign, np.int32)
    offsets = np.empty(nlist + 1, np.int64)
    ids = np.empty(assign.shape[0], np.uint32)
    lib().orc_ivf_lists(_p(assign), assign.shape[0], nlist, _p(offsets), _p(ids))
    return offsets, ids


class IVFPartition:
    """IVFFlatSearch.Partition restated (IVFFlatSearch.swift:39-95, 517-631),
    built from given centroids."""

    def __init__(self, rows, centroids, metric):
        rows, centroids = _c(rows, np.float32), _c(centroids, np.float32)
        self.metric = metric
        self.dim = rows.shape[1]
        self.count = rows.shape[0]
        self.nlist = centroids.shape[0]
        self.centroids = centroids
        self.cnorms = row_norms(centroids)
        self.assign = ivf_assign(rows, centroids, metric)
        self.offsets, self.list_ids = ivf_lists(self.assign, self.nlist)
        self.packed = _c(rows[self.list_ids], np.float32)
        self.packed_norms = row_norms(self.packed)

    def probe(self, q, nprobe):
        q = _c(q, np.float32)
        out = np.empty(max(1, min(nprobe, self.nlist)), np.int32)
        m = lib().orc_ivf_probe(_p(self.centroids), _p(self.cnorms), self.nlist, self.dim, _p(q),
                                nprobe, self.metric, _p(out))
        return out[:m]

    def search(self, q, k, nprobe):
        q = _c(q, np.float32)
        dist = np.empty(k, np.float32)
        ids = np.empty(k, np.uint32)
        probes = np.empty(max(1, min(nprobe, self.nlist)), np.int32)
        m = lib().orc_ivf_search(_p(self.packed), _p(self.packed_norms), _p(self.offsets),
                                 _p(self.list_ids), _p(self.centroids), _p(self.cnorms),
                                 self.nlist, self.count, self.dim, _p(q), k, nprobe, self.metric,
                                 _p(dist), _p(ids), _p(probes))
        return dist[:m], ids[:m], probes


def kmeans(rows, k, iters, metric):
    rows = _c(rows, np.float32)
    cent = np.empty((k, rows.shape[1]), np.float32)
    assign = np.empty(rows.shape[0], np.int32)
    lib().orc_kmeans(_p(rows), rows.shape[0], rows.shape[1], k, iters, metric, _p(cent),
                     _p(assign))
    return cent, assign


def ivf_flat_train(rows, nlist, metric):
    """buildPartition's sampled k-means: (L x dim centroids)."""
    rows = _c(rows, np.float32)
    n, d = rows.shape
    cent = np.empty((max(1, min(max(1, nlist), n)), d), np.float32)
    lists = lib().orc_ivf_flat_train(_p(rows), n, d, nlist, metric, _p(cent))
    return cent[:lists]


def ivfpq_train(rows, nlist, m, iters, metric):
    """_IVFPQIndex.train: (coarse nlist x dim, codebooks m x 256 x dim/m)."""
    rows = _c(rows, np.float32)
    n, d = rows.shape
    coarse = np.empty((nlist, d), np.float32)
    books = np.empty((m, 256, d // m), np.float32)
    lib().orc_ivfpq_train(_p(rows), n, d, nlist, m, iters, metric, _p(coarse), _p(books))
    return coarse, books


def simd_distance(a, b, metric):
    a, b = _c(a, np.float32), _c(b, np.float32)
    return lib().orc_simd_distance(_p(a), _p(b), a.shape[0], metric)


def pq_encode_rows(rows, coarse, codebooks, metric):
    rows, coarse, codebooks = _c(rows, np.float32), _c(coarse, np.float32), _c(codebooks, np.float32)
    n, d = rows.shape
    m = codebooks.shape[0]
    assign = np.empty(n, np.int32)
    codes = np.empty((n, m), np.uint8)
    lib().orc_ivfpq_encode_rows(_p(rows), n, d, _p(coarse), coarse.shape[0], _p(codebooks), m,
                                metric, _p(assign), _p(codes))
    return assign, codes


def pq_lut(qres, codebooks, metric):
    qres, codebooks = _c(qres, np.float32), _c(codebooks, np.float32)
    m, _, dsub = codebooks.shape
    lut = np.empty((m, 256), np.float32)
    lib().orc_pq_lut(_p(qres), _p(codebooks), m, dsub, metric, _p(lut))
    return lut


def sorted_list_run(scores, ids, cap):
    scores, ids = _c(scores, np.float32), _c(ids, np.uint32)
    os_ = np.empty(max(cap, 1), np.float32)
    oi = np.empty(max(cap, 1), np.uint32)
    m = lib().orc_sorted_list_run(_p(scores), _p(ids), scores.shape[0], cap, _p(os_), _p(oi))
    return os_[:m], oi[:m]


def ivfpq_probe(coarse, q, nprobe, metric):
    coarse, q = _c(coarse, np.float32), _c(q, np.float32)
    out = np.empty(max(1, min(nprobe, coarse.shape[0])), np.int32)
    dist = np.empty_like(out, dtype=np.float32)
    m = lib().orc_ivfpq_probe(_p(coarse), coarse.shape[0], coarse.shape[1], _p(q), nprobe, metric,
                              _p(out), _p(dist))
    return out[:m], dist[:m]


def ivfpq_search(coarse, codebooks, codes, offsets, list_ids, metric, q, k, nprobe, rows=None,
                 rerank_k=0):
    coarse, codebooks, codes = (_c(coarse, np.float32), _c(codebooks, np.float32),
                                _c(codes, np.uint8))
    offsets, list_ids, q = _c(offsets, np.int64), _c(list_ids, np.uint32), _c(q, np.float32)
    rows = _c(rows, np.float32) if rows is not None else None
    kout = rerank_k if (rows is not None and rerank_k > 0) else k
    score = np.empty(max(k, kout), np.float32)
    ids = np.empty(max(k, kout), np.uint32)
    m = lib().orc_ivfpq_search(_p(coarse), coarse.shape[0], coarse.shape[1], _p(codebooks),
                               codebooks.shape[0], _p(codes), _p(offsets), _p(list_ids), metric,
                               _p(q), k, nprobe, _p(rows), rerank_k, _p(score), _p(ids))
    return score[:m], ids[:m]


def distances_for_ids(corpus, norms, q, ids, metric):
    corpus, q, ids = _c(corpus, np.float32), _c(q, np.float32), _c(ids, np.uint32)
    norms = _c(norms, np.float32) if norms is not None else None
    out = np.empty(ids.shape[0], np.float32)
    lib().orc_distances_for_ids(_p(corpus), _p(norms), corpus.shape[1], _p(q), _p(ids),
                                ids.shape[0], metric, _p(out))
    return out
