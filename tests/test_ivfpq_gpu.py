"""Parity of the HIP IVF-PQ build and ADC probe scan.

The bar (IVFPQIndex.swift:106-226, 418-452, 484-550; ProductQuantizer.swift:
120-169, 223-253; BoundedSelection.swift:158-214):
  - coarse assignments and PQ codes bit-identical to the oracle's
    restatement for the same coarse centroids and codebooks;
  - ADC results identical to the oracle's: the same scores bit for bit and
    the same ids in the same order (BoundedSortedList order, newest first
    among equal scores), including inputs built to tie;
  - with rerank_k > 0 (a step with no counterpart in the reference), the
    exact host distances of the k_adc candidates, best rerank_k by
    (distance, id), equal the oracle's.
"""
import numpy as np
import pytest

import meltan_amd as M
from meltan_amd import workloads
from oracle import oracle
from test_flat_gpu import COS, IP, L2

pytestmark = pytest.mark.gpu


def _books_from_rows(rows, m, seed):
    """Codebooks [m][256][dsub] taken from row subvectors (any fixed codebook
    pins the encode and ADC arithmetic)."""
    n, d = rows.shape
    dsub = d // m
    rng = np.random.default_rng(seed)
    pick = rng.choice(n, size=256, replace=False)
    return np.ascontiguousarray(rows[pick].reshape(256, m, dsub).transpose(1, 0, 2)).astype(np.float32)


def _oracle_index(rows, coarse, books, metric):
    assign, codes = oracle.pq_encode_rows(rows, coarse, books, metric)
    offsets, ids = oracle.ivf_lists(assign, coarse.shape[0])
    return assign, codes, offsets, ids


@pytest.mark.parametrize("metric", [L2, IP, COS])
@pytest.mark.parametrize("dim,m", [(32, 8), (96, 48)])
def test_ivfpq_codes_and_adc_match_oracle(gpu_ctx, metric, dim, m):
    n, nlist = 6000, 24
    rows = workloads.lcg_vectors(1, n, dim, seed=700 + dim + metric)
    coarse = rows[:: n // nlist][:nlist].copy()
    books = _books_from_rows(rows, m, seed=701 + dim)
    assign, codes, offsets, ids = _oracle_index(rows, coarse, books, metric)
    c = gpu_ctx.upload(rows)
    pq = c.ivfpq_build(coarse, books, metric)
    gcodes, gassign = pq.codes()
    assert np.array_equal(gassign, assign)
    assert np.array_equal(gcodes, codes)
    queries = workloads.lcg_vectors(1, 12, dim, seed=702 + dim)
    for nprobe in (1, 3, 8):
        for k in (1, 10, 100):
            print(f"ivfpq m{metric} d{dim} np{nprobe} k{k}", flush=True)
            gs, gi = pq.search(queries, k, nprobe)
            for qi in range(queries.shape[0]):
                os_, oi = oracle.ivfpq_search(coarse, books, codes, offsets, ids, metric,
                                              queries[qi], k, nprobe)
                kk = len(os_)
                assert np.array_equal(gs[qi, :kk], os_), f"scores q{qi}"
                assert np.array_equal(gi[qi, :kk], oi), f"ids q{qi}"
                assert np.all(gi[qi, kk:] == M.EMPTY_ID)
    pq.release()
    c.release()


def test_ivfpq_ties_follow_bounded_sorted_list(gpu_ctx):
    # Duplicated rows share codes and scores: the kept ids and their order
    # among equal scores follow the newest-first insertion rule.
    dim, m, n, nlist = 32, 8, 4000, 8
    base = workloads.lcg_vectors(0, n // 8, dim, seed=711)
    rows = np.repeat(base, 8, axis=0)
    coarse = base[:nlist].copy()
    books = _books_from_rows(base, m, seed=712)
    assign, codes, offsets, ids = _oracle_index(rows, coarse, books, L2)
    c = gpu_ctx.upload(rows)
    pq = c.ivfpq_build(coarse, books, L2)
    queries = np.concatenate([base[:4], workloads.lcg_vectors(0, 4, dim, seed=713)])
    for k in (3, 10, 37):
        gs, gi = pq.search(queries, k, 3)
        for qi in range(queries.shape[0]):
            os_, oi = oracle.ivfpq_search(coarse, books, codes, offsets, ids, L2, queries[qi], k, 3)
            assert np.array_equal(gs[qi, :len(os_)], os_)
            assert np.array_equal(gi[qi, :len(oi)], oi), f"k{k} q{qi}"
    pq.release()
    c.release()


@pytest.mark.parametrize("metric", [IP, L2])
def test_ivfpq_exact_rerank_matches_oracle(gpu_ctx, metric):
    dim, m, n, nlist = 96, 48, 8000, 32
    rows = workloads.lcg_vectors(1, n, dim, seed=721 + metric)
    coarse = rows[:: n // nlist][:nlist].copy()
    books = _books_from_rows(rows, m, seed=722)
    assign, codes, offsets, ids = _oracle_index(rows, coarse, books, metric)
    c = gpu_ctx.upload(rows)
    pq = c.ivfpq_build(coarse, books, metric)
    queries = workloads.lcg_vectors(1, 10, dim, seed=723)
    gs, gi = pq.search(queries, 100, 6, rerank_k=10)
    for qi in range(queries.shape[0]):
        os_, oi = oracle.ivfpq_search(coarse, books, codes, offsets, ids, metric, queries[qi], 100,
                                      6, rows=rows, rerank_k=10)
        assert np.array_equal(gs[qi, :len(os_)], os_)
        assert np.array_equal(gi[qi, :len(oi)], oi)
    pq.release()
    c.release()


def test_ivfpq_mixture_96_sample(gpu_ctx):
    # The 8,192-centre mixture at 262,144 rows x 96, nlist 256, m 48 (dsub
    # 2), nprobe 16, top-100 ADC then exact rerank to 10: a sample of
    # queries equals the oracle, and the reranked results find most of the
    # exact top-10.  (Recall need not grow with nprobe here: with inner
    # product, more probed lists bring more ADC false positives into the
    # top-100.)
    print("ivfpq 262144 x 96 mixture", flush=True)
    db, q, _ = workloads.mixture_10m_96(nq=32, n=262144)
    c = gpu_ctx.upload(db)
    coarse = c.kmeans(256, 2, L2)
    books = _books_from_rows(db, 48, seed=731)
    pq = c.ivfpq_build(coarse, books, IP)
    gcodes, gassign = pq.codes()
    sample = np.arange(0, db.shape[0], 4099)
    a_s, c_s = oracle.pq_encode_rows(db[sample], coarse, books, IP)
    assert np.array_equal(gassign[sample], a_s) and np.array_equal(gcodes[sample], c_s)
    offsets, ids = oracle.ivf_lists(gassign, 256)
    gs, gi = pq.search(q, 100, 16, rerank_k=10)
    for qi in range(0, q.shape[0], 8):
        os_, oi = oracle.ivfpq_search(coarse, books, gcodes, offsets, ids, IP, q[qi], 100, 16,
                                      rows=db, rerank_k=10)
        assert np.array_equal(gs[qi], os_) and np.array_equal(gi[qi], oi)
    fd, fi = c.flat_search(q, 10, IP)
    recall = []
    for nprobe in (2, 16, 64):
        _, ri = pq.search(q, 100, nprobe, rerank_k=10)
        recall.append(np.mean([len(set(ri[i]) & set(fi[i])) / 10 for i in range(q.shape[0])]))
    print("recall@10 at nprobe 2/16/64:", recall, flush=True)
    assert min(recall) > 0.5
    pq.release()
    c.release()


@pytest.mark.parametrize("metric", [IP, COS, L2])
def test_ivfpq_probe_ties_beyond_the_kept_centroids(gpu_ctx, metric):
    # nlist far above nprobe + 64, with 200 copies of one centroid and a zero
    # query (every inner-product distance is -0, every cosine distance 1):
    # more centroids tie at the nprobe-th distance than the first selection
    # keeps, and the BoundedSortedList order over every centroid decides.
    dim, m, n, nlist = 32, 8, 20000, 512
    rows = workloads.lcg_vectors(1, n, dim, seed=741 + metric)
    coarse = rows[:: n // nlist][:nlist].copy()
    coarse[100:300] = coarse[5]
    books = _books_from_rows(rows, m, seed=742)
    assign, codes, offsets, ids = _oracle_index(rows, coarse, books, metric)
    c = gpu_ctx.upload(rows)
    pq = c.ivfpq_build(coarse, books, metric)
    queries = np.stack([np.zeros(dim, np.float32), coarse[5], coarse[5] + np.float32(1e-3),
                        rows[123]]).astype(np.float32)
    for nprobe in (8, 16, 100):
        gs, gi = pq.search(queries, 10, nprobe)
        for qi in range(queries.shape[0]):
            os_, oi = oracle.ivfpq_search(coarse, books, codes, offsets, ids, metric, queries[qi],
                                          10, nprobe)
            assert np.array_equal(gs[qi, :len(os_)], os_), f"np{nprobe} q{qi}"
            assert np.array_equal(gi[qi, :len(oi)], oi), f"np{nprobe} q{qi}"
    pq.release()
    c.release()


@pytest.mark.parametrize("metric", [L2, IP, COS])
def test_ivfpq_score_ties_beyond_the_kept_candidates(gpu_ctx, metric):
    # 300 copies of one row share its code and score, and a query equal to a
    # coarse centroid has a zero residual (its list's LUT ties for inner
    # product and cosine): more rows tie at the k_adc-th score than the
    # k_adc + 64 the scan keeps, so ivfpq_tie_replay finishes those queries.
    dim, m, n, nlist = 32, 8, 12000, 16
    rows = workloads.lcg_vectors(1, n, dim, seed=751 + metric)
    rows[2000:2300] = rows[77]
    coarse = rows[:: n // nlist][:nlist].copy()
    books = _books_from_rows(rows, m, seed=752)
    assign, codes, offsets, ids = _oracle_index(rows, coarse, books, metric)
    c = gpu_ctx.upload(rows)
    pq = c.ivfpq_build(coarse, books, metric)
    queries = np.stack([rows[77], coarse[3], coarse[9], rows[5]]).astype(np.float32)
    gpu_ctx.timing(True)
    gpu_ctx.timing_reset()
    for k, nprobe, rerank in ((10, 4, 0), (100, 2, 0), (100, 3, 10), (100, 1, 0)):
        gs, gi = pq.search(queries, k, nprobe, rerank_k=rerank)
        for qi in range(queries.shape[0]):
            os_, oi = oracle.ivfpq_search(coarse, books, codes, offsets, ids, metric, queries[qi],
                                          k, nprobe, rows=rows if rerank else None,
                                          rerank_k=rerank)
            assert np.array_equal(gs[qi, :len(os_)], os_), f"k{k} q{qi}"
            assert np.array_equal(gi[qi, :len(oi)], oi), f"k{k} q{qi}"
    _, replays = gpu_ctx.timing_read("ivfpq_tie_replay")
    gpu_ctx.timing(False)
    # L2: the 301 equal rows tie at the top; cosine: coarse[3] probed alone
    # scores every row of its list m * 1.0.
    if metric != IP:
        assert replays > 0
    pq.release()
    c.release()


@pytest.mark.parametrize("metric", [IP, L2])
def test_ivfpq_train_matches_oracle(gpu_ctx, metric):
    # _IVFPQIndex.train (IVFPQIndex.swift:54-104): coarse k-means, residuals
    # against the last pass's assignment, per-subspace k-means with 256
    # centroids -- bit for bit.
    ctr = workloads.centers(761, 40, 32)
    rows, _ = workloads.mixture_rows(762, ctr, 0.3, 3000, False)
    c = gpu_ctx.upload(rows)
    for nlist, m, iters in ((16, 8, 6), (1, 4, 3), (40, 16, 25)):
        gcoarse, gbooks = c.ivfpq_train(nlist, m, iters, metric)
        ocoarse, obooks = oracle.ivfpq_train(rows, nlist, m, iters, metric)
        assert np.array_equal(gcoarse, ocoarse), (nlist, m, iters)
        assert np.array_equal(gbooks, obooks), (nlist, m, iters)
    with pytest.raises(M.ANNSError):
        gpu_ctx.upload(rows[:255]).ivfpq_train(4, 8, 2, metric)  # needs 256 rows
    c.release()


def test_ivfpq_save_load_round_trip_and_corruption(gpu_ctx, tmp_path):
    dim, m, n, nlist = 32, 8, 6000, 24
    rows = workloads.lcg_vectors(1, n, dim, seed=771)
    coarse = rows[:: n // nlist][:nlist].copy()
    books = _books_from_rows(rows, m, seed=772)
    c = gpu_ctx.upload(rows)
    pq = c.ivfpq_build(coarse, books, IP)
    queries = workloads.lcg_vectors(1, 8, dim, seed=773)
    want = pq.search(queries, 50, 4, rerank_k=10)
    want_adc = pq.search(queries, 50, 4)
    path = tmp_path / "index.ivpb"
    pq.save(path)
    loaded = M.ivfpq_load(gpu_ctx, path, c)
    got = loaded.search(queries, 50, 4, rerank_k=10)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    assert all(np.array_equal(a, b) for a, b in zip(loaded.codes(), pq.codes()))
    # Without rows the ADC search works and the rerank is refused.
    bare = M.ivfpq_load(gpu_ctx, path)
    got = bare.search(queries, 50, 4)
    assert np.array_equal(got[0], want_adc[0]) and np.array_equal(got[1], want_adc[1])
    with pytest.raises(M.ANNSError):
        bare.search(queries, 50, 4, rerank_k=10)
    data = path.read_bytes()

    def corrupt(blob, reason):
        bad = tmp_path / "bad.ivpb"
        bad.write_bytes(blob)
        with pytest.raises(M.ANNSError) as ei:
            M.ivfpq_load(gpu_ctx, bad)
        assert ei.value.code == M.CORRUPT_FILE and reason in str(ei.value), str(ei.value)

    corrupt(b"IVPX" + data[4:], "Invalid file magic")
    corrupt(data[:-1], "File size does not match")
    corrupt(data[:20], "Unexpected EOF")
    hdr = M.IVPB_HEADER
    fields = list(hdr.unpack(data[:hdr.size]))
    fields[1] = 9
    corrupt(hdr.pack(*fields) + data[hdr.size:], "version 9")
    # A list id moved to another list: ids and assignments disagree.
    off_at = hdr.size + 4 * nlist * dim + 4 * m * 256 * (dim // m)
    ids_at = off_at + 8 * (nlist + 1)
    tampered = bytearray(data)
    first, second = tampered[ids_at:ids_at + 4], tampered[ids_at + 4 * (n - 1):ids_at + 4 * n]
    tampered[ids_at:ids_at + 4], tampered[ids_at + 4 * (n - 1):ids_at + 4 * n] = second, first
    corrupt(bytes(tampered), "disagree")
    small = gpu_ctx.upload(rows[:100])
    with pytest.raises(M.ANNSError) as ei:
        M.ivfpq_load(gpu_ctx, path, small)
    assert ei.value.code == M.DIMENSION_MISMATCH
    for h in (loaded, bare, pq, small, c):
        h.release()
