"""Parity of the HIP exact flat scan (mans_flat_search) with the oracle.

The bar: each returned distance is bit-identical to the oracle's host-formula
distance of that id (dots.c summation order), the returned distances are
exactly the k smallest the oracle finds, and ids agree wherever distances
are not exactly tied.  Cases follow FlatSearchTests.swift:73-233,
ExactSearchIntegrationTests.swift:91-189 and BoundedExactScanTests.swift:211-272.
"""
import sys
import threading

import numpy as np
import pytest

import meltan_amd as M
from meltan_amd import workloads
from oracle import oracle

pytestmark = pytest.mark.gpu

COS, L2, IP = 0, 1, 2
FMAX = np.finfo(np.float32).max


def check_flat(corpus, norms, queries, k, metric, gdist, gids, what=""):
    """Asserts the GPU rows are a valid exact top-k for every query."""
    n = corpus.shape[0]
    odist, oids, counts = oracle.flat_search_batch(corpus, norms, queries, k, metric)
    for i in range(queries.shape[0]):
        kk = int(counts[i])
        assert kk == min(k, 256, n), what
        # distances: the k smallest, bit for bit
        assert np.array_equal(gdist[i, :kk], odist[i, :kk]), (
            f"{what} q{i}: dist {gdist[i, :kk][:5]} vs {odist[i, :kk][:5]}")
        # each id carries its own exact distance
        redo = oracle.distances_for_ids(corpus, norms, queries[i], gids[i, :kk], metric)
        assert np.array_equal(redo, gdist[i, :kk]), f"{what} q{i}: ids do not carry their distances"
        assert len(set(gids[i, :kk].tolist())) == kk, f"{what} q{i}: duplicate ids"
        # ids equal wherever the distance is not tied
        d = odist[i, :kk]
        for j in range(kk):
            tied = (j > 0 and d[j - 1] == d[j]) or (j + 1 < kk and d[j + 1] == d[j]) or j == kk - 1
            if not tied:
                assert gids[i, j] == oids[i, j], f"{what} q{i} rank {j}"
        # ascending by (distance, id)
        order = np.lexsort((gids[i, :kk], gdist[i, :kk]))
        assert np.array_equal(order, np.arange(kk)), f"{what} q{i}: not sorted by (distance, id)"
        # padding past min(k, 256, n)
        assert np.all(gdist[i, kk:] == FMAX) and np.all(gids[i, kk:] == M.EMPTY_ID)


@pytest.mark.parametrize("dim", [16, 64, 66, 128, 333, 384])
@pytest.mark.parametrize("n", [64, 100, 2049, 5000])
def test_flat_parity_across_dims_sizes_metrics(gpu_ctx, dim, n):
    print(f"flat parity dim={dim} n={n}", flush=True)
    corpus = workloads.lcg_vectors(0, n, dim, seed=n * 31 + dim)
    queries = workloads.lcg_vectors(0, 4, dim, seed=n * 31 + dim + 1)
    norms = oracle.row_norms(corpus)
    c = gpu_ctx.upload(corpus)
    for metric in (COS, L2, IP):
        for k in (1, 10, 100):
            gd, gi = c.flat_search(queries, k, metric)
            check_flat(corpus, norms, queries, k, metric, gd, gi, f"dim{dim} n{n} m{metric} k{k}")
    c.release()


def test_flat_k_edges(gpu_ctx):
    corpus = workloads.lcg_vectors(0, 400, 32, seed=9)
    norms = oracle.row_norms(corpus)
    c = gpu_ctx.upload(corpus)
    q = workloads.lcg_vectors(0, 3, 32, seed=10)
    for k in (256, 300, 399, 400, 401, 1000):
        gd, gi = c.flat_search(q, k, L2)
        check_flat(corpus, norms, q, k, L2, gd, gi, f"k{k}")
    small = workloads.lcg_vectors(0, 5, 32, seed=11)
    cs = gpu_ctx.upload(small)
    gd, gi = cs.flat_search(q, 10, COS)
    check_flat(small, oracle.row_norms(small), q, 10, COS, gd, gi, "n<k")


def test_flat_rejects_hamming_and_handles_empty(gpu_ctx):
    corpus = workloads.lcg_vectors(0, 100, 8, seed=1)
    c = gpu_ctx.upload(corpus)
    with pytest.raises(M.ANNSError) as e:
        c.flat_search(corpus[:1], 5, M.METRIC_HAMMING)
    assert e.value.code == M.SEARCH_FAILED and e.value.is_tier_degradeable
    empty = gpu_ctx.upload(np.zeros((0, 8), np.float32))
    gd, gi = empty.flat_search(corpus[:2], 5, COS)
    assert np.all(gi == M.EMPTY_ID) and np.all(gd == FMAX)


def test_flat_10k_batch_1000(gpu_ctx):
    print("flat 10k x 384 batch 1000", flush=True)
    db, q = workloads.flat_10k(1000)
    norms = oracle.row_norms(db)
    c = gpu_ctx.upload(db)
    gd, gi = c.flat_search(q, 10, COS)
    check_flat(db, norms, q, 10, COS, gd, gi, "10k")


def test_flat_100k_noisy_queries(gpu_ctx):
    print("flat 100k x 384", flush=True)
    db, q = workloads.flat_100k(64)
    norms = oracle.row_norms(db)
    c = gpu_ctx.upload(db)
    for batch in (1, 32, 64):
        gd, gi = c.flat_search(q[:batch], 10, COS)
        check_flat(db, norms, q[:batch], 10, COS, gd, gi, f"100k batch {batch}")
    # noisy copies find their source row first
    _, src = workloads.noisy_queries(2002, db, 64)
    gd, gi = c.flat_search(q, 1, COS)
    even = np.arange(0, 64, 2)
    assert np.mean(gi[even, 0] == src[even]) > 0.9


def test_flat_adversarial_duplicates_zeros_extremes(gpu_ctx):
    # BoundedExactScanTests.swift:211-250 layout: quarter zeros, quarter copies
    # of one row, the rest random with magnitudes 1e-5 / 1 / 1e5.
    dim, n = 64, 16384 + 512
    rng_rows = workloads.lcg_vectors(1, n, dim, seed=2024)
    base = rng_rows[0].copy()
    corpus = rng_rows.copy()
    corpus[0::4] = 0.0
    corpus[1::4] = base
    idx = np.arange(n)
    corpus[(idx % 8 == 2)] *= 1e-5
    corpus[(idx % 8 == 6)] *= 1e5
    norms = oracle.row_norms(corpus)
    c = gpu_ctx.upload(corpus)
    q = workloads.lcg_vectors(1, 2, dim, seed=2025)
    for metric in (COS, L2, IP):
        for k in (24, 256):
            gd, gi = c.flat_search(q, k, metric)
            check_flat(corpus, norms, q, k, metric, gd, gi, f"adversarial m{metric} k{k}")


def test_flat_zero_query(gpu_ctx):
    corpus = workloads.lcg_vectors(1, 5000, 96, seed=31)
    norms = oracle.row_norms(corpus)
    c = gpu_ctx.upload(corpus)
    q = np.zeros((1, 96), np.float32)
    for metric in (COS, L2, IP):
        gd, gi = c.flat_search(q, 24, metric)
        check_flat(corpus, norms, q, 24, metric, gd, gi, f"zero query m{metric}")


def test_flat_write_rows_refreshes_norms(gpu_ctx):
    corpus = workloads.lcg_vectors(0, 3000, 48, seed=88)
    c = gpu_ctx.upload(corpus)
    q = workloads.lcg_vectors(0, 1, 48, seed=89)
    c.flat_search(q, 10, COS)
    corpus2 = corpus.copy()
    corpus2[7] = q[0] * 10
    c.write_rows(7, corpus2[7:8])
    for metric in (COS, L2, IP):
        gd, gi = c.flat_search(q, 10, metric)
        check_flat(corpus2, oracle.row_norms(corpus2), q, 10, metric, gd, gi, f"mutated m{metric}")
    gd, gi = c.flat_search(q, 1, COS)
    assert gi[0, 0] == 7


def test_flat_device_api_matches_host_api(gpu_ctx):
    from meltan_amd import hip

    db, q = workloads.flat_10k(64)
    c = gpu_ctx.upload(db)
    hd, hi = c.flat_search(q, 10, COS)
    dq = hip.DeviceArray.from_numpy(q)
    dd = hip.DeviceArray((64, 10), np.float32)
    di = hip.DeviceArray((64, 10), np.uint32)
    s = hip.Stream()
    c.flat_search_device(dq.ptr, 64, 10, COS, dd.ptr, di.ptr, s.handle)
    assert np.array_equal(dd.numpy(), hd)
    assert np.array_equal(di.numpy(), hi)
    # default (pooled) stream, and an unaligned query pointer (scalar kernel path)
    c.flat_search_device(dq.ptr, 64, 10, COS, dd.ptr, di.ptr, None)
    assert np.array_equal(dd.numpy(), hd)
    q2 = np.concatenate([np.zeros(1, np.float32), q.ravel()])
    dq2 = hip.DeviceArray.from_numpy(q2)
    c.flat_search_device(dq2.offset(1), 64, 10, COS, dd.ptr, di.ptr, None)
    assert np.array_equal(dd.numpy(), hd) and np.array_equal(di.numpy(), hi)
    s.destroy()


def test_flat_concurrent_callers_share_a_context(gpu_ctx):
    # ExactSearchIntegrationTests.swift:193-230: many concurrent searches.
    db, q = workloads.flat_10k(32)
    c = gpu_ctx.upload(db)
    want = c.flat_search(q, 10, COS)
    results = [None] * 8
    errors = []

    def worker(i):
        try:
            results[i] = c.flat_search(q, 10, COS)
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors
    for r in results:
        assert np.array_equal(r[0], want[0]) and np.array_equal(r[1], want[1])


def test_flat_1m_full_size_properties(gpu_ctx):
    # 1,000,000 x 384 mixture: self queries find themselves; a sample of
    # queries matches the oracle exactly.
    print("flat 1M x 384", flush=True)
    db, q = workloads.mixture_1m_384(nq=8)
    c = gpu_ctx.upload(db)
    rows = np.array([0, 1, 499_999, 999_999])
    gd, gi = c.flat_search(db[rows], 10, COS)
    assert np.all(gi[:, 0] == rows) and np.all(gd[:, 0] <= 1e-6)
    assert np.all(np.diff(gd, axis=1) >= 0)
    norms = oracle.row_norms(db)
    gd, gi = c.flat_search(q[:4], 10, COS)
    check_flat(db, norms, q[:4], 10, COS, gd, gi, "1M")


def test_flat_threshold_merge_paths(gpu_ctx):
    # Single queries and small batches (below the batched path) merge the
    # block lists by threshold: few candidates on random rows; thousands of
    # equal keys (a duplicated row) overflow the candidate buffer and take
    # the full selection; corpora with fewer block lists than candidates
    # take every list.
    print("flat threshold merge", flush=True)
    dim = 64
    db = workloads.lcg_vectors(0, 200_000, dim, seed=4242)
    dup = db.copy()
    pos = np.random.default_rng(7).choice(200_000, 5000, replace=False)
    dup[pos] = db[123]
    same = np.repeat(db[5:6], 200_000, axis=0)  # every key ties: the full selection
    q = workloads.lcg_vectors(0, 3, dim, seed=4243)
    qd = np.concatenate([db[123:124] + 1e-3 * q[:1], q[1:]]).astype(np.float32)
    for corpus, queries, what in ((db, q, "random"), (dup, qd, "duplicates"), (same, q, "same")):
        norms = oracle.row_norms(corpus)
        c = gpu_ctx.upload(corpus)
        for metric in (COS, L2, IP):
            for k in (1, 10, 32):
                for b in (1, 3):
                    gd, gi = c.flat_search(queries[:b], k, metric)
                    check_flat(corpus, norms, queries[:b], k, metric, gd, gi,
                               f"{what} m{metric} k{k} b{b}")
        c.release()
    for n in (700, 3000):
        small = db[:n].copy()
        c = gpu_ctx.upload(small)
        for k in (10, 32):
            gd, gi = c.flat_search(q, k, COS)
            check_flat(small, oracle.row_norms(small), q, k, COS, gd, gi, f"n{n} k{k}")
        c.release()
