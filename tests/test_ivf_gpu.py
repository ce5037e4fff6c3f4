"""Parity of the HIP IVF-flat build, probe scan and k-means.

The bar (IVFFlatSearch.swift:115-311, 517-703; SURVEY contract for IVF):
  - lists (CSR offsets and ids in row order) bit-identical to the oracle's
    partition built from the same centroids;
  - probe lists identical (the nprobe smallest centroid distances by
    (distance, index), ascending ids);
  - results: distances bit-identical to the oracle's scan of the probed
    lists, ids equal except on exact ties;
  - nprobe >= nlist gives the exact flat result (IVFFlatSearchTests.swift:193-216);
  - device k-means centroids bit-identical to the oracle's Lloyd iterations.
"""
import numpy as np
import pytest

import meltan_amd as M
from meltan_amd import workloads
from oracle import oracle
from test_flat_gpu import COS, IP, L2, check_flat

pytestmark = pytest.mark.gpu


def _assert_rows(gd, gi, od, oi, what):
    kk = len(od)
    assert np.array_equal(gd[:kk], od), f"{what}: {gd[:kk][:4]} vs {od[:4]}"
    for j in range(kk):
        tied = (j > 0 and od[j - 1] == od[j]) or (j + 1 < kk and od[j + 1] == od[j]) or j == kk - 1
        if not tied:
            assert gi[j] == oi[j], f"{what} rank {j}"
    assert np.all(gd[kk:] == np.finfo(np.float32).max)
    assert np.all(gi[kk:] == M.EMPTY_ID)


@pytest.mark.parametrize("metric", [L2, COS, IP])
def test_ivf_lists_probes_and_results_match_oracle(gpu_ctx, metric):
    dim, n, nlist = 64, 6000, 48
    rows = workloads.lcg_vectors(1, n, dim, seed=601 + metric)
    cents = rows[::n // nlist][:nlist].copy()
    part = oracle.IVFPartition(rows, cents, metric)
    c = gpu_ctx.upload(rows)
    ivf = c.ivf_flat_build(cents, metric)
    off, ids = ivf.lists()
    assert np.array_equal(off, part.offsets)
    assert np.array_equal(ids, part.list_ids)
    queries = workloads.lcg_vectors(1, 40, dim, seed=602 + metric)
    for nprobe in (1, 4, 13):
        for k in (1, 10, 64):
            print(f"ivf m{metric} nprobe{nprobe} k{k}", flush=True)
            gd, gi, gp = ivf.search(queries, k, nprobe, want_probes=True)
            for qi in range(queries.shape[0]):
                od, oi, op = part.search(queries[qi], k, nprobe)
                assert np.array_equal(gp[qi], op), f"probes q{qi}"
                _assert_rows(gd[qi], gi[qi], od, oi, f"m{metric} np{nprobe} k{k} q{qi}")
    ivf.release()
    c.release()


@pytest.mark.parametrize("dim", [64, 100, 128, 192, 256])
def test_ivf_list_major_batch_matches_oracle(gpu_ctx, dim):
    # Batches of 64 queries and more scan each probed list once for all the
    # queries probing it (chunks of 512 rows, 16 queries per work item);
    # results must equal the oracle's per-query scan exactly, for every
    # metric, with lists larger than a chunk, k up to 32 and some queries
    # whose probes reach only empty lists.
    n, nlist, nq = 9000, 12, 80
    rows = workloads.lcg_vectors(1, n, dim, seed=640 + dim)
    cents = np.concatenate([rows[:nlist - 2], np.full((2, dim), 1e3, np.float32)])
    queries = workloads.lcg_vectors(1, nq, dim, seed=641 + dim)
    queries[5] = 1e3  # nearest centroids: the two empty lists
    for metric in (L2, COS, IP):
        part = oracle.IVFPartition(rows, cents, metric)
        c = gpu_ctx.upload(rows)
        ivf = c.ivf_flat_build(cents, metric)
        for nprobe, k in ((1, 10), (2, 1), (5, 32), (12, 10)):
            print(f"ivf list-major dim{dim} m{metric} nprobe{nprobe} k{k}", flush=True)
            gd, gi, gp = ivf.search(queries, k, nprobe, want_probes=True)
            for qi in range(nq):
                od, oi, op = part.search(queries[qi], k, nprobe)
                assert np.array_equal(gp[qi], op), f"probes q{qi}"
                _assert_rows(gd[qi], gi[qi], od, oi, f"lm dim{dim} m{metric} np{nprobe} k{k} q{qi}")
        ivf.release()
        c.release()


def test_ivf_probe_selection_both_paths_and_ties(gpu_ctx):
    # nprobe <= 64 selects with per-wave lists, above it with the radix cut;
    # every centroid appears twice (rows 0..149 repeated), so each query's
    # keys come in equal pairs and the (distance, index) order decides.
    dim, n = 64, 8000
    rows = workloads.lcg_vectors(1, n, dim, seed=631)
    base = rows[:150].copy()
    cents = np.concatenate([base, base])
    part = oracle.IVFPartition(rows, cents, L2)
    c = gpu_ctx.upload(rows)
    ivf = c.ivf_flat_build(cents, L2)
    queries = workloads.lcg_vectors(1, 70, dim, seed=632)
    for nprobe in (63, 64, 65, 200):
        print(f"ivf probe selection nprobe{nprobe}", flush=True)
        gd, gi, gp = ivf.search(queries, 10, nprobe, want_probes=True)
        for qi in range(queries.shape[0]):
            od, oi, op = part.search(queries[qi], 10, nprobe)
            assert np.array_equal(gp[qi], op), f"probes np{nprobe} q{qi}"
            _assert_rows(gd[qi], gi[qi], od, oi, f"np{nprobe} q{qi}")
    ivf.release()
    c.release()


def test_ivf_full_probe_equals_flat(gpu_ctx):
    dim, n, nlist = 128, 5000, 20
    rows = workloads.lcg_vectors(0, n, dim, seed=611)
    cents = rows[:nlist].copy()
    c = gpu_ctx.upload(rows)
    ivf = c.ivf_flat_build(cents, L2)
    q = workloads.lcg_vectors(0, 16, dim, seed=612)
    gd, gi = ivf.search(q, 10, nlist)
    check_flat(rows, oracle.row_norms(rows), q, 10, L2, gd, gi, "nprobe=nlist")
    gd2, gi2 = ivf.search(q, 10, nlist + 5)
    assert np.array_equal(gd, gd2) and np.array_equal(gi, gi2)
    ivf.release()
    c.release()


def test_ivf_empty_lists_and_small_k(gpu_ctx):
    # Centroids far away from every row leave lists empty; a probe of only
    # empty lists returns padding.
    dim, n = 32, 3000
    rows = workloads.lcg_vectors(1, n, dim, seed=621)
    cents = np.concatenate([rows[:6], np.full((4, dim), 1e3, np.float32)])
    part = oracle.IVFPartition(rows, cents, L2)
    c = gpu_ctx.upload(rows)
    ivf = c.ivf_flat_build(cents, L2)
    off, ids = ivf.lists()
    assert np.array_equal(off, part.offsets) and np.array_equal(ids, part.list_ids)
    q = np.full((2, dim), 1e3, np.float32)  # nearest centroids are the empty ones
    gd, gi, gp = ivf.search(q, 5, 2, want_probes=True)
    for qi in range(2):
        od, oi, op = part.search(q[qi], 5, 2)
        assert np.array_equal(gp[qi], op)
        _assert_rows(gd[qi], gi[qi], od, oi, f"empty q{qi}")
    ivf.release()
    c.release()


@pytest.mark.parametrize("metric", [L2, COS, IP])
@pytest.mark.parametrize("dim", [32, 128, 7])
def test_kmeans_matches_oracle(gpu_ctx, metric, dim):
    # KMeans.cluster (KMeans.swift:53-257): first-wins SIMDDistance
    # assignment, stop at the first unchanged pass, Float sums in row order
    # times 1 / Float(count), empty clusters kept -- bit for bit, including
    # runs long enough to settle.
    n, k = 4000, 24
    ctr = workloads.centers(630 + dim, 30, dim)
    rows, _ = workloads.mixture_rows(631 + metric, ctr, 0.4, n, False)
    rows[n // k] = rows[0]  # two initial centroids coincide: one stays empty
    c = gpu_ctx.upload(rows)
    for iters in (0, 1, 6, 200):
        got = c.kmeans(k, iters, metric)
        ref, _ = oracle.kmeans(rows, k, iters, metric)
        assert np.array_equal(got, ref), f"iters {iters}"
    c.release()


@pytest.mark.parametrize("metric", [L2, IP])
def test_ivf_flat_train_matches_oracle(gpu_ctx, metric):
    # buildPartition's sample and 8 k-means iterations (IVFFlatSearch.swift:
    # 517-551): small nlist (a 16 nlist-row sample), nlist >= 4096 (the
    # sample rows themselves) and nlist above n.
    rows = workloads.gauss_rows(641, 3 * 4096 + 5, 16, False)
    c = gpu_ctx.upload(rows)
    for nlist in (8, 64, 4096):
        got = c.ivf_flat_train(nlist, metric)
        want = oracle.ivf_flat_train(rows, nlist, metric)
        assert np.array_equal(got, want), nlist
    small = gpu_ctx.upload(rows[:100])
    got = small.ivf_flat_train(256, metric)
    assert np.array_equal(got, oracle.ivf_flat_train(rows[:100], 256, metric))
    if metric == L2:  # every row is its own nearest centroid
        assert np.array_equal(got, rows[:100])
    small.release()
    c.release()


def test_ivf_mixture_1m_128_properties(gpu_ctx):
    # The 4,096-centre mixture at full size with device k-means centroids:
    # a sample of rows sits in its nearest list, probes and results of a
    # sample of queries equal the oracle's over the same lists, and recall
    # against the exact result grows with nprobe.
    print("ivf 1M x 128 mixture", flush=True)
    db, q = workloads.mixture_1m_128(nq=64)
    c = gpu_ctx.upload(db)
    cents = c.ivf_flat_train(4096, L2)  # the reference's sampled build
    ivf = c.ivf_flat_build(cents, L2)
    off, ids = ivf.lists()
    assert off[-1] == db.shape[0] and np.all(np.diff(off) >= 0)
    assign = np.empty(db.shape[0], np.int64)
    for lst in range(4096):
        assign[ids[off[lst]:off[lst + 1]]] = lst
    sample = np.arange(0, db.shape[0], 9973)
    ref = oracle.ivf_assign(db[sample], cents, L2)
    assert np.array_equal(assign[sample], ref)
    # oracle scan over the device lists
    part = oracle.IVFPartition.__new__(oracle.IVFPartition)
    part.metric, part.dim, part.count, part.nlist = L2, db.shape[1], db.shape[0], 4096
    part.centroids, part.cnorms = cents, oracle.row_norms(cents)
    part.offsets, part.list_ids = off, ids
    part.packed = np.ascontiguousarray(db[ids])
    part.packed_norms = oracle.row_norms(part.packed)
    fd, fi = c.flat_search(q, 10, L2)
    recalls = []
    for nprobe in (4, 8, 32):
        gd, gi, gp = ivf.search(q, 10, nprobe, want_probes=True)
        for qi in range(0, q.shape[0], 8):
            od, oi, op = part.search(q[qi], 10, nprobe)
            assert np.array_equal(gp[qi], op)
            _assert_rows(gd[qi], gi[qi], od, oi, f"1M np{nprobe} q{qi}")
        recalls.append(np.mean([len(set(gi[i]) & set(fi[i])) / 10 for i in range(q.shape[0])]))
    assert recalls[0] <= recalls[1] <= recalls[2]
    ivf.release()
    c.release()
