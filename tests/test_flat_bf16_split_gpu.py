"""Parity of the batched flat path on split-bf16 MFMA.

Batches of at least 16 queries with k <= 32 run the contraction on
v_mfma_f32_32x32x16_bf16 with the queries split into two bf16 parts and the
rows kept as their bf16 high parts plus the norm of the remainder (two
partial products).  Its keys are lower bounds with the split's error and
the rows' remainder term included, so the results must meet the streaming
scan's bar: distances
bit-identical to the oracle's (dots.c order, host formulas), ids equal
except on exact ties.  A corpus with values outside the split range keeps
the fp32 contraction; a query outside it is re-run by the streaming scan.
The timing counters show which kernels ran ("flat_bound" is the sampled
launch of the split path).
"""
import numpy as np
import pytest

from meltan_amd import workloads
from oracle import oracle
from test_flat_gpu import COS, IP, L2, check_flat

pytestmark = pytest.mark.gpu


def _search(ctx, corpus, queries, k, metric):
    ctx.timing(True)
    ctx.timing_reset()
    try:
        gd, gi = corpus.flat_search(queries, k, metric)
        launches = {name: ctx.timing_read(name)[1] for name in ("flat_bound", "flat_gemm", "flat_scan")}
    finally:
        ctx.timing(False)
    return gd, gi, launches


@pytest.mark.parametrize("dim", [64, 96, 128, 192, 256, 384])
def test_split_parity_dims_metrics(gpu_ctx, dim):
    for n, nq in ((5000, 16), (20011, 130)):
        print(f"split parity dim={dim} n={n} nq={nq}", flush=True)
        corpus = workloads.lcg_vectors(1, n, dim, seed=3 * n + dim)
        queries = workloads.lcg_vectors(1, nq, dim, seed=3 * n + dim + 1)
        norms = oracle.row_norms(corpus)
        c = gpu_ctx.upload(corpus)
        for metric in (COS, L2, IP):
            for k in (1, 10, 32):
                gd, gi, launches = _search(gpu_ctx, c, queries, k, metric)
                assert launches["flat_bound"] == 1 and launches["flat_gemm"] == 1, launches
                check_flat(corpus, norms, queries, k, metric, gd, gi, f"split dim{dim} n{n} m{metric} k{k}")
        c.release()


def test_split_near_duplicates(gpu_ctx):
    # Rows that differ from each other by a few ulps: the keys' slack covers
    # many rows at once, proofs fail and queries are re-run, and the result
    # must still be exact.
    dim, n = 128, 12000
    base = workloads.lcg_vectors(1, 50, dim, seed=11)
    rng = np.random.default_rng(12)
    corpus = base[rng.integers(0, 50, n)].copy()
    corpus *= (1.0 + rng.integers(-8, 9, (n, 1)) * 2.0 ** -23).astype(np.float32)
    queries = base[:20] + np.float32(1e-3) * workloads.lcg_vectors(1, 20, dim, seed=13)
    norms = oracle.row_norms(corpus)
    c = gpu_ctx.upload(corpus)
    for metric in (COS, L2, IP):
        gd, gi, launches = _search(gpu_ctx, c, queries, 10, metric)
        assert launches["flat_bound"] == 1
        check_flat(corpus, norms, queries, 10, metric, gd, gi, f"near-dup m{metric}")
    c.release()


def test_split_corpus_outside_split_range_keeps_fp32(gpu_ctx):
    dim, n = 96, 6000
    corpus = workloads.lcg_vectors(0, n, dim, seed=21)
    corpus[17, 5] = 1e-30  # below 2^-50: the split could lose it
    queries = workloads.lcg_vectors(0, 24, dim, seed=22)
    norms = oracle.row_norms(corpus)
    c = gpu_ctx.upload(corpus)
    gd, gi, launches = _search(gpu_ctx, c, queries, 10, L2)
    assert launches["flat_bound"] == 0 and launches["flat_gemm"] == 1, launches
    check_flat(corpus, norms, queries, 10, L2, gd, gi, "fp32 fallback")
    # Rewriting the row back into range re-enables the split path.
    fixed = corpus[17:18].copy()
    fixed[0, 5] = 0.25
    c.write_rows(17, fixed)
    corpus[17] = fixed[0]
    gd, gi, launches = _search(gpu_ctx, c, queries, 10, L2)
    assert launches["flat_bound"] == 1, launches
    check_flat(corpus, oracle.row_norms(corpus), queries, 10, L2, gd, gi, "after write")
    c.release()


def test_split_query_outside_split_range_is_rerun(gpu_ctx):
    dim, n = 128, 8000
    corpus = workloads.lcg_vectors(1, n, dim, seed=31)
    queries = workloads.lcg_vectors(1, 33, dim, seed=32)
    queries[3, 0] = 4e15     # above 2^50 (its square still fits fp32)
    queries[4, 7] = 1e-30    # below 2^-50
    queries[5] = 0.0         # zero is in range
    norms = oracle.row_norms(corpus)
    c = gpu_ctx.upload(corpus)
    for metric in (COS, L2, IP):
        gd, gi, launches = _search(gpu_ctx, c, queries, 10, metric)
        assert launches["flat_bound"] == 1 and launches["flat_scan"] >= 1, launches
        check_flat(corpus, norms, queries, 10, metric, gd, gi, f"bad query m{metric}")
    c.release()


def test_split_mixture_1m_384_batch_1024(gpu_ctx):
    # The batch-1024 workload at full size: every query's ids carry their
    # exact distances in (distance, id) order; a sample of 64 queries equals
    # the oracle's exact top-10.
    print("split 1M x 384 mixture, 1024 queries", flush=True)
    db, q = workloads.mixture_1m_384(nq=1024)
    norms = oracle.row_norms(db)
    c = gpu_ctx.upload(db)
    gd, gi, launches = _search(gpu_ctx, c, q, 10, COS)
    assert launches["flat_bound"] == 1 and launches["flat_gemm"] == 1
    for i in range(1024):
        redo = oracle.distances_for_ids(db, norms, q[i], gi[i], COS)
        assert np.array_equal(redo, gd[i]), f"query {i}"
        order = np.lexsort((gi[i], gd[i]))
        assert np.array_equal(order, np.arange(10)), f"query {i} order"
    sel = np.arange(0, 1024, 16)
    check_flat(db, norms, q[sel], 10, COS, gd[sel], gi[sel], "1M batch 1024")
    c.release()
