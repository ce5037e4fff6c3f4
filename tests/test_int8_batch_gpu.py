"""Parity of the batched int8 prefilter (i8 MFMA contraction + fused key
selection, then the per-query merge, exact rescore and proof).

Batches of at least 16 queries go through the matrix-core kernel.  Its dots
are exact integer sums, its keys are the reference's formulas
(BoundedExactScan.swift:178-228) in the same operation order, and its
selection must be the kc smallest (key, row) slots, so every batched result
must equal the oracle's restatement of BoundedExactScan bit for bit: mode 0
(adaptive budget, margin proof) and mode 1 (one round at a fixed budget,
including the approximate answers a small budget gives).  The timing
counters show which kernels ran.
"""
import numpy as np
import pytest

from meltan_amd import workloads
from oracle import oracle
from test_flat_gpu import COS, IP, L2
from test_int8_gpu import _assert_same, _oracle_rows

pytestmark = pytest.mark.gpu


def _rounds_for(final_budget, k, n):
    """Rounds of BoundedExactScan.swift:95-118 that end at `final_budget`."""
    b, r = min(max(256, 16 * k), n), 1
    while b < final_budget:
        b, r = min(4 * b, n), r + 1
    return r


def _batched(ctx, corpus, queries, k, metric, mode, budget):
    ctx.timing(True)
    ctx.timing_reset()
    try:
        gd, gi, rounds = corpus.int8_search(queries, k, metric, mode=mode, budget=budget)
        launches = {name: ctx.timing_read(name)[1] for name in ("int8_gemm", "int8_merge", "int8_scan")}
    finally:
        ctx.timing(False)
    return gd, gi, rounds, launches


@pytest.mark.parametrize("dim", [64, 80, 96, 128, 384])
def test_int8_batched_matches_oracle(gpu_ctx, dim):
    # dim 80: a 16-byte code stride that is not a whole number of 32-byte
    # MFMA steps (the kernel pads the last step with zero codes).
    n, nq = 20000, 40
    corpus = workloads.lcg_vectors(1, n, dim, seed=900 + dim)
    queries = workloads.lcg_vectors(1, nq, dim, seed=901 + dim)
    norms = oracle.row_norms(corpus)
    planes = oracle.int8_build(corpus)
    c = gpu_ctx.upload(corpus)
    for metric in (COS, L2, IP):
        for mode, k, budget in ((0, 10, 0), (1, 10, 100), (1, 5, 7)):
            print(f"int8 batched dim{dim} m{metric} mode{mode} k{k} b{budget}", flush=True)
            gd, gi, rounds, launches = _batched(gpu_ctx, c, queries, k, metric, mode, budget)
            assert launches["int8_gemm"] == 1, launches
            if mode == 1:
                assert np.all(rounds == 1)
            ref = _oracle_rows(corpus, norms, planes, queries, k, metric, mode=mode, budget=budget)
            _assert_same(gd, gi, ref, k, f"dim{dim} m{metric} mode{mode} b{budget}")
            if mode == 0:
                finals = [oracle.int8_search(corpus, norms, planes, q, k, metric)[2] for q in queries]
                assert list(rounds) == [_rounds_for(f, k, n) for f in finals]
    c.release()


def test_int8_batched_ragged(gpu_ctx):
    # n not a multiple of the 64-row stage, nq not a multiple of the
    # 128-query block, segments that end inside a stage.
    dim = 96
    for n, nq in ((16384 + 37, 17), (30011, 129), (70001, 300)):
        print(f"int8 batched ragged n={n} nq={nq}", flush=True)
        corpus = workloads.lcg_vectors(0, n, dim, seed=n)
        queries = workloads.lcg_vectors(0, nq, dim, seed=n + 1)
        norms = oracle.row_norms(corpus)
        planes = oracle.int8_build(corpus)
        c = gpu_ctx.upload(corpus)
        gd, gi, _, launches = _batched(gpu_ctx, c, queries, 10, COS, 1, 64)
        assert launches["int8_gemm"] == 1
        ref = _oracle_rows(corpus, norms, planes, queries, 10, COS, mode=1, budget=64)
        _assert_same(gd, gi, ref, 10, f"ragged n{n} nq{nq}")
        c.release()


def test_int8_batched_crowded_segment_is_selected_again(gpu_ctx):
    # Every query's best rows sit in the first segment (near-copies of the
    # queries in rows 0..399), more than its two 8-slot lane lists hold: in
    # mode 1 the merge cannot show an exact selection, and the streaming
    # scan selects those queries again at the same budget.  In mode 0 the
    # contraction gathers into 128-slot regions, which hold them.
    dim, n, nq = 64, 40000, 20
    rng = np.random.default_rng(77)
    corpus = workloads.lcg_vectors(1, n, dim, seed=78)
    queries = workloads.lcg_vectors(1, nq, dim, seed=79)
    for i in range(400):
        corpus[i] = queries[i % nq] + rng.normal(0, 1e-3, dim).astype(np.float32)
    norms = oracle.row_norms(corpus)
    planes = oracle.int8_build(corpus)
    c = gpu_ctx.upload(corpus)
    for metric, mode, budget in ((COS, 1, 100), (L2, 0, 0)):
        print(f"int8 crowded m{metric} mode{mode}", flush=True)
        gd, gi, rounds, launches = _batched(gpu_ctx, c, queries, 10, metric, mode, budget)
        assert launches["int8_gemm"] == 1, launches
        if mode == 1:
            assert launches["int8_scan"] >= 1, launches
        ref = _oracle_rows(corpus, norms, planes, queries, 10, metric, mode=mode, budget=budget)
        _assert_same(gd, gi, ref, 10, f"crowded m{metric}")
        if mode == 1:
            assert np.all(rounds == 1)
    c.release()


def test_int8_batched_mixture_1m_384(gpu_ctx):
    # The C3 workload at full size: 1,000,000 x 384 (1,000-centre mixture),
    # 1024 queries, top-100 prefilter then rerank to 10.  A sample of queries
    # is checked against the oracle bit for bit; every query's ids must
    # carry their exact distances.
    print("int8 batched 1M x 384 mixture, 1024 queries", flush=True)
    db, q = workloads.mixture_1m_384(nq=1024)
    c = gpu_ctx.upload(db)
    gd, gi, rounds, launches = _batched(gpu_ctx, c, q, 10, COS, 1, 100)
    assert launches["int8_gemm"] == 1
    assert np.all(rounds == 1)
    norms = oracle.row_norms(db)
    for i in range(0, 1024, 97):
        redo = oracle.distances_for_ids(db, norms, q[i], gi[i], COS)
        assert np.array_equal(redo, gd[i]), f"query {i}"
        assert np.all(np.diff(gd[i]) >= 0)
    planes = oracle.int8_build(db)
    sample = [0, 1, 511, 1023]
    ref = _oracle_rows(db, norms, planes, q[sample], 10, COS, mode=1, budget=100)
    _assert_same(gd[sample], gi[sample], ref, 10, "1M mode1 batch")
    c.release()


def test_int8_batched_mode0_rounds_on_gathered_slots(gpu_ctx):
    # Mode 0 on the 1M x 384 mixture with 24 queries: the MFMA contraction
    # gathers every slot at or below a bound from 256 sampled slots, and one
    # block per query runs the budget rounds (256, 1024, ...) on what was
    # gathered; the mixture needs budget 1024 for most queries.  Results
    # equal the exact flat search and the round counts equal the oracle's
    # restatement of BoundedExactScan.
    print("int8 batched mode 0, 1M x 384 mixture, 24 queries", flush=True)
    db, q = workloads.mixture_1m_384(nq=24)
    c = gpu_ctx.upload(db)
    gd, gi, rounds, launches = _batched(gpu_ctx, c, q, 10, COS, 0, 0)
    assert launches["int8_gemm"] == 1, launches
    fd, fi = c.flat_search(q, 10, COS)
    assert np.array_equal(gd, fd) and np.array_equal(gi, fi)
    assert np.any(rounds > 1)
    norms = oracle.row_norms(db)
    planes = oracle.int8_build(db)
    for i in (0, 7, 23):
        final = oracle.int8_search(db, norms, planes, q[i], 10, COS)[2]
        assert rounds[i] == _rounds_for(final, 10, len(db)), f"query {i}"
    c.release()
