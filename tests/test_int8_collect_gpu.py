"""Parity of the threshold-collect int8 scan.

Single queries and small groups (up to 64 queries) over corpora of at least
256 rows per block (about 131,000 rows and up), at budgets up to 1024, run
in two launches: a sampled launch over a sixteenth of each block's rows
gives each query a bound (the min(kc, nblk / 2)-th smallest block minimum:
at least that many rows lie at or below it), then every row at or below the
bound is collected and rescored, and the query's last block runs the budget
rounds of BoundedExactScan on what was collected: while the budget is at
most the number of rows collected, the budget smallest slots are among them,
so each round selects them (radix select), takes the k best exact slots and
checks the proof.  The answers and the round counts must equal the oracle's
restatement of BoundedExactScan bit for bit, as the list-based scan does.  A
bound that lets more rows through than the candidate buffer holds (many
equal keys) sends the query back to the list-based scan.
"""
import numpy as np
import pytest

from meltan_amd import workloads
from oracle import oracle
from test_flat_gpu import COS, IP, L2, check_flat
from test_int8_batch_gpu import _rounds_for
from test_int8_gpu import _assert_same, _oracle_rows

pytestmark = pytest.mark.gpu


def _run(ctx, corpus, queries, k, metric, mode, budget):
    ctx.timing(True)
    ctx.timing_reset()
    try:
        gd, gi, rounds = corpus.int8_search(queries, k, metric, mode=mode, budget=budget)
        launches = {name: ctx.timing_read(name)[1] for name in ("int8_bound", "int8_scan", "int8_gemm")}
    finally:
        ctx.timing(False)
    return gd, gi, rounds, launches


@pytest.mark.parametrize("dim", [64, 100, 384])
def test_int8_collect_matches_oracle(gpu_ctx, dim):
    # dim 100: an int8 row of 112 bytes (seven 16-byte chunks) and a last
    # rescore piece of four floats.
    n, nq = 150000, 3
    corpus = workloads.lcg_vectors(1, n, dim, seed=700 + dim)
    queries = workloads.lcg_vectors(1, nq, dim, seed=701 + dim)
    norms = oracle.row_norms(corpus)
    planes = oracle.int8_build(corpus)
    c = gpu_ctx.upload(corpus)
    for metric in (COS, L2, IP):
        for mode, k, budget in ((0, 10, 0), (1, 10, 100), (1, 5, 7), (1, 16, 256)):
            print(f"int8 collect dim{dim} m{metric} mode{mode} k{k} b{budget}", flush=True)
            gd, gi, rounds, launches = _run(gpu_ctx, c, queries, k, metric, mode, budget)
            assert launches["int8_bound"] == 1 and launches["int8_gemm"] == 0, launches
            ref = _oracle_rows(corpus, norms, planes, queries, k, metric, mode=mode, budget=budget)
            _assert_same(gd, gi, ref, k, f"collect dim{dim} m{metric} mode{mode} b{budget}")
            if mode == 1:
                assert np.all(rounds == 1)
                assert launches["int8_scan"] == 1, launches
            else:
                finals = [oracle.int8_search(corpus, norms, planes, q, k, metric)[2] for q in queries]
                assert list(rounds) == [_rounds_for(f, k, n) for f in finals]
                check_flat(corpus, norms, queries, k, metric, gd, gi, f"collect exact m{metric}")
    c.release()


def test_int8_collect_many_equal_keys(gpu_ctx):
    # Every row of the first corpus is the same vector: all keys are equal,
    # slots order by row id, and the bound lets about kc blocks' worth of
    # rows through (more than 4,096: the radix select reads them from
    # global memory).  In the second, with more rows per block than blocks,
    # they overflow the candidate buffer and the query is selected again by
    # the list-based scan.
    dim = 32
    base = workloads.lcg_vectors(1, 1, dim, seed=81)[0]
    queries = workloads.lcg_vectors(1, 2, dim, seed=82)
    for n, overflow in ((150000, False), (400000, True)):
        print(f"int8 collect equal keys n={n}", flush=True)
        corpus = np.tile(base, (n, 1))
        norms = oracle.row_norms(corpus)
        planes = oracle.int8_build(corpus)
        c = gpu_ctx.upload(corpus)
        for metric in (COS, L2):
            gd, gi, rounds, launches = _run(gpu_ctx, c, queries, 10, metric, 1, 100)
            assert launches["int8_bound"] == 1
            assert launches["int8_scan"] == (2 if overflow else 1), launches
            assert np.all(rounds == 1)
            ref = _oracle_rows(corpus, norms, planes, queries, 10, metric, mode=1, budget=100)
            _assert_same(gd, gi, ref, 10, f"equal keys n{n} m{metric}")
            assert np.array_equal(gi, np.tile(np.arange(10, dtype=np.uint32), (2, 1)))
        c.release()


def test_int8_collect_small_batch_and_zero_query(gpu_ctx):
    # A batch below the matrix-core threshold (15 queries, one grid row
    # each), with a zero query (cosine keys of 1 for every row) among them.
    dim, n, nq = 96, 140000, 15
    corpus = workloads.lcg_vectors(0, n, dim, seed=91)
    queries = workloads.lcg_vectors(0, nq, dim, seed=92)
    queries[4] = 0.0
    norms = oracle.row_norms(corpus)
    planes = oracle.int8_build(corpus)
    c = gpu_ctx.upload(corpus)
    for metric, mode, budget in ((COS, 1, 100), (L2, 0, 0), (IP, 1, 50)):
        print(f"int8 collect batch m{metric} mode{mode}", flush=True)
        gd, gi, _, launches = _run(gpu_ctx, c, queries, 10, metric, mode, budget)
        assert launches["int8_bound"] == 1 and launches["int8_gemm"] == 0, launches
        ref = _oracle_rows(corpus, norms, planes, queries, 10, metric, mode=mode, budget=budget)
        _assert_same(gd, gi, ref, 10, f"batch m{metric} mode{mode}")
    c.release()


def test_int8_collect_adversarial_rounds(gpu_ctx):
    # The zero / duplicate / extreme-magnitude layout of
    # BoundedExactScanTests.swift:211-250 at a size that takes the collect
    # path: proofs that fail in the first round re-run on the list-based
    # scan with the codes the sampled launch stored, and every round count
    # and result must still equal the oracle's.
    dim, n = 64, 140000
    rows = workloads.lcg_vectors(1, n, dim, seed=3024)
    corpus = rows.copy()
    corpus[0::4] = 0.0
    corpus[1::4] = rows[0]
    idx = np.arange(n)
    corpus[idx % 8 == 2] *= 1e-5
    corpus[idx % 8 == 6] *= 1e5
    norms = oracle.row_norms(corpus)
    planes = oracle.int8_build(corpus)
    c = gpu_ctx.upload(corpus)
    q = workloads.lcg_vectors(1, 3, dim, seed=3025)
    for metric in (COS, L2, IP):
        for k in (10, 16):  # mode 0 starts at kc = max(256, 16 k)
            print(f"int8 collect adversarial m{metric} k{k}", flush=True)
            gd, gi, rounds, launches = _run(gpu_ctx, c, q, k, metric, 0, 0)
            assert launches["int8_bound"] == 1, launches
            ref = _oracle_rows(corpus, norms, planes, q, k, metric)
            _assert_same(gd, gi, ref, k, f"collect adversarial m{metric} k{k}")
            # Rounds past a budget of 1024 end in the exact scan, so the
            # round counts are compared where the oracle stops by then.
            finals = [oracle.int8_search(corpus, norms, planes, qq, k, metric)[2] for qq in q]
            for r, f in zip(rounds, finals):
                if f <= 1024:
                    assert r == _rounds_for(f, k, n)
            check_flat(corpus, norms, q, k, metric, gd, gi, f"collect adversarial exact m{metric} k{k}")
    c.release()
