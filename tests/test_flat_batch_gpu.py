"""Parity of the batched flat path (fp32 MFMA contraction + fused selection).

Batches of at least 16 queries with k <= 32 at dims 64/96/128/192/256/384 go
through the matrix-core kernel; its keys are lower bounds, so the returned
rows must meet the same bar as the streaming scan: distances bit-identical to
the oracle's (dots.c order, host formulas), ids equal except on exact ties.
Every case also checks through the timing counters that the batched kernel
is the one that ran.
"""
import numpy as np
import pytest

from oracle import oracle
from meltan_amd import workloads
from test_flat_gpu import COS, IP, L2, check_flat

pytestmark = pytest.mark.gpu


def _search_batched(ctx, corpus, queries, k, metric):
    ctx.timing(True)
    ctx.timing_reset()
    try:
        gd, gi = corpus.flat_search(queries, k, metric)
        _, launches = ctx.timing_read("flat_gemm")
    finally:
        ctx.timing(False)
    return gd, gi, launches


@pytest.mark.parametrize("dim", [64, 96, 128, 192, 256, 384])
def test_batched_parity_dims_metrics(gpu_ctx, dim):
    print(f"batched parity dim={dim}", flush=True)
    for n, nq in ((4100, 16), (7777, 130)):
        corpus = workloads.lcg_vectors(0, n, dim, seed=n + dim)
        queries = workloads.lcg_vectors(0, nq, dim, seed=n + dim + 7)
        norms = oracle.row_norms(corpus)
        c = gpu_ctx.upload(corpus)
        for metric in (COS, L2, IP):
            for k in (1, 10, 16, 32):
                gd, gi, launches = _search_batched(gpu_ctx, c, queries, k, metric)
                assert launches >= 1, "the batched kernel did not run"
                check_flat(corpus, norms, queries, k, metric, gd, gi,
                           f"dim{dim} n{n} nq{nq} m{metric} k{k}")
        c.release()


def test_batched_ragged_sizes(gpu_ctx):
    # n not a multiple of the 32-row tile, segments past the end, nq not a
    # multiple of the 128-query block.
    dim = 96
    for n, nq in ((4097, 17), (5000, 129), (20000, 257), (65569, 300)):
        print(f"batched ragged n={n} nq={nq}", flush=True)
        corpus = workloads.lcg_vectors(1, n, dim, seed=n)
        queries = workloads.lcg_vectors(1, nq, dim, seed=n + 1)
        norms = oracle.row_norms(corpus)
        c = gpu_ctx.upload(corpus)
        gd, gi, launches = _search_batched(gpu_ctx, c, queries, 10, L2)
        assert launches >= 1
        check_flat(corpus, norms, queries, 10, L2, gd, gi, f"ragged n{n} nq{nq}")
        c.release()


def test_batched_adversarial_duplicates_zeros_tiny(gpu_ctx):
    # Zero rows, exact duplicates (ties broken by id) and rows scaled to
    # 1e-20 (products below the smallest normal) next to large ones.
    dim, n = 128, 9000
    rows = workloads.lcg_vectors(1, n, dim, seed=77)
    corpus = rows.copy()
    corpus[0::5] = 0.0
    corpus[1::5] = rows[3]
    idx = np.arange(n)
    corpus[idx % 7 == 2] *= 1e-20
    corpus[idx % 7 == 4] *= 1e4
    norms = oracle.row_norms(corpus)
    queries = workloads.lcg_vectors(1, 40, dim, seed=78)
    queries[5] = 0.0
    queries[6] = corpus[1]
    queries[7] *= 1e-20
    c = gpu_ctx.upload(corpus)
    for metric in (COS, L2, IP):
        gd, gi, launches = _search_batched(gpu_ctx, c, queries, 16, metric)
        assert launches >= 1
        check_flat(corpus, norms, queries, 16, metric, gd, gi, f"adversarial m{metric}")
    c.release()


def test_batched_100k_noisy_batch_1024(gpu_ctx):
    print("batched 100k x 384 batch 1024", flush=True)
    db, q = workloads.flat_100k(1024)
    norms = oracle.row_norms(db)
    c = gpu_ctx.upload(db)
    gd, gi, launches = _search_batched(gpu_ctx, c, q, 10, COS)
    assert launches >= 1
    sel = np.arange(0, 1024, 8)  # the oracle checks an eighth of the batch
    check_flat(db, norms, q[sel], 10, COS, gd[sel], gi[sel], "100k batch 1024")
    c.release()


def test_batched_small_corpus_uses_streaming_path(gpu_ctx):
    corpus = workloads.lcg_vectors(0, 4000, 64, seed=15)
    queries = workloads.lcg_vectors(0, 40, 64, seed=16)
    c = gpu_ctx.upload(corpus)
    gd, gi, launches = _search_batched(gpu_ctx, c, queries, 10, L2)
    assert launches == 0
    check_flat(corpus, oracle.row_norms(corpus), queries, 10, L2, gd, gi, "n4000")
    c.release()


def test_batched_large_k_uses_streaming_path(gpu_ctx):
    # k > 32 needs more candidates than the batched kernel keeps per lane.
    corpus = workloads.lcg_vectors(0, 5000, 64, seed=5)
    queries = workloads.lcg_vectors(0, 20, 64, seed=6)
    c = gpu_ctx.upload(corpus)
    gd, gi, launches = _search_batched(gpu_ctx, c, queries, 40, COS)
    assert launches == 0
    check_flat(corpus, oracle.row_norms(corpus), queries, 40, COS, gd, gi, "k40")
    c.release()
