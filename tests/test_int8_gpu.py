"""Parity of the HIP int8 prefilter + fp32 rerank (mans_int8_search).

The bar (BoundedExactScan.swift:30-369, Int8CodeCache.swift:64-99):
  - the device codes and planes are bit-identical to the oracle's
    Int8CodeBuffer.fill restatement;
  - mode 0 (adaptive budget with the margin proof) returns exactly what the
    oracle's restatement returns, which is the exact top-k (bit-identical
    distances, ids equal except on exact ties);
  - mode 1 (one round at a fixed budget, no proof) returns the oracle's
    top-k of the rescored budget candidates, bit for bit, including the
    approximate answers a too-small budget gives.
Cases follow BoundedExactScanTests.swift:175-393 (LCG data, zero rows,
duplicates, extreme magnitudes, every metric).
"""
import numpy as np
import pytest

import meltan_amd as M
from meltan_amd import workloads
from oracle import oracle
from test_flat_gpu import COS, IP, L2, check_flat

pytestmark = pytest.mark.gpu


def _oracle_rows(corpus, norms, planes, queries, k, metric, mode=0, budget=0):
    out = []
    for q in queries:
        d, i, _ = oracle.int8_search(corpus, norms, planes, q, k, metric, mode=mode, budget=budget)
        out.append((d, i))
    return out


def _assert_same(gd, gi, ref, k, what):
    for qi, (od, oi) in enumerate(ref):
        kk = len(od)
        assert np.array_equal(gd[qi, :kk], od), f"{what} q{qi}: {gd[qi, :kk][:4]} vs {od[:4]}"
        for j in range(kk):
            tied = (j > 0 and od[j - 1] == od[j]) or (j + 1 < kk and od[j + 1] == od[j]) or j == kk - 1
            if not tied:
                assert gi[qi, j] == oi[j], f"{what} q{qi} rank {j}"
        assert np.all(gd[qi, kk:] == np.finfo(np.float32).max)
        assert np.all(gi[qi, kk:] == M.EMPTY_ID)


@pytest.mark.parametrize("dim", [64, 96, 384])
def test_int8_codes_bit_exact(gpu_ctx, dim):
    n = 16384 + 100
    corpus = workloads.lcg_vectors(1, n, dim, seed=dim)
    corpus[7] = 0.0                      # zero row: scale 1, codes 0
    corpus[8] *= 1e-30                   # tiny row
    corpus[9, :3] = [1e30, -1e30, 0.5]   # huge magnitudes
    c = gpu_ctx.upload(corpus)
    got = c.int8_codes()
    ref = oracle.int8_build(corpus)
    for name, g, r in zip(("codes", "u", "w", "normSq", "invSqrt"), got, ref):
        assert np.array_equal(g, r), f"dim {dim}: {name} differs"
    c.release()


@pytest.mark.parametrize("metric", [COS, L2, IP])
def test_int8_mode0_matches_oracle_and_flat(gpu_ctx, metric):
    dim, n = 128, 20000
    corpus = workloads.lcg_vectors(1, n, dim, seed=401 + metric)
    queries = workloads.lcg_vectors(1, 6, dim, seed=402 + metric)
    norms = oracle.row_norms(corpus)
    planes = oracle.int8_build(corpus)
    c = gpu_ctx.upload(corpus)
    for k in (1, 10, 100):
        print(f"int8 mode0 m{metric} k{k}", flush=True)
        gd, gi, rounds = c.int8_search(queries, k, metric, mode=0)
        assert np.all(rounds >= 1)
        ref = _oracle_rows(corpus, norms, planes, queries, k, metric)
        _assert_same(gd, gi, ref, k, f"m{metric} k{k}")
        check_flat(corpus, norms, queries, k, metric, gd, gi, f"exact m{metric} k{k}")
    c.release()


@pytest.mark.parametrize("metric", [COS, L2, IP])
def test_int8_mode1_fixed_budget_matches_oracle(gpu_ctx, metric):
    dim, n = 96, 30000
    corpus = workloads.lcg_vectors(0, n, dim, seed=501 + metric)
    queries = workloads.lcg_vectors(0, 5, dim, seed=502 + metric)
    norms = oracle.row_norms(corpus)
    planes = oracle.int8_build(corpus)
    c = gpu_ctx.upload(corpus)
    for k, budget in ((10, 100), (10, 10), (5, 3), (16, 1000)):
        print(f"int8 mode1 m{metric} k{k} budget{budget}", flush=True)
        gd, gi, rounds = c.int8_search(queries, k, metric, mode=1, budget=budget)
        assert np.all(rounds == 1)
        ref = _oracle_rows(corpus, norms, planes, queries, k, metric, mode=1, budget=budget)
        _assert_same(gd, gi, ref, k, f"m{metric} k{k} b{budget}")
    c.release()


def test_int8_adversarial_zeros_duplicates_extremes(gpu_ctx):
    # BoundedExactScanTests.swift:211-250 layout.
    dim, n = 64, 16384 + 512
    rows = workloads.lcg_vectors(1, n, dim, seed=2024)
    corpus = rows.copy()
    corpus[0::4] = 0.0
    corpus[1::4] = rows[0]
    idx = np.arange(n)
    corpus[idx % 8 == 2] *= 1e-5
    corpus[idx % 8 == 6] *= 1e5
    norms = oracle.row_norms(corpus)
    planes = oracle.int8_build(corpus)
    c = gpu_ctx.upload(corpus)
    q = workloads.lcg_vectors(1, 3, dim, seed=2025)
    for metric in (COS, L2, IP):
        for k in (24, 256):
            print(f"int8 adversarial m{metric} k{k}", flush=True)
            gd, gi, _ = c.int8_search(q, k, metric, mode=0)
            ref = _oracle_rows(corpus, norms, planes, q, k, metric)
            _assert_same(gd, gi, ref, k, f"adversarial m{metric} k{k}")
            check_flat(corpus, norms, q, k, metric, gd, gi, f"adversarial exact m{metric} k{k}")
    c.release()


def test_int8_small_corpus_is_tier_degradeable(gpu_ctx):
    corpus = workloads.lcg_vectors(0, 16383, 32, seed=3)
    c = gpu_ctx.upload(corpus)
    with pytest.raises(M.ANNSError) as ei:
        c.int8_search(corpus[:1], 10, COS)
    assert ei.value.code == M.PIPELINE_UNAVAILABLE and ei.value.is_tier_degradeable
    with pytest.raises(M.ANNSError):
        c.int8_search(corpus[:1], 10, 3)  # hamming
    c.release()


def test_int8_write_rows_refreshes_codes(gpu_ctx):
    dim, n = 64, 17000
    corpus = workloads.lcg_vectors(1, n, dim, seed=71)
    c = gpu_ctx.upload(corpus)
    c.int8_codes()  # build
    new = workloads.lcg_vectors(1, 300, dim, seed=72) * 3.0
    c.write_rows(1000, new)
    corpus[1000:1300] = new
    got = c.int8_codes()
    ref = oracle.int8_build(corpus)
    for g, r in zip(got, ref):
        assert np.array_equal(g, r)
    q = corpus[1100:1103].copy()
    gd, gi, _ = c.int8_search(q, 5, L2)
    check_flat(corpus, oracle.row_norms(corpus), q, 5, L2, gd, gi, "after write")
    c.invalidate()
    got = c.int8_codes()
    assert np.array_equal(got[0], ref[0])
    c.release()


def test_int8_unsupported_dim_mode0_is_exact(gpu_ctx):
    # dim % 4 != 0: the proof-checked search still returns the exact answer.
    dim, n = 66, 16400
    corpus = workloads.lcg_vectors(0, n, dim, seed=81)
    q = workloads.lcg_vectors(0, 2, dim, seed=82)
    c = gpu_ctx.upload(corpus)
    gd, gi, _ = c.int8_search(q, 10, COS, mode=0)
    check_flat(corpus, oracle.row_norms(corpus), q, 10, COS, gd, gi, "dim66")
    with pytest.raises(M.ANNSError):
        c.int8_search(q, 10, COS, mode=1, budget=100)
    c.release()


def test_int8_mixture_1m_384_sample(gpu_ctx):
    # The 1,000-centre mixture at full size: mode 0 equals the exact flat
    # result; mode 1 with the top-100 prefilter equals the oracle's.
    print("int8 1M x 384 mixture", flush=True)
    db, q = workloads.mixture_1m_384(nq=8)
    c = gpu_ctx.upload(db)
    fd, fi = c.flat_search(q, 10, COS)
    gd, gi, rounds = c.int8_search(q, 10, COS, mode=0)
    assert np.array_equal(gd, fd)
    assert np.array_equal(gi, fi)
    norms = oracle.row_norms(db)
    planes = oracle.int8_build(db)
    # Single queries: one collect launch whose last block runs every budget
    # round the proof needs; the round counts equal the oracle's.
    from test_int8_batch_gpu import _rounds_for
    for i in range(3):
        _, gi1, r1 = c.int8_search(q[i:i + 1], 10, COS, mode=0)
        final = oracle.int8_search(db, norms, planes, q[i], 10, COS)[2]
        assert r1[0] == _rounds_for(final, 10, len(db)), f"query {i}"
        assert np.array_equal(gi1[0], fi[i])
    gd1, gi1, _ = c.int8_search(q[:3], 10, COS, mode=1, budget=100)
    ref = _oracle_rows(db, norms, planes, q[:3], 10, COS, mode=1, budget=100)
    _assert_same(gd1, gi1, ref, 10, "1M mode1")
    c.release()
