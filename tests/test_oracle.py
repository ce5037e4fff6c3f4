"""Pins the CPU oracle before it is trusted as the parity checker.

Each check is chosen so that a plausible slip in the restatement (a dropped
term, a wrong sign or index, a transposed operand) fails it: golden vectors
of the reference's own dots.c, literal known-answer cases of the reference's
tests, closed forms, and brute force in float64 on small inputs.
"""
import json
import math

import numpy as np
import pytest

from conftest import GOLDEN
from meltan_amd import workloads
from oracle import oracle

COS, L2, IP = 0, 1, 2
DIMS = [1, 3, 16, 66, 128, 333, 384]


# ---- dots.c golden vectors (bit-exact) --------------------------------------------

@pytest.mark.parametrize("dim", DIMS)
def test_dots_match_reference_golden(golden_dots, dim):
    g = golden_dots
    corpus, q = g[f"corpus_{dim}"], g[f"query_{dim}"]
    assert np.array_equal(oracle.f32_dot_rows(corpus, q).view(np.uint32),
                          g[f"f32_{dim}"].view(np.uint32))
    assert np.array_equal(oracle.f32_dot_rows_gather(corpus, q, g[f"idx_{dim}"]).view(np.uint32),
                          g[f"gather_{dim}"].view(np.uint32))
    assert np.array_equal(oracle.i8_dot_rows(g[f"codes_{dim}"], g[f"qcodes_{dim}"]),
                          g[f"i8_{dim}"])


def test_dots_match_reference_library_on_fresh_inputs():
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    rng = np.random.default_rng(5)
    for dim in (7, 64, 385):
        corpus = rng.standard_normal((50, dim)).astype(np.float32)
        q = rng.standard_normal(dim).astype(np.float32)
        out = np.empty(50, np.float32)
        ref.mans_f32_dot_rows(corpus.ctypes.data, q.ctypes.data, 50, dim, out.ctypes.data)
        assert np.array_equal(out.view(np.uint32), oracle.f32_dot_rows(corpus, q).view(np.uint32))


def test_dot_order_is_sequential_not_pairwise():
    # 1 + 2^-24 + 2^-24 sums to 1 left-to-right, to 1 + 2^-23 pairwise.
    corpus = np.array([[1.0, 2.0 ** -24, 2.0 ** -24]], np.float32)
    q = np.ones(3, np.float32)
    assert oracle.f32_dot_rows(corpus, q)[0] == np.float32(1.0)


# ---- distance known answers ----------------------------------------------------------

def _kat_vec(v):
    if v == "ones128":
        return np.ones(128, np.float32)
    if v == "unit1536":
        return np.full(1536, 1.0 / math.sqrt(1536), np.float32)
    return np.asarray(v, np.float32)


def test_distance_kats():
    kats = json.loads((GOLDEN / "reference_kats.json").read_text())
    for case in kats["distance"]:
        q, v = _kat_vec(case["query"]), _kat_vec(case["vector"])
        m = case["metric"]
        dot = oracle.f32_dot_rows(v[None, :], q)[0]
        d = oracle.host_distance(dot, oracle.row_norms(q[None, :])[0],
                                 oracle.row_norms(v[None, :])[0], m)
        assert abs(d - case["expect"]) <= case["tol"], case["from"]
        assert abs(oracle.simd_distance(q, v, m) - case["expect"]) <= case["tol"], case["from"]


def test_cosine_degenerate_denominator_is_one():
    z = np.zeros((1, 8), np.float32)
    q = np.ones(8, np.float32)
    assert oracle.host_distance(0.0, 8.0, 0.0, COS) == 1.0
    dist, ids = oracle.flat_search(z, oracle.row_norms(z), q, 1, COS)
    assert dist[0] == 1.0 and ids[0] == 0


# ---- selection semantics (BoundedSelectionTests literal cases) -----------------

def test_sorted_list_kats():
    kats = json.loads((GOLDEN / "reference_kats.json").read_text())
    for case in kats["sorted_list"]:
        tags = {}
        scores, ids = [], []
        for step in case["steps"]:
            for s, t in step["insert"]:
                tid = tags.setdefault(t, len(tags))
                scores.append(np.inf if s == "inf" else float(s))
                ids.append(tid)
            _, got = oracle.sorted_list_run(np.array(scores), np.array(ids), case["capacity"])
            names = {v: k for k, v in tags.items()}
            assert [names[i] for i in got] == step["expect"], case["from"]


def test_sorted_list_matches_linear_reference():
    # BoundedSelectionTests.swift:104-145 reference insert, on quarter-rounded
    # scores so ties are frequent.
    rng = np.random.default_rng(4096)
    for trial in range(24):
        length, cap = int(rng.integers(1, 200)), int(rng.integers(1, 40))
        scores = rng.uniform(-10, 10, length).astype(np.float32)
        if trial % 2 == 0:
            scores = (np.round(scores * 4) / 4).astype(np.float32)
        ref = []
        for i, s in enumerate(scores):
            if len(ref) == cap and not (s < ref[-1][0]):
                continue
            j = 0
            while j < len(ref) and ref[j][0] < s:
                j += 1
            ref.insert(j, (s, i))
            if len(ref) > cap:
                ref.pop()
        got_s, got_i = oracle.sorted_list_run(scores, np.arange(length), cap)
        assert got_i.tolist() == [i for _, i in ref]


# ---- exact flat scan -------------------------------------------------------------

def _brute(corpus, q, metric):
    c, qq = corpus.astype(np.float64), q.astype(np.float64)
    dot = c @ qq
    if metric == IP:
        d = -dot
    elif metric == L2:
        d = ((c - qq) ** 2).sum(1)
    else:
        den = np.sqrt((c * c).sum(1) * (qq @ qq))
        d = np.where(den < 1e-10, 1.0, 1.0 - dot / np.where(den == 0, 1, den))
    order = np.lexsort((np.arange(len(d)), d))
    return d, order


@pytest.mark.parametrize("metric", [COS, L2, IP])
@pytest.mark.parametrize("n,dim", [(64, 128), (100, 128), (2049, 128), (5000, 66), (4200, 16)])
def test_flat_oracle_matches_bruteforce(metric, n, dim):
    corpus = workloads.lcg_vectors(0, n, dim, seed=n)
    q = workloads.lcg_vectors(0, 1, dim, seed=n + 1)[0]
    k = 100
    dist, ids = oracle.flat_search(corpus, oracle.row_norms(corpus), q, k, metric, cores=8)
    d64, order = _brute(corpus, q, metric)
    kk = min(k, n)
    assert len(ids) == kk
    assert np.all(np.diff(dist) >= 0)
    # the reference's own checker: set equality unless the k-boundary is a near tie
    gap = d64[order[kk]] - d64[order[kk - 1]] if n > kk else np.inf
    if gap > 1e-5:
        assert set(ids.tolist()) == set(order[:kk].tolist())
    assert np.allclose(dist, d64[ids], rtol=1e-5, atol=1e-5)


def test_flat_oracle_slicing_does_not_change_results():
    corpus = workloads.gauss_rows(77, 40000, 64, True)
    q = workloads.gauss_rows(78, 1, 64, True)[0]
    norms = oracle.row_norms(corpus)
    a = oracle.flat_search(corpus, norms, q, 24, COS, cores=1)
    b = oracle.flat_search(corpus, norms, q, 24, COS, cores=19, threads=4)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_flat_oracle_k_larger_than_n_and_cap():
    corpus = workloads.lcg_vectors(0, 70, 8, seed=3)
    q = corpus[5]
    d, ids = oracle.flat_search(corpus, oracle.row_norms(corpus), q, 500, L2)
    assert len(ids) == 70 and ids[0] == 5 and d[0] == 0.0
    corpus = workloads.lcg_vectors(0, 400, 8, seed=4)
    d, ids = oracle.flat_search(corpus, oracle.row_norms(corpus), corpus[0], 300, L2)
    assert len(ids) == 256  # FlatGPUSearch.maxTopK


# ---- int8 codes and the bounded scan ---------------------------------------------

def test_int8_codes_error_model():
    rng = np.random.default_rng(11)
    corpus = (rng.standard_normal((300, 96)) * rng.uniform(1e-3, 1e3, (300, 1))).astype(np.float32)
    corpus[0] = 0.0
    codes, u, w, ns, inv = oracle.int8_build(corpus)
    assert codes[0].tolist() == [0] * 96 and u[0] == 1.0 and inv[0] == 0.0
    c64, u64 = codes.astype(np.float64), u.astype(np.float64)[:, None]
    # |v - u c| <= u/2 (+ float rounding of v * (1/u)), |c| <= 127, max |c| == 127
    err = np.abs(corpus - u64 * c64)
    assert np.all(err[1:] <= u64[1:] * (0.5 + 1e-5))
    assert np.abs(codes).max() <= 127 and np.all(np.abs(codes[1:]).max(1) == 127)
    assert np.allclose(ns, (corpus.astype(np.float64) ** 2).sum(1), rtol=1e-5)
    absum = np.abs(c64).sum(1)
    assert np.allclose(w / u, (absum / 2 + 96 / 4) * (1 + 1e-6) + 16, rtol=1e-6)


def test_int8_dot_bound_contains_true_dot():
    # Int8CodeCache.swift:18-20 contract: dot(q,v) in qs*u*D +- qs*(w + u*|q|_1/2)
    rng = np.random.default_rng(12)
    corpus = rng.standard_normal((500, 128)).astype(np.float32)
    codes, u, w, ns, inv = oracle.int8_build(corpus)
    for seed in range(5):
        q = np.random.default_rng(seed).standard_normal(128).astype(np.float32)
        qs = np.abs(q).max() / 127.0
        qc = np.clip(np.trunc(q / qs + np.where(q >= 0, 0.5, -0.5)), -127, 127)
        D = codes.astype(np.float64) @ qc
        true = corpus.astype(np.float64) @ q.astype(np.float64)
        half = qs * (w + u * np.abs(qc).sum() / 2)
        assert np.all(np.abs(true - qs * u * D) <= half)


def _assert_exact(dist, ids, corpus, q, metric, k):
    d64, order = _brute(corpus, q, metric)
    kk = min(k, 256, len(d64))
    bd = d64[order[kk - 1]]
    gap = d64[order[kk]] - bd if len(d64) > kk else np.inf
    if gap > 2e-3:
        assert set(ids[:kk].tolist()) == set(order[:kk].tolist())
    else:
        assert set(ids[:kk].tolist()) <= set(np.nonzero(d64 <= bd + 2e-3)[0].tolist())
    tol = np.maximum(2e-3, np.abs(d64[ids[:kk]]) * 2e-3)
    assert np.all(np.abs(dist[:kk] - d64[ids[:kk]]) <= tol)


@pytest.mark.parametrize("dim", [16, 128, 333])
@pytest.mark.parametrize("metric", [COS, L2, IP])
def test_int8_oracle_is_exact(dim, metric):
    n = 16384 + 512  # BoundedExactScanTests.swift:169
    corpus = workloads.lcg_vectors(1, n, dim, seed=7)
    planes = oracle.int8_build(corpus)
    norms = oracle.row_norms(corpus)
    q = workloads.lcg_vectors(1, 1, dim, seed=7 + 123)[0]
    for k in (1, 24, 97):
        dist, ids, budget = oracle.int8_search(corpus, norms, planes, q, k, metric, cores=8)
        _assert_exact(dist, ids, corpus, q, metric, k)
        # and identical to the oracle's own fp32 scan, ties aside
        fd, fi = oracle.flat_search(corpus, norms, q, k, metric, cores=8)
        assert np.array_equal(np.sort(dist), np.sort(fd))


def test_int8_oracle_nil_below_threshold():
    corpus = workloads.lcg_vectors(1, 2048, 64, seed=12)
    planes = oracle.int8_build(corpus)
    assert oracle.int8_search(corpus, oracle.row_norms(corpus), planes,
                              np.full(64, 0.25, np.float32), 10, COS) is None


def test_int8_oracle_detects_a_dropped_bound_term():
    """Plants a mistake in the oracle's inputs (the w plane zeroed, i.e. the
    error term dropped) and checks the exactness test would catch it."""
    dim, n = 64, 16384 + 512
    corpus = workloads.lcg_vectors(1, n, dim, seed=99)
    codes, u, w, ns, inv = oracle.int8_build(corpus)
    norms = oracle.row_norms(corpus)
    caught = False
    for s in range(20):
        q = workloads.lcg_vectors(1, 1, dim, seed=500 + s)[0]
        d, ids, _ = oracle.int8_search(corpus, norms, (codes, u, np.zeros_like(w), ns, inv), q,
                                       97, IP, cores=8, mode=1, budget=100)
        fd, fi = oracle.flat_search(corpus, norms, q, 97, IP)
        if set(ids.tolist()) != set(fi.tolist()):
            caught = True
            break
    assert caught


# ---- IVF-flat --------------------------------------------------------------------

def test_ivf_probe_matches_reference_dots():
    ref = oracle.ref_lib()
    rng = np.random.default_rng(3)
    cent = rng.standard_normal((200, 32)).astype(np.float32)
    cent[17] = cent[3]  # a tie: lower index must win
    for metric in (COS, L2, IP):
        part_c = oracle.row_norms(cent)
        for s in range(5):
            q = rng.standard_normal(32).astype(np.float32)
            if ref is not None:
                dots = np.empty(200, np.float32)
                ref.mans_f32_dot_rows(cent.ctypes.data, q.ctypes.data, 200, 32, dots.ctypes.data)
            else:
                dots = oracle.f32_dot_rows(cent, q)
            qn = oracle.row_norms(q[None, :])[0]
            keys = np.array([oracle.host_distance(dots[c], qn, part_c[c], metric)
                             for c in range(200)], np.float32)
            want = np.sort(np.lexsort((np.arange(200), keys))[:12])
            p = oracle.IVFPartition(rng.standard_normal((10, 32)).astype(np.float32), cent, metric)
            assert p.probe(q, 12).tolist() == want.tolist()


@pytest.mark.parametrize("metric", [L2, COS, IP])
def test_ivf_full_probe_equals_bruteforce(metric):
    # IVFFlatSearchTests.swift:193-216: nprobe >= nlist gives brute force, in order.
    corpus = workloads.lcg_vectors(0, 3000, 24, seed=5)
    cent, _ = oracle.kmeans(corpus, 16, 4, metric)
    part = oracle.IVFPartition(corpus, cent, metric)
    norms = oracle.row_norms(corpus)
    for s in range(4):
        q = workloads.lcg_vectors(0, 1, 24, seed=50 + s)[0]
        d, ids, _ = part.search(q, 10, 16)
        fd, fi = oracle.flat_search(corpus, norms, q, 10, metric)
        assert ids.tolist() == fi.tolist() and np.array_equal(d, fd)


def test_ivf_lists_are_a_partition():
    corpus = workloads.gauss_rows(9, 5000, 16, False)
    cent, assign = oracle.kmeans(corpus, 32, 5, L2)
    off, ids = oracle.ivf_lists(assign, 32)
    assert off[0] == 0 and off[-1] == 5000 and np.all(np.diff(off) >= 0)
    assert np.array_equal(np.sort(ids), np.arange(5000))
    for c in range(32):
        seg = ids[off[c]:off[c + 1]]
        assert np.all(assign[seg] == c) and np.all(np.diff(seg.astype(np.int64)) > 0)
    # k-means returns the assignment of its last pass, before that pass's
    # update (KMeans.swift:253-256); each row's list is its nearest centroid
    # among the centroids that pass saw (float64 check, ties aside).
    prev, _ = oracle.kmeans(corpus, 32, 4, L2)
    d = ((corpus[:, None, :].astype(np.float64) - prev[None].astype(np.float64)) ** 2).sum(2)
    best = d.min(1)
    assert np.all(d[np.arange(5000), assign] <= best + 1e-4)


# ---- k-means (KMeans.swift:53-257) -------------------------------------------------

def _seq_mean(rows):
    """KMeans.swift:224-250: the Float sum in row order times 1 / Float(count)."""
    acc = np.zeros(rows.shape[1], np.float32)
    for r in rows:
        acc = (acc + r).astype(np.float32)
    return (acc * (np.float32(1.0) / np.float32(len(rows)))).astype(np.float32)


def _dist64(rows, cent, metric):
    a, b = rows.astype(np.float64), cent.astype(np.float64)
    if metric == L2:
        return ((a[:, None, :] - b[None]) ** 2).sum(2)
    dot = a @ b.T
    if metric == IP:
        return -dot
    return 1.0 - dot / (np.linalg.norm(a, axis=1)[:, None] * np.linalg.norm(b, axis=1)[None])


@pytest.mark.parametrize("metric", [L2, IP, COS])
def test_kmeans_update_is_the_float_mean_of_the_previous_assignment(metric):
    n, k = 3000, 20
    rows = workloads.gauss_rows(41, n, 12, False)
    init, a0 = oracle.kmeans(rows, k, 0, metric)
    assert np.all(a0 == -1)  # Result.assignments before any pass
    assert np.array_equal(init, rows[(np.arange(k) * (n // k)) % n])
    c1, a1 = oracle.kmeans(rows, k, 1, metric)
    d = _dist64(rows, init, metric)
    assert np.all(d[np.arange(n), a1] <= d.min(1) + 1e-5 * (1 + np.abs(d.min(1))))
    for c in range(k):
        members = rows[a1 == c]
        if len(members) == 0:
            assert np.array_equal(c1[c], init[c])
        else:
            assert np.array_equal(c1[c], _seq_mean(members)), c


def test_kmeans_returns_the_last_pass_and_stops_when_settled():
    n, k = 4000, 16
    ctr = workloads.centers(45, 16, 8)
    rows = workloads.mixture_rows(46, ctr, 0.3, n, False)[0]
    for t in (2, 3, 5):
        before, _ = oracle.kmeans(rows, k, t - 1, L2)
        _, at = oracle.kmeans(rows, k, t, L2)
        assert np.array_equal(at, _dist64(rows, before, L2).argmin(1))
    # Once a pass changes nothing the loop stops: more iterations change nothing.
    settled = None
    for t in range(2, 60):
        a, _ = oracle.kmeans(rows, k, t, L2)
        b, _ = oracle.kmeans(rows, k, t + 1, L2)
        if np.array_equal(a, b):
            settled = t
            break
    assert settled is not None
    c_many, a_many = oracle.kmeans(rows, k, 500, L2)
    c_set, _ = oracle.kmeans(rows, k, settled, L2)
    assert np.array_equal(c_many, c_set)
    assert np.array_equal(a_many, _dist64(rows, c_many, L2).argmin(1))


def test_kmeans_ties_go_to_the_first_centroid_and_empty_clusters_keep_theirs():
    n, k = 1000, 10
    rows = workloads.gauss_rows(47, n, 6, False)
    rows[n // k] = rows[0]  # initial centroids 0 and 1 coincide
    c, a = oracle.kmeans(rows, k, 1, L2)
    assert not np.any(a == 1) and a[n // k] == 0
    assert np.array_equal(c[1], rows[0])


def test_ivf_flat_train_uses_the_reference_sample():
    # IVFFlatSearch.swift:528-551.  With L >= 4096 the sample holds exactly L
    # rows at stride n // L; k-means with k equal to the sample size leaves
    # every (distinct) sample row as its own centroid.
    n = 3 * 4096 + 5
    rows = workloads.gauss_rows(48, n, 4, False)
    cent = oracle.ivf_flat_train(rows, 4096, L2)
    assert np.array_equal(cent, rows[0:3 * 4096:3])
    # Fewer rows than lists: L = n and every row is a centroid.
    cent = oracle.ivf_flat_train(rows[:100], 256, L2)
    assert np.array_equal(cent, rows[:100])
    # Small nlist: min(n, max(L, min(4096, 16 L))) rows at stride n // count,
    # clustered with 8 iterations.
    want, _ = oracle.kmeans(rows[0:n:n // 128][:128], 8, 8, IP)
    assert np.array_equal(oracle.ivf_flat_train(rows, 8, IP), want)


def test_ivfpq_train_closed_form_and_composition():
    # IVFPQIndex.swift:54-104, ProductQuantizer.swift:10-85.  With one coarse
    # list the centroid is the mean of all rows; with 256 rows every
    # codebook is the residuals' subvectors themselves.
    rng = np.random.default_rng(49)
    rows = rng.standard_normal((256, 16)).astype(np.float32)
    for metric in (L2, IP):
        coarse, books = oracle.ivfpq_train(rows, 1, 4, 5, metric)
        mean = _seq_mean(rows)
        assert np.array_equal(coarse[0], mean)
        res = (rows - mean).astype(np.float32)
        for sub in range(4):
            assert np.array_equal(books[sub], res[:, 4 * sub:4 * sub + 4])
    # Larger: coarse = k-means of the rows; codebooks = k-means of the
    # residual subvectors against the last pass's assignment.
    rows = workloads.gauss_rows(50, 1500, 12, False)
    coarse, books = oracle.ivfpq_train(rows, 6, 3, 4, IP)
    want_c, assign = oracle.kmeans(rows, 6, 4, IP)
    assert np.array_equal(coarse, want_c)
    res = (rows - want_c[assign]).astype(np.float32)
    for sub in range(3):
        want_b, _ = oracle.kmeans(np.ascontiguousarray(res[:, 4 * sub:4 * sub + 4]), 256, 4, L2)
        assert np.array_equal(books[sub], want_b)


# ---- PQ ----------------------------------------------------------------------------

def test_pq_encode_subtracting_equals_encode_residual():
    # ProductQuantizerTests.swift:91-109
    rng = np.random.default_rng(8)
    m, dsub, dim = 8, 4, 32
    books = rng.standard_normal((m, 256, dsub)).astype(np.float32)
    rows = rng.standard_normal((200, dim)).astype(np.float32)
    coarse = rng.standard_normal((1, dim)).astype(np.float32)
    _, c1 = oracle.pq_encode_rows(rows, coarse, books, L2)
    _, c2 = oracle.pq_encode_rows(rows - coarse, np.zeros_like(coarse), books, L2)
    assert np.array_equal(c1, c2)
    # brute force in float64: the chosen code is the nearest sub-centroid
    res = (rows - coarse).astype(np.float64).reshape(200, m, 1, dsub)
    dd = ((res - books.astype(np.float64)[None]) ** 2).sum(3)
    best = dd.min(2)
    chosen = np.take_along_axis(dd, c1.astype(np.int64)[:, :, None], 2)[:, :, 0]
    assert np.all(chosen <= best + 1e-5)


def test_pq_lut_sum_equals_reconstruction_distance_l2():
    rng = np.random.default_rng(9)
    m, dsub = 6, 2
    books = rng.standard_normal((m, 256, dsub)).astype(np.float32)
    q = rng.standard_normal(m * dsub).astype(np.float32)
    lut = oracle.pq_lut(q, books, L2)
    ipl = oracle.pq_lut(q, books, IP)
    code = rng.integers(0, 256, m)
    recon = np.concatenate([books[s, code[s]] for s in range(m)]).astype(np.float64)
    assert abs(sum(lut[s, code[s]] for s in range(m)) - ((q - recon) ** 2).sum()) < 1e-4
    assert abs(sum(ipl[s, code[s]] for s in range(m)) + q.astype(np.float64) @ recon) < 1e-4


def test_ivfpq_probe_newest_first_ties():
    coarse = np.array([[1, 0], [0, 1], [1, 0], [5, 5]], np.float32)
    q = np.array([2, 0], np.float32)
    probes, dist = oracle.ivfpq_probe(coarse, q, 3, L2)
    # centroids 0 and 2 tie; the later index ranks first (BoundedSelection.swift:199-213)
    assert probes.tolist() == [2, 0, 1]


def test_ivfpq_search_is_the_sorted_list_over_probed_adc_scores():
    """_IVFPQIndex.search (IVFPQIndex.swift:177-226) composed from its
    parts, computed here independently: probes in BoundedSortedList order,
    per probe the residual LUT, each row's score the Float sum of its m LUT
    entries in code order, all candidates inserted in arrival order into
    BoundedSortedList(k).  Duplicate rows make ties at every k."""
    rng = np.random.default_rng(51)
    n, dim, m, nlist = 700, 8, 4, 6
    rows = rng.standard_normal((n, dim)).astype(np.float32)
    rows[100:160] = rows[7]
    coarse = rows[[0, 50, 200, 300, 400, 500]].copy()
    books = rng.standard_normal((m, 256, dim // m)).astype(np.float32)
    norms = oracle.row_norms(rows)
    for metric in (L2, IP, COS):
        assign, codes = oracle.pq_encode_rows(rows, coarse, books, metric)
        off, ids = oracle.ivf_lists(assign, nlist)
        for qi in range(4):
            q = rows[7] if qi == 0 else rng.standard_normal(dim).astype(np.float32)
            for k, nprobe in ((5, 2), (30, 3), (64, 6)):
                got_s, got_i = oracle.ivfpq_search(coarse, books, codes, off, ids, metric, q, k,
                                                   nprobe)
                probes, _ = oracle.ivfpq_probe(coarse, q, nprobe, metric)
                cs, ci = [], []
                for p in probes:
                    lut = oracle.pq_lut((q - coarse[p]).astype(np.float32), books, metric)
                    members = ids[off[p]:off[p + 1]]
                    sc = np.zeros(len(members), np.float32)
                    for sub in range(m):
                        sc = (sc + lut[sub, codes[members, sub]]).astype(np.float32)
                    cs.append(sc)
                    ci.append(members)
                cs, ci = np.concatenate(cs), np.concatenate(ci)
                want_s, want_i = oracle.sorted_list_run(cs, ci, k)
                assert got_i.tolist() == want_i.tolist() and np.array_equal(got_s, want_s)
                # No candidate left out scores below the kept ones; equal
                # scores come newest first.
                assert np.all(cs[~np.isin(ci, want_i)] >= want_s[-1])
                pos = {int(i): j for j, i in enumerate(ci)}
                for a in range(len(want_i) - 1):
                    if want_s[a] == want_s[a + 1]:
                        assert pos[int(want_i[a])] > pos[int(want_i[a + 1])]
                # The exact rerank: the kept ids' host distances, (distance, id) order.
                rk = min(5, k)
                rs, ri = oracle.ivfpq_search(coarse, books, codes, off, ids, metric, q, k, nprobe,
                                             rows=rows, rerank_k=rk)
                exact = oracle.distances_for_ids(rows, norms, q, want_i, metric)
                order = np.lexsort((want_i, exact))[:rk]
                assert ri.tolist() == want_i[order].tolist() and np.array_equal(rs, exact[order])


@pytest.mark.parametrize("metric", [COS, L2, IP])
def test_int8_fixed_budget_over_every_row_is_the_exact_result(metric):
    """Mode 1 with budget = n selects every row, so the rescored top-k is
    the exact fp32 scan's (BoundedExactScan.swift:96-122, 320-369)."""
    n, dim = 16384 + 256, 48
    corpus = workloads.lcg_vectors(1, n, dim, seed=31)
    planes = oracle.int8_build(corpus)
    norms = oracle.row_norms(corpus)
    for sd in range(3):
        q = workloads.lcg_vectors(1, 1, dim, seed=310 + sd)[0]
        d, ids, _ = oracle.int8_search(corpus, norms, planes, q, 10, metric, cores=8, mode=1,
                                       budget=n)
        fd, fi = oracle.flat_search(corpus, norms, q, 10, metric, cores=8)
        assert np.array_equal(d, fd) and ids.tolist() == fi.tolist()


def test_host_batch_route_takes_the_int8_scan_from_16384_rows():
    # HostBatchWork.run (FlatGPUSearch.swift:1024-1036): boundedExactSearch
    # for n >= 16384, the fp32 host scan below; both are exact, so the
    # distances equal the fp32 scan's either way.
    for n, want_route in ((16384, 1), (16383, 0)):
        corpus = workloads.lcg_vectors(1, n, 32, seed=77)
        planes = oracle.int8_build(corpus)
        norms = oracle.row_norms(corpus)
        q = workloads.lcg_vectors(1, 6, 32, seed=78)
        d, ids, counts, route = oracle.host_batch_search(corpus, norms, planes, q, 10, COS, cores=8,
                                                         threads=4)
        assert np.all(route == want_route)
        fd, fi, fc = oracle.flat_search_batch(corpus, norms, q, 10, COS, cores=8, threads=4)
        assert np.array_equal(counts, fc) and np.array_equal(d, fd)
        for i in range(q.shape[0]):
            assert set(ids[i].tolist()) == set(fi[i].tolist())
