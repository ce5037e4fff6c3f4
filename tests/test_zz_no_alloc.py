"""mans_flat_search_device_noalloc against mans_flat_search_device.

The no-allocation entry point takes every workspace from the library's
fixed device array and must give the same results, bit for bit, as the
entry point that allocates -- here on two calls in a row (the second with a
smaller input, so the array holds the first call's leftovers), on the
streaming scan's proof loop (k up to the 256 cap), on an odd dimension (the
exact-key path), on an empty corpus, and on a null stream.
"""
import numpy as np
import pytest

import meltan_amd as M
from meltan_amd import workloads
from meltan_amd.hip import DeviceArray, hip
from oracle import oracle
from test_flat_gpu import COS, IP, L2, check_flat

pytestmark = pytest.mark.gpu


def _both(corpus, q, k, metric):
    nq = q.shape[0]
    dq = DeviceArray.from_numpy(q)
    outs = []
    for fn in (corpus.flat_search_device, corpus.flat_search_device_noalloc):
        dd = DeviceArray((nq, k), np.float32)
        di = DeviceArray((nq, k), np.uint32)
        fn(dq.ptr, nq, k, metric, dd.ptr, di.ptr, None)
        outs.append((dd.numpy(), di.numpy()))
    (ad, ai), (bd, bi) = outs
    return ad, ai, bd, bi


def test_noalloc_matches_the_allocating_entry_point(gpu_ctx):
    print("noalloc: 200k x 384, two calls", flush=True)
    db = workloads.gauss_rows(951, 200_000, 384, True)
    norms = oracle.row_norms(db)
    c = gpu_ctx.upload(db)
    q1 = workloads.gauss_rows(952, 300, 384, True)
    q2 = workloads.gauss_rows(953, 7, 384, True)
    for q, k, metric in ((q1, 10, COS), (q2, 5, L2)):
        ad, ai, bd, bi = _both(c, q, k, metric)
        assert np.array_equal(ad, bd) and np.array_equal(ai, bi), (q.shape, k)
        check_flat(db, norms, q, k, metric, bd, bi, f"noalloc nq{q.shape[0]}")
    # k at and above the cap, one query (the largest per-query workspace).
    ad, ai, bd, bi = _both(c, q2[:1], 300, IP)
    assert np.array_equal(ad, bd) and np.array_equal(ai, bi)
    c.release()


def test_noalloc_exact_path_small_and_empty(gpu_ctx):
    rows = workloads.lcg_vectors(0, 5000, 66, seed=961)  # dim % 4 != 0: exact keys
    c = gpu_ctx.upload(rows)
    q = workloads.lcg_vectors(0, 9, 66, seed=962)
    for metric in (COS, L2, IP):
        ad, ai, bd, bi = _both(c, q, 20, metric)
        assert np.array_equal(ad, bd) and np.array_equal(ai, bi)
    c.release()
    empty = gpu_ctx.upload(np.zeros((0, 16), np.float32))
    ad, ai, bd, bi = _both(empty, np.ones((3, 16), np.float32), 4, COS)
    assert np.all(bi == M.EMPTY_ID) and np.all(bd == np.finfo(np.float32).max)
    assert np.array_equal(ad, bd) and np.array_equal(ai, bi)
    empty.release()


def test_noalloc_argument_errors(gpu_ctx):
    rows = workloads.lcg_vectors(0, 1000, 16, seed=963)
    c = gpu_ctx.upload(rows)
    dq = DeviceArray((2, 16), np.float32)
    dd = DeviceArray((2, 4), np.float32)
    di = DeviceArray((2, 4), np.uint32)
    with pytest.raises(M.ANNSError) as ei:
        c.flat_search_device_noalloc(dq.ptr, 2, 1 << 31, COS, dd.ptr, di.ptr)
    assert ei.value.code == M.SEARCH_FAILED
    with pytest.raises(M.ANNSError) as ei:
        c.flat_search_device_noalloc(dq.ptr, 1 << 32, 4, COS, dd.ptr, di.ptr)
    assert ei.value.code == M.SEARCH_FAILED
    c.release()
