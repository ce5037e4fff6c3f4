"""The benchmark workloads are reproducible: their SHA-256 digests match the
committed ones (tests/golden/workloads_sha256.json, written by
tests/golden/make_workload_sha256.py), and the bytes do not depend on the
thread split, because every row has its own random stream."""
import json
from pathlib import Path

import numpy as np

from meltan_amd import workloads as W

GOLD = json.loads((Path(__file__).parent / "golden" / "workloads_sha256.json").read_text())


def test_flat_10k_digest():
    db, q = W.flat_10k()
    assert W.sha256(db) == GOLD["flat_10k_384"]["rows"]
    assert W.sha256(q) == GOLD["flat_10k_384"]["queries"]


def test_flat_100k_digest():
    db, q = W.flat_100k()
    assert W.sha256(db) == GOLD["flat_100k_384"]["rows"]
    assert W.sha256(q) == GOLD["flat_100k_384"]["queries"]


def test_mixture_query_digests():
    ctr = W.centers(3001, 1000, 384)
    q, _ = W.mixture_rows(3002, ctr, 0.3, 1024, True)
    assert W.sha256(q) == GOLD["mixture_1m_384"]["queries"]
    ctr = W.centers(4001, 4096, 128)
    q, _ = W.mixture_rows(4002, ctr, 0.25, 1024, False)
    assert W.sha256(q) == GOLD["mixture_1m_128"]["queries"]
    ctr = W.centers(5001, 8192, 96)
    assert W.sha256(ctr) == GOLD["mixture_10m_96"]["centres"]
    q, _ = W.mixture_rows(5002, ctr, 0.25, 1024, False)
    assert W.sha256(q) == GOLD["mixture_10m_96"]["queries"]
    tr, _ = W.mixture_rows(5003, ctr, 0.25, 262_144, False)
    assert W.sha256(tr) == GOLD["mixture_10m_96_train"]["rows"]


def test_bytes_do_not_depend_on_the_split():
    a = W.gauss_rows(1001, 3000, 384, True, threads=1)
    b = W.gauss_rows(1001, 3000, 384, True, threads=7)
    assert np.array_equal(a, b)
    ctr = W.centers(3001, 1000, 384)
    whole, wid = W.mixture_rows(3001, ctr, 0.3, 1000, True, threads=3)
    tail, tid = W.mixture_rows(3001, ctr, 0.3, 400, True, row0=600, threads=1)
    assert np.array_equal(whole[600:], tail) and np.array_equal(wid[600:], tid)
