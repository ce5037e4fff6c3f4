"""Degradeable failures (Errors.swift:21-31) through the C ABI.

MANS_HIP_FAIL=alloc makes every workspace allocation of a new context fail
and MANS_HIP_FAIL=launch every search's launch: searches through such a
context return gpuResourceExhausted (-4) / gpuExecutionFailed (-5), both
tier-degradeable, for the flat, int8, IVF-flat and IVF-PQ scans, and a
normal context keeps returning oracle-exact results afterwards.
"""
import ctypes as C

import numpy as np
import pytest

import meltan_amd as M
from meltan_amd import workloads
from oracle import oracle
from test_flat_gpu import COS, IP, L2, check_flat

pytestmark = pytest.mark.gpu


def _call(fn, *args):
    rc = fn(*args)
    return rc, M.lib().mans_last_error().decode(errors="replace")


def test_injected_alloc_and_launch_failures(gpu_ctx, monkeypatch):
    n, dim = 16384 + 512, 64
    rows = workloads.lcg_vectors(1, n, dim, seed=901)
    q = workloads.lcg_vectors(1, 8, dim, seed=902)
    norms = oracle.row_norms(rows)
    c = gpu_ctx.upload(rows)
    c.int8_search(q, 10, COS)  # builds the int8 planes through the normal context
    ivf = c.ivf_flat_build(rows[:: n // 32][:32].copy(), L2)
    books = np.ascontiguousarray(rows[:256].reshape(256, 16, 4).transpose(1, 0, 2))
    pq = c.ivfpq_build(rows[:: n // 16][:16].copy(), books, IP)
    L = M.lib()
    out_d = np.empty((8, 10), np.float32)
    out_i = np.empty((8, 10), np.uint32)
    p = lambda a: a.ctypes.data
    for mode, code in (("alloc", M.RESOURCE_EXHAUSTED), ("launch", M.EXECUTION_FAILED)):
        monkeypatch.setenv("MANS_HIP_FAIL", mode)
        bad = M.Context(0)
        monkeypatch.delenv("MANS_HIP_FAIL")
        h = bad.handle
        calls = {
            "flat": (L.mans_flat_search, h, c.handle, p(q), 8, 10, COS, p(out_d), p(out_i)),
            "int8": (L.mans_int8_search, h, c.handle, p(q), 8, 10, COS, 0, 0, p(out_d), p(out_i),
                     None),
            "ivf": (L.mans_ivf_flat_search, h, ivf.handle, p(q), 8, 10, 4, p(out_d), p(out_i), None),
            "ivfpq": (L.mans_ivfpq_search, h, pq.handle, p(q), 8, 10, 4, 0, p(out_d), p(out_i)),
        }
        for name, (fn, *args) in calls.items():
            rc, msg = _call(fn, *args)
            assert rc == code, f"{mode} {name}: {rc} {msg}"
            assert rc in M.DEGRADEABLE
        if mode == "alloc":
            with pytest.raises(M.ANNSError) as ei:
                bad.upload(rows[:100])
            assert ei.value.code == M.RESOURCE_EXHAUSTED
        bad.close()
    # The normal context is untouched.
    for metric in (COS, L2, IP):
        gd, gi = c.flat_search(q, 10, metric)
        check_flat(rows, norms, q, 10, metric, gd, gi, f"after faults m{metric}")
    pq.release()
    ivf.release()
    c.release()


def test_search_arguments_are_checked_before_any_work(gpu_ctx):
    rows = workloads.lcg_vectors(1, 1000, 16, seed=903)
    c = gpu_ctx.upload(rows)
    L = M.lib()
    q = np.zeros((1, 16), np.float32)
    d = np.empty(4, np.float32)
    i = np.empty(4, np.uint32)
    # k beyond the 32-bit output stride
    rc, msg = _call(L.mans_flat_search, gpu_ctx.handle, c.handle, q.ctypes.data, 1, 1 << 31, COS,
                    d.ctypes.data, i.ctypes.data)
    assert rc == M.SEARCH_FAILED and "2^31" in msg
    rc, msg = _call(L.mans_flat_search, gpu_ctx.handle, c.handle, q.ctypes.data, 1, 4, 3,
                    d.ctypes.data, i.ctypes.data)
    assert rc == M.SEARCH_FAILED  # hamming
    c.release()
