"""The loadReadOnly(.mmap) path onto the device (mans_corpus_upload_mann).

A corpus loaded from a MANN v3 file's vector section must equal, bit for
bit, the corpus uploaded from the same rows in memory: same exact flat top-k
(distances and ids), same int8 planes.  Files written with 4 KiB and 16 KiB
pages (Apple silicon's) load with the matching page size.  Only fp32
storage reaches the device scan (FlatGPUSearch.isEligible); f16 and binary
files are tier-degradeable.
"""
import numpy as np
import pytest

import meltan_amd as M
from meltan_amd import workloads
from mann_writer import write_mann_v3
from oracle import oracle
from test_flat_gpu import COS, IP, L2, check_flat

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("page", [4096, 16384])
def test_mann_upload_equals_memory_upload(gpu_ctx, tmp_path, page):
    n, dim = 20000, 96
    rows = workloads.lcg_vectors(1, n, dim, seed=page)
    path = tmp_path / "index.mann"
    write_mann_v3(path, rows, degree=8, metric=1, page=page, entry_point=3)
    fc, metric = gpu_ctx.upload_mann(path, page)
    assert metric == 1 and (fc.n, fc.dim) == (n, dim)
    mc = gpu_ctx.upload(rows)
    q = np.ascontiguousarray(np.concatenate([rows[:5], workloads.lcg_vectors(1, 40, dim, seed=9)]))
    for metric_code in (COS, L2):
        fd, fi = fc.flat_search(q, 10, metric_code)
        md, mi = mc.flat_search(q, 10, metric_code)
        assert np.array_equal(fd, md) and np.array_equal(fi, mi)
    # Stored rows find themselves at distance 0.
    d0, i0 = fc.flat_search(rows[:5], 1, L2)
    assert np.array_equal(i0[:, 0], np.arange(5)) and np.all(d0[:, 0] == 0)
    for a, b in zip(fc.int8_codes(), mc.int8_codes()):
        assert np.array_equal(a, b)
    fc.release()
    mc.release()


@pytest.mark.parametrize("metric", [COS, L2, IP])
def test_mann_loaded_corpus_matches_the_oracle(gpu_ctx, tmp_path, metric):
    # The corpus read from the file's vector section searched against the
    # oracle over the rows that were written: exact top-k, bit for bit.
    n, dim = 30000, 384
    rows = workloads.gauss_rows(811, n, dim, True)
    path = tmp_path / "c.mann"
    write_mann_v3(path, rows, degree=4, metric=metric, page=16384)
    fc, got_metric = gpu_ctx.upload_mann(path, 16384)
    assert got_metric == metric
    q = workloads.gauss_rows(812, 24, dim, True)
    norms = oracle.row_norms(rows)
    for k in (1, 10, 100):
        gd, gi = fc.flat_search(q, k, metric)
        check_flat(rows, norms, q, k, metric, gd, gi, f"mann k{k}")
    fc.release()


def test_mann_upload_larger_than_one_staging_chunk(gpu_ctx, tmp_path):
    # 70 MB of vectors: three 32 MiB staging chunks, both buffers reused.
    n, dim = 45000, 384
    rows = workloads.gauss_rows(11, n, dim, True)
    path = tmp_path / "big.mann"
    write_mann_v3(path, rows, degree=2, metric=0)
    fc, _ = gpu_ctx.upload_mann(path)
    idx = np.array([0, 1, n // 2, n - 1])
    d, i = fc.flat_search(rows[idx], 1, L2)
    assert np.array_equal(i[:, 0], idx) and np.all(d[:, 0] == 0)
    fc.release()


def test_mann_non_fp32_storage_is_tier_degradeable(gpu_ctx, tmp_path):
    path = tmp_path / "half.mann"
    write_mann_v3(path, np.ones((100, 16), np.float16))
    with pytest.raises(M.ANNSError) as ei:
        gpu_ctx.upload_mann(path)
    assert ei.value.code == M.PIPELINE_UNAVAILABLE and ei.value.is_tier_degradeable
    path = tmp_path / "bits.mann"
    write_mann_v3(path, np.ones((100, 4), np.uint8))
    with pytest.raises(M.ANNSError):
        gpu_ctx.upload_mann(path)
    path = tmp_path / "bad.mann"
    path.write_bytes(b"MANN" + b"\0" * 10)
    with pytest.raises(M.ANNSError) as ei:
        gpu_ctx.upload_mann(path)
    assert ei.value.code == M.CORRUPT_FILE
