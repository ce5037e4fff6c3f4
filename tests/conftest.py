import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden_dots():
    return np.load(GOLDEN / "dots_golden.npz", allow_pickle=False)


@pytest.fixture(scope="session")
def gpu_ctx():
    import meltan_amd as M

    ctx = M.Context(0)  # raises ANNSError(deviceNotSupported) loudly without a gfx950 GPU
    yield ctx
    ctx.close()


def tie_tolerant_equal(ref_dist, ref_ids, got_dist, got_ids, rel=1e-5):
    """ids equal except where the reference distances tie within `rel`
    (relative) at the same rank or across the k boundary."""
    ref_dist = np.asarray(ref_dist, np.float64)
    got_dist = np.asarray(got_dist, np.float64)
    k = len(ref_ids)
    assert len(got_ids) == k
    for i in range(k):
        if ref_ids[i] == got_ids[i]:
            continue
        tol = rel * max(abs(ref_dist[i]), 1e-30)
        if abs(ref_dist[i] - got_dist[i]) > tol:
            return False, f"rank {i}: ids {ref_ids[i]} vs {got_ids[i]}, dist {ref_dist[i]} vs {got_dist[i]}"
    boundary = ref_dist[-1] if k else 0.0
    missing = set(ref_ids.tolist()) - set(got_ids.tolist())
    for m in missing:
        j = list(ref_ids).index(m)
        if abs(ref_dist[j] - boundary) > rel * max(abs(boundary), 1e-30):
            return False, f"id {m} (dist {ref_dist[j]}) missing away from the boundary {boundary}"
    return True, ""
