"""The C ABI library loads and exports every function include/mans_hip.h
declares; without a GPU, creating a context reports deviceNotSupported (no
CPU fallback exists)."""
import ctypes as C
import re
from pathlib import Path

import pytest

import meltan_amd as M

HEADER = Path(__file__).resolve().parents[1] / "include" / "mans_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(mans_[a-z0-9_]+)\s*\(", text, flags=re.M)


def test_header_and_binding_agree():
    decl = declared_functions()
    assert len(decl) >= 28
    assert decl == M.EXPORTS


def test_library_exports_every_declared_symbol():
    lib = M.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name


def _gpu_present() -> bool:
    import subprocess
    try:
        out = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=30).stdout
    except Exception:
        return False
    return "gfx950" in out


def test_context_without_gpu_fails_loudly():
    if _gpu_present():
        pytest.skip("a GPU is present")
    with pytest.raises(M.ANNSError) as err:
        M.Context(0)
    assert err.value.code == M.DEVICE_NOT_SUPPORTED
    assert not err.value.is_tier_degradeable


def test_error_codes_match_anns_error_degrade_set():
    # Errors.swift:21-31: pipeline/resource/execution/search failures degrade.
    assert M.DEGRADEABLE == {M.PIPELINE_UNAVAILABLE, M.RESOURCE_EXHAUSTED, M.EXECUTION_FAILED,
                             M.SEARCH_FAILED}
    assert M.DEVICE_NOT_SUPPORTED not in M.DEGRADEABLE
    assert M.DIMENSION_MISMATCH not in M.DEGRADEABLE
