"""Builds the native pieces in-tree.

- ``meltan_amd/libmans_hip.so``: the HIP kernels and the C ABI of
  ``include/mans_hip.h``, compiled for gfx950 only.
- ``meltan_amd/libmans_datagen.so``: the seeded workload generator.

The oracle (``oracle/``) has its own Makefile; ``__graft_entry__.build``
drives both.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    noisy = [l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if noisy:
        sys.stderr.write("\n".join(noisy) + "\n")


def build_datagen() -> Path:
    out = PKG / "libmans_datagen.so"
    _run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-std=c11",
          "-Wall", "-o", str(out), str(PKG / "datagen.c"), "-lm"])
    return out


def _stale(src: Path, obj: Path) -> bool:
    """True when obj is missing or older than src or any shared header."""
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    deps = [src, *CSRC.glob("*.hpp"), ROOT / "include" / "mans_hip.h"]
    return any(d.stat().st_mtime > t for d in deps)


def build_hip(jobs: int | None = None, incremental: bool = False) -> Path:
    """Compiles every .hip source (only the stale ones when incremental)."""
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objects = [OBJ / (s.stem + ".o") for s in sources]
    todo = [(s, o) for s, o in zip(sources, objects) if not incremental or _stale(s, o)]
    jobs = jobs or min(max(1, len(todo)), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)]) for s, o in todo]
        for f in futs:
            f.result()
    out = PKG / "libmans_hip.so"
    tmp = PKG / "libmans_hip.so.tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp),
          *[str(o) for o in objects]])
    os.replace(tmp, out)
    return out


def build_all(incremental: bool = False) -> None:
    build_datagen()
    build_hip(incremental=incremental)


if __name__ == "__main__":
    build_all(incremental="--incremental" in sys.argv)
    print("built", PKG / "libmans_hip.so", PKG / "libmans_datagen.so")
