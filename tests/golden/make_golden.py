"""Writes the golden vectors under tests/golden/.

dots_golden.npz: inputs and outputs of the reference's own C kernels
(Sources/MetalANNSC/dots.c, built by `make -C oracle ref` into
oracle/_ref/libdots_ref.so): mans_f32_dot_rows, mans_i8_dot_rows_f32 and
mans_f32_dot_rows_gather on seeded inputs (LCG of FlatSearchTests.swift:15-22)
at dims 1, 3, 16, 66, 128, 333, 384.  Run from the repository root:

    make -C oracle ref && python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from meltan_amd import workloads  # noqa: E402
from oracle import oracle  # noqa: E402

DIMS = [1, 3, 16, 66, 128, 333, 384]
ROWS = 64


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libdots_ref.so missing: run `make -C oracle ref`")
    out = {}
    for dim in DIMS:
        corpus = workloads.lcg_vectors(0, ROWS, dim, seed=1000 + dim)
        q = workloads.lcg_vectors(0, 1, dim, seed=2000 + dim)[0]
        f = np.empty(ROWS, np.float32)
        ref.mans_f32_dot_rows(corpus.ctypes.data, q.ctypes.data, ROWS, dim, f.ctypes.data)
        idx = np.array([(7 * i + 3) % ROWS for i in range(ROWS // 2)], dtype=np.uint32)
        g = np.empty(idx.shape[0], np.float32)
        ref.mans_f32_dot_rows_gather(corpus.ctypes.data, q.ctypes.data, idx.ctypes.data,
                                     idx.shape[0], dim, g.ctypes.data)
        codes = np.clip(np.rint(corpus * 127), -127, 127).astype(np.int8)
        qcodes = np.clip(np.rint(q * 127), -127, 127).astype(np.int8)
        i8 = np.empty(ROWS, np.float32)
        ref.mans_i8_dot_rows_f32(codes.ctypes.data, qcodes.ctypes.data, ROWS, dim, i8.ctypes.data)
        out[f"corpus_{dim}"] = corpus
        out[f"query_{dim}"] = q
        out[f"f32_{dim}"] = f
        out[f"idx_{dim}"] = idx
        out[f"gather_{dim}"] = g
        out[f"codes_{dim}"] = codes
        out[f"qcodes_{dim}"] = qcodes
        out[f"i8_{dim}"] = i8
    np.savez_compressed(Path(__file__).with_name("dots_golden.npz"), **out)
    print("wrote dots_golden.npz", sorted(out)[:4], "...")


if __name__ == "__main__":
    main()
