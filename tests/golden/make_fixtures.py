"""Writes the committed golden fixtures under tests/golden/.

The expected outputs come from numpy / scipy float64 (independent of oracle/ and of
the HIP library), so they pin both. The reference ships no golden vectors for this
path (its tests never call MatMul/Transpose/SparseMatMul/SparseMatVec), and it
cannot be built or run here (Go + Objective-C + Metal), so these are the build's own.

Run:  python tests/golden/make_fixtures.py
"""
import os

import numpy as np
import scipy.sparse as sp

HERE = os.path.dirname(os.path.abspath(__file__))


def gemm_small():
    rng = np.random.default_rng(42)
    out = {}
    shapes = [(1, 1, 1), (8, 8, 8), (3, 5, 7), (17, 33, 9), (64, 48, 40), (33, 65, 130)]
    for (M, N, K) in shapes:
        A = rng.uniform(-1, 1, size=(M, K)).astype(np.float32)
        B = rng.uniform(-1, 1, size=(K, N)).astype(np.float32)
        C = A.astype(np.float64) @ B.astype(np.float64)
        key = f"{M}x{N}x{K}"
        out[f"A_{key}"] = A
        out[f"B_{key}"] = B
        out[f"C64_{key}"] = C
    np.savez_compressed(os.path.join(HERE, "gemm_small.npz"), **out)


def gemm_256():
    # Config C1: M=N=K=256, U[-1,1], fixed seed; float64 reference product.
    rng = np.random.default_rng(20240601)
    A = rng.uniform(-1, 1, size=(256, 256)).astype(np.float32)
    B = rng.uniform(-1, 1, size=(256, 256)).astype(np.float32)
    C = A.astype(np.float64) @ B.astype(np.float64)
    np.savez_compressed(os.path.join(HERE, "gemm_256.npz"), A=A, B=B, C64=C)


def csr_64():
    """64x64 COO with duplicates, explicit zeros and empty rows."""
    rng = np.random.default_rng(7)
    rows, cols = 64, 64
    ri, ci, v = [], [], []
    empty = {0, 5, 6, 31, 63}
    for r in range(rows):
        if r in empty:
            continue
        n = int(rng.integers(1, 9))
        for _ in range(n):
            ri.append(r)
            ci.append(int(rng.integers(0, cols)))
            v.append(float(rng.uniform(-1, 1)))
    # explicit duplicates and explicit zeros
    for (r, c, val) in [(3, 7, 0.5), (3, 7, -0.25), (3, 7, 2.0), (10, 0, 0.0), (10, 63, 0.0), (62, 62, 1.0), (62, 62, 1.0)]:
        ri.append(r)
        ci.append(c)
        v.append(val)
    perm = rng.permutation(len(v))  # COO input order is arbitrary
    ri = np.array(ri, dtype=np.int32)[perm]
    ci = np.array(ci, dtype=np.int32)[perm]
    v = np.array(v, dtype=np.float32)[perm]
    # expected CSR: stable sort by (row, col)
    order = np.lexsort((ci, ri))
    rowptr = np.zeros(rows + 1, dtype=np.int32)
    np.cumsum(np.bincount(ri, minlength=rows), out=rowptr[1:])
    D = rng.standard_normal((cols, 8)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    S = sp.coo_matrix((v.astype(np.float64), (ri, ci)), shape=(rows, cols)).tocsr()  # sums duplicates
    C64 = S @ D.astype(np.float64)
    y64 = S @ x.astype(np.float64)
    np.savez_compressed(os.path.join(HERE, "csr_64.npz"), ri=ri, ci=ci, v=v, rowptr=rowptr,
                        idx=ci[order], data=v[order], D=D, x=x, C64=C64, y64=y64)


if __name__ == "__main__":
    gemm_small()
    gemm_256()
    csr_64()
    print("fixtures written to", HERE)
