"""Synthetic workload shapes for the bench (host-side structure generation only;
dense values are generated on the device by gn_fill_uniform_f32 / gn_fill_normal_f32)."""
import numpy as np


def csr_uniform(M, K, mean_row, seed):
    """CSR with row lengths ~ Poisson(mean_row), uniform distinct columns sorted per
    row, values U[-1,1) (float32). Vectorised: draws (row, col) keys, removes the
    rare duplicate keys (a fraction ~ mean_row/K of entries) and sorts."""
    rng = np.random.default_rng(seed)
    lens = rng.poisson(mean_row, size=M).astype(np.int64)
    rows = np.repeat(np.arange(M, dtype=np.int64), lens)
    cols = rng.integers(0, K, size=rows.size, dtype=np.int64)
    keys = np.unique(rows * K + cols)  # sorted by (row, col), duplicates dropped
    rows = keys // K
    col = (keys % K).astype(np.int32)
    rowptr = np.zeros(M + 1, dtype=np.int64)
    np.cumsum(np.bincount(rows, minlength=M), out=rowptr[1:])
    val = rng.uniform(-1.0, 1.0, size=col.size).astype(np.float32)
    return rowptr.astype(np.int32), col, val


def host_normal(shape, seed, mean=0.0, std=1.0):
    """float32 N(mean, std^2) host array (numpy's generator; for inputs that start on the host)."""
    return np.random.default_rng(seed).normal(mean, std, size=shape).astype(np.float32)


def host_uniform(shape, seed, lo=-1.0, hi=1.0):
    """float32 U[lo, hi) host array."""
    return np.random.default_rng(seed).uniform(lo, hi, size=shape).astype(np.float32)
