"""Randomised parity sweep of the CSR kernels on the device API: 120 structures with fixed
seeds, drawn over row counts (1 .. 20000), column counts (1 .. 70000, past the packed
layout's 65536), mean row lengths (0.3 .. 300, empty rows included), sorted or unsorted
columns with duplicates, and now and then one row of 5000-20000 entries.

* gn_spmm_csr (N of 1 .. 256) is compared bit for bit with the oracle's restatement of the
  reference loop with fmaf (orc_spmm_csr_f32, one fma per entry in CSR order).
* The grouped-layout SpMV of a plan (gn_spmv_plan_*) is compared bit for bit with the
  oracle's SpMV loop when every row has at most 4096 entries; with a longer row the plan
  runs the flat kernel, which sums rows in another order: relFrob <= 1e-5 against float64.
* The flat SpMV (gn_spmv_csr) is compared with float64 within relFrob 1e-5."""
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _structure(rng):
    M = int(rng.choice([1, 7, 100, 1000, 5000, 20000]))
    K = int(rng.choice([1, 5, 300, 4096, 65536, 70000]))
    mean = float(rng.choice([0.3, 2.0, 10.0, 65.0, 300.0]))
    lens = rng.poisson(mean, size=M).astype(np.int64)
    if M > 1 and rng.random() < 0.2:
        lens[int(rng.integers(M))] = int(rng.integers(5000, 20001))
    while lens.sum() > 1_500_000:  # keep the CPU oracle quick
        lens //= 2
    rowptr = np.zeros(M + 1, dtype=np.int64)
    np.cumsum(lens, out=rowptr[1:])
    nnz = int(rowptr[-1])
    col = rng.integers(0, K, size=nnz).astype(np.int32)
    if rng.random() < 0.7:  # sorted within each row (duplicates kept)
        rows = np.repeat(np.arange(M), lens)
        col = col[np.lexsort((col, rows))]
    val = rng.uniform(-1.0, 1.0, size=nnz).astype(np.float32)
    return M, K, rowptr.astype(np.int32), col, val, int(lens.max()) if M else 0


def _rel(got, ref):
    den = np.linalg.norm(ref)
    return np.linalg.norm(got - ref) / den if den > 0 else np.linalg.norm(got)


@pytest.mark.parametrize("seed", [201, 202, 203])
def test_csr_random_sweep(dev, seed):
    import torch

    rng = np.random.default_rng(seed)
    for case in range(40):
        M, K, rp, col, val, maxrow = _structure(rng)
        nnz = val.size
        N = int(rng.choice([1, 2, 3, 7, 16, 64, 256]))
        while nnz * N > 60_000_000 and N > 1:
            N //= 2
        desc = f"seed {seed} case {case}: M={M} K={K} nnz={nnz} longest row {maxrow} N={N}"
        print(desc, flush=True)
        sys.stdout.flush()
        d_rp, d_col = torch.from_numpy(rp).to(dev), torch.from_numpy(col).to(dev)
        d_val = torch.from_numpy(val).to(dev)
        D = rng.standard_normal((K, N)).astype(np.float32)
        x = rng.standard_normal(K).astype(np.float32)
        d_D, d_x = torch.from_numpy(D).to(dev), torch.from_numpy(x).to(dev)
        C = torch.full((M, N), float("nan"), device=dev)
        y = torch.full((M,), float("nan"), device=dev)
        yp = torch.full((M,), float("nan"), device=dev)
        G.spmm_csr(M, N, K, nnz, d_rp, d_col, d_val, d_D, C)
        G.spmv_csr(M, K, nnz, d_rp, d_col, d_val, d_x, y)
        plan = G.SpmvPlan(M, K, nnz, d_rp, d_col) if nnz > 0 else None
        if plan is not None:
            plan.run(d_val, d_x, yp)
        torch.cuda.synchronize()
        if plan is not None:
            plan.release()
        np.testing.assert_array_equal(C.cpu().numpy(), O.spmm_f32_par(rp, col, val, D, O.threads(), use_fma=True),
                                      err_msg=desc)
        ref64 = O.spmv_f64(rp, col, val, x)
        assert _rel(y.cpu().numpy().astype(np.float64), ref64) <= 1e-5, desc
        if plan is not None:
            got = yp.cpu().numpy()
            if maxrow <= 4096:
                np.testing.assert_array_equal(got, O.spmv_f32(rp, col, val, x, use_fma=True), err_msg=desc)
            else:
                assert _rel(got.astype(np.float64), ref64) <= 1e-5, desc
