"""Random call sequences through the Part-1 sparse entries (perform_sparse_matvec,
perform_sparse_dense_matmul) on one values buffer, as a Go caller makes them: the host
row-pointer and column arrays are passed on every call, and the library keeps their device
copy (and, for SpMV, the grouped layout built for the call's column count) with the values
buffer. Between calls the sequence changes row pointers in place, changes columns in place
and announces it with gn_csr_indices_changed, switches the column count (past 65536 too, the
layout's unpacked form), passes a column count the columns do not fit (refused with -3 and
not kept), scales the values on the device, and releases and re-creates the values buffer.
Every result must equal the oracle's fmaf loop on the current arrays bit for bit (the
structure has 2^18+ entries and rows of at most 4096, so SpMV runs the grouped layout)."""
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [301, 302])
def test_part1_sparse_cache_random_sequence(dev, seed):
    rng = np.random.default_rng(seed)
    rows, K = 6000, 9000
    rp, col, val = O.random_csr(rows, K, 50.0, seed=seed)
    assert val.size >= 1 << 18
    kmax = int(col.max()) + 1
    val_cur = val.copy()
    bv = G.Buffer.from_array(val)
    N = 16
    n_checked = 0
    for step in range(30):
        action = rng.choice(["spmv", "spmv", "spmm", "rowptr", "cols", "kswitch", "badk", "scale", "rebuffer"])
        print(f"seed {seed} step {step}: {action}", flush=True)
        sys.stdout.flush()
        if action == "rowptr":  # move one row boundary by one entry, in place
            k = int(rng.integers(1, rows))
            if rp[k] > rp[k - 1] and rng.random() < 0.5:
                rp[k] -= 1
            elif rp[k] < rp[k + 1]:
                rp[k] += 1
            continue
        if action == "cols":  # in place, announced as the reference's caller would re-upload
            sel = rng.integers(0, col.size, size=1000)
            col[sel] = rng.integers(0, K, size=sel.size).astype(np.int32)
            kmax = int(col.max()) + 1
            assert G.load().gn_csr_indices_changed(bv.handle) == 0
            continue
        if action == "scale":  # values changed on the device; the cache holds indices only
            f = float(rng.choice([-0.5, 2.0]))
            G.call("perform_sparse_scalar_multiply", bv.handle, rp.ctypes.data, rp.size, col.ctypes.data, col.size,
                   rows, K, val.size, f, None)
            val_cur = val_cur * np.float32(f)
            continue
        if action == "rebuffer":
            bv.release()
            bv = G.Buffer.from_array(val_cur)
            continue
        kc = K
        if action == "kswitch":
            kc = int(rng.choice([K, K + 1000, 70000]))
        if action == "badk":
            kc = max(1, kmax - 1)  # a column count the columns do not fit
        if action in ("spmv", "kswitch", "badk"):
            x = rng.standard_normal(kc).astype(np.float32)
            bx, by = G.Buffer.from_array(x), G.Buffer(rows * 4)
            rc, msg = G.call_rc("perform_sparse_matvec", bv.handle, rp.ctypes.data, rp.size, col.ctypes.data,
                                col.size, rows, kc, val.size, bx.handle, kc, by.handle, rows, None)
            if action == "badk":
                assert rc == -3 and "column index" in msg, (rc, msg)
            else:
                assert rc == 0, (rc, msg)
                np.testing.assert_array_equal(by.to_array((rows,)), O.spmv_f32(rp, col, val_cur, x, use_fma=True),
                                              err_msg=f"seed {seed} step {step} K={kc}")
                n_checked += 1
            bx.release()
            by.release()
        else:  # spmm
            D = rng.standard_normal((K, N)).astype(np.float32)
            bd, bc = G.Buffer.from_array(D), G.Buffer(rows * N * 4)
            G.call("perform_sparse_dense_matmul", bv.handle, rp.ctypes.data, rp.size, col.ctypes.data, col.size, rows,
                   K, val.size, bd.handle, K, N, bc.handle, rows, N, None)
            np.testing.assert_array_equal(bc.to_array((rows, N)), O.spmm_f32(rp, col, val_cur, D, use_fma=True),
                                          err_msg=f"seed {seed} step {step}")
            n_checked += 1
            bd.release()
            bc.release()
    bv.release()
    assert n_checked >= 5
