"""GPU parity of CSR SpMM / SpMV against the oracle's restatement of the reference
loops (internal/cgo/metal_bridge_sparse.m:117-133, :325-339).

SpMM accumulates in CSR order with one fma per stored entry, so it is compared
bit-for-bit with the fmaf restatement; SpMV uses a parallel reduction and is held
to relFrob <= 1e-5 against float64."""
import os
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _spmm_abi(rp, col, val, D, rows, cols):
    N = D.shape[1]
    bv = G.Buffer.from_array(val) if val.size else None
    bd, bc = G.Buffer.from_array(D), G.Buffer(rows * N * 4)
    col_ptr = col.ctypes.data if col.size else None
    G.call("perform_sparse_dense_matmul", bv.handle if bv else None, rp.ctypes.data, rp.size, col_ptr, col.size, rows,
           cols, val.size, bd.handle, cols, N, bc.handle, rows, N, None)
    return bc.to_array((rows, N))


def _spmv_abi(rp, col, val, x, rows, cols):
    bv = G.Buffer.from_array(val) if val.size else None
    bx, by = G.Buffer.from_array(x), G.Buffer(rows * 4)
    col_ptr = col.ctypes.data if col.size else None
    G.call("perform_sparse_matvec", bv.handle if bv else None, rp.ctypes.data, rp.size, col_ptr, col.size, rows, cols,
           val.size, bx.handle, x.size, by.handle, rows, None)
    return by.to_array((rows,))


def test_spmm_golden_duplicates_zeros_empty_rows(dev):
    z = np.load(os.path.join(GOLD, "csr_64.npz"))
    rp, idx, data, D = z["rowptr"], z["idx"], z["data"], z["D"]
    C = _spmm_abi(rp, idx, data, D, 64, 64)
    np.testing.assert_array_equal(C, O.spmm_f32(rp, idx, data, D, use_fma=True))
    assert O.rel_frob(C, z["C64"]) <= 1e-5
    for r in (0, 5, 6, 31, 63):
        assert np.all(C[r] == 0)


@pytest.mark.parametrize("N", [1, 3, 4, 8, 20, 64, 100, 256, 300, 512])
def test_spmm_widths_bit_exact(dev, N):
    rp, col, val = O.random_csr(700, 900, 9.0, seed=N)
    D = O.normal((900, N), 5, N)
    C = _spmm_abi(rp, col, val, D, 700, 900)
    np.testing.assert_array_equal(C, O.spmm_f32(rp, col, val, D, use_fma=True))


def _shuffle_rows(rp, col, seed):
    rng = np.random.default_rng(seed)
    col = col.copy()
    for r in range(rp.size - 1):
        rng.shuffle(col[rp[r]:rp[r + 1]])
    return col


@pytest.mark.parametrize("N,ldd,ldc,order", [(32, 32, 32, "sorted"), (36, 40, 36, "unsorted"),
                                             (96, 96, 100, "duplicates"), (256, 256, 256, "sorted"),
                                             (260, 272, 264, "unsorted")])
def test_spmm_column_bands_long_rows_bit_exact(dev, N, ldd, ldc, order):
    """Rows long enough for several full 16-entry batches plus a tail, a partial last
    column band (N % 32 != 0), pitches wider than N, unsorted or repeated columns; the
    device-pointer entry. Columns past N in C keep their contents."""
    import torch

    M, K = 1000, 3000
    rp, col, val = O.random_csr(M, K, 45.0, seed=N, distinct=order != "duplicates")
    if order == "unsorted":
        col = _shuffle_rows(rp, col, N)
    assert (rp[1:] - rp[:-1]).max() >= 48
    D = O.normal((K, N), 7, N)
    ref = O.spmm_f32(rp, col, val, D, use_fma=True)
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val)]
    Dd = torch.zeros((K, ldd), dtype=torch.float32, device=dev)
    Dd[:, :N] = torch.from_numpy(D).to(dev)
    Cd = torch.full((M, ldc), float("nan"), dtype=torch.float32, device=dev)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    G.spmm_csr(M, N, K, val.size, d[0], d[1], d[2], Dd, Cd, flags, ldd=ldd, ldc=ldc)
    assert flags.cpu().tolist() == [0, 0]
    C = Cd.cpu().numpy()
    np.testing.assert_array_equal(C[:, :N], ref)
    assert np.isnan(C[:, N:]).all()


def test_spmm_column_bands_skip_bad_columns_in_full_batches(dev):
    """An out-of-range column inside a full 16-entry batch and another in a row's tail
    are skipped (the rest of the row keeps CSR order) and reported in flags[1]."""
    import torch

    M, K, N = 64, 500, 64
    rp, col, val = O.random_csr(M, K, 40.0, seed=9)
    lens = rp[1:] - rp[:-1]
    assert lens[3] >= 16 and lens[7] >= 33
    bad = col.copy()
    drop = [rp[3] + 5, rp[7] + lens[7] - 1]  # batch entry of row 3, last (tail) entry of row 7
    bad[drop[0]], bad[drop[1]] = K + 5, -1
    keep = np.ones(col.size, bool)
    keep[drop] = False
    rp_keep = np.concatenate([[0], np.cumsum([keep[rp[r]:rp[r + 1]].sum() for r in range(M)])]).astype(np.int32)
    D = O.normal((K, N), 8, 1)
    ref = O.spmm_f32(rp_keep, col[keep], val[keep], D, use_fma=True)
    d = [torch.from_numpy(a).to(dev) for a in (rp, bad, val, D)]
    Cd = torch.empty((M, N), dtype=torch.float32, device=dev)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    G.spmm_csr(M, N, K, val.size, d[0], d[1], d[2], d[3], Cd, flags)
    assert flags.cpu().tolist() == [0, 1]
    np.testing.assert_array_equal(Cd.cpu().numpy(), ref)


def _with_row_lengths(rp, col, val, lengths):
    """The CSR with the first rows cut to the given lengths (entries dropped from their ends)."""
    keep = np.ones(col.size, bool)
    for r, n in enumerate(lengths):
        keep[rp[r] + n:rp[r + 1]] = False
    rp2 = np.concatenate([[0], np.cumsum([keep[rp[r]:rp[r + 1]].sum() for r in range(rp.size - 1)])]).astype(np.int32)
    return rp2, col[keep], val[keep]


@pytest.mark.parametrize("N,ldd,ldc,order", [(32, 32, 32, "sorted"), (100, 104, 100, "unsorted"),
                                             (256, 256, 260, "duplicates")])
def test_spmm_two_launch_split_bit_exact(dev, N, ldd, ldc, order):
    """From 65536 stored entries the band path runs in two launches, over the first and the
    second half of each row's entries, with the partial sum passing through C. Rows of 0, 1,
    2 and 3 entries, unsorted or repeated columns, pitches wider than N, a partial last band,
    the last entries of the arrays (inside the final 16-entry batch), and out-of-range
    columns in either half of a row and in the arrays' last entry: bit for bit against the
    fmaf restatement of the reference loop (bad entries skipped), flags[1] raised."""
    import torch

    M, K = 2500, 3000
    rp, col, val = O.random_csr(M, K, 40.0, seed=N + 1, distinct=order != "duplicates")
    rp, col, val = _with_row_lengths(rp, col, val, [0, 1, 2, 3, 0])
    if order == "unsorted":
        col = _shuffle_rows(rp, col, N)
    assert col.size >= 1 << 16
    lens = rp[1:] - rp[:-1]
    long_row = int(np.argmax(lens))
    bad = col.copy()
    drop = [rp[long_row] + 3, rp[long_row] + lens[long_row] * 3 // 4, rp[3] + 2, col.size - 1]
    bad[drop[0]], bad[drop[1]], bad[drop[2]], bad[drop[3]] = K, -7, K + 100, 2 * K
    keep = np.ones(col.size, bool)
    keep[drop] = False
    rp_keep = np.concatenate([[0], np.cumsum([keep[rp[r]:rp[r + 1]].sum() for r in range(M)])]).astype(np.int32)
    D = O.normal((K, N), 9, N)
    ref = O.spmm_f32(rp_keep, col[keep], val[keep], D, use_fma=True)
    d = [torch.from_numpy(a).to(dev) for a in (rp, bad, val)]
    Dd = torch.zeros((K, ldd), dtype=torch.float32, device=dev)
    Dd[:, :N] = torch.from_numpy(D).to(dev)
    Cd = torch.full((M, ldc), float("nan"), dtype=torch.float32, device=dev)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    _say("spmm two-launch split", N, ldd, ldc, order, col.size)
    G.spmm_csr(M, N, K, val.size, d[0], d[1], d[2], Dd, Cd, flags, ldd=ldd, ldc=ldc)
    assert flags.cpu().tolist() == [0, 1]
    C = Cd.cpu().numpy()
    np.testing.assert_array_equal(C[:, :N], ref)
    assert np.isnan(C[:, N:]).all()
    assert np.all(C[[0, 4], :N] == 0)


def test_spmm_column_cut_edges_bit_exact(dev):
    """The two-launch SpMM outside graph capture cuts each row at its first column >= K / 2:
    rows wholly below or above the cut, cuts at and around the 16-entry batch boundary, a row
    whose first column is already past the cut (unsorted), a cut inside the arrays' last
    16 entries, and a decreasing row-pointer pair (that row empty, flags[0]); every row bit for
    bit against the fmaf restatement of the reference loop."""
    import torch

    rng = np.random.default_rng(77)
    M, K, N = 2000, 3001, 64
    cut = K // 2
    lo = lambda n: np.sort(rng.choice(cut, n, replace=False))
    hi = lambda n: np.sort(cut + rng.choice(K - cut, n, replace=False))
    rows = [lo(40), hi(40), np.concatenate([lo(16), hi(20)]), np.concatenate([lo(17), hi(5)]),
            np.concatenate([lo(15), hi(1)]), np.concatenate([hi(3), lo(30)]), np.array([cut]), np.array([cut - 1])]
    while len(rows) < M - 1:
        rows.append(np.sort(rng.choice(K, 40, replace=False)))
    rows.append(np.concatenate([lo(5), hi(5)]))  # ends inside the arrays' last 16 entries
    rp = np.concatenate([[0], np.cumsum([r.size for r in rows])]).astype(np.int32)
    col = np.concatenate(rows).astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    assert col.size >= 1 << 16
    rp[101] = rp[100] - 3  # row 100: s > e, invalid; row 101 starts 3 entries into row 99
    s_e = []
    for r in range(M):
        s, e = int(rp[r]), int(rp[r + 1])
        s_e.append((s, e) if 0 <= s <= e <= col.size else (0, 0))
    rp_eff = np.concatenate([[0], np.cumsum([e - s for s, e in s_e])]).astype(np.int32)
    col_eff = np.concatenate([col[s:e] for s, e in s_e]).astype(np.int32)
    val_eff = np.concatenate([val[s:e] for s, e in s_e]).astype(np.float32)
    D = O.normal((K, N), 4, N)
    ref = O.spmm_f32(rp_eff, col_eff, val_eff, D, use_fma=True)
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val, D)]
    Cd = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    _say("spmm column cut edges", col.size)
    G.spmm_csr(M, N, K, val.size, d[0], d[1], d[2], d[3], Cd, flags)
    assert flags.cpu().tolist() == [1, 0]
    C = Cd.cpu().numpy()
    np.testing.assert_array_equal(C, ref)
    assert np.all(C[100] == 0)


def test_spmm_with_duplicates_unsorted_columns(dev):
    rp, col, val = O.random_csr(300, 50, 20.0, seed=3, distinct=False)  # many duplicate columns
    D = O.normal((50, 256), 6, 1)
    C = _spmm_abi(rp, col, val, D, 300, 50)
    np.testing.assert_array_equal(C, O.spmm_f32(rp, col, val, D, use_fma=True))
    assert O.rel_frob(C, O.spmm_f64(rp, col, val, D)) <= 1e-5


def test_spmm_nnz_zero_gives_zero(dev):
    rp = np.zeros(11, np.int32)
    D = O.normal((7, 16), 1, 1)
    C = _spmm_abi(rp, np.zeros(0, np.int32), np.zeros(0, np.float32), D, 10, 7)
    assert np.all(C == 0)


def test_spmm_malformed_csr_is_an_error(dev):
    rp = np.array([0, 2, 3], np.int32)
    col = np.array([0, 9, 1], np.int32)  # 9 >= cols
    val = np.ones(3, np.float32)
    D = np.ones((4, 8), np.float32)
    bv, bd, bc = G.Buffer.from_array(val), G.Buffer.from_array(D), G.Buffer(2 * 8 * 4)
    rc, msg = G.call_rc("perform_sparse_dense_matmul", bv.handle, rp.ctypes.data, 3, col.ctypes.data, 3, 2, 4, 3,
                        bd.handle, 4, 8, bc.handle, 2, 8, None)
    assert rc == -3 and "column" in msg
    rp_bad = np.array([0, 3, 2], np.int32)  # decreasing
    col_ok = np.array([0, 1, 2], np.int32)
    rc, msg = G.call_rc("perform_sparse_dense_matmul", bv.handle, rp_bad.ctypes.data, 3, col_ok.ctypes.data, 3, 2, 4, 3,
                        bd.handle, 4, 8, bc.handle, 2, 8, None)
    assert rc == -3 and "row pointers" in msg
    # dimension mismatch: A cols != B rows
    rc, _ = G.call_rc("perform_sparse_dense_matmul", bv.handle, rp.ctypes.data, 3, col_ok.ctypes.data, 3, 2, 5, 3,
                      bd.handle, 4, 8, bc.handle, 2, 8, None)
    assert rc == -2


def test_spmm_c5_full_size_device_api(dev):
    """Config C5: 65536x65536 CSR at 0.1% density (~4.3M nnz) x 65536x256."""
    import torch

    M = K = 65536
    N = 256
    rp, col, val = O.random_csr(M, K, 65.536, seed=42)
    nnz = val.size
    _say("C5 nnz", nnz)
    d_rp = torch.from_numpy(rp).to(dev)
    d_col = torch.from_numpy(col).to(dev)
    d_val = torch.from_numpy(val).to(dev)
    Dd = torch.empty((K, N), dtype=torch.float32, device=dev)
    G.fill_normal(Dd, 42, 41)
    Cd = torch.empty((M, N), dtype=torch.float32, device=dev)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    G.spmm_csr(M, N, K, nnz, d_rp, d_col, d_val, Dd, Cd, flags)
    assert flags.cpu().tolist() == [0, 0]
    D = Dd.cpu().numpy()
    C = Cd.cpu().numpy()
    # sampled rows: bit-exact against the CSR-order fmaf loop
    rows = np.random.default_rng(1).choice(M, 512, replace=False)
    sub_rp = np.zeros(rows.size + 1, np.int32)
    sub_rp[1:] = np.cumsum(rp[rows + 1] - rp[rows])
    sub_col = np.concatenate([col[rp[r]:rp[r + 1]] for r in rows])
    sub_val = np.concatenate([val[rp[r]:rp[r + 1]] for r in rows])
    np.testing.assert_array_equal(C[rows], O.spmm_f32(sub_rp, sub_col, sub_val, D, use_fma=True))
    # whole-output property: column sums 1^T C = (1^T S) D, in float64
    colsum_S = np.bincount(col, weights=val.astype(np.float64), minlength=K)
    lhs = C.astype(np.float64).sum(axis=0)
    rhs = colsum_S @ D.astype(np.float64)
    assert np.linalg.norm(lhs - rhs) / np.linalg.norm(rhs) <= 1e-5


def test_spmv_golden_and_random(dev):
    z = np.load(os.path.join(GOLD, "csr_64.npz"))
    y = _spmv_abi(z["rowptr"], z["idx"], z["data"], z["x"], 64, 64)
    assert O.rel_frob(y, z["y64"]) <= 1e-5
    # mean row lengths on both sides of the 32-entry switch to the wave-per-row kernel;
    # 1003 rows leave a partial group of rows in the last wave, 300 spans 5 chunks of 64
    for M, mean in ((1000, 0.5), (1000, 3.0), (1003, 31.0), (1003, 40.0), (1000, 300.0)):
        rp, col, val = O.random_csr(M, 2000, mean, seed=int(mean * 10))
        x = O.normal((2000,), 3, int(mean))
        y = _spmv_abi(rp, col, val, x, M, 2000)
        assert O.rel_frob(y, O.spmv_f64(rp, col, val, x)) <= 1e-5, mean
        assert O.rel_frob(y, O.spmv_f32(rp, col, val, x).astype(np.float64)) <= 1e-5, mean


def test_spmv_dimension_and_csr_errors(dev):
    rp = np.array([0, 1], np.int32)
    col = np.array([5], np.int32)
    val = np.ones(1, np.float32)
    bv, bx, by = G.Buffer.from_array(val), G.Buffer.from_array(np.ones(3, np.float32)), G.Buffer(4)
    rc, _ = G.call_rc("perform_sparse_matvec", bv.handle, rp.ctypes.data, 2, col.ctypes.data, 1, 1, 3, 1, bx.handle, 4,
                      by.handle, 1, None)
    assert rc == -1  # aCols != xSize
    rc, msg = G.call_rc("perform_sparse_matvec", bv.handle, rp.ctypes.data, 2, col.ctypes.data, 1, 1, 3, 1, bx.handle,
                        3, by.handle, 1, None)
    assert rc == -3 and "column" in msg


def test_spmv_c5_full_size(dev):
    import torch

    M = K = 65536
    rp, col, val = O.random_csr(M, K, 65.536, seed=42)
    x = O.normal((K,), 42, 51)
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val, x)]
    y = torch.empty(M, dtype=torch.float32, device=dev)
    G.spmv_csr(M, K, val.size, d[0], d[1], d[2], d[3], y)
    assert O.rel_frob(y.cpu().numpy(), O.spmv_f64(rp, col, val, x)) <= 1e-5


def test_transpose_reference_abi(dev):
    """perform_mps_matrix_transpose (metal_bridge.h:36-41)."""
    for (r, c) in [(1, 1), (3, 70), (64, 64), (257, 129), (1000, 3)]:
        X = O.normal((r, c), 9, r * 1000 + c)
        bi, bo = G.Buffer.from_array(X), G.Buffer(r * c * 4)
        G.call("perform_mps_matrix_transpose", bi.handle, r, c, bo.handle, c, r, None)
        np.testing.assert_array_equal(bo.to_array((c, r)), O.transpose_f32(X))
    rc, _ = G.call_rc("perform_mps_matrix_transpose", bi.handle, 1000, 3, bo.handle, 1000, 3, None)
    assert rc == -2


def test_spmv_wave_kernel_empty_rows_and_bad_columns(dev):
    """Long rows (wave-per-row kernel) mixed with empty rows; an out-of-range column is
    skipped and reported."""
    import torch

    rng = np.random.default_rng(61)
    M, K = 37, 500
    lens = rng.integers(40, 200, M)
    lens[[0, 5, 6, 36]] = 0
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    col = np.concatenate([np.sort(rng.choice(K, n, replace=False)) for n in lens]).astype(np.int32)
    val = rng.standard_normal(col.size).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    y = _spmv_abi(rp, col, val, x, M, K)
    assert np.all(y[[0, 5, 6, 36]] == 0)
    assert O.rel_frob(y, O.spmv_f64(rp, col, val, x)) <= 1e-5
    # same answer bit for bit through the device-pointer entry (gn_spmv_csr)
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val, x)]
    yd = torch.empty(M, dtype=torch.float32, device=dev)
    G.spmv_csr(M, K, val.size, d[0], d[1], d[2], d[3], yd)
    np.testing.assert_array_equal(yd.cpu().numpy(), y)
    bad = col.copy()
    bad[rp[1] + 3] = K + 7
    bv, bx, by = G.Buffer.from_array(val), G.Buffer.from_array(x), G.Buffer(M * 4)
    rc, msg = G.call_rc("perform_sparse_matvec", bv.handle, rp.ctypes.data, rp.size, bad.ctypes.data, bad.size, M, K,
                        val.size, bx.handle, K, by.handle, M, None)
    assert rc == -3 and "column" in msg


@pytest.mark.parametrize("K,mean", [(20000, 100.0), (70001, 280.0)])
def test_spmv_long_rows_skew_unsorted_and_errors(dev, K, mean):
    """Wide x (K = 20000 and 70001) with unsorted columns and duplicates, one row of
    200000 entries among rows of ~100-280 and 100 empty rows. The device-pointer entry with
    x 4 bytes past 16-byte alignment gives the same bits; an out-of-range column is
    reported."""
    import torch

    rng = np.random.default_rng(K)
    M = 4096
    lens = rng.poisson(mean, M).astype(np.int64)
    lens[100] = 200000
    lens[500:600] = 0
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    col = rng.integers(0, K, int(rp[-1])).astype(np.int32)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    y = _spmv_abi(rp, col, val, x, M, K)
    assert np.all(y[500:600] == 0)
    err = O.rel_frob(y, O.spmv_f64(rp, col, val, x))
    _say("spmv wide/skewed", K, col.size, err)
    assert err <= 1e-5
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val)]
    xt = torch.empty(K + 1, dtype=torch.float32, device=dev)
    xt[1:].copy_(torch.from_numpy(x))
    yd = torch.empty(M, dtype=torch.float32, device=dev)
    G.spmv_csr(M, K, val.size, d[0], d[1], d[2], xt[1:], yd)
    np.testing.assert_array_equal(yd.cpu().numpy(), y)
    bad = col.copy()
    bad[rp[7] + 2] = K + 5
    bv, bx, by = G.Buffer.from_array(val), G.Buffer.from_array(x), G.Buffer(M * 4)
    rc, msg = G.call_rc("perform_sparse_matvec", bv.handle, rp.ctypes.data, rp.size, bad.ctypes.data, bad.size, M, K,
                        val.size, bx.handle, K, by.handle, M, None)
    assert rc == -3 and "column" in msg


def test_spmm_index_cache_reuse_and_invalidation(dev):
    """The Part-1 SpMM keeps the device copy of the index arrays with the values buffer:
    the second call allocates and uploads nothing; new host arrays, changed row pointers
    and gn_csr_indices_changed after an in-place column change are all seen; a malformed
    structure is refused and not kept; release_gpu_buffer of the values drops the copy."""
    rows, cols, N = 500, 700, 64
    rp, col, val = O.random_csr(rows, cols, 12.0, seed=77)
    D = O.normal((cols, N), 7, 1)
    bv, bd, bc = G.Buffer.from_array(val), G.Buffer.from_array(D), G.Buffer(rows * N * 4)

    def run(rp_, col_, expect_rc=0):
        rc, msg = G.call_rc("perform_sparse_dense_matmul", bv.handle, rp_.ctypes.data, rp_.size, col_.ctypes.data,
                            col_.size, rows, cols, val.size, bd.handle, cols, N, bc.handle, rows, N, None)
        assert rc == expect_rc, (rc, msg)
        return bc.to_array((rows, N)) if rc == 0 else None

    n0 = G.memory_stats()[2]
    C1 = run(rp, col)
    n1 = G.memory_stats()[2]
    assert n1 == n0 + 2  # the cached row pointers and column indices
    C2 = run(rp, col)
    assert G.memory_stats()[2] == n1  # nothing uploaded or allocated
    np.testing.assert_array_equal(C1, O.spmm_f32(rp, col, val, D, use_fma=True))
    np.testing.assert_array_equal(C2, C1)
    # columns changed in place: announced with gn_csr_indices_changed
    col[:] = (col + 13) % cols
    assert G.load().gn_csr_indices_changed(bv.handle) == 0
    np.testing.assert_array_equal(run(rp, col), O.spmm_f32(rp, col, val, D, use_fma=True))
    # new host arrays are a new structure: seen without any call
    col_new = ((col + 5) % cols).astype(np.int32)
    np.testing.assert_array_equal(run(rp, col_new), O.spmm_f32(rp, col_new, val, D, use_fma=True))
    # row pointers changed in place are compared on every call
    k = int(np.argmax(np.diff(rp) > 0))  # a row with at least one entry
    rp[k + 1] -= 1  # its last entry moves to the next row
    np.testing.assert_array_equal(run(rp, col_new), O.spmm_f32(rp, col_new, val, D, use_fma=True))
    assert G.memory_stats()[2] == n1  # each replaced copy was released
    # a malformed structure is refused and not kept; the corrected one then runs
    col_new[3] = cols + 4
    assert G.load().gn_csr_indices_changed(bv.handle) == 0
    run(rp, col_new, expect_rc=-3)
    assert G.memory_stats()[2] == n0
    col_new[3] = 0
    np.testing.assert_array_equal(run(rp, col_new), O.spmm_f32(rp, col_new, val, D, use_fma=True))
    # values scaled in place (perform_sparse_scalar_multiply) are read on the next call: the
    # cache holds the index arrays only
    G.call("perform_sparse_scalar_multiply", bv.handle, rp.ctypes.data, rp.size, col_new.ctypes.data, col_new.size,
           rows, cols, val.size, -2.0, None)
    np.testing.assert_array_equal(run(rp, col_new), O.spmm_f32(rp, col_new, val * np.float32(-2.0), D, use_fma=True))
    G.call("perform_sparse_scalar_multiply", bv.handle, rp.ctypes.data, rp.size, col_new.ctypes.data, col_new.size,
           rows, cols, val.size, -0.5, None)
    # SpMV with the same values buffer shares the cached structure
    x = O.normal((cols,), 8, 1)
    bx, by = G.Buffer.from_array(x), G.Buffer(rows * 4)
    G.call("perform_sparse_matvec", bv.handle, rp.ctypes.data, rp.size, col_new.ctypes.data, col_new.size, rows, cols,
           val.size, bx.handle, cols, by.handle, rows, None)
    assert O.rel_frob(by.to_array((rows,)), O.spmv_f64(rp, col_new, val, x)) <= 1e-5
    nmid = G.memory_stats()[2]
    bv.release()
    assert G.memory_stats()[2] == nmid - 3  # the values and their cached index arrays
    for b in (bd, bc, bx, by):
        b.release()


def test_spmm_index_cache_revalidates_for_a_smaller_column_count(dev):
    """An index copy validated for K columns is not trusted for a call with fewer columns:
    the same arrays with aCols below the largest column index are refused with -3, as the
    uncached path refuses them, instead of silently dropping the out-of-range entries."""
    rows, cols, N = 300, 400, 32
    rp, col, val = O.random_csr(rows, cols, 10.0, seed=78)
    D = O.normal((cols, N), 7, 2)
    bv, bd, bc = G.Buffer.from_array(val), G.Buffer.from_array(D), G.Buffer(rows * N * 4)

    def run(k):
        return G.call_rc("perform_sparse_dense_matmul", bv.handle, rp.ctypes.data, rp.size, col.ctypes.data, col.size,
                         rows, k, val.size, bd.handle, k, N, bc.handle, rows, N, None)

    assert run(cols) == (0, "")
    assert run(cols) == (0, "")  # cached and validated for K = cols
    k_small = int(col.max())  # at least one column index is now out of range
    rc, msg = run(k_small)
    assert rc == -3 and "column" in msg, (rc, msg)
    # SpMV through the same cached structure with the smaller K is refused too
    x = O.normal((k_small,), 8, 2)
    bx, by = G.Buffer.from_array(x), G.Buffer(rows * 4)
    rc, msg = G.call_rc("perform_sparse_matvec", bv.handle, rp.ctypes.data, rp.size, col.ctypes.data, col.size, rows,
                        k_small, val.size, bx.handle, k_small, by.handle, rows, None)
    assert rc == -3, (rc, msg)
    assert run(cols) == (0, "")  # and the full K still runs
    np.testing.assert_array_equal(bc.to_array((rows, N)), O.spmm_f32(rp, col, val, D, use_fma=True))
    for b in (bv, bd, bc, bx, by):
        b.release()
