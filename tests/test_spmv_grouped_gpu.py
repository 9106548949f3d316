"""GPU parity of the grouped-layout SpMV (gn_spmv_plan_*, and perform_sparse_matvec once
the index arrays kept with the values buffer are validated) against the oracle's CSR-order
fmaf restatement of the reference loop (internal/cgo/metal_bridge_sparse.m:325-339).

The grouped kernel gathers x in an order sorted by cache line but sums every row in CSR
order with one fused multiply-add per entry, so it is compared bit for bit with
oracle.spmv_f32(use_fma=True); the row-block cut, rows at the 4096-entry limit, the packed
(K <= 65536) and two-array (wider x) layouts, the sort-key coarsening for wide x and the
flag for a bad column are each exercised. A structure with a longer row takes no layout
and runs the flat kernel (relFrob <= 1e-5 against float64, the same bits as gn_spmv_csr)."""
import ctypes
import sys
import zlib

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _csr_from_lens(lens, K, rng, offset=0, sort=True):
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64) + offset
    nnz = int(rp[-1])
    col = rng.integers(0, K, nnz).astype(np.int32)
    if sort:
        for i in range(len(lens)):
            col[rp[i]:rp[i + 1]].sort()
    val = rng.uniform(-1, 1, nnz).astype(np.float32)
    return rp.astype(np.int32), col, val


def _plan_run(dev, rp, col, val, x, K, flags=None):
    import torch

    M = rp.size - 1
    d_rp, d_col, d_val, d_x = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (rp, col, val, x))
    y = torch.full((M,), float("nan"), dtype=torch.float32, device=dev)
    plan = G.SpmvPlan(M, K, val.size, d_rp, d_col)
    try:
        plan.run(d_val, d_x, y, flags)
        out = y.cpu().numpy()
        # a second run on the same plan with other values and x gives their product
        val2 = (val * np.float32(0.5) - np.float32(0.25)).astype(np.float32)
        x2 = (x[::-1] * np.float32(1.5)).astype(np.float32).copy()
        d_val.copy_(torch.from_numpy(val2))
        d_x.copy_(torch.from_numpy(x2))
        plan.run(d_val, d_x, y, flags)
        out2 = y.cpu().numpy()
    finally:
        plan.release()
    return out, out2, val2, x2


CASES = {
    # C5's density on a quarter of its rows: one or two row blocks per CU
    "c5_quarter": dict(M=16384, K=65536, lens=("poisson", 65.5)),
    # rows at and just under the 4096-entry limit among rows of ~100, empty rows; K above
    # 65536 (two-array layout)
    "long_rows": dict(M=4096, K=70001, lens=("poisson", 100.0), long={7: 4096, 100: 4095, 101: 4096},
                      empty=(slice(500, 600),)),
    # K = 65536 exactly: the largest packed layout (columns in 16 bits)
    "k65536_long": dict(M=6000, K=65536, lens=("poisson", 70.0), long={0: 4096, 5999: 4096}),
    # x of 2^20 columns: the sort key is coarsened to 4096 bins of 256 columns
    "wide_x": dict(M=3000, K=1 << 20, lens=("poisson", 80.0)),
    # a single column
    "k1": dict(M=5000, K=1, lens=("poisson", 3.0)),
    # one row of 4096 entries
    "one_row": dict(M=1, K=30000, lens=("fixed", 4096)),
    # mostly empty rows
    "sparse_rows": dict(M=20000, K=5000, lens=("poisson", 0.05)),
    # row pointers starting at an offset (the entries before it are never read)
    "offset_rowptr": dict(M=2000, K=4000, lens=("poisson", 40.0), offset=1000),
    "tiny": dict(M=3, K=4, lens=("list", [2, 0, 3])),
    "unsorted": dict(M=3000, K=9000, lens=("poisson", 50.0), sort=False),
}

# rows longer than 4096 entries: no layout, the flat kernel
FLAT_CASES = {
    "row_4097": dict(M=4096, K=70001, lens=("poisson", 100.0), long={7: 4097}),
    "row_100000": dict(M=2048, K=30000, lens=("poisson", 30.0), long={1000: 100000}),
}


def _make(name):
    c = CASES[name] if name in CASES else FLAT_CASES[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    M, K = c["M"], c["K"]
    kind, p = c["lens"]
    if kind == "poisson":
        lens = rng.poisson(p, M).astype(np.int64)
    elif kind == "fixed":
        lens = np.full(M, p, np.int64)
    else:
        lens = np.array(p, np.int64)
    for r, n in c.get("long", {}).items():
        lens[r] = n
    for sl in c.get("empty", ()):
        lens[sl] = 0
    offset = c.get("offset", 0)
    rp, col, val = _csr_from_lens(lens, K, rng, offset=offset, sort=c.get("sort", True))
    val[:offset] = np.nan  # entries before the first row pointer are never read
    x = rng.standard_normal(K).astype(np.float32)
    return rp, col, val, x, K


@pytest.mark.parametrize("name", list(CASES))
def test_spmv_plan_bit_exact(dev, name):
    import torch

    rp, col, val, x, K = _make(name)
    _say("spmv plan", name, "M", rp.size - 1, "K", K, "nnz", val.size)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    y, y2, val2, x2 = _plan_run(dev, rp, col, val, x, K, flags)
    assert flags.cpu().tolist() == [0, 0]
    np.testing.assert_array_equal(y, O.spmv_f32(rp, col, val, x, use_fma=True))
    np.testing.assert_array_equal(y2, O.spmv_f32(rp, col, val2, x2, use_fma=True))


@pytest.mark.parametrize("name", list(FLAT_CASES))
def test_spmv_plan_flat_kernel_for_rows_over_the_limit(dev, name):
    import torch

    rp, col, val, x, K = _make(name)
    _say("spmv plan (flat)", name, "M", rp.size - 1, "K", K, "nnz", val.size)
    y, y2, val2, x2 = _plan_run(dev, rp, col, val, x, K)
    assert O.rel_frob(y, O.spmv_f64(rp, col, val, x)) <= 1e-5
    assert O.rel_frob(y2, O.spmv_f64(rp, col, val2, x2)) <= 1e-5
    d = [torch.from_numpy(a).to(dev) for a in (rp, col, val, x)]
    yd = torch.empty(rp.size - 1, dtype=torch.float32, device=dev)
    G.spmv_csr(rp.size - 1, K, val.size, d[0], d[1], d[2], d[3], yd)
    np.testing.assert_array_equal(yd.cpu().numpy(), y)


def test_spmv_plan_c5_full_size(dev):
    """Config C5: 65536 x 65536 at 0.1% density (~4.3M entries), bit-exact."""
    rp, col, val = O.random_csr(65536, 65536, 65.536, seed=42)
    x = O.normal((65536,), 42, 51)
    _say("spmv plan C5 nnz", val.size)
    y, y2, val2, x2 = _plan_run(dev, rp, col, val, x, 65536)
    np.testing.assert_array_equal(y, O.spmv_f32(rp, col, val, x, use_fma=True))
    np.testing.assert_array_equal(y2, O.spmv_f32(rp, col, val2, x2, use_fma=True))


def test_spmv_plan_bad_columns_are_flagged(dev):
    """A column outside [0, K) (above K, or negative) raises flags[1], reads nothing and
    contributes nothing; the other entries are summed as usual (packed and two-array
    layouts)."""
    import torch

    for name in ("long_rows", "k65536_long"):
        rp, col, val, x, K = _make(name)
        for bad_at, bad in ((int(rp[3]) + 1, K + 3), (int(rp[7]) + 5, -1)):
            colb = col.copy()
            colb[bad_at] = bad
            flags = torch.zeros(2, dtype=torch.int32, device=dev)
            y, _, _, _ = _plan_run(dev, rp, colb, val, x, K, flags)
            assert flags.cpu().tolist()[1] == 1, (name, bad)
            keep = np.ones(col.size, bool)
            keep[bad_at] = False
            kept_before = np.concatenate([[0], np.cumsum(keep)])  # kept entries before each position
            rp_k = kept_before[rp].astype(np.int32)
            np.testing.assert_array_equal(y, O.spmv_f32(rp_k, colb[keep], val[keep], x, use_fma=True))


def test_spmv_plan_rejects_malformed_row_pointers(dev):
    import torch

    col = torch.zeros(4, dtype=torch.int32, device=dev)
    for rp in ([0, 3, 2, 4], [0, 2, 5], [-1, 2, 4]):
        d_rp = torch.tensor(rp, dtype=torch.int32, device=dev)
        torch.cuda.synchronize()  # the plan reads the row pointers on the library stream
        h = ctypes.c_void_p()
        rc, msg = G.call_rc("gn_spmv_plan_create", len(rp) - 1, 4, 4, d_rp.data_ptr(), col.data_ptr(),
                            ctypes.byref(h), None)
        assert rc == -1 and "monotone" in msg, (rp, rc, msg)
        assert not h.value


def test_spmv_part1_uses_grouped_layout(dev):
    """perform_sparse_matvec with host index arrays: the first call uploads the indices,
    builds the grouped layout and validates the columns through its kernel; every call,
    the first included, gives the CSR-order fmaf bits. A call with a larger column count
    validates again and rebuilds the layout for it; a bad column is refused; releasing the
    values buffer frees the cached copy and the layout."""
    rng = np.random.default_rng(5)
    M, K = 8192, 16384
    lens = rng.poisson(40.0, M).astype(np.int64)  # ~330K entries: above the 2^18 threshold
    rp, col, val = _csr_from_lens(lens, K, rng)
    x = rng.standard_normal(K).astype(np.float32)
    ref = O.spmv_f32(rp, col, val, x, use_fma=True)
    bv, bx, by = G.Buffer.from_array(val), G.Buffer.from_array(x), G.Buffer(M * 4)

    def run(k, xb, c=col):
        rc, msg = G.call_rc("perform_sparse_matvec", bv.handle, rp.ctypes.data, rp.size, c.ctypes.data, c.size, M, k,
                            val.size, xb.handle, k, by.handle, M, None)
        return rc, msg, (by.to_array((M,)) if rc == 0 else None)

    n0 = G.memory_stats()[2]
    rc, _, y1 = run(K, bx)
    assert rc == 0
    np.testing.assert_array_equal(y1, ref)
    # the cached row pointers and columns, and the packed layout (K <= 65536): block
    # offsets and grouped words
    assert G.memory_stats()[2] == n0 + 4
    for _ in range(2):
        np.testing.assert_array_equal(run(K, bx)[2], ref)
    assert G.memory_stats()[2] == n0 + 4
    # a larger column count (x extended with values the indices never reach)
    K2 = K + 4096
    x_big = np.concatenate([x, rng.standard_normal(4096).astype(np.float32)])
    bxb = G.Buffer.from_array(x_big)
    ref2 = O.spmv_f32(rp, col, val, x_big, use_fma=True)
    for _ in range(2):
        np.testing.assert_array_equal(run(K2, bxb)[2], ref2)
    # a column outside [0, K) in a new host array: refused, through the grouped kernel's flag
    bad = col.copy()
    bad[12345] = K + 1
    rc, msg, _ = run(K, bx, bad)
    assert rc == -3 and "column" in msg
    bv.release()
    for b in (bx, bxb, by):
        b.release()
    G.call("gn_synchronize", None)
    assert G.memory_stats()[2] == n0 - 3  # bv, bx, by, and the cached indices and layout, are gone
