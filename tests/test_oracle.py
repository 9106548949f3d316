"""Pins for the CPU checker (oracle/). Each check compares the oracle with something
other than itself: numpy/scipy float64, hand-derived bit tables, closed forms, the
reference's own test vectors, or brute force on tiny inputs."""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------ generator
def _splitmix_py(state):
    """Published SplitMix64 step (Steele, Lea, Flood 2014): returns (next_state, output)."""
    M = (1 << 64) - 1
    state = (state + 0x9E3779B97F4A7C15) & M
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return state, z ^ (z >> 31)


def _mix(z):
    M = (1 << 64) - 1
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return z ^ (z >> 31)


def test_splitmix_known_answer_and_counter_form():
    # Published first outputs of SplitMix64 from state 0.
    s, o1 = _splitmix_py(0)
    s, o2 = _splitmix_py(s)
    assert o1 == 0xE220A8397B1DCDAF
    assert o2 == 0x6E789E6AA1B965F4
    # The oracle's counter form equals the sequential generator started at its base.
    for seed, stream in [(42, 0), (42, 1), (7, 123456789)]:
        base = seed ^ _mix((stream + 0x632BE59BD9B4E019) & ((1 << 64) - 1))
        st = base
        for i in range(5):
            st, out = _splitmix_py(st)
            assert O.lib().orc_splitmix64(seed, stream, i) == out


def test_uniform_normal_moments_and_determinism():
    u = O.uniform((1 << 16,), 42, 1, -1.0, 1.0)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert abs(u.mean()) < 0.02 and abs(u.var() - 1.0 / 3.0) < 0.01
    n = O.normal((1 << 16,), 42, 2, 0.0, 0.02)
    assert abs(n.mean()) < 0.02 * 0.02 and abs(n.std() - 0.02) < 0.02 * 0.02
    assert np.array_equal(n, O.normal((1 << 16,), 42, 2, 0.0, 0.02))
    assert not np.array_equal(n, O.normal((1 << 16,), 42, 3, 0.0, 0.02))


# ------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_f64_matches_numpy_all_transposes(tA, tB):
    z = np.load(os.path.join(GOLD, "gemm_small.npz"))
    for key in ["1x1x1", "8x8x8", "3x5x7", "17x33x9", "64x48x40", "33x65x130"]:
        A, B, C = z[f"A_{key}"], z[f"B_{key}"], z[f"C64_{key}"]
        As = np.ascontiguousarray(A.T) if tA else A
        Bs = np.ascontiguousarray(B.T) if tB else B
        R = O.gemm_f64(As, Bs, transA=bool(tA), transB=bool(tB))
        np.testing.assert_allclose(R, C, rtol=1e-12, atol=1e-12)


def test_gemm_f64_alpha_beta_and_closed_forms():
    rng = np.random.default_rng(1)
    A = rng.standard_normal((20, 30)).astype(np.float32)
    B = rng.standard_normal((30, 10)).astype(np.float32)
    C0 = rng.standard_normal((20, 10))
    R = O.gemm_f64(A, B, alpha=0.5, beta=-2.0, C=C0)
    np.testing.assert_allclose(R, 0.5 * (A.astype(np.float64) @ B) - 2.0 * C0, rtol=1e-12, atol=1e-12)
    # identity and permutation
    I = np.eye(30, dtype=np.float32)
    np.testing.assert_array_equal(O.gemm_f64(A, I), A.astype(np.float64))
    P = np.eye(30, dtype=np.float32)[rng.permutation(30)]
    np.testing.assert_array_equal(O.gemm_f64(A, P), A.astype(np.float64) @ P)
    # rank-1 outer product is exact in float64
    u = rng.standard_normal((12, 1)).astype(np.float32)
    v = rng.standard_normal((1, 9)).astype(np.float32)
    np.testing.assert_array_equal(O.gemm_f64(u, v), u.astype(np.float64) * v.astype(np.float64))
    # small integers: exact
    Ai = rng.integers(-8, 8, size=(16, 24)).astype(np.float32)
    Bi = rng.integers(-8, 8, size=(24, 7)).astype(np.float32)
    np.testing.assert_array_equal(O.gemm_f64(Ai, Bi), Ai.astype(np.float64) @ Bi)
    # (AB)^T = B^T A^T through the transpose flags
    np.testing.assert_allclose(O.gemm_f64(B, A, transA=True, transB=True), (A.astype(np.float64) @ B).T, rtol=1e-12)


def test_gemm_f64_rows_subset():
    rng = np.random.default_rng(2)
    A = rng.standard_normal((50, 40)).astype(np.float32)
    B = rng.standard_normal((40, 30)).astype(np.float32)
    rows = np.array([0, 7, 49, 13])
    full = A.astype(np.float64) @ B
    np.testing.assert_allclose(O.gemm_f64_rows(A, B, rows), full[rows], rtol=1e-12)
    np.testing.assert_allclose(O.gemm_f64_rows(np.ascontiguousarray(A.T), B, rows, transA=True), full[rows], rtol=1e-12)


def test_gemm_f64_k_zero():
    A = np.zeros((3, 0), np.float32)
    B = np.zeros((0, 4), np.float32)
    np.testing.assert_array_equal(O.gemm_f64(A, B), np.zeros((3, 4)))


# ------------------------------------------------------------------ fp16
def test_f16_table_hand_derived():
    t = json.load(open(os.path.join(GOLD, "f16_table.json")))
    for c in t["cases"]:
        # array entry points carry raw bits (a scalar ctypes float would quiet an sNaN)
        x = np.array([int(c["f32"], 16)], dtype=np.uint32).view(np.float32)
        assert int(O.f32_to_f16_bits(x, rtz=True)[0]) == int(c["rtz"], 16), c["what"]
        got = int(O.f32_to_f16_bits(x, rtz=False)[0])
        if c["rne"] == "nan":
            assert (got & 0x7C00) == 0x7C00 and (got & 0x3FF) != 0, c["what"]
        else:
            assert got == int(c["rne"], 16), c["what"]


def _rtz_numpy(x):
    """Independent IEEE round-toward-zero via numpy's RNE cast + one nextafter step."""
    x = np.asarray(x, dtype=np.float32)
    h = x.astype(np.float16)
    over = np.abs(h.astype(np.float64)) > np.abs(x.astype(np.float64))
    h = np.where(over, np.nextafter(h, np.float16(0)), h)
    return h.view(np.uint16)


def test_rtz_equals_ieee_round_toward_zero():
    rng = np.random.default_rng(3)
    # log-uniform magnitudes spanning fp16 subnormals .. just below overflow, both signs
    mag = np.exp2(rng.uniform(-26, 15.99, size=200000)).astype(np.float32)
    x = (mag * rng.choice([-1, 1], size=mag.size)).astype(np.float32)
    got = O.f32_to_f16_bits(x, rtz=True)
    np.testing.assert_array_equal(got, _rtz_numpy(x))
    # every fp16 value, and the fp32 just above/below it, truncates to the right code
    allh = np.arange(0, 0x7C00, dtype=np.uint16)
    hv = allh.view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(O.f32_to_f16_bits(hv, True), allh)
    up = np.nextafter(hv, np.float32(np.inf))
    np.testing.assert_array_equal(O.f32_to_f16_bits(up[up < 65536], True), allh[up < 65536])


def test_rne_equals_numpy():
    rng = np.random.default_rng(4)
    mag = np.exp2(rng.uniform(-27, 16.5, size=200000)).astype(np.float32)
    x = (mag * rng.choice([-1, 1], size=mag.size)).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(O.f32_to_f16_bits(x, rtz=False), ref)
    # exact midpoints between consecutive fp16 values (ties to even)
    h = np.arange(0, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(O.f32_to_f16_bits(mid, False), mid.astype(np.float16).view(np.uint16))


def test_f16_to_f32_all_patterns():
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(allh)
    ref = allh.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ------------------------------------------------------------------ CSR
def test_coo_to_csr_golden():
    z = np.load(os.path.join(GOLD, "csr_64.npz"))
    rc, rowptr, idx, data = O.coo_to_csr(64, 64, z["ri"], z["ci"], z["v"])
    assert rc == 0
    np.testing.assert_array_equal(rowptr, z["rowptr"])
    np.testing.assert_array_equal(idx, z["idx"])
    np.testing.assert_array_equal(data, z["data"])  # stable order keeps duplicate order
    assert rowptr[0] == 0 and rowptr[-1] == z["v"].size and np.all(np.diff(rowptr) >= 0)
    for r in range(64):
        assert np.all(np.diff(idx[rowptr[r]:rowptr[r + 1]]) >= 0)


def test_coo_validation_errors():
    ri = np.array([0, 1], np.int32)
    ci = np.array([0, 1], np.int32)
    v = np.ones(2, np.float32)
    assert O.coo_to_csr(2, 2, ri, ci, v)[0] == 0
    assert O.coo_to_csr(1, 2, ri, ci, v)[0] == -2   # row out of range
    assert O.coo_to_csr(2, 1, ri, ci, v)[0] == -3   # col out of range
    rc, rowptr, idx, data = O.coo_to_csr(4, 4, ri[:0], ci[:0], v[:0])
    assert rc == 0 and np.array_equal(rowptr, np.zeros(5, np.int32)) and idx.size == 0


def test_csr_to_dense_last_duplicate_wins():
    rowptr = np.array([0, 2, 2], np.int32)
    idx = np.array([1, 1], np.int32)
    data = np.array([3.0, 5.0], np.float32)
    np.testing.assert_array_equal(O.csr_to_dense(2, 2, rowptr, idx, data), [[0, 5], [0, 0]])


# ------------------------------------------------------------------ SpMM / SpMV
def _fma_f32(a, b, c):
    """Correctly rounded fp32 fma via exact rationals (brute force for tiny cases)."""
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    f = np.float32(float(exact))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda y: (abs(Fraction(float(y)) - exact), int(np.array(y).view(np.uint32)) & 1))
    return np.float32(best)


def test_spmm_golden_and_semantics():
    z = np.load(os.path.join(GOLD, "csr_64.npz"))
    rp, idx, data, D = z["rowptr"], z["idx"], z["data"], z["D"]
    C64 = O.spmm_f64(rp, idx, data, D)
    np.testing.assert_allclose(C64, z["C64"], rtol=1e-12, atol=1e-12)  # duplicates summed (scipy)
    for fma in (True, False):
        C = O.spmm_f32(rp, idx, data, D, use_fma=fma)
        assert O.rel_frob(C, z["C64"]) < 1e-6
        for r in (0, 5, 6, 31, 63):  # empty rows
            assert np.all(C[r] == 0)


def test_spmm_f32_rounding_order_brute_force():
    z = np.load(os.path.join(GOLD, "csr_64.npz"))
    rp, idx, data, D = z["rowptr"], z["idx"], z["data"], z["D"]
    Cf = O.spmm_f32(rp, idx, data, D, use_fma=True)
    Cn = O.spmm_f32(rp, idx, data, D, use_fma=False)
    for i in (1, 3, 10, 62):
        for j in range(D.shape[1]):
            accf = np.float32(0)
            accn = np.float32(0)
            for k in range(rp[i], rp[i + 1]):
                accf = _fma_f32(data[k], D[idx[k], j], accf)
                accn = np.float32(accn + np.float32(data[k] * D[idx[k], j]))
            assert Cf[i, j] == accf
            assert Cn[i, j] == accn


def test_spmm_equals_dense_gemm_without_duplicates():
    rp, col, val = O.random_csr(200, 300, 6.0, seed=11)
    D = O.normal((300, 32), 11, 5)
    dense = O.csr_to_dense(200, 300, rp, col, val)
    np.testing.assert_allclose(O.spmm_f64(rp, col, val, D), O.gemm_f64(dense, D), rtol=1e-12, atol=1e-12)
    S = sp.csr_matrix((val.astype(np.float64), col, rp), shape=(200, 300))
    np.testing.assert_allclose(O.spmm_f64(rp, col, val, D), S @ D.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_spmv_golden():
    z = np.load(os.path.join(GOLD, "csr_64.npz"))
    rp, idx, data, x = z["rowptr"], z["idx"], z["data"], z["x"]
    np.testing.assert_allclose(O.spmv_f64(rp, idx, data, x), z["y64"], rtol=1e-12, atol=1e-12)
    y = O.spmv_f32(rp, idx, data, x, use_fma=False)
    # sequential fp32 sum, brute force
    for i in range(64):
        acc = np.float32(0)
        for k in range(rp[i], rp[i + 1]):
            acc = np.float32(acc + np.float32(data[k] * x[idx[k]]))
        assert y[i] == acc
    assert O.rel_frob(O.spmv_f32(rp, idx, data, x, use_fma=True), z["y64"]) < 1e-6


# ------------------------------------------------------------------ activations / linear
def test_activation_reference_vectors():
    # gpu/matrix/activation_test.go:32-51 (ReLU), :200-220 (LeakyReLU alpha=0.1)
    x = np.array([-2.0, -1.0, 0.0, 1.0, 2.0, 3.0], np.float32)
    np.testing.assert_allclose(O.act_f32(0, x), [0, 0, 0, 1, 2, 3], atol=1e-6)
    np.testing.assert_allclose(O.act_f32(4, x[:4], 0.1), [-0.2, -0.1, 0.0, 1.0], atol=1e-6)
    x4 = np.array([-2.0, -1.0, 0.0, 1.0], np.float32)
    assert abs(O.act_f32(7, x4)[2]) <= 1e-6   # GELU(0)=0, activation_test.go:282-285
    assert abs(O.act_f32(1, x4)[2] - 0.5) <= 1e-6  # Sigmoid(0)=0.5, :96-98
    assert abs(O.act_f32(2, x4)[2]) <= 1e-6   # Tanh(0)=0, :124-126
    assert abs(O.act_f32(6, x4)[2]) <= 1e-6   # Swish(0)=0
    e = O.act_f32(5, x4, 1.0)
    assert abs(e[3] - 1.0) <= 1e-6 and e[0] < 0  # ELU, :236-244


def test_activation_closed_forms():
    xs = np.array([-30.0, -3.0, -0.5, 0.0, 0.25, 2.0, 30.0])
    for x in xs:
        g = O.lib().orc_act_f64(7, 0.0, x)
        assert g == pytest.approx(0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3))), abs=1e-12)
        assert O.lib().orc_act_f64(1, 0.0, x) == pytest.approx(1 / (1 + math.exp(-x)), rel=1e-12)
        assert O.lib().orc_act_f64(2, 0.0, x) == pytest.approx(math.tanh(x), rel=1e-12)
    # GELU limits: x for large x, 0 for large negative x; ReLU/GELU agree asymptotically
    assert O.lib().orc_act_f64(7, 0.0, 50.0) == 50.0
    assert O.lib().orc_act_f64(7, 0.0, -50.0) == 0.0
    assert math.isnan(O.lib().orc_act_f64(3, 0.0, 1.0))  # softmax is not an epilogue
    # fp32 restatement tracks the float64 one
    x = np.linspace(-8, 8, 1001).astype(np.float32)
    for code in (0, 1, 2, 4, 5, 6, 7):
        np.testing.assert_allclose(O.act_f32(code, x, 0.1), O.act_f64(code, x.astype(np.float64), 0.1), rtol=2e-6, atol=2e-6)


def test_softmax_rows_pins():
    """orc_softmax_rows_f64 against what fixes softmax independently: scipy's routine, rows
    summing to 1, invariance to a per-row shift, the two-element closed form
    1 / (1 + exp(b - a)), a constant row giving 1/n, and NaN handling (fmax skips NaN in
    the maximum, exp then spreads it over the row)."""
    from scipy.special import softmax

    rng = np.random.default_rng(17)
    x = (3.0 * rng.standard_normal((37, 129))).astype(np.float32)
    y = O.softmax_rows_f64(x)
    np.testing.assert_allclose(y, softmax(x.astype(np.float64), axis=1), rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, rtol=1e-12)
    np.testing.assert_allclose(O.softmax_rows_f64(x + np.float32(5.0)), y, rtol=1e-5)  # x+5 rounds in fp32
    two = np.array([[1.5, -0.25], [-30.0, 30.0]], np.float32)
    t = O.softmax_rows_f64(two)
    for r in range(2):
        a, b = float(two[r, 0]), float(two[r, 1])
        assert t[r, 0] == pytest.approx(1.0 / (1.0 + math.exp(b - a)), rel=1e-12)
    np.testing.assert_allclose(O.softmax_rows_f64(np.full((1, 8), 2.5, np.float32)), 1.0 / 8, rtol=1e-15)
    one = O.softmax_rows_f64(np.array([3.0, 1.0, 0.5], np.float32))  # 1-D is one row
    assert one.shape == (3,) and one.sum() == pytest.approx(1.0)
    nan_row = O.softmax_rows_f64(np.array([[np.nan, 1.0, 2.0]], np.float32))
    assert np.isnan(nan_row).all()


@pytest.mark.parametrize("w_out_in", [0, 1])
def test_linear_f64_matches_numpy(w_out_in):
    rng = np.random.default_rng(5)
    X = rng.standard_normal((9, 33)).astype(np.float32)
    W = (rng.standard_normal((17, 33)) if w_out_in else rng.standard_normal((33, 17))).astype(np.float32)
    b = rng.standard_normal(17).astype(np.float32)
    Wm = W.T.astype(np.float64) if w_out_in else W.astype(np.float64)
    pre = X.astype(np.float64) @ Wm + b
    np.testing.assert_allclose(O.linear_f64(X, W, b, 0, w_out_in), np.maximum(pre, 0), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(O.linear_f64(X, W, None, -1, w_out_in), X.astype(np.float64) @ Wm, rtol=1e-12, atol=1e-12)


def test_transpose():
    X = np.arange(12, dtype=np.float32).reshape(3, 4)
    np.testing.assert_array_equal(O.transpose_f32(X), X.T)


def test_rel_frob():
    R = np.array([3.0, 4.0])
    assert O.rel_frob(np.array([3.0, 4.0], np.float32), R) == 0.0
    assert O.rel_frob(np.array([3.0, 4.5], np.float32), R) == pytest.approx(0.1)


# ------------------------------------------------------------------ activation / linear backward
GRAD_CODES = [-1, 0, 1, 2, 4, 5, 6, 7]


@pytest.mark.parametrize("code", GRAD_CODES)
def test_act_grad_matches_finite_differences(code):
    """orc_act_grad_f64 against central differences of the forward restatement
    orc_act_f64 (an independent check: a dropped term or wrong sign fails)."""
    rng = np.random.default_rng(71 + code)
    x = rng.uniform(-4, 4, 200)
    x = x[np.abs(x) > 1e-2]  # away from the ReLU / LeakyReLU / ELU kink at 0
    h = 1e-6
    fd = (O.act_f64(code, x + h, 0.1) - O.act_f64(code, x - h, 0.1)) / (2 * h)
    g = O.act_grad_f64(code, x, 0.1)
    np.testing.assert_allclose(g, fd, rtol=1e-6, atol=1e-8)


def test_act_grad_closed_forms():
    assert O.act_grad_f64(7, 0.0) == 0.5     # GELU'(0)
    assert O.act_grad_f64(1, 0.0) == 0.25    # sigmoid'(0)
    assert O.act_grad_f64(2, 0.0) == 1.0     # tanh'(0)
    assert O.act_grad_f64(6, 0.0) == 0.5     # swish'(0)
    assert O.act_grad_f64(0, 2.0) == 1.0 and O.act_grad_f64(0, -2.0) == 0.0
    assert O.act_grad_f64(4, -2.0, 0.2) == 0.2
    assert abs(O.act_grad_f64(5, -1.0, 0.5) - 0.5 * np.exp(-1.0)) < 1e-15
    assert abs(O.act_grad_f64(7, 50.0) - 1.0) < 1e-12 and abs(O.act_grad_f64(7, -50.0)) < 1e-12


@pytest.mark.parametrize("code", [0, 1, 2, 4, 7])
def test_linear_backward_matches_finite_differences(code):
    """(dX, dW, db) of L = sum(G * act(X W + b)) by central differences, W [in, out]:
    pins the transposes and the bias reduction of the backward restatement."""
    rng = np.random.default_rng(91 + code)
    B_, I_, O_ = 3, 4, 5
    X = rng.standard_normal((B_, I_))
    W = rng.standard_normal((I_, O_))
    b = rng.standard_normal(O_)
    Gout = rng.standard_normal((B_, O_))

    def loss(X_, W_, b_):
        return float((Gout * O.act_f64(code, X_ @ W_ + b_, 0.1)).sum())

    pre = (X @ W + b)
    # the restatement works on fp32 storage: feed values exactly representable in fp32
    X32, W32, pre32, G32 = (a.astype(np.float32) for a in (X, W, pre, Gout))
    dX, dW, db, _ = O.linear_backward_f64(X32, W32, pre32, G32, code, alpha=0.1)
    h = 1e-6

    def fd(arr, idx, which):
        a_p, a_m = arr.copy(), arr.copy()
        a_p[idx] += h
        a_m[idx] -= h
        args_p = {"X": (a_p, W, b), "W": (X, a_p, b), "b": (X, W, a_p)}[which]
        args_m = {"X": (a_m, W, b), "W": (X, a_m, b), "b": (X, W, a_m)}[which]
        return (loss(*args_p) - loss(*args_m)) / (2 * h)

    fdX = np.array([[fd(X, (i, j), "X") for j in range(I_)] for i in range(B_)])
    fdW = np.array([[fd(W, (i, j), "W") for j in range(O_)] for i in range(I_)])
    fdb = np.array([fd(b, (j,), "b") for j in range(O_)])
    # tolerance covers the fp32 rounding of the restatement's inputs
    np.testing.assert_allclose(dX, fdX, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(dW, fdW, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(db, fdb, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ remaining sparse entry points
def _rand_csr(rng, M, K, density):
    D = np.where(rng.random((M, K)) < density, rng.standard_normal((M, K)), 0.0).astype(np.float32)
    rows, cols = np.nonzero(D)
    rp = np.zeros(M + 1, np.int32)
    np.cumsum(np.bincount(rows, minlength=M), out=rp[1:])
    return D, rp, cols.astype(np.int32), D[rows, cols]


def test_csr_to_csc_round_trip():
    rng = np.random.default_rng(201)
    D, rp, ci, v = _rand_csr(rng, 30, 41, 0.2)
    cp, ri, cv = O.csr_to_csc(30, 41, rp, ci, v)
    back = np.zeros_like(D)
    for j in range(41):
        back[ri[cp[j]:cp[j + 1]], j] = cv[cp[j]:cp[j + 1]]
    np.testing.assert_array_equal(back, D)


def test_spgemm_matches_dense_product_and_merge_pairing():
    rng = np.random.default_rng(203)
    A, arp, acol, aval = _rand_csr(rng, 40, 60, 0.15)
    Bd, brp, bcol, bval = _rand_csr(rng, 60, 35, 0.15)
    bcp, brow, bv = O.csr_to_csc(60, 35, brp, bcol, bval)
    C = O.spgemm_csr_csc_f32(arp, acol, aval, bcp, brow, bv)
    ref = A.astype(np.float64) @ Bd.astype(np.float64)
    assert O.rel_frob(C, ref) <= 1e-6
    # duplicates pair up in merge order: A row (col 1: 2, col 1: 3), B column (row 1: 5, row 1: 7)
    C2 = O.spgemm_csr_csc_f32(np.array([0, 2], np.int32), np.array([1, 1], np.int32), np.array([2, 3], np.float32),
                              np.array([0, 2], np.int32), np.array([1, 1], np.int32), np.array([5, 7], np.float32))
    assert C2[0, 0] == 2 * 5 + 3 * 7
    # a zero sum leaves +0 (the reference stores only nonzero sums)
    C3 = O.spgemm_csr_csc_f32(np.array([0, 2], np.int32), np.array([0, 1], np.int32), np.array([1, -1], np.float32),
                              np.array([0, 2], np.int32), np.array([0, 1], np.int32), np.array([1, 1], np.float32))
    assert C3[0, 0] == 0.0 and not np.signbit(C3[0, 0])


def test_dense_csc_matches_dense_product():
    rng = np.random.default_rng(205)
    A = rng.standard_normal((23, 50)).astype(np.float32)
    Bd, brp, bcol, bval = _rand_csr(rng, 50, 31, 0.2)
    bcp, brow, bv = O.csr_to_csc(50, 31, brp, bcol, bval)
    C = O.dense_csc_f32(A, bcp, brow, bv)
    assert O.rel_frob(C, A.astype(np.float64) @ Bd.astype(np.float64)) <= 1e-6


def test_sparse_add_merge_cases():
    rng = np.random.default_rng(207)
    A, arp, acol, aval = _rand_csr(rng, 25, 33, 0.3)
    B, brp, bcol, bval = _rand_csr(rng, 25, 33, 0.3)
    # force some exact cancellations
    both = np.argwhere((A != 0) & (B != 0))[:5]
    for i, j in both:
        B[i, j] = -A[i, j]
    rows, cols = np.nonzero(B)
    brp = np.zeros(26, np.int32)
    np.cumsum(np.bincount(rows, minlength=25), out=brp[1:])
    bcol, bval = cols.astype(np.int32), B[rows, cols]
    rc, ri, ci, vv = O.sparse_add(arp, acol, aval, brp, bcol, bval)
    assert rc == 0
    S = np.zeros((25, 33), np.float32)
    S[ri, ci] = vv
    np.testing.assert_array_equal(S, A + B)
    # order: rows non-decreasing, columns increasing within a row; cancelled entries dropped
    key = ri.astype(np.int64) * 33 + ci
    assert np.all(np.diff(key) > 0)
    assert not np.any(vv == 0)
    assert ri.size == np.count_nonzero(A + B)
    rc2, *_ = O.sparse_add(arp, acol, aval, brp, bcol, bval, max_nnz=ri.size - 1)
    assert rc2 == -2


def test_dense_to_coo_threshold_order_nan():
    rng = np.random.default_rng(209)
    D = rng.standard_normal((17, 29)).astype(np.float32)
    D[3, 4] = np.nan
    rc, ri, ci, vv = O.dense_to_coo(D, 0.5)
    assert rc == 0
    rr, cc = np.nonzero(np.abs(np.nan_to_num(D, nan=0.0)) > 0.5)
    np.testing.assert_array_equal(ri, rr)
    np.testing.assert_array_equal(ci, cc)
    np.testing.assert_array_equal(vv, D[rr, cc])
    assert O.dense_to_coo(D, 0.5, max_nnz=3)[0] == -2


def test_parallel_sparse_loops_equal_the_serial_ones():
    """The CPU baseline's OpenMP row split computes each row exactly as the reference's
    single-threaded loop does (metal_bridge_sparse.m:117-133, :325-339)."""
    rp, col, val = O.random_csr(3000, 2000, 9.0, seed=5, distinct=False)
    D = O.normal((2000, 40), 3, 1)
    x = O.normal((2000,), 3, 2)
    for fma in (True, False):
        np.testing.assert_array_equal(O.spmm_f32_par(rp, col, val, D, 8, use_fma=fma),
                                      O.spmm_f32(rp, col, val, D, use_fma=fma))
        np.testing.assert_array_equal(O.spmv_f32_par(rp, col, val, x, 8, use_fma=fma),
                                      O.spmv_f32(rp, col, val, x, use_fma=fma))


# ---------------------------------------------------------------- backward from the output
@pytest.mark.parametrize("code,alpha,lo,hi,atol", [
    (0, 0.0, -4, 4, 0.0), (1, 0.0, -6, 6, 2e-7), (2, 0.0, -4, 4, 1e-6), (4, 0.1, -4, 4, 1e-7),
    (5, 1.0, -6, 4, 5e-7), (6, 0.0, -0.3, 6, 3e-6), (7, 0.0, -0.3, 3, 5e-6)])
def test_act_backward_out_equals_derivative_at_the_input(code, alpha, lo, hi, atol):
    """The reference's backward formulas in terms of the OUTPUT y = act(x) are identities of
    act'(x): y(1-y), 1-y^2, y+alpha (ELU, x<0), 1 or alpha; for Swish and GELU the three
    Newton steps from x = y converge on [lo, hi] (two steps leave errors of 1e-4 to 1e-3
    there, so a wrong step count fails). Checked against orc_act_grad_f64, itself pinned
    by finite differences above."""
    rng = np.random.default_rng(90 + code)
    x = rng.uniform(lo, hi, 4000)
    x = x[np.abs(x) > 1e-3]
    g = rng.standard_normal(x.size).astype(np.float32)
    y = O.act_f64(code, x, alpha).astype(np.float32)
    got = O.act_backward_out_f32(code, g, y, alpha)
    ref = g.astype(np.float64) * O.act_grad_f64(code, x, alpha)
    np.testing.assert_allclose(got, ref, rtol=2e-6 if code != 2 else 0, atol=atol * 4)


def test_act_backward_out_special_cases():
    one = np.ones(1, np.float32)
    # Swish: |y| < 1e-8 short-cuts to g/2 (metal_bridge_activation.m:573-577); GELU: y = 0 gives x = 0.
    assert O.act_backward_out_f32(6, 3 * one, np.float32([5e-9]))[0] == 1.5
    assert O.act_backward_out_f32(7, 3 * one, np.float32([0.0]))[0] == 1.5
    # ReLU passes g where y > 0 only; LeakyReLU / ELU use the output's sign.
    y = np.float32([-1.0, 0.0, 2.0])
    g = np.float32([5.0, 6.0, 7.0])
    assert list(O.act_backward_out_f32(0, g, y)) == [0.0, 0.0, 7.0]
    assert list(O.act_backward_out_f32(4, g, y, 0.5)) == [2.5, 3.0, 7.0]
    assert list(O.act_backward_out_f32(5, g, y, 2.0)) == [5.0, 12.0, 7.0]  # g * (y + alpha) for y <= 0
    # Sigmoid at y = 1/2 is g/4, Tanh at y = 0 is g.
    assert O.act_backward_out_f32(1, 4 * one, np.float32([0.5]))[0] == 1.0
    assert O.act_backward_out_f32(2, 4 * one, np.float32([0.0]))[0] == 4.0


def test_softmax_backward_matches_finite_differences():
    """y * (g - <g, y>) is the gradient of x -> <g, softmax(x)> at y = softmax(x): checked by
    float64 central differences (a dropped term or a wrong sign fails)."""
    rng = np.random.default_rng(123)
    for rows, cols in ((1, 7), (3, 33), (2, 300)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        g = rng.standard_normal((rows, cols)).astype(np.float32)
        y = O.softmax_rows_f64(x)
        got = O.softmax_backward_f32(g, y.astype(np.float32))
        h = 1e-4
        fd = np.empty((rows, cols))
        for j in range(cols):
            xp = x.astype(np.float64).copy()
            xm = xp.copy()
            xp[:, j] += h
            xm[:, j] -= h
            sp_ = np.exp(xp - xp.max(1, keepdims=True))
            sp_ /= sp_.sum(1, keepdims=True)
            sm_ = np.exp(xm - xm.max(1, keepdims=True))
            sm_ /= sm_.sum(1, keepdims=True)
            fd[:, j] = ((g * sp_).sum(1) - (g * sm_).sum(1)) / (2 * h)
        np.testing.assert_allclose(got, fd, rtol=1e-4, atol=1e-6)
