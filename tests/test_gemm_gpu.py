"""GPU parity of the MFMA GEMMs (fp32 and fp16-in/fp32-acc) against the oracle.

Tolerances: fp32 relFrob <= 1e-5 vs float64 GEMM; fp16-in
relFrob <= 2e-2 vs float64 GEMM of the unrounded fp32 inputs. The fp16 path is also
checked at 1e-5 against the float64 product of the fp16-ROUNDED inputs, which pins
the GEMM itself rather than the input cast."""
import os
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
VARIANTS = [(False, False), (False, True), (True, False), (True, True)]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _stored(X, trans):
    return np.ascontiguousarray(X.T) if trans else X


def _gemm_dev(dev, A, B, tA, tB, dtype, **kw):
    import torch

    As, Bs = _stored(A, tA), _stored(B, tB)
    ad = torch.from_numpy(As).to(dev)
    bd = torch.from_numpy(Bs).to(dev)
    if dtype == G.GN_F16:
        a16 = torch.empty(ad.shape, dtype=torch.float16, device=dev)
        b16 = torch.empty(bd.shape, dtype=torch.float16, device=dev)
        mode = kw.pop("round_mode", G.ROUND_NEAREST_EVEN)
        G.cast_f32_f16(ad, a16, mode)
        G.cast_f32_f16(bd, b16, mode)
        ad, bd = a16, b16
    M, N = A.shape[0], B.shape[1]
    C = kw.pop("C", None)
    cd = torch.from_numpy(C).to(dev) if C is not None else torch.empty((M, N), dtype=torch.float32, device=dev)
    bias = kw.pop("bias", None)
    bd_bias = torch.from_numpy(bias).to(dev) if bias is not None else None
    G.gemm(ad, bd, cd, transA=tA, transB=tB, bias=bd_bias, **kw)
    return cd.cpu().numpy()


def _nan_like(dev, M, N):
    """An output buffer filled with NaN, so a tile the kernel never writes fails the checks."""
    import torch

    return torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)


def _sum_invariants(A, B, C, tA=False, tB=False):
    """Whole-output checks in float64 on the device: row sums C.1 = op(A)(op(B).1) and column
    sums 1^T C = (1^T op(A)) op(B), each within 1e-5 relative (2-norm). A, B are the stored
    device operands (already rounded to their input precision), C the fp32 result. Every
    output element enters one row sum and one column sum, so a tile that is wrong, missing
    or written to the wrong place fails one of them (NaN fails both)."""
    import torch

    a = A.double()
    b = B.double()
    opA = a.t() if tA else a
    opB = b.t() if tB else b
    c = C.double()
    row_ref = opA @ opB.sum(dim=1)
    col_ref = opA.sum(dim=0) @ opB
    row_err = (torch.linalg.vector_norm(c.sum(dim=1) - row_ref) / torch.linalg.vector_norm(row_ref)).item()
    col_err = (torch.linalg.vector_norm(c.sum(dim=0) - col_ref) / torch.linalg.vector_norm(col_ref)).item()
    return row_err, col_err


# ------------------------------------------------------------------ fp32
@pytest.mark.parametrize("tA,tB", VARIANTS)
def test_f32_golden_small_all_transposes(dev, tA, tB):
    z = np.load(os.path.join(GOLD, "gemm_small.npz"))
    for key in ["1x1x1", "8x8x8", "3x5x7", "17x33x9", "64x48x40", "33x65x130"]:
        _say("f32 golden", key, tA, tB)
        C = _gemm_dev(dev, z[f"A_{key}"], z[f"B_{key}"], tA, tB, G.GN_F32)
        assert O.rel_frob(C, z[f"C64_{key}"]) <= 1e-5, key


def test_f32_c1_256_reference_abi(dev):
    """Config C1 through perform_mps_matrix_multiplication (metal_bridge.h:28-34)."""
    z = np.load(os.path.join(GOLD, "gemm_256.npz"))
    A, B = z["A"], z["B"]
    ba, bb, bc = G.Buffer.from_array(A), G.Buffer.from_array(B), G.Buffer(256 * 256 * 4)
    G.call("perform_mps_matrix_multiplication", ba.handle, 256, 256, bb.handle, 256, 256, bc.handle, 256, 256, None)
    C = bc.to_array((256, 256))
    err = O.rel_frob(C, z["C64"])
    _say("C1 relFrob", err)
    assert err <= 1e-5
    # the oracle generator's inputs too (seed 42, U[-1,1])
    A2, B2 = O.uniform((256, 256), 42, 1), O.uniform((256, 256), 42, 2)
    ba2, bb2 = G.Buffer.from_array(A2), G.Buffer.from_array(B2)
    G.call("perform_mps_matrix_multiplication", ba2.handle, 256, 256, bb2.handle, 256, 256, bc.handle, 256, 256, None)
    assert O.rel_frob(bc.to_array((256, 256)), O.gemm_f64(A2, B2)) <= 1e-5


def test_f32_closed_forms(dev):
    rng = np.random.default_rng(3)
    A = rng.integers(-8, 8, size=(96, 160)).astype(np.float32)
    B = rng.integers(-8, 8, size=(160, 72)).astype(np.float32)
    # small integers: every partial sum is exact in fp32, so the product is exact
    np.testing.assert_array_equal(_gemm_dev(dev, A, B, False, False, G.GN_F32), A.astype(np.float64) @ B)
    I = np.eye(160, dtype=np.float32)
    X = rng.standard_normal((96, 160)).astype(np.float32)
    np.testing.assert_array_equal(_gemm_dev(dev, X, I, False, False, G.GN_F32), X)
    P = np.eye(160, dtype=np.float32)[rng.permutation(160)]
    np.testing.assert_array_equal(_gemm_dev(dev, X, P, False, True, G.GN_F32), X @ P)


@pytest.mark.parametrize("tA,tB", VARIANTS)
def test_f32_c2_4096_all_transposes(dev, tA, tB):
    """Config C2: 4096^3, N(0,1), four transpose variants; rows sampled against float64."""
    n = 4096
    A = O.normal((n, n), 42, 11)
    B = O.normal((n, n), 42, 12)
    import torch

    _say("C2", tA, tB)
    ad = torch.from_numpy(_stored(A, tA)).to(dev)
    bd = torch.from_numpy(_stored(B, tB)).to(dev)
    cd = _nan_like(dev, n, n)
    G.gemm(ad, bd, cd, transA=tA, transB=tB)
    row_err, col_err = _sum_invariants(ad, bd, cd, tA, tB)
    _say("C2 row/col-sum relative errors", tA, tB, row_err, col_err)
    assert row_err <= 1e-5 and col_err <= 1e-5
    C = cd.cpu().numpy()
    rows = np.random.default_rng(7).choice(n, 48, replace=False)
    ref = O.gemm_f64_rows(A, B, rows)
    err = O.rel_frob(C[rows], ref)
    _say("C2 relFrob", tA, tB, err)
    assert err <= 1e-5
    assert np.isfinite(C).all()


@pytest.mark.parametrize("K", [32, 96])
def test_f32_ring_ragged_all_transposes_bit_identical(dev, K):
    """fp32 shapes that fill the CUs with one round of 256x256 ring tiles (16 x 16 of them). M
    and N are not multiples of 256 and K is one or three 32-deep K-tile pairs, so rows and
    columns past M, N must read as zeros and the pairs the ring issues past the end of K must
    not be used. Every tile is checked (NaN start, row and column sums), sampled rows against
    float64, and all four layouts agree bit for bit."""
    import torch

    rng = np.random.default_rng(K)
    M, N = 4000, 4000
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    outs = []
    for tA, tB in VARIANTS:
        _say("f32 ring ragged", K, tA, tB)
        ad = torch.from_numpy(_stored(A, tA)).to(dev)
        bd = torch.from_numpy(_stored(B, tB)).to(dev)
        cd = _nan_like(dev, M, N)
        G.gemm(ad, bd, cd, transA=tA, transB=tB)
        row_err, col_err = _sum_invariants(ad, bd, cd, tA, tB)
        assert row_err <= 1e-5 and col_err <= 1e-5, (tA, tB, row_err, col_err)
        outs.append(cd.cpu().numpy())
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])
    rows = np.concatenate([np.arange(0, 8), rng.choice(M, 16, replace=False), np.arange(M - 8, M)])
    err = O.rel_frob(outs[0][rows], O.gemm_f64_rows(A, B, rows))
    _say("f32 ring ragged relFrob", K, err)
    assert err <= 1e-5


@pytest.mark.parametrize("M,N,K", [(2000, 2010, 96), (2000, 4000, 96), (2000, 2100, 96), (600, 700, 64),
                                   (520, 1100, 96)])
def test_f32_ring_small_tiles_all_transposes_bit_identical(dev, M, N, K):
    """The fp32 ring's smaller tiles with ragged M, N and K of one or three 32-deep K-tile
    pairs: 128x128 with 8 waves (2000 x 2010: 256 tiles, one round), 128x128 with 4 waves
    (2000 x 4000: 512 tiles, two per CU), 64x64 (the other shapes; 2000 x 2100 has 1056 of
    them, 600 x 700 has 110, more than the small-product kernel takes). NaN start, row and
    column sums, rows against float64, all four layouts bit for bit."""
    import torch

    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    outs = []
    for tA, tB in VARIANTS:
        _say("f32 ring small tiles", M, N, K, tA, tB)
        ad = torch.from_numpy(_stored(A, tA)).to(dev)
        bd = torch.from_numpy(_stored(B, tB)).to(dev)
        cd = _nan_like(dev, M, N)
        G.gemm(ad, bd, cd, transA=tA, transB=tB)
        row_err, col_err = _sum_invariants(ad, bd, cd, tA, tB)
        assert row_err <= 1e-5 and col_err <= 1e-5, (tA, tB, row_err, col_err)
        outs.append(cd.cpu().numpy())
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])
    rows = np.unique(np.concatenate([np.arange(0, min(M, 6)), rng.choice(M, min(M, 10), replace=False),
                                     np.arange(max(0, M - 6), M)]))
    assert O.rel_frob(outs[0][rows], O.gemm_f64_rows(A, B, rows)) <= 1e-5


@pytest.mark.parametrize("M,N,K,pad", [(600, 700, 64, 4), (2000, 2100, 32, 8)])
def test_f32_ring_padded_leading_dims(dev, M, N, K, pad):
    """Leading dimensions wider than the rows (views into wider buffers, still 16-byte
    aligned) on the fp32 ring, all four layouts: the copies step by lda / ldb, not by the
    logical extent, and the columns past the view are never read."""
    import torch

    rng = np.random.default_rng(M + pad)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    ref_rows = np.unique(np.concatenate([np.arange(0, 6), rng.choice(M, 10, replace=False), np.arange(M - 6, M)]))
    ref = O.gemm_f64_rows(A, B, ref_rows)
    for tA, tB in VARIANTS:
        As, Bs = _stored(A, tA), _stored(B, tB)
        aw = torch.full((As.shape[0], As.shape[1] + pad), float("nan"), dtype=torch.float32, device=dev)
        bw = torch.full((Bs.shape[0], Bs.shape[1] + pad), float("nan"), dtype=torch.float32, device=dev)
        aw[:, :As.shape[1]] = torch.from_numpy(As).to(dev)
        bw[:, :Bs.shape[1]] = torch.from_numpy(Bs).to(dev)
        cd = _nan_like(dev, M, N)
        G.gemm(aw[:, :As.shape[1]], bw[:, :Bs.shape[1]], cd, transA=tA, transB=tB)
        C = cd.cpu().numpy()
        assert np.isfinite(C).all(), (tA, tB)
        assert O.rel_frob(C[ref_rows], ref) <= 1e-5, (tA, tB)


def test_f32_ring_small_tiles_batched(dev):
    """Batched strides on the 64x64 fp32 ring (6 x 256^2 x 64: 96 tiles)."""
    import torch

    rng = np.random.default_rng(47)
    bs, M, N, K = 6, 256, 256, 64
    A = rng.standard_normal((bs, M, K)).astype(np.float32)
    B = rng.standard_normal((bs, K, N)).astype(np.float32)
    C = torch.full((bs, M, N), float("nan"), dtype=torch.float32, device=dev)
    G.gemm(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), C, batch=bs, strideA=M * K, strideB=K * N,
           strideC=M * N)
    Cn = C.cpu().numpy()
    for z in range(bs):
        assert O.rel_frob(Cn[z], A[z].astype(np.float64) @ B[z]) <= 1e-5, z


@pytest.mark.parametrize("tA,tB", [(False, True), (True, True)])
def test_f32_ring_batched_alpha_beta_bias_act(dev, tA, tB):
    """Batched strides and the alpha / beta / bias / GELU epilogue on the fp32 ring
    (4 x 2048^2 x 128: 256 tiles of 256x256)."""
    import torch

    rng = np.random.default_rng(43)
    bs, M, N, K = 4, 2048, 2048, 128
    A = rng.standard_normal((bs, M, K)).astype(np.float32)
    B = rng.standard_normal((bs, K, N)).astype(np.float32)
    C0 = rng.standard_normal((bs, M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    As = np.ascontiguousarray(A.transpose(0, 2, 1)) if tA else A
    Bs = np.ascontiguousarray(B.transpose(0, 2, 1)) if tB else B
    ad, bd = torch.from_numpy(As).to(dev), torch.from_numpy(Bs).to(dev)
    C = torch.from_numpy(C0).to(dev)
    G.gemm(ad, bd, C, transA=tA, transB=tB, batch=bs, strideA=M * K, strideB=K * N, strideC=M * N, alpha=0.5,
           beta=0.25, bias=torch.from_numpy(bias).to(dev), act=G.ACT_GELU)
    Cn = C.cpu().numpy()
    rows = rng.choice(M, 12, replace=False)
    for z in range(bs):
        pre = 0.5 * O.gemm_f64_rows(A[z], B[z], rows) + 0.25 * C0[z][rows].astype(np.float64) + bias
        assert O.rel_frob(Cn[z][rows], O.act_f64(G.ACT_GELU, pre)) <= 1e-5, z


@pytest.mark.parametrize("M,N,K,tA,tB", [(1000, 1000, 1000, False, False), (1000, 1000, 1000, False, True),
                                           (1000, 1000, 1000, True, True), (600, 700, 100, False, False),
                                           (2000, 2012, 1001, True, False), (4000, 4000, 40, True, False),
                                           (2048, 2048, 36, False, True)])
def test_f32_k_tail_split_alpha_beta_bias_act(dev, M, N, K, tA, tB):
    """A K that is not a multiple of 32 runs as the ring over the first K - K % 32 and the
    register-staged kernel over the rest, the partial result passing through C: alpha, beta,
    bias and GELU must apply once. K = 1000, 100, 40 and 36 leave 8, 4, 8 and 4; TN takes any
    K (1001: a tail of 9). Every tile: NaN-free output and row sums against float64; sampled
    rows in full."""
    import torch

    rng = np.random.default_rng(K + M)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    ad = torch.from_numpy(_stored(A, tA)).to(dev)
    bd = torch.from_numpy(_stored(B, tB)).to(dev)
    C = torch.from_numpy(C0).to(dev)
    _say("f32 K tail", M, N, K, tA, tB)
    G.gemm(ad, bd, C, transA=tA, transB=tB, alpha=0.5, beta=0.25, bias=torch.from_numpy(bias).to(dev),
           act=G.ACT_GELU)
    Cn = C.cpu().numpy()
    assert np.isfinite(Cn).all()
    rows = np.concatenate([np.arange(0, 4), rng.choice(M, 12, replace=False), np.arange(M - 4, M)])
    pre = 0.5 * O.gemm_f64_rows(A, B, rows) + 0.25 * C0[rows].astype(np.float64) + bias
    assert O.rel_frob(Cn[rows], O.act_f64(G.ACT_GELU, pre)) <= 1e-5
    # the same product with no epilogue: whole-output row and column sums
    C2 = _nan_like(dev, M, N)
    G.gemm(ad, bd, C2, transA=tA, transB=tB)
    row_err, col_err = _sum_invariants(ad, bd, C2, tA, tB)
    assert row_err <= 1e-5 and col_err <= 1e-5, (row_err, col_err)


@pytest.mark.parametrize("dtype,M,N,K,tA,tB", [(G.GN_F16, 777, 1234, 4099, False, False), (G.GN_F16, 777, 1234, 4099, False, True),
                                                 (G.GN_F16, 777, 1234, 4099, True, False), (G.GN_F16, 777, 1234, 4099, True, True),
                                                 (G.GN_F32, 513, 1027, 999, False, False), (G.GN_F32, 513, 1027, 999, True, True),
                                                 (G.GN_F32, 1023, 1023, 1023, False, True), (G.GN_F32, 1023, 1023, 1023, True, False)])
def test_unaligned_packed_alpha_beta_bias_act(dev, dtype, M, N, K, tA, tB):
    """Operands whose rows are not 16-byte multiples are packed into zero-padded K-contiguous
    copies and multiplied on the aligned path: alpha, beta, bias and GELU against float64 of
    the rounded inputs on sampled rows, and whole-output row and column sums (no epilogue)."""
    import torch

    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    half = dtype == G.GN_F16
    ad = torch.from_numpy(_stored(A, tA)).to(dev)
    bd = torch.from_numpy(_stored(B, tB)).to(dev)
    if half:
        ad, bd = ad.half(), bd.half()
    Ar, Br = (O.round_f16(A, False), O.round_f16(B, False)) if half else (A, B)
    C = torch.from_numpy(C0).to(dev)
    _say("unaligned packed", dtype, M, N, K, tA, tB)
    G.gemm(ad, bd, C, transA=tA, transB=tB, alpha=0.5, beta=0.25, bias=torch.from_numpy(bias).to(dev), act=G.ACT_GELU)
    Cn = C.cpu().numpy()
    assert np.isfinite(Cn).all()
    rows = np.concatenate([np.arange(0, 4), rng.choice(M, 12, replace=False), np.arange(M - 4, M)])
    pre = 0.5 * O.gemm_f64_rows(Ar, Br, rows) + 0.25 * C0[rows].astype(np.float64) + bias
    assert O.rel_frob(Cn[rows], O.act_f64(G.ACT_GELU, pre)) <= 1e-5
    C2 = _nan_like(dev, M, N)
    G.gemm(ad, bd, C2, transA=tA, transB=tB)
    row_err, col_err = _sum_invariants(ad, bd, C2, tA, tB)
    assert row_err <= 1e-5 and col_err <= 1e-5, (row_err, col_err)


@pytest.mark.parametrize("dtype,M,N,K,tA,tB", [(G.GN_F16, 300, 1000, 8192, False, False), (G.GN_F16, 300, 1000, 8192, False, True),
                                                 (G.GN_F16, 300, 1000, 8192, True, False), (G.GN_F16, 300, 1000, 8192, True, True),
                                                 (G.GN_F32, 300, 1000, 8192, False, False), (G.GN_F32, 300, 1000, 8192, True, True),
                                                 (G.GN_F16, 512, 512, 16384, False, True), (G.GN_F32, 64, 4096, 4096, True, False)])
def test_splitk_alpha_beta_bias_act(dev, dtype, M, N, K, tA, tB):
    """Few output tiles and a long K: the product runs as slices of K into fp32 partial
    buffers and a reduce applies alpha, beta*C, bias and GELU. Every row against float64 of
    the rounded inputs, and whole-output row and column sums without the epilogue."""
    import torch

    rng = np.random.default_rng(M * 7 + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    half = dtype == G.GN_F16
    ad = torch.from_numpy(_stored(A, tA)).to(dev)
    bd = torch.from_numpy(_stored(B, tB)).to(dev)
    if half:
        ad, bd = ad.half(), bd.half()
    Ar, Br = (O.round_f16(A, False), O.round_f16(B, False)) if half else (A, B)
    C = torch.from_numpy(C0).to(dev)
    _say("split-K", dtype, M, N, K, tA, tB)
    G.gemm(ad, bd, C, transA=tA, transB=tB, alpha=0.5, beta=0.25, bias=torch.from_numpy(bias).to(dev), act=G.ACT_GELU)
    Cn = C.cpu().numpy()
    assert np.isfinite(Cn).all()
    rows = np.arange(M) if M * N * K <= (1 << 32) else rng.choice(M, 48, replace=False)
    pre = 0.5 * O.gemm_f64_rows(Ar, Br, rows) + 0.25 * C0[rows].astype(np.float64) + bias
    assert O.rel_frob(Cn[rows], O.act_f64(G.ACT_GELU, pre)) <= 1e-5
    C2 = _nan_like(dev, M, N)
    G.gemm(ad, bd, C2, transA=tA, transB=tB)
    row_err, col_err = _sum_invariants(ad, bd, C2, tA, tB)
    assert row_err <= 1e-5 and col_err <= 1e-5, (row_err, col_err)


@pytest.mark.parametrize("dtype", [G.GN_F16, G.GN_F32])
def test_splitk_layouts_bit_identical_and_repeatable(dev, dtype):
    """The slice count does not depend on the layout, and the partials are summed in slice
    order: all four transpose layouts of a split product, each called twice, give one result."""
    import torch

    rng = np.random.default_rng(91)
    M, N, K = 300, 1000, 8192
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    outs = []
    for tA, tB in VARIANTS:
        ad = torch.from_numpy(_stored(A, tA)).to(dev)
        bd = torch.from_numpy(_stored(B, tB)).to(dev)
        if dtype == G.GN_F16:
            ad, bd = ad.half(), bd.half()
        for _ in range(2):
            C = _nan_like(dev, M, N)
            G.gemm(ad, bd, C, transA=tA, transB=tB)
            outs.append(C.cpu().numpy())
    _say("split-K layouts", dtype, [bool(np.array_equal(o, outs[0])) for o in outs])
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


@pytest.mark.parametrize("dtype", [G.GN_F16, G.GN_F32])
def test_splitk_scalar_reduce_strided_c(dev, dtype):
    """Split-K into an output whose row length (N = 999) and pitch (ldc = 1004) rule out
    16-byte rows: the reduce takes its element-wise form, beta reads C through the pitch, and
    the columns between N and ldc keep their NaN sentinel."""
    import torch

    rng = np.random.default_rng(41)
    M, N, K, ldc = 200, 999, 8192, 1004
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    half = dtype == G.GN_F16
    ad, bd = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    if half:
        ad, bd = ad.half(), bd.half()
    Ar, Br = (O.round_f16(A, False), O.round_f16(B, False)) if half else (A, B)
    Cbig = torch.full((M, ldc), float("nan"), dtype=torch.float32, device=dev)
    Cbig[:, :N] = torch.from_numpy(C0).to(dev)
    C = Cbig[:, :N]
    assert C.stride(0) == ldc
    _say("split-K scalar reduce", dtype, M, N, K, ldc)
    G.gemm(ad, bd, C, alpha=2.0, beta=-0.5, act=G.ACT_RELU)
    out = Cbig.cpu().numpy()
    assert np.isnan(out[:, N:]).all()
    ref = np.maximum(2.0 * O.gemm_f64_rows(Ar, Br, np.arange(M)) - 0.5 * C0.astype(np.float64), 0.0)
    assert O.rel_frob(out[:, :N], ref) <= 1e-5


def test_splitk_linear_backward_shape_relu(dev):
    """grad_input = G W^T of the 512 x 11008 -> 4096 linear layer (fp16, K = 11008 split in
    four), ReLU epilogue: sampled rows against float64 and whole-output sums."""
    import torch

    rng = np.random.default_rng(23)
    M, N, K = 512, 4096, 11008
    Gd = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev).half()
    W = torch.from_numpy((0.02 * rng.standard_normal((N, K))).astype(np.float32)).to(dev).half()
    C = _nan_like(dev, M, N)
    G.gemm(Gd, W, C, transB=True, act=G.ACT_RELU)
    Cn = C.cpu().numpy()
    rows = np.concatenate([np.arange(0, 4), rng.choice(M, 12, replace=False), np.arange(M - 4, M)])
    Ar = Gd.float().cpu().numpy()
    Br = W.float().cpu().numpy().T.copy()
    assert O.rel_frob(Cn[rows], np.maximum(O.gemm_f64_rows(Ar, Br, rows), 0.0)) <= 1e-5
    C2 = _nan_like(dev, M, N)
    G.gemm(Gd, W, C2, transB=True)
    row_err, col_err = _sum_invariants(Gd, W, C2, False, True)
    assert row_err <= 1e-5 and col_err <= 1e-5, (row_err, col_err)


def test_splitk_shape_under_graph_capture(dev):
    """Under HIP graph capture the split (whose scratch may need an allocation) is not taken:
    the captured product replays within tolerance of float64, the same on every replay."""
    import torch

    rng = np.random.default_rng(29)
    M, N, K = 300, 1000, 8192
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    ad = torch.from_numpy(A).to(dev).half()
    bd = torch.from_numpy(B).to(dev).half()
    C = torch.empty(M, N, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        G.gemm(ad, bd, C)  # eager, split
    torch.cuda.synchronize()
    eager = C.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        G.gemm(ad, bd, C)
    torch.cuda.synchronize()
    ref = O.gemm_f64_rows(O.round_f16(A, False), O.round_f16(B, False), np.arange(M))
    reps = []
    for rep in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        reps.append(C.cpu().numpy())
        _say("captured split-K shape, replay", rep)
        assert O.rel_frob(reps[-1], ref) <= 1e-5
    for r in reps[1:]:
        np.testing.assert_array_equal(r, reps[0])
    assert O.rel_frob(eager.cpu().numpy(), ref) <= 1e-5


def test_unaligned_packed_batched_and_offset_pointer(dev):
    """The packed path with a batch (strides of unaligned rows) and an aligned shape whose A
    starts one element into its buffer (so no 16-byte loads), fp32 and fp16."""
    import torch

    rng = np.random.default_rng(17)
    bs, M, N, K = 3, 300, 500, 257
    A = rng.standard_normal((bs, M, K)).astype(np.float32)
    B = rng.standard_normal((bs, K, N)).astype(np.float32)
    C = _nan_like(dev, bs * M, N).reshape(bs, M, N)
    G.gemm(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), C, batch=bs, strideA=M * K, strideB=K * N,
           strideC=M * N)
    Cn = C.cpu().numpy()
    for z in range(bs):
        assert O.rel_frob(Cn[z], A[z].astype(np.float64) @ B[z]) <= 1e-5, z
    for half in (False, True):
        M, N, K = 1024, 1024, 512
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
        buf = torch.zeros(M * K + 1, dtype=torch.float32, device=dev)
        buf[1:] = torch.from_numpy(A.reshape(-1)).to(dev)
        if half:
            buf = buf.half()
        ad = buf[1:].view(M, K)
        bd = torch.from_numpy(B).to(dev)
        bd = bd.half() if half else bd
        C = _nan_like(dev, M, N)
        G.gemm(ad, bd, C)
        Ar, Br = (O.round_f16(A, False), O.round_f16(B, False)) if half else (A, B)
        rows = rng.choice(M, 16, replace=False)
        assert O.rel_frob(C.cpu().numpy()[rows], O.gemm_f64_rows(Ar, Br, rows)) <= 1e-5, half


def test_unaligned_gemm_under_graph_capture(dev):
    """Under HIP graph capture an unaligned GEMM takes the element-wise-load kernel (the
    packed path's scratch could need an allocation): the captured graph replays correctly."""
    import torch

    rng = np.random.default_rng(23)
    M, N, K = 777, 1234, 1027
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    ad = torch.from_numpy(A).to(dev).half()
    bd = torch.from_numpy(B).to(dev).half()
    C = _nan_like(dev, M, N)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        G.gemm(ad, bd, C)
    torch.cuda.synchronize()
    rows = rng.choice(M, 16, replace=False)
    for rep in range(2):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        Cn = C.cpu().numpy()
        assert np.isfinite(Cn).all(), rep
        err = O.rel_frob(Cn[rows], O.gemm_f64_rows(O.round_f16(A, False), O.round_f16(B, False), rows))
        assert err <= 1e-5, (rep, err)


def test_f32_transpose_variants_bit_identical(dev):
    """All four load paths feed MFMA the same operands in the same order."""
    rng = np.random.default_rng(5)
    A = rng.standard_normal((640, 384)).astype(np.float32)
    B = rng.standard_normal((384, 512)).astype(np.float32)
    outs = [_gemm_dev(dev, A, B, tA, tB, G.GN_F32) for tA, tB in VARIANTS]
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


def test_f32_alpha_beta_bias_activation(dev):
    rng = np.random.default_rng(9)
    A = rng.standard_normal((130, 70)).astype(np.float32)
    B = rng.standard_normal((70, 90)).astype(np.float32)
    C0 = rng.standard_normal((130, 90)).astype(np.float32)
    bias = rng.standard_normal(90).astype(np.float32)
    base = A.astype(np.float64) @ B
    out = _gemm_dev(dev, A, B, False, False, G.GN_F32, alpha=0.5, beta=-1.5, C=C0)
    assert O.rel_frob(out, 0.5 * base - 1.5 * C0) <= 1e-5
    for act, alpha in [(G.ACT_RELU, 0.0), (G.ACT_GELU, 0.0), (G.ACT_SIGMOID, 0.0), (G.ACT_TANH, 0.0),
                       (G.ACT_LEAKY_RELU, 0.1), (G.ACT_ELU, 1.0), (G.ACT_SWISH, 0.0)]:
        out = _gemm_dev(dev, A, B, False, False, G.GN_F32, bias=bias, act=act, act_alpha=alpha)
        ref = O.act_f64(act, base + bias, alpha)
        assert O.rel_frob(out, ref) <= 1e-5, act


def test_f32_unaligned_leading_dims_and_batch(dev):
    import torch

    rng = np.random.default_rng(11)
    # leading dimensions larger than the row length (views into wider buffers)
    Aw = torch.from_numpy(rng.standard_normal((50, 37)).astype(np.float32)).to(dev)
    Bw = torch.from_numpy(rng.standard_normal((29, 45)).astype(np.float32)).to(dev)
    A, B = Aw[:, :29], Bw[:, :41]
    C = torch.zeros((50, 41), dtype=torch.float32, device=dev)
    G.gemm(A, B, C)
    ref = A.cpu().numpy().astype(np.float64) @ B.cpu().numpy().astype(np.float64)
    assert O.rel_frob(C.cpu().numpy(), ref) <= 1e-5
    # strided batch through perform_batch_matmul_optimized (metal_bridge.h:1432-1437)
    bs, M, N, K = 3, 33, 20, 17
    A3 = rng.standard_normal((bs, M, K)).astype(np.float32)
    B3 = rng.standard_normal((bs, K, N)).astype(np.float32)
    ba, bb, bc = G.Buffer.from_array(A3), G.Buffer.from_array(B3), G.Buffer(bs * M * N * 4)
    G.call("perform_batch_matmul_optimized", ba.handle, bb.handle, bc.handle, bs, M, N, K, None)
    C3 = bc.to_array((bs, M, N))
    for i in range(bs):
        assert O.rel_frob(C3[i], A3[i].astype(np.float64) @ B3[i]) <= 1e-5


# Products the fp32 small-product kernel takes (at most 64 tiles of 64 x 64), one per shape
# of it: 16 x 16 workgroup tiles with 4 / 8 / 16 K-splitting waves, 32 x 32 tiles with 4 / 8.
SMALL_SHAPES = [
    (256, 256, 256),   # config C1: 256 tiles of 16 x 16, 4 waves
    (37, 53, 71),      # ragged M, N and a K tail inside a 16-element step
    (17, 200, 5),      # K shorter than one step
    (100, 100, 500),   # 8 waves
    (64, 128, 784),    # 16 waves
    (512, 512, 256),   # 32 x 32 tiles, 4 waves
    (384, 384, 1024),  # 32 x 32 tiles, 8 waves
    (512, 512, 32),    # K of two steps: 16 x 16 tiles, 1024 workgroups
    (16, 16, 16384),   # long K under 2^24 multiply-adds
    (128, 128, 4096),  # 4 tiles of 64 x 64, K up to 4096
]


# The fp16 kernel's shapes (16 x 16 tiles, at most 16 tiles of 64 x 64): 4, 8 and 16 waves.
SMALL_SHAPES_F16 = [
    (37, 53, 71),      # 4 waves, ragged, K tail inside a 32-element step
    (17, 200, 5),      # K shorter than one step
    (256, 256, 256),   # 8 waves
    (100, 130, 1000),  # 16 waves
    (64, 128, 784),    # 16 waves
    (16, 16, 4096),    # long K under 2^24 multiply-adds
]


@pytest.mark.parametrize("dtype,M,N,K", [(G.GN_F32,) + s for s in SMALL_SHAPES] +
                         [(G.GN_F16,) + s for s in SMALL_SHAPES_F16])
def test_small_kernel_all_layouts_aligned_or_not(dev, dtype, M, N, K):
    """The small-product kernel: NaN start, the whole output against float64 of the stored
    (for fp16 the rounded) operands (relFrob 1e-5), all four layouts bit for bit, and the
    unaligned loads (leading dimensions one wider than the rows, so no 16-byte vectors) bit
    for bit with the aligned ones: each element's summation order depends on K alone."""
    import torch

    tdt = torch.float16 if dtype == G.GN_F16 else torch.float32
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    if dtype == G.GN_F16:
        A, B = A.astype(np.float16).astype(np.float32), B.astype(np.float16).astype(np.float32)
    ref = A.astype(np.float64) @ B
    outs = []
    for pad in (0, 1):
        for tA, tB in VARIANTS:
            _say("small kernel", dtype, M, N, K, tA, tB, "pad", pad)
            As, Bs = _stored(A, tA), _stored(B, tB)
            aw = torch.full((As.shape[0], As.shape[1] + pad), float("nan"), dtype=tdt, device=dev)
            bw = torch.full((Bs.shape[0], Bs.shape[1] + pad), float("nan"), dtype=tdt, device=dev)
            aw[:, :As.shape[1]] = torch.from_numpy(As).to(dev).to(tdt)
            bw[:, :Bs.shape[1]] = torch.from_numpy(Bs).to(dev).to(tdt)
            cd = _nan_like(dev, M, N)
            G.gemm(aw[:, :As.shape[1]], bw[:, :Bs.shape[1]], cd, transA=tA, transB=tB, dtype=dtype)
            C = cd.cpu().numpy()
            err = O.rel_frob(C, ref)
            assert err <= 1e-5, (tA, tB, pad, err)
            outs.append(C)
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


@pytest.mark.parametrize("tA,tB", VARIANTS)
@pytest.mark.parametrize("dtype", [G.GN_F32, G.GN_F16])
def test_small_kernel_batched_alpha_beta_bias_act(dev, dtype, tA, tB):
    """Batched strides and the alpha / beta / bias / activation epilogue on the small-product
    kernel (5 x 96 x 80 x 300: 20 tiles of 64 x 64 in fp32, too many for the fp16 rule; 3 x 96
    x 80 x 300: 12; and in fp32 4 x 200 x 150 x 40 on 32 x 32 tiles), against float64 of the
    stored operands with the oracle's activation formulas."""
    import torch

    tdt = torch.float16 if dtype == G.GN_F16 else torch.float32
    cases = [(5, 96, 80, 300), (4, 200, 150, 40)] if dtype == G.GN_F32 else [(3, 96, 80, 300)]
    for bs, M, N, K in cases:
        rng = np.random.default_rng(bs + M + K)
        A = rng.standard_normal((bs, M, K)).astype(np.float32)
        B = rng.standard_normal((bs, K, N)).astype(np.float32)
        if dtype == G.GN_F16:
            A, B = A.astype(np.float16).astype(np.float32), B.astype(np.float16).astype(np.float32)
        C0 = rng.standard_normal((bs, M, N)).astype(np.float32)
        bias = rng.standard_normal(N).astype(np.float32)
        As = np.ascontiguousarray(A.transpose(0, 2, 1)) if tA else A
        Bs = np.ascontiguousarray(B.transpose(0, 2, 1)) if tB else B
        ad, bd = torch.from_numpy(As).to(dev).to(tdt), torch.from_numpy(Bs).to(dev).to(tdt)
        base = np.einsum("zmk,zkn->zmn", A.astype(np.float64), B.astype(np.float64))
        for act, aa in [(G.ACT_NONE, 0.0), (G.ACT_RELU, 0.0), (G.ACT_GELU, 0.0), (G.ACT_LEAKY_RELU, 0.1)]:
            _say("small kernel epilogue", dtype, bs, M, N, K, tA, tB, act)
            C = torch.from_numpy(C0).to(dev)
            G.gemm(ad, bd, C, transA=tA, transB=tB, alpha=0.75, beta=-0.5, bias=torch.from_numpy(bias).to(dev),
                   act=act, act_alpha=aa, M=M, N=N, K=K, batch=bs, strideA=M * K, strideB=K * N, strideC=M * N,
                   dtype=dtype)
            pre = 0.75 * base - 0.5 * C0 + bias
            ref = pre if act == G.ACT_NONE else O.act_f64(act, pre, aa)
            assert O.rel_frob(C.cpu().numpy(), ref) <= 1e-5, (bs, M, act)


@pytest.mark.parametrize("dtype,M,N,K", [(G.GN_F32, 1, 4096, 2048), (G.GN_F32, 2, 2048, 3000),
                                         (G.GN_F32, 8, 4100, 4096), (G.GN_F32, 13, 11008, 2048),
                                         (G.GN_F16, 1, 2048, 4096), (G.GN_F16, 2, 11008, 2048),
                                         (G.GN_F16, 16, 4096, 2056), (G.GN_F16, 5, 3001, 2048)])
def test_skinny_linear_layer_all_layouts(dev, dtype, M, N, K):
    """Skinny products Y = act(X W^T + b) (a few rows, W of N x K): in the NT layout (W
    K-contiguous) they run the small-product kernel with 4 to 16 K-splitting waves, in the
    other layouts the tiled kernels. NaN start, bias + ReLU and then alpha / beta, each layout
    against float64 of the stored operands (relFrob 1e-5), and the layouts against each other
    within the same bar (they sum K in different orders)."""
    import torch

    tdt = torch.float16 if dtype == G.GN_F16 else torch.float32
    rng = np.random.default_rng(M * 11 + N + K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    if dtype == G.GN_F16:
        X, W = X.astype(np.float16).astype(np.float32), W.astype(np.float16).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    pre = X.astype(np.float64) @ W.T.astype(np.float64)
    outs = []
    for tA, tB in VARIANTS:
        _say("skinny", dtype, M, N, K, tA, tB)
        ad = torch.from_numpy(_stored(X, tA)).to(dev).to(tdt)
        bd = torch.from_numpy(W if tB else np.ascontiguousarray(W.T)).to(dev).to(tdt)
        cd = _nan_like(dev, M, N)
        G.gemm(ad, bd, cd, transA=tA, transB=tB, bias=torch.from_numpy(bias).to(dev), act=G.ACT_RELU, dtype=dtype)
        C = cd.cpu().numpy()
        assert O.rel_frob(C, np.maximum(pre + bias, 0.0)) <= 1e-5, (tA, tB)
        outs.append(C)
        cd = torch.from_numpy(C0).to(dev)
        G.gemm(ad, bd, cd, transA=tA, transB=tB, alpha=-0.5, beta=2.0, dtype=dtype)
        assert O.rel_frob(cd.cpu().numpy(), -0.5 * pre + 2.0 * C0) <= 1e-5, (tA, tB)
    for o in outs[1:]:
        assert O.rel_frob(o, outs[0]) <= 1e-5


@pytest.mark.parametrize("dtype,M,N,K", [(G.GN_F32, 1, 4096, 4096), (G.GN_F32, 2, 8192, 2048),
                                         (G.GN_F32, 3, 11008, 1000), (G.GN_F32, 4, 16384, 777),
                                         (G.GN_F16, 1, 2048, 2048), (G.GN_F16, 2, 1024, 3001),
                                         (G.GN_F16, 2, 8200, 1024), (G.GN_F16, 4, 16384, 515)])
def test_gemv_nn_rows_all_layouts(dev, dtype, M, N, K):
    """Products of 1-4 rows with W stored K x N (NN, the reference LinearLayer's input @ Weight)
    run on the GEMV kernel (K split over 16 waves, fp32 sums on the VALU). NaN start; bias +
    GELU, then alpha / beta with a prior C, each against float64 of the stored operands (relFrob
    1e-5); the same product in the other layouts (other kernels, other summation orders) within
    the same bar; and two runs bit for bit."""
    import torch

    tdt = torch.float16 if dtype == G.GN_F16 else torch.float32
    rng = np.random.default_rng(M * 13 + N + K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    if dtype == G.GN_F16:
        X, W = X.astype(np.float16).astype(np.float32), W.astype(np.float16).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    pre = X.astype(np.float64) @ W.astype(np.float64)
    outs = []
    for tA, tB in VARIANTS:
        _say("gemv nn", dtype, M, N, K, tA, tB)
        ad = torch.from_numpy(_stored(X, tA)).to(dev).to(tdt)
        bd = torch.from_numpy(_stored(W, tB)).to(dev).to(tdt)
        cd = _nan_like(dev, M, N)
        G.gemm(ad, bd, cd, transA=tA, transB=tB, bias=torch.from_numpy(bias).to(dev), act=G.ACT_GELU, dtype=dtype)
        C = cd.cpu().numpy()
        assert O.rel_frob(C, O.act_f64(G.ACT_GELU, pre + bias, 0.0)) <= 1e-5, (tA, tB)
        outs.append(C)
        if not tA and not tB:
            cd2 = _nan_like(dev, M, N)
            G.gemm(ad, bd, cd2, transA=tA, transB=tB, bias=torch.from_numpy(bias).to(dev), act=G.ACT_GELU,
                   dtype=dtype)
            np.testing.assert_array_equal(cd2.cpu().numpy(), C)
        cd = torch.from_numpy(C0).to(dev)
        G.gemm(ad, bd, cd, transA=tA, transB=tB, alpha=1.5, beta=-1.0, dtype=dtype)
        assert O.rel_frob(cd.cpu().numpy(), 1.5 * pre - C0) <= 1e-5, (tA, tB)
    for o in outs[1:]:
        assert O.rel_frob(o, outs[0]) <= 1e-5


def test_f32_k_zero_and_empty(dev):
    import torch

    A = torch.zeros((4, 0), dtype=torch.float32, device=dev)
    B = torch.zeros((0, 3), dtype=torch.float32, device=dev)
    C = torch.full((4, 3), 7.0, dtype=torch.float32, device=dev)
    G.gemm(A, B, C, K=0)
    assert torch.count_nonzero(C).item() == 0
    bias = torch.arange(3, dtype=torch.float32, device=dev)
    G.gemm(A, B, C, K=0, bias=bias, act=G.ACT_RELU)
    np.testing.assert_array_equal(C.cpu().numpy(), np.tile(np.arange(3, dtype=np.float32), (4, 1)))


# ------------------------------------------------------------------ fp16 cast
def test_cast_f32_f16_bit_exact(dev):
    import json

    import torch

    rng = np.random.default_rng(13)
    mag = np.exp2(rng.uniform(-27, 17, size=1 << 20)).astype(np.float32)
    x = (mag * rng.choice([-1, 1], size=mag.size)).astype(np.float32)
    t = json.load(open(os.path.join(GOLD, "f16_table.json")))
    special = np.array([int(c["f32"], 16) for c in t["cases"]], dtype=np.uint32).view(np.float32)
    x = np.concatenate([special, x, special[:3]])  # odd length: exercises the scalar path too
    xd = torch.from_numpy(x).to(dev)
    for mode in (G.ROUND_NEAREST_EVEN, G.ROUND_TOWARD_ZERO):
        for arr in (xd, xd[: (xd.numel() // 4) * 4]):
            out = torch.empty(arr.shape, dtype=torch.float16, device=dev)
            G.cast_f32_f16(arr, out, mode)
            got = out.cpu().numpy().view(np.uint16)
            ref = O.f32_to_f16_bits(arr.cpu().numpy(), rtz=bool(mode))
            nan = np.isnan(arr.cpu().numpy())
            if mode == G.ROUND_NEAREST_EVEN:
                np.testing.assert_array_equal(got[~nan], ref[~nan])
                assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)
            else:
                np.testing.assert_array_equal(got, ref)  # incl. the reference's NaN/overflow handling
    # f16 -> f32 widening over all patterns
    allh = torch.from_numpy(np.arange(65536, dtype=np.int32).astype(np.uint16).view(np.int16)).to(dev)
    out = torch.empty(65536, dtype=torch.float32, device=dev)
    G.cast_f16_f32(allh.view(torch.float16), out)
    ref = O.f16_bits_to_f32(np.arange(65536, dtype=np.int32).astype(np.uint16))
    got = out.cpu().numpy()
    nan = np.isnan(ref)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


# ------------------------------------------------------------------ fp16 GEMM
@pytest.mark.parametrize("tA,tB", VARIANTS)
def test_f16_golden_small_all_transposes(dev, tA, tB):
    z = np.load(os.path.join(GOLD, "gemm_small.npz"))
    for key in ["1x1x1", "8x8x8", "3x5x7", "17x33x9", "64x48x40", "33x65x130"]:
        A, B = z[f"A_{key}"], z[f"B_{key}"]
        C = _gemm_dev(dev, A, B, tA, tB, G.GN_F16)
        assert O.rel_frob(C, z[f"C64_{key}"]) <= 2e-2, key
        ref_r = O.gemm_f64(O.round_f16(A, False), O.round_f16(B, False))
        assert O.rel_frob(C, ref_r) <= 1e-5, key


@pytest.mark.parametrize("tA,tB", VARIANTS)
def test_f16_medium_all_transposes_rne_and_rtz(dev, tA, tB):
    rng = np.random.default_rng(17)
    A = rng.standard_normal((768, 1024)).astype(np.float32)
    B = (0.02 * rng.standard_normal((1024, 640))).astype(np.float32)
    for rtz in (False, True):
        mode = G.ROUND_TOWARD_ZERO if rtz else G.ROUND_NEAREST_EVEN
        C = _gemm_dev(dev, A, B, tA, tB, G.GN_F16, round_mode=mode)
        assert O.rel_frob(C, O.gemm_f64(A, B)) <= 2e-2
        assert O.rel_frob(C, O.gemm_f64(O.round_f16(A, rtz), O.round_f16(B, rtz))) <= 1e-5


def test_f16_transpose_variants_bit_identical(dev):
    rng = np.random.default_rng(19)
    A = rng.standard_normal((512, 576)).astype(np.float32)
    B = rng.standard_normal((576, 768)).astype(np.float32)
    outs = [_gemm_dev(dev, A, B, tA, tB, G.GN_F16) for tA, tB in VARIANTS]
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


def test_f16_c3_8192(dev):
    """Config C3: 8192^3, A ~ N(0,1), B ~ N(0,0.02^2), cast to fp16 (RNE); rows sampled."""
    import torch

    n = 8192
    ad = torch.empty((n, n), dtype=torch.float32, device=dev)
    bd = torch.empty((n, n), dtype=torch.float32, device=dev)
    G.fill_normal(ad, 42, 21, 0.0, 1.0)
    G.fill_normal(bd, 42, 22, 0.0, 0.02)
    a16 = torch.empty((n, n), dtype=torch.float16, device=dev)
    b16 = torch.empty((n, n), dtype=torch.float16, device=dev)
    G.cast_f32_f16(ad, a16)
    G.cast_f32_f16(bd, b16)
    C = _nan_like(dev, n, n)
    _say("C3 gemm")
    G.gemm(a16, b16, C)
    row_err, col_err = _sum_invariants(a16, b16, C)
    _say("C3 row/col-sum relative errors", row_err, col_err)
    assert row_err <= 1e-5 and col_err <= 1e-5
    rows = np.random.default_rng(23).choice(n, 16, replace=False)
    A = ad.cpu().numpy()
    B = bd.cpu().numpy()
    Cr = C[torch.from_numpy(rows).to(dev)].cpu().numpy()
    err = O.rel_frob(Cr, O.gemm_f64_rows(A, B, rows))
    err_r = O.rel_frob(Cr, O.gemm_f64_rows(O.round_f16(A[rows], False), O.round_f16(B, False), np.arange(16)))
    _say("C3 relFrob vs fp32 inputs", err, "vs fp16-rounded inputs", err_r)
    assert err <= 2e-2 and err_r <= 1e-5
    assert torch.isfinite(C).all().item()


@pytest.mark.parametrize("act", [G.ACT_RELU, G.ACT_GELU])
def test_f16_c4_fused_linear(dev, act):
    """Config C4: Y = act(X W^T + b), X 512x4096, W 11008x4096 (fp16), b fp32."""
    import torch

    X = O.normal((512, 4096), 42, 31)
    W = O.normal((11008, 4096), 42, 32, 0.0, 0.02)
    b = O.normal((11008,), 42, 33, 0.0, 0.01)
    x16 = torch.empty((512, 4096), dtype=torch.float16, device=dev)
    w16 = torch.empty((11008, 4096), dtype=torch.float16, device=dev)
    G.cast_f32_f16(torch.from_numpy(X).to(dev), x16)
    G.cast_f32_f16(torch.from_numpy(W).to(dev), w16)
    bd = torch.from_numpy(b).to(dev)
    Yd = _nan_like(dev, 512, 11008)
    G.gemm(x16, w16, Yd, transB=True, bias=bd, act=act)
    # Whole output: the pre-activation's row / column sums (the epilogue's input) cannot be
    # read back, so every element is compared with act(X16 W16^T + b) from a float64
    # product of the same fp16 operands on the device (relative Frobenius error).
    pre64 = x16.double() @ w16.double().t().contiguous() + bd.double()
    ref64 = torch.relu(pre64) if act == G.ACT_RELU else torch.from_numpy(O.act_f64(act, pre64.cpu().numpy())).to(dev)
    full_err = (torch.linalg.matrix_norm(Yd.double() - ref64) / torch.linalg.matrix_norm(ref64)).item()
    _say("C4", act, "whole-output relFrob vs float64 of the fp16 operands", full_err)
    assert full_err <= 1e-5
    Y = Yd.cpu().numpy()
    assert Y.shape == (512, 11008)
    assert np.isfinite(Y).all()
    rows = np.arange(0, 512, 37)
    pre = O.gemm_f64_rows(X, W, rows, transB=True) + b
    ref = O.act_f64(act, pre)
    err = O.rel_frob(Y[rows], ref)
    _say("C4", act, "relFrob", err)
    assert err <= 2e-2
    pre_r = O.gemm_f64_rows(O.round_f16(X[rows], False), O.round_f16(W, False), np.arange(rows.size), transB=True) + b
    ref_r = np.maximum(pre_r, 0) if act == G.ACT_RELU else O.act_f64(act, pre_r)
    assert O.rel_frob(Y[rows], ref_r) <= 1e-5


def test_fused_linear_reference_abi(dev):
    """perform_fused_linear_activation (metal_bridge.h:1348-1353): W is [in, out]."""
    rng = np.random.default_rng(29)
    X = rng.standard_normal((40, 96)).astype(np.float32)
    W = rng.standard_normal((96, 70)).astype(np.float32)
    b = rng.standard_normal(70).astype(np.float32)
    bx, bw, bb, by = G.Buffer.from_array(X), G.Buffer.from_array(W), G.Buffer.from_array(b), G.Buffer(40 * 70 * 4)
    for act in (0, 7, 1, 2, 4, 5, 6):
        G.call("perform_fused_linear_activation", bx.handle, 40, 96, bw.handle, 70, bb.handle, act, 0.2, by.handle, None)
        Y = by.to_array((40, 70))
        assert O.rel_frob(Y, O.linear_f64(X, W, b, act, 0, alpha=0.2)) <= 1e-5, act
    # bias omitted (nullable)
    G.call("perform_fused_linear_activation", bx.handle, 40, 96, bw.handle, 70, None, 0, 0.0, by.handle, None)
    assert O.rel_frob(by.to_array((40, 70)), O.linear_f64(X, W, None, 0, 0)) <= 1e-5
    # Softmax (3) is not an element-wise epilogue
    rc, msg = G.call_rc("perform_fused_linear_activation", bx.handle, 40, 96, bw.handle, 70, None, 3, 0.0, by.handle,
                        None)
    assert rc == -1


def test_fused_linear_nil_activation_call_sequence(dev):
    """The reference's FusedLinearActivation.Forward with config.Activation == nil sends
    C.int(OpReLU) and alpha 0 (fused-operations.go:433-434). OpReLU is 6 in the OpType enum
    (gradient.go:27-39). The reference kernel would read 6 as no activation
    (default.metal:488-506, codes 0-4 only); this entry reads every code as an ActivationType
    (activation.go:20-29), where 6 is Swish. The unchanged call therefore runs Swish here; the
    one-line Go edit of the integration (ActivationType ReLU, 0) runs ReLU, the comment's
    "Default to ReLU", a deliberate deviation from the kernel's identity."""
    rng = np.random.default_rng(31)
    X = rng.standard_normal((24, 64)).astype(np.float32)
    W = rng.standard_normal((64, 40)).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    bx, bw, bb, by = G.Buffer.from_array(X), G.Buffer.from_array(W), G.Buffer.from_array(b), G.Buffer(24 * 40 * 4)
    op_relu = 6  # OpReLU: OpAdd, OpSub, OpMul, OpDiv, OpMatMul, OpTranspose, OpReLU
    G.call("perform_fused_linear_activation", bx.handle, 24, 64, bw.handle, 40, bb.handle, op_relu, 0.0, by.handle,
           None)
    Y6 = by.to_array((24, 40))
    swish = O.linear_f64(X, W, b, G.ACT_SWISH, 0)
    assert O.rel_frob(Y6, swish) <= 1e-5
    assert O.rel_frob(Y6, O.linear_f64(X, W, b, G.ACT_RELU, 0)) > 1e-2  # not ReLU: the Go edit is needed
    G.call("perform_fused_linear_activation", bx.handle, 24, 64, bw.handle, 40, bb.handle, G.ACT_RELU, 0.0, by.handle,
           None)
    Y0 = by.to_array((24, 40))
    assert O.rel_frob(Y0, O.linear_f64(X, W, b, G.ACT_RELU, 0)) <= 1e-5
    assert (Y0 >= 0).all()
    for buf in (bx, bw, bb, by):
        buf.release()


# ------------------------------------------------------------------ fp16 ring kernel (large aligned shapes)
@pytest.mark.parametrize("M,N", [(4000, 4000), (2500, 2600)])
@pytest.mark.parametrize("tA,tB", VARIANTS)
def test_f16_ring_ragged_all_transposes(dev, tA, tB, M, N):
    """The ring kernel at 256x256 tiles (4000 x 4000: one round of 256) and at 128x128 tiles
    with two workgroups per CU (2500 x 2600: 420 tiles), M, N not multiples of the tile and K
    not a multiple of the 32-deep K tile: out-of-range rows, columns and the K tail must read
    as zeros."""
    rng = np.random.default_rng(31)
    K = 1000
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    C = _gemm_dev(dev, A, B, tA, tB, G.GN_F16)
    rows = np.concatenate([np.arange(0, 16), rng.choice(M, 24, replace=False), np.arange(M - 16, M)])
    ref_r = O.gemm_f64_rows(O.round_f16(A[rows], False), O.round_f16(B, False), np.arange(rows.size))
    err = O.rel_frob(C[rows], ref_r)
    _say("ring ragged", tA, tB, err)
    assert err <= 1e-5
    assert np.isfinite(C).all()


@pytest.mark.parametrize("M,N,K", [(4000, 4000, 1000), (4096, 4096, 4096)])
def test_f16_mfma32_variant_nn(dev, monkeypatch, M, N, K):
    """GONNGPU_F16_MFMA32=1 runs NN products on the 256x256 tiles through the 32x32x16 MFMA
    kernel (kept for measurement). Ragged M, N and a K tail (4000 x 4000 x 1000, one round of
    256 tiles) and a square case: sampled rows within 1e-5 of the float64 product of the
    rounded inputs, whole-output row and column sums from a NaN-filled output, and the same
    bits as the 16x16x32 kernel (the matrix unit accumulates K in the same order for both
    instruction shapes)."""
    import torch

    rng = np.random.default_rng(53)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    base = _gemm_dev(dev, A, B, False, False, G.GN_F16)
    monkeypatch.setenv("GONNGPU_F16_MFMA32", "1")
    a16 = torch.empty((M, K), dtype=torch.float16, device=dev)
    b16 = torch.empty((K, N), dtype=torch.float16, device=dev)
    G.cast_f32_f16(torch.from_numpy(A).to(dev), a16)
    G.cast_f32_f16(torch.from_numpy(B).to(dev), b16)
    cd = _nan_like(dev, M, N)
    G.gemm(a16, b16, cd)
    torch.cuda.synchronize()
    row_err, col_err = _sum_invariants(a16, b16, cd)
    C = cd.cpu().numpy()
    rows = np.concatenate([np.arange(0, 16), rng.choice(M, 24, replace=False), np.arange(M - 16, M)])
    ref_r = O.gemm_f64_rows(O.round_f16(A[rows], False), O.round_f16(B, False), np.arange(rows.size))
    err = O.rel_frob(C[rows], ref_r)
    _say("mfma32 variant", M, N, K, err, row_err, col_err)
    assert np.isfinite(C).all()
    assert err <= 1e-5 and row_err <= 1e-5 and col_err <= 1e-5
    np.testing.assert_array_equal(C, base)


def test_f16_ring_transpose_variants_bit_identical(dev):
    rng = np.random.default_rng(37)
    A = rng.standard_normal((4096, 512)).astype(np.float32)
    B = rng.standard_normal((512, 4096)).astype(np.float32)
    outs = [_gemm_dev(dev, A, B, tA, tB, G.GN_F16) for tA, tB in VARIANTS]
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 1024), (1536, 1536, 512)])
def test_f16_one_round_tiles_all_layouts(dev, M, N, K):
    """Products that one round of 128x128 tiles holds: 2048^2 runs on 128x128 tiles with 8
    waves in every layout; 1536^2 on 128x96 tiles when B is K-contiguous and 128x128
    otherwise. The four layouts must agree bit for bit, start from NaN, and match float64 of
    the fp16-rounded inputs in whole-output row and column sums and on sampled rows."""
    import torch

    rng = np.random.default_rng(M + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    outs = []
    for tA, tB in VARIANTS:
        ad = torch.from_numpy(_stored(A, tA)).to(dev).half()
        bd = torch.from_numpy(_stored(B, tB)).to(dev).half()
        C = _nan_like(dev, M, N)
        _say("one-round tiles", M, N, K, tA, tB)
        G.gemm(ad, bd, C, transA=tA, transB=tB)
        row_err, col_err = _sum_invariants(ad, bd, C, tA, tB)
        assert row_err <= 1e-5 and col_err <= 1e-5, (tA, tB, row_err, col_err)
        outs.append(C.cpu().numpy())
    rows = np.concatenate([np.arange(0, 3), rng.choice(M, 8, replace=False), np.arange(M - 3, M)])
    ref = O.gemm_f64_rows(O.round_f16(A, False), O.round_f16(B, False), rows)
    assert O.rel_frob(outs[0][rows], ref) <= 1e-5
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


def test_f16_row_split_all_transposes_bit_identical(dev):
    """A shape whose last round of 256x256 tiles would be mostly empty (4600 x 4608: 18 x 18
    tiles) runs as two launches over row blocks: rows below 3072 (NN, TN) or 3584 (NT, TT) on
    256x256 tiles, the rest on 128-row tiles. M and K are ragged. NaN start and whole-output
    row and column sums for every layout, sampled rows (both sides of each split) against
    float64 of the fp16-rounded inputs, and the four layouts bit for bit."""
    import torch

    rng = np.random.default_rng(4600)
    M, N, K = 4600, 4608, 96
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    outs = []
    for tA, tB in VARIANTS:
        _say("f16 row split", tA, tB)
        ad = torch.from_numpy(_stored(A, tA)).to(dev).half()
        bd = torch.from_numpy(_stored(B, tB)).to(dev).half()
        cd = _nan_like(dev, M, N)
        G.gemm(ad, bd, cd, transA=tA, transB=tB)
        row_err, col_err = _sum_invariants(ad, bd, cd, tA, tB)
        assert row_err <= 1e-5 and col_err <= 1e-5, (tA, tB, row_err, col_err)
        outs.append(cd.cpu().numpy())
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])
    rows = np.concatenate([np.arange(3064, 3080), np.arange(3576, 3592), rng.choice(M, 16, replace=False),
                           np.arange(M - 8, M)])
    ref_r = O.gemm_f64_rows(O.round_f16(A[rows], False), O.round_f16(B, False), np.arange(rows.size))
    err = O.rel_frob(outs[0][rows], ref_r)
    _say("f16 row split relFrob", err)
    assert err <= 1e-5


@pytest.mark.parametrize("K", [8, 40, 968])
def test_f16_ring_odd_k_tiles_all_layouts(dev, K):
    """The ring takes K-tiles two at a time. One 32-deep K-tile (K = 8), two with a tail
    (K = 40) and 31 with a tail (K = 968) leave the last pair half or wholly zero; TN, NT
    and TT equal the NN result bit for bit (same summation order per element), and TN
    meets the oracle within the fp16-input bar."""
    rng = np.random.default_rng(K)
    M, N = 4096, 4000
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    c_tn = _gemm_dev(dev, A, B, True, False, G.GN_F16)
    c_nn = _gemm_dev(dev, A, B, False, False, G.GN_F16)
    np.testing.assert_array_equal(c_tn, c_nn)
    # K-contiguous B (NT, TT) takes the 8-row x 128-byte chunk layout with its K tail
    np.testing.assert_array_equal(_gemm_dev(dev, A, B, False, True, G.GN_F16), c_nn)
    np.testing.assert_array_equal(_gemm_dev(dev, A, B, True, True, G.GN_F16), c_nn)
    rows = np.concatenate([np.arange(0, 8), rng.choice(M, 16, replace=False), np.arange(M - 8, M)])
    ref_r = O.gemm_f64_rows(O.round_f16(A[rows], False), O.round_f16(B, False), np.arange(rows.size))
    err = O.rel_frob(c_tn[rows], ref_r)
    _say("ring odd K tiles", K, err)
    assert err <= 1e-5


def test_f16_ring_batched_and_epilogue(dev):
    """Batched strides and the bias + GELU epilogue on the ring kernel (4 x 2048^2)."""
    import torch

    rng = np.random.default_rng(41)
    bs, M, N, K = 4, 2048, 2048, 512
    A = rng.standard_normal((bs, M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((bs, K, N))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    a16 = torch.from_numpy(A).to(dev).half()
    b16 = torch.from_numpy(B).to(dev).half()
    C = torch.empty((bs, M, N), dtype=torch.float32, device=dev)
    G.gemm(a16, b16, C, batch=bs, strideA=M * K, strideB=K * N, strideC=M * N,
           bias=torch.from_numpy(bias).to(dev), act=G.ACT_GELU)
    Cn = C.cpu().numpy()
    rows = rng.choice(M, 12, replace=False)
    for z in range(bs):
        pre = O.gemm_f64_rows(O.round_f16(A[z][rows], False), O.round_f16(B[z], False), np.arange(rows.size)) + bias
        assert O.rel_frob(Cn[z][rows], O.act_f64(G.ACT_GELU, pre)) <= 1e-5, z


# ------------------------------------------------------------------ fp16, fewer 256x256 tiles than CUs
@pytest.mark.parametrize("tA,tB", VARIANTS)
def test_f16_few_tiles_ragged_all_transposes(dev, tA, tB):
    """3 x 12 tiles of 256: the 128-wide ring kernels take it (128x128 tiles with 8 waves for
    NN and TN, 128x96 for NT and TT), with M, N ragged and an 8-deep K tail (K = 5000)."""
    rng = np.random.default_rng(43)
    M, N, K = 704, 3000, 5000
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    C = _gemm_dev(dev, A, B, tA, tB, G.GN_F16)
    rows = np.concatenate([np.arange(0, 8), rng.choice(M, 16, replace=False), np.arange(M - 8, M)])
    ref_r = O.gemm_f64_rows(O.round_f16(A[rows], False), O.round_f16(B, False), np.arange(rows.size))
    err = O.rel_frob(C[rows], ref_r)
    _say("few tiles ragged", tA, tB, err)
    assert err <= 1e-5
    assert np.isfinite(C).all()


def test_f16_deterministic_batched_epilogue(dev):
    """Batched fp16 GEMM with beta*C + bias + GELU: two runs agree bit for bit and the
    epilogue is applied once."""
    import torch

    rng = np.random.default_rng(47)
    bs, M, N, K = 3, 512, 1024, 8192
    A = rng.standard_normal((bs, M, K)).astype(np.float32)
    B = (0.02 * rng.standard_normal((bs, K, N))).astype(np.float32)
    C0 = rng.standard_normal((bs, M, N)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    a16 = torch.from_numpy(A).to(dev).half()
    b16 = torch.from_numpy(B).to(dev).half()
    outs = []
    for _ in range(2):
        C = torch.from_numpy(C0).to(dev)
        G.gemm(a16, b16, C, batch=bs, strideA=M * K, strideB=K * N, strideC=M * N, beta=0.5,
               bias=torch.from_numpy(bias).to(dev), act=G.ACT_GELU)
        outs.append(C.cpu().numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    rows = rng.choice(M, 10, replace=False)
    for z in range(bs):
        pre = (O.gemm_f64_rows(O.round_f16(A[z][rows], False), O.round_f16(B[z], False), np.arange(rows.size))
               + 0.5 * C0[z][rows] + bias)
        err = O.rel_frob(outs[0][z][rows], O.act_f64(G.ACT_GELU, pre))
        _say("batched epilogue", z, err)
        assert err <= 1e-5, z


@pytest.mark.parametrize("tA", [False, True])
def test_f16_128x96_tiles_ragged(dev, tA):
    """K-contiguous B with a tile count that favours 128x96 tiles (168 of them, fewer than one
    per CU): N = 2000 leaves a partial 96-wide tile, M = 1000 a partial 128-row tile."""
    rng = np.random.default_rng(59)
    M, N, K = 1000, 2000, 1032
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    C = _gemm_dev(dev, A, B, tA, True, G.GN_F16)
    rows = np.concatenate([np.arange(0, 4), rng.choice(M, 12, replace=False), np.arange(M - 4, M)])
    ref_r = O.gemm_f64_rows(O.round_f16(A[rows], False), O.round_f16(B, False), np.arange(rows.size))
    err = O.rel_frob(C[rows], ref_r)
    _say("128x96 tiles", tA, err)
    assert err <= 1e-5
    assert np.isfinite(C).all()



@pytest.mark.parametrize("tA", [False, True])
def test_f16_ring_128x192_three_slots_ragged(dev, tA):
    """K-contiguous B with enough 128x192 tiles for the 8-wave, three-slot ring (the C4 path):
    M = 1000 and N = 5000 leave partial tiles in both directions, K = 1000 a partial K-tile
    pair; alpha, beta, bias and GELU in the epilogue. Every output element is compared with a
    float64 product of the same fp16 operands on the device, and NaN marks unwritten tiles."""
    import torch

    rng = np.random.default_rng(61)
    M, N, K = 1000, 5000, 1000
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    a16 = torch.from_numpy(_stored(A, tA)).to(dev).half()
    b16 = torch.from_numpy(np.ascontiguousarray(B.T)).to(dev).half()  # K-contiguous B: stored [N, K]
    bd = torch.from_numpy(bias).to(dev)
    for trial, beta in enumerate((0.0, 0.25)):
        Cd = torch.from_numpy(C0).to(dev) if beta else _nan_like(dev, M, N)
        G.gemm(a16, b16, Cd, transA=tA, transB=True, alpha=0.5, beta=beta, bias=bd, act=G.ACT_GELU)
        opA = a16.double().t() if tA else a16.double()
        pre = 0.5 * (opA @ b16.double().t().contiguous()) + bd.double()
        if beta:
            pre = pre + beta * torch.from_numpy(C0).to(dev).double()
        ref = torch.from_numpy(O.act_f64(G.ACT_GELU, pre.cpu().numpy())).to(dev)
        err = (torch.linalg.matrix_norm(Cd.double() - ref) / torch.linalg.matrix_norm(ref)).item()
        _say("128x192 ring", tA, beta, err)
        assert err <= 1e-5
        assert torch.isfinite(Cd).all().item()


def test_f16_register_staged_when_ring_offsets_overflow(dev):
    """A leading dimension of 2^21 halves or more overflows the ring kernels' 32-bit DMA
    offsets, so the register-staged kernel takes the 128x128 tiles. Its result equals the
    ring kernel's on a compact copy of the operand, bit for bit (same summation order)."""
    import torch

    torch.manual_seed(61)
    M, N, K = 128, 16384, 64
    lda = (1 << 21) + 64
    a_big = torch.zeros(M * lda, dtype=torch.float16, device=dev)  # 512 MiB
    a = torch.randn(M, K, device=dev).half()
    a_view = a_big.as_strided((M, K), (lda, 1))
    a_view.copy_(a)
    b = (0.05 * torch.randn(K, N, device=dev)).half()
    c_wide = torch.empty(M, N, device=dev)
    c_compact = torch.empty(M, N, device=dev)
    G.gemm(a_view, b, c_wide)
    G.gemm(a, b, c_compact)
    torch.cuda.synchronize()
    same = torch.equal(c_wide, c_compact)
    _say("register-staged vs ring (lda 2^21+64)", same)
    assert same
    ref = a.float() @ b.float()
    assert ((c_wide - ref).norm() / ref.norm()).item() <= 1e-5


@pytest.mark.parametrize("tA,tB", VARIANTS)
def test_f16_ring128_batched_alpha_beta_bias_act(dev, tA, tB):
    """The 128-wide ring tiles (128x128, or 128x96 when B is K-contiguous) with a batch of
    2, alpha, beta*C, bias and Leaky ReLU, ragged M and N: every batch against float64 of
    the fp16-rounded inputs."""
    import torch

    rng = np.random.default_rng(79)
    bs, M, N, K = 2, 520, 2000, 264
    A = rng.standard_normal((bs, M, K)).astype(np.float32)
    B = (0.05 * rng.standard_normal((bs, K, N))).astype(np.float32)
    C0 = rng.standard_normal((bs, M, N)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    As = np.ascontiguousarray(A.transpose(0, 2, 1)) if tA else A
    Bs = np.ascontiguousarray(B.transpose(0, 2, 1)) if tB else B
    a16 = torch.from_numpy(As).to(dev).half()
    b16 = torch.from_numpy(Bs).to(dev).half()
    C = torch.from_numpy(C0).to(dev)
    G.gemm(a16, b16, C, transA=tA, transB=tB, M=M, N=N, K=K, batch=bs, strideA=M * K, strideB=K * N,
           strideC=M * N, alpha=0.75, beta=-0.5, bias=torch.from_numpy(bias).to(dev), act=G.ACT_LEAKY_RELU,
           act_alpha=0.1)
    Cn = C.cpu().numpy()
    Ar = a16.float().cpu().numpy()
    Br = b16.float().cpu().numpy()
    for z in range(bs):
        Az = Ar[z].T if tA else Ar[z]
        Bz = Br[z].T if tB else Br[z]
        pre = 0.75 * (Az.astype(np.float64) @ Bz.astype(np.float64)) - 0.5 * C0[z] + bias
        err = O.rel_frob(Cn[z], O.act_f64(G.ACT_LEAKY_RELU, pre, 0.1))
        _say("ring128 epilogue", tA, tB, z, err)
        assert err <= 1e-5, (z, err)


def test_batch_beyond_one_launch(dev):
    """70000 small problems (more than the 65535 batches of one launch's grid.z): the
    launcher runs chunks with offset operands; every problem matches float64 and the
    chunk boundary (problems 65534..65536) is exact for small integers."""
    import torch

    rng = np.random.default_rng(83)
    bs, M, N, K = 70000, 5, 3, 4
    A = rng.integers(-4, 5, size=(bs, M, K)).astype(np.float32)
    B = rng.integers(-4, 5, size=(bs, K, N)).astype(np.float32)
    ad, bd = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    C = torch.full((bs, M, N), float("nan"), device=dev)
    G.gemm(ad, bd, C, batch=bs, strideA=M * K, strideB=K * N, strideC=M * N)
    got = C.cpu().numpy()
    ref = np.einsum("bmk,bkn->bmn", A.astype(np.float64), B.astype(np.float64))
    np.testing.assert_array_equal(got, ref)  # small integers: exact in fp32
    a16, b16 = ad.half(), bd.half()
    C16 = torch.full((bs, M, N), float("nan"), device=dev)
    G.gemm(a16, b16, C16, batch=bs, strideA=M * K, strideB=K * N, strideC=M * N)
    np.testing.assert_array_equal(C16.cpu().numpy(), ref)
