"""Randomised parity sweeps of gn_gemm. The first: 600 products with fixed seeds, each drawn over fp32 /
fp16 inputs, both transposes, leading dimensions padded past the operand width, ragged and
degenerate sizes (1..8 up to 5120, capped at 2^35 multiply-adds), alpha, beta with a prior C,
an optional bias and every activation code. These reach the dispatch's paths (ring tiles of
every shape, the fp16 row split, split-K with its reduce, the unaligned pack, the small-tile
fp32 kernels) in combinations the fixed cases do not.

Reference: float64 on the device from the stored (fp16-rounded) operands. Outputs with no
activation or ReLU are compared whole (relFrob <= 1e-5, the fp32 bar; for fp16 inputs the
reference uses the rounded operands, as the fixed fp16 tests do); for the other activations
1024 sampled elements are compared with the oracle's activation (orc_act_f64, the
reference's formulas) applied to the float64 pre-activation. The padding columns of C must be
left as they were.

The second: 120 products of 1-16 rows with wide N and long K (test_gemm_random_few_rows),
where the dispatch chooses between the GEMV, small-product and tiled kernels."""
import random
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ACTS = [G.ACT_NONE, G.ACT_RELU, G.ACT_SIGMOID, G.ACT_TANH, G.ACT_LEAKY_RELU, G.ACT_ELU, G.ACT_SWISH, G.ACT_GELU]


def _pick_dim(rng):
    r = rng.random()
    if r < 0.1:
        return rng.randint(1, 8)
    if r < 0.5:
        return rng.randint(9, 700)
    if r < 0.9:
        return rng.randint(700, 3000)
    return rng.choice([1024, 2048, 4096, 5120])


@pytest.mark.parametrize("seed", [101, 102, 103])
def test_gemm_random_sweep(dev, seed):
    import torch

    rng = random.Random(seed)
    torch.manual_seed(seed)
    for case in range(200):
        dtype = rng.choice([G.GN_F32, G.GN_F16])
        M, N, K = _pick_dim(rng), _pick_dim(rng), _pick_dim(rng)
        if M * N * K > 2 ** 35:
            K = max(1, 2 ** 35 // (M * N))
        tA, tB = rng.random() < 0.5, rng.random() < 0.5
        padA, padB, padC = rng.choice([0, 0, 0, 1, 3, 8]), rng.choice([0, 0, 0, 1, 3, 8]), rng.choice([0, 0, 1, 4])
        alpha = rng.choice([1.0, 1.0, 0.5, -2.0])
        beta = rng.choice([0.0, 0.0, 0.0, 1.0, -0.5])
        act = rng.choice(ACTS)
        act_alpha = rng.choice([0.01, 0.2])
        use_bias = rng.random() < 0.4
        tdt = torch.float16 if dtype == G.GN_F16 else torch.float32
        ar, ac = (K, M) if tA else (M, K)
        br, bc = (N, K) if tB else (K, N)
        A_full = torch.randn(ar, ac + padA, device=dev).to(tdt)
        B_full = (0.1 * torch.randn(br, bc + padB, device=dev)).to(tdt)
        A, B = A_full[:, :ac], B_full[:, :bc]
        C_full = torch.randn(M, N + padC, device=dev)
        C = C_full[:, :N]
        C0 = C.double().clone()
        pad_before = C_full[:, N:].clone()
        bias = torch.randn(N, device=dev) if use_bias else None
        desc = (f"seed {seed} case {case}: {'f16' if dtype == G.GN_F16 else 'f32'} M={M} N={N} K={K} tA={tA} "
                f"tB={tB} pads={padA},{padB},{padC} alpha={alpha} beta={beta} act={act} bias={use_bias}")
        print(desc, flush=True)
        sys.stdout.flush()
        G.gemm(A, B, C, transA=tA, transB=tB, alpha=alpha, beta=beta, bias=bias, act=act, act_alpha=act_alpha,
               M=M, N=N, K=K, lda=A_full.stride(0), ldb=B_full.stride(0), ldc=C_full.stride(0), dtype=dtype)
        torch.cuda.synchronize()
        a64, b64 = A.double(), B.double()
        pre = alpha * ((a64.t() if tA else a64) @ (b64.t() if tB else b64)) + beta * C0
        if use_bias:
            pre = pre + bias.double()
        got = C.double()
        assert bool(torch.isfinite(got).all()), desc
        assert torch.equal(C_full[:, N:], pad_before), desc
        if act in (G.ACT_NONE, G.ACT_RELU):
            ref = pre if act == G.ACT_NONE else torch.clamp(pre, min=0.0)
            den = torch.linalg.vector_norm(ref).item()
            err = torch.linalg.vector_norm(got - ref).item() / den if den > 0 else torch.linalg.vector_norm(got).item()
        else:
            n = M * N
            idx = torch.from_numpy(np.random.default_rng(seed * 1000 + case).integers(0, n, size=min(n, 1024))).to(dev)
            ref = O.act_f64(act, pre.reshape(-1)[idx].cpu().numpy(), act_alpha)
            g = got.reshape(-1)[idx].cpu().numpy()
            den = np.linalg.norm(ref)
            err = np.linalg.norm(g - ref) / den if den > 0 else np.linalg.norm(g)
        assert err <= 1e-5, (desc, err)


@pytest.mark.parametrize("seed", [111, 112, 113])
def test_gemm_random_few_rows(dev, seed):
    """120 products of 1-16 rows with wide N (256 .. 20000) and long K (1 .. 9000), drawn over
    dtypes, all four layouts, padded leading dimensions, alpha, beta with a prior C, bias and
    ReLU / GELU: the range where the dispatch chooses between the NN GEMV kernel, the
    small-product kernel (its skinny linear-layer branch included) and the tiled kernels. Each
    against float64 of the stored operands (relFrob <= 1e-5; GELU through the oracle's
    formula), C's padding columns untouched."""
    import torch

    rng = random.Random(seed)
    torch.manual_seed(seed)
    for case in range(40):
        dtype = rng.choice([G.GN_F32, G.GN_F16])
        M = rng.choice([1, 1, 2, 3, 4, rng.randint(5, 16)])
        N = rng.choice([256, 1024, 2048, 4096, 8192, 11008, 16384, rng.randint(257, 20000)])
        K = rng.choice([1, 7, 512, 1024, 2048, 4096, 8192, rng.randint(2, 9000)])
        tA, tB = rng.random() < 0.3, rng.random() < 0.5
        padA, padB, padC = rng.choice([0, 0, 1, 8]), rng.choice([0, 0, 1, 8]), rng.choice([0, 0, 3])
        alpha = rng.choice([1.0, -0.5])
        beta = rng.choice([0.0, 0.0, 1.5])
        act = rng.choice([G.ACT_NONE, G.ACT_RELU, G.ACT_GELU])
        use_bias = rng.random() < 0.5
        tdt = torch.float16 if dtype == G.GN_F16 else torch.float32
        ar, ac = (K, M) if tA else (M, K)
        br, bc = (N, K) if tB else (K, N)
        A_full = torch.randn(ar, ac + padA, device=dev).to(tdt)
        B_full = (0.05 * torch.randn(br, bc + padB, device=dev)).to(tdt)
        A, B = A_full[:, :ac], B_full[:, :bc]
        C_full = torch.randn(M, N + padC, device=dev)
        C = C_full[:, :N]
        C0 = C.double().clone()
        pad_before = C_full[:, N:].clone()
        bias = torch.randn(N, device=dev) if use_bias else None
        desc = (f"seed {seed} case {case}: {'f16' if dtype == G.GN_F16 else 'f32'} M={M} N={N} K={K} tA={tA} "
                f"tB={tB} pads={padA},{padB},{padC} alpha={alpha} beta={beta} act={act} bias={use_bias}")
        print(desc, flush=True)
        sys.stdout.flush()
        G.gemm(A, B, C, transA=tA, transB=tB, alpha=alpha, beta=beta, bias=bias, act=act, M=M, N=N, K=K,
               lda=A_full.stride(0), ldb=B_full.stride(0), ldc=C_full.stride(0), dtype=dtype)
        torch.cuda.synchronize()
        a64, b64 = A.double(), B.double()
        pre = alpha * ((a64.t() if tA else a64) @ (b64.t() if tB else b64)) + beta * C0
        if use_bias:
            pre = pre + bias.double()
        got = C.double().cpu().numpy()
        pre = pre.cpu().numpy()
        ref = pre if act == G.ACT_NONE else (np.maximum(pre, 0.0) if act == G.ACT_RELU else O.act_f64(act, pre, 0.0))
        assert np.isfinite(got).all(), desc
        assert torch.equal(C_full[:, N:], pad_before), desc
        den = np.linalg.norm(ref)
        err = np.linalg.norm(got - ref) / den if den > 0 else np.linalg.norm(got)
        assert err <= 1e-5, (desc, err)
