"""GPU parity of the linear-layer backward (FusedLinearActivation.Backward,
gpu/matrix/fused-operations.go:467-578; matmulBackward, gpu/matrix/gradient.go:601-637)
against the oracle's float64 restatement: gn_activation_backward (activation derivative
at the pre-activation, dropout scale, bias column sums) plus the NT / TN GEMMs.
Tolerance: relFrob <= 1e-5 (fp32); ReLU / LeakyReLU / identity gradients are products
by 0, 1 or alpha and are compared bit for bit."""
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu
CODES = [G.ACT_NONE, G.ACT_RELU, G.ACT_SIGMOID, G.ACT_TANH, G.ACT_LEAKY_RELU, G.ACT_ELU, G.ACT_SWISH, G.ACT_GELU]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _act_bwd(dev, dy, pre, act, alpha=0.0, scale=1.0, bias=True):
    import torch

    t_dy, t_pre = torch.from_numpy(dy).to(dev), torch.from_numpy(pre).to(dev)
    gi = torch.empty_like(t_pre)
    gb = torch.full((pre.shape[1],), float("nan"), device=dev) if bias else None
    G.activation_backward(t_dy, t_pre, act, gi, gb, alpha=alpha, scale=scale)
    return gi.cpu().numpy(), (gb.cpu().numpy() if bias else None)


@pytest.mark.parametrize("act", CODES)
@pytest.mark.parametrize("shape", [(1, 7), (300, 1000), (513, 11)])
def test_activation_backward_all_codes(dev, act, shape):
    rng = np.random.default_rng(101 + act + shape[0])
    pre = (2.0 * rng.standard_normal(shape)).astype(np.float32)
    dy = rng.standard_normal(shape).astype(np.float32)
    gi, gb = _act_bwd(dev, dy, pre, act, alpha=0.1, scale=1.0 / 0.9)
    ref = O.act_backward_f64(act, dy, pre, 0.1, 1.0 / 0.9)
    _say("act bwd", act, shape, O.rel_frob(gi, ref))
    if act in (G.ACT_NONE, G.ACT_RELU, G.ACT_LEAKY_RELU):
        d = np.where(pre > 0, np.float32(1), np.float32(0.1 if act == G.ACT_LEAKY_RELU else 0.0))
        if act == G.ACT_NONE:
            d = np.ones_like(pre)
        np.testing.assert_array_equal(gi, (dy * d) * np.float32(1.0 / 0.9))
    assert O.rel_frob(gi, ref) <= 1e-5
    assert O.rel_frob(gb, ref.sum(axis=0)) <= 1e-5


def test_activation_backward_bias_deterministic_and_empty(dev):
    rng = np.random.default_rng(7)
    pre = rng.standard_normal((2048, 777)).astype(np.float32)
    dy = rng.standard_normal((2048, 777)).astype(np.float32)
    _, b1 = _act_bwd(dev, dy, pre, G.ACT_GELU)
    _, b2 = _act_bwd(dev, dy, pre, G.ACT_GELU)
    np.testing.assert_array_equal(b1, b2)
    _, b0 = _act_bwd(dev, np.zeros((0, 9), np.float32), np.zeros((0, 9), np.float32), G.ACT_RELU)
    np.testing.assert_array_equal(b0, np.zeros(9, np.float32))
    rc, msg = G.call_rc("gn_activation_backward", None, None, 4, 4, 3, 0.0, 1.0, None, None, None)
    assert rc == -1 and "activation" in msg  # Softmax is not element-wise


@pytest.mark.parametrize("act", [G.ACT_RELU, G.ACT_GELU])
def test_linear_backward_full(dev, act):
    """Backward of Y = act(X W + b) with W [in, out] (the reference layout): grad_input
    = G W^T (gn_gemm NT), grad_weight = X^T G (gn_gemm TN), grad_bias = column sums."""
    import torch

    rng = np.random.default_rng(113 + act)
    Bn, In, Out = 512, 768, 1024
    X = rng.standard_normal((Bn, In)).astype(np.float32)
    W = (0.05 * rng.standard_normal((In, Out))).astype(np.float32)
    b = (0.1 * rng.standard_normal(Out)).astype(np.float32)
    dY = rng.standard_normal((Bn, Out)).astype(np.float32)
    pre = (X.astype(np.float64) @ W.astype(np.float64) + b).astype(np.float32)
    tX, tW, tdY, tpre = (torch.from_numpy(a).to(dev) for a in (X, W, dY, pre))
    Gd = torch.empty_like(tdY)
    gb = torch.empty(Out, device=dev)
    G.activation_backward(tdY, tpre, act, Gd, gb)
    dX = torch.empty((Bn, In), device=dev)
    dW = torch.empty((In, Out), device=dev)
    G.gemm(Gd, tW, dX, transB=True)          # [Bn,Out] x [In,Out]^T
    G.gemm(tX, Gd, dW, transA=True)          # [Bn,In]^T x [Bn,Out]
    rdX, rdW, rdb, _ = O.linear_backward_f64(X, W, pre, dY, act)
    e = (O.rel_frob(dX.cpu().numpy(), rdX), O.rel_frob(dW.cpu().numpy(), rdW), O.rel_frob(gb.cpu().numpy(), rdb))
    _say("linear backward", act, e)
    assert max(e) <= 1e-5
