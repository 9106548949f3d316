"""GPU parity of ActivationForward (gpu/matrix/activation.go:56-175): the Part-1 entries
perform_activation_*_forward (metal_bridge.h:257-396) and the device-pointer
gn_activation_forward / gn_softmax_rows, against the oracle (orc_act_f64,
orc_softmax_rows_f64). Bar: relFrob <= 1e-5 against float64 and every element within
1e-5 absolute (fp32 transcendental functions round differently from the reference's)."""
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ENTRY = {0: "relu", 1: "sigmoid", 2: "tanh", 4: "leaky_relu", 5: "elu", 6: "swish", 7: "gelu"}
ALPHA = {4: 0.1, 5: 1.0}


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _inputs(n, seed):
    rng = np.random.default_rng(seed)
    x = (3.0 * rng.standard_normal(n)).astype(np.float32)
    # clamp edges and special points of the reference formulas
    x[:12] = [0.0, -0.0, 88.0, -88.0, 100.0, -100.0, 1e-30, -1e-30, 20.0, -20.0, 5.5, -5.5]
    return x


def _check(got, ref):
    err = O.rel_frob(got, ref)
    assert err <= 1e-5, err
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5)
    return err


@pytest.mark.parametrize("code", sorted(ENTRY))
def test_activation_forward_reference_abi(dev, code):
    n = 100003  # not a multiple of 4: the vector body and the scalar tail
    x = _inputs(n, code)
    bx, by = G.Buffer.from_array(x), G.Buffer(n * 4)
    name = f"perform_activation_{ENTRY[code]}_forward"
    if code in ALPHA:
        G.call(name, bx.handle, n, ALPHA[code], by.handle, None)
    else:
        G.call(name, bx.handle, n, by.handle, None)
    y = by.to_array((n,))
    err = _check(y, O.act_f64(code, x, ALPHA.get(code, 0.0)))
    _say(name, err)
    # the reference's own vectors (gpu/matrix/activation_test.go:32-51, :282-285)
    v = np.array([-2.0, -1.0, 0.0, 1.0, 2.0, 3.0], np.float32)
    bv, bo = G.Buffer.from_array(v), G.Buffer(v.nbytes)
    if code in ALPHA:
        G.call(name, bv.handle, v.size, ALPHA[code], bo.handle, None)
    else:
        G.call(name, bv.handle, v.size, bo.handle, None)
    out = bo.to_array((v.size,))
    if code == 0:
        np.testing.assert_array_equal(out, [0, 0, 0, 1, 2, 3])
    if code == 7:
        assert out[2] == 0.0


def test_activation_forward_in_place_and_errors(dev):
    x = _inputs(4096, 3)
    b = G.Buffer.from_array(x)
    G.call("perform_activation_gelu_forward", b.handle, x.size, b.handle, None)  # in place
    _check(b.to_array((x.size,)), O.act_f64(7, x))
    small = G.Buffer(16)
    rc, msg = G.call_rc("perform_activation_relu_forward", b.handle, x.size, small.handle, None)
    assert rc == -1 and "smaller" in msg
    rc, msg = G.call_rc("perform_activation_relu_forward", None, 4, b.handle, None)
    assert rc == -1 and "Invalid buffer pointers for ReLU forward" in msg
    rc, _ = G.call_rc("perform_activation_tanh_forward", b.handle, -1, b.handle, None)
    assert rc == -1
    assert G.call_rc("perform_activation_sigmoid_forward", b.handle, 0, b.handle, None)[0] == 0


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 100000), (300, 10), (64, 4099), (2, 3)])
def test_softmax_forward_reference_abi(dev, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    x = (4.0 * rng.standard_normal((rows, cols))).astype(np.float32)
    bx, by = G.Buffer.from_array(x), G.Buffer(x.nbytes)
    if rows == 1:
        G.call("perform_activation_softmax_1d_forward", bx.handle, cols, by.handle, None)
    else:
        G.call("perform_activation_softmax_2d_forward", bx.handle, rows, cols, by.handle, None)
    y = by.to_array((rows, cols))
    ref = O.softmax_rows_f64(x)
    err = _check(y, ref)
    np.testing.assert_allclose(y.sum(axis=1, dtype=np.float64), 1.0, rtol=1e-5)
    _say("softmax", rows, cols, err)


def test_softmax_nan_and_shift(dev):
    x = np.array([[np.nan, 1.0, 2.0], [1.0, 2.0, 3.0], [101.0, 102.0, 103.0]], np.float32)
    bx, by = G.Buffer.from_array(x), G.Buffer(x.nbytes)
    G.call("perform_activation_softmax_2d_forward", bx.handle, 3, 3, by.handle, None)
    y = by.to_array((3, 3))
    assert np.isnan(y[0]).all()
    np.testing.assert_allclose(y[1], y[2], rtol=1e-6)


def test_device_pointer_entries_unaligned(dev):
    """gn_activation_forward on a pointer 4 bytes past a 16-byte boundary (scalar path)
    and gn_softmax_rows on torch tensors."""
    import torch

    x = _inputs(10001, 9)
    xt = torch.from_numpy(x).to(dev)
    out = torch.empty(10001, device=dev)
    G.activation_forward(xt[1:], out[1:], G.ACT_GELU)  # 10000 values, both 4 bytes past 16-byte alignment
    torch.cuda.synchronize()
    _check(out[1:].cpu().numpy(), O.act_f64(7, x[1:]))
    G.activation_forward(xt, out, G.ACT_NONE)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), x)
    m = torch.from_numpy((2.0 * np.random.default_rng(1).standard_normal((33, 77))).astype(np.float32)).to(dev)
    sm = torch.empty_like(m)
    G.softmax_rows(m, sm)
    torch.cuda.synchronize()
    _check(sm.cpu().numpy(), O.softmax_rows_f64(m.cpu().numpy()))
    rc, msg = G.call_rc("gn_activation_forward", G._ptr(xt), G._ptr(out), 4, 3, 0.0, None)
    assert rc == -1 and "unsupported" in msg  # Softmax is row-wise, not element-wise
