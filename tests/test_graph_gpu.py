"""HIP graph capture of the device-pointer API: the GEMM (fp16 ring and register-staged
kernels, fp32, the small-product kernel in fp32 and for a skinny fp16 X W^T, the NN GEMV), CSR SpMM, SpMV and the grouped-layout SpMV of a plan built before the capture
launch no memset and allocate nothing, so a caller can capture them once and replay the graph. Each replay is compared with the eager result
for inputs changed between replays (with the program's own eager work and
synchronisations in between), bit for bit."""
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_graph_replays_match_eager(dev):
    import torch

    torch.manual_seed(5)
    a16 = torch.randn(4096, 512, device=dev).half()      # ring kernel: 16 x 16 tiles of 256
    b16 = torch.randn(512, 4096, device=dev).half()
    x32 = torch.randn(700, 300, device=dev)              # fp32 register-staged kernel
    xs = torch.randn(96, 200, device=dev)                # fp32 small-product kernel
    ws = torch.randn(200, 80, device=dev)
    xk = torch.randn(2, 4096, device=dev).half()         # fp16 skinny X W^T: small-product kernel
    wk = (0.05 * torch.randn(2048, 4096, device=dev)).half()
    xg = torch.randn(1, 2048, device=dev)                 # fp32 NN GEMV (one row)
    wg = 0.05 * torch.randn(2048, 8192, device=dev)
    w32 = torch.randn(300, 500, device=dev)
    bias = torch.randn(500, device=dev)
    a2 = torch.randn(4600, 64, device=dev).half()        # fp16 row split: two launches
    b2 = torch.randn(64, 4608, device=dev).half()
    rp, col, val = O.random_csr(4000, 3000, 20.0, seed=3)  # > 65536 entries: SpMM in two launches
    d_rp, d_col, d_val = (torch.from_numpy(v).to(dev) for v in (rp, col, val))
    D = torch.randn(3000, 64, device=dev)
    xv = torch.randn(3000, device=dev)

    c16 = torch.empty(4096, 4096, device=dev)
    c2 = torch.empty(4600, 4608, device=dev)
    y32 = torch.empty(700, 500, device=dev)
    ys = torch.empty(96, 80, device=dev)
    yk = torch.empty(2, 2048, device=dev)
    yg = torch.empty(1, 8192, device=dev)
    S = torch.empty(4000, 64, device=dev)
    yv = torch.empty(4000, device=dev)
    yp = torch.empty(4000, device=dev)
    torch.cuda.synchronize()
    plan = G.SpmvPlan(4000, 3000, val.size, d_rp, d_col)  # reads the row pointers back: not capturable

    def work():
        G.gemm(a16, b16, c16)
        G.gemm(a2, b2, c2)
        G.gemm(x32, w32, y32, bias=bias, act=G.ACT_GELU)
        G.gemm(xs, ws, ys, bias=bias[:80], act=G.ACT_RELU)
        G.gemm(xk, wk, yk, transB=True)
        G.gemm(xg, wg, yg, bias=bias.repeat(17)[:8192], act=G.ACT_RELU)
        G.spmm_csr(4000, 64, 3000, val.size, d_rp, d_col, d_val, D, S)
        G.spmv_csr(4000, 3000, val.size, d_rp, d_col, d_val, xv, yv)
        plan.run(d_val, xv, yp)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        work()  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        work()
    torch.cuda.synchronize()

    assert val.size >= 1 << 16
    outs = (c16, c2, y32, S, yv, yp, ys, yk, yg)
    for rep in range(3):
        # new inputs, eager work and a synchronisation between replays
        with torch.no_grad():
            a16.copy_(torch.randn_like(a16, dtype=torch.float32).half())
            b2.copy_(torch.randn_like(b2, dtype=torch.float32).half())
            w32.mul_(0.5).add_(0.1)
            ws.mul_(-0.5).add_(0.2)
            xk.copy_(torch.randn_like(xk, dtype=torch.float32).half())
            xg.mul_(-1.25)
            D.copy_(torch.randn_like(D))
            xv.mul_(-1.5)
            d_val.mul_(0.75)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        work()  # eager, on the current stream
        torch.cuda.synchronize()
        for name, gt, ref in zip(("gemm f16", "gemm f16 row split", "gemm f32", "spmm", "spmv", "spmv plan",
                                  "gemm f32 small", "gemm f16 skinny", "gemv f32"), got,
                                 outs):
            same = torch.equal(gt, ref)
            _say("replay", rep, name, "bit-identical" if same else "DIFFERS")
            assert same, (rep, name)
        # the plan's replayed result is also the reference loop's, bit for bit
        np.testing.assert_array_equal(got[5].cpu().numpy(),
                                      O.spmv_f32(rp, col, d_val.cpu().numpy(), xv.cpu().numpy(), use_fma=True))
    plan.release()


def test_synchronize_on_a_capturing_stream_is_an_error(dev):
    """gn_synchronize (the completion wait every synchronous entry uses) on a stream under
    capture has nothing to wait for: it returns -6 without touching the stream, and the capture
    goes on. The captured GEMM then replays with the eager result's bits."""
    import torch

    torch.manual_seed(11)
    a = torch.randn(512, 256, device=dev)
    b = torch.randn(256, 384, device=dev)
    c = torch.empty(512, 384, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        G.gemm(a, b, c)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        G.gemm(a, b, c)
        rc, msg = G.call_rc("gn_synchronize", s.cuda_stream)
        G.gemm(a, b, c, beta=1.0)  # c = ab + ab after the refused wait
    _say("gn_synchronize under capture:", rc, msg)
    assert rc == -6 and "device execution" in msg
    torch.cuda.synchronize()
    for rep in range(2):
        with torch.no_grad():
            a.mul_(0.5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = c.clone()
        G.gemm(a, b, c)
        G.gemm(a, b, c, beta=1.0)
        torch.cuda.synchronize()
        assert torch.equal(got, c), rep


def _ptrs(*bufs):
    import ctypes

    return (ctypes.c_void_p * len(bufs))(*[b.handle.value for b in bufs])


def test_mpsgraph_abi_matmul_relu_chain(dev):
    """createMPSGraph / createMatMulNode / createReLUNode / compileGraph /
    executeCompiledGraph (metal_bridge.h:1800-1826): Y = relu(X W1) W2 (the MatMul + ReLU
    pair runs as one GEMM with a ReLU epilogue) against float64, executed twice with new
    inputs through the same compiled HIP graph."""
    L = G.load()
    g = L.createMPSGraph()
    assert g
    X = L.gn_graph_placeholder(g, 70, 96, G.GN_F32)
    W1 = L.gn_graph_placeholder(g, 96, 130, G.GN_F32)
    W2 = L.gn_graph_placeholder(g, 130, 40, G.GN_F32)
    y = L.createMatMulNode(g, L.createReLUNode(g, L.createMatMulNode(g, X, W1)), W2)
    assert y
    assert not L.createMatMulNode(g, X, W2)  # inner dimensions 96 and 130
    g2 = L.createMPSGraph()  # shapes whose byte counts wrap around 2^64 are refused
    assert not L.gn_graph_placeholder(g2, 1 << 40, 1 << 40, G.GN_F32)
    tall, wide = L.gn_graph_placeholder(g2, 1 << 31, 1, G.GN_F32), L.gn_graph_placeholder(g2, 1, 1 << 40, G.GN_F32)
    assert tall and wide and not L.createMatMulNode(g2, tall, wide)  # a 2^71-value product
    L.gn_graph_release(g2)
    c = L.compileGraph(g, None)
    assert c
    rng = np.random.default_rng(71)
    for rep in range(2):
        x = rng.standard_normal((70, 96)).astype(np.float32)
        w1 = rng.standard_normal((96, 130)).astype(np.float32)
        w2 = rng.standard_normal((130, 40)).astype(np.float32)
        bx, b1, b2, by = G.Buffer.from_array(x), G.Buffer.from_array(w1), G.Buffer.from_array(w2), G.Buffer(70 * 40 * 4)
        L.executeCompiledGraph(c, None, _ptrs(bx, b1, b2), 3, _ptrs(by), 1)
        h = np.maximum(x.astype(np.float64) @ w1, 0.0).astype(np.float32)
        err = O.rel_frob(by.to_array((70, 40)), h.astype(np.float64) @ w2)
        _say("mpsgraph chain", rep, err)
        assert err <= 1e-5
    rc, msg = G.call_rc("gn_graph_execute", c, None, _ptrs(bx), 1, _ptrs(by), 1)
    assert rc == -1 and "expected 3 inputs" in msg
    L.gn_graph_release(c)
    L.gn_graph_release(g)


def test_graph_subgraph_fp16_transposed_gelu(dev):
    """gn_graph_compile of a subgraph: GELU(A16 * B16^T) with fp16 placeholders and a
    transposed B, plus a second output (the unfused MatMul result read twice)."""
    import ctypes

    L = G.load()
    g = L.createMPSGraph()
    A = L.gn_graph_placeholder(g, 300, 256, G.GN_F16)
    B = L.gn_graph_placeholder(g, 520, 256, G.GN_F16)
    unused = L.gn_graph_placeholder(g, 8, 8, G.GN_F32)
    m = L.gn_graph_matmul(g, A, B, 0, 1)
    act = L.gn_graph_activation(g, m, G.ACT_GELU, 0.0)
    tanh = L.gn_graph_activation(g, m, G.ACT_TANH, 0.0)
    assert m and act and tanh
    assert not L.gn_graph_activation(g, A, G.ACT_RELU, 0.0)  # fp16 tensors only feed MatMuls
    comp = ctypes.c_void_p()
    ins = (ctypes.c_void_p * 3)(A, B, unused)
    outs = (ctypes.c_void_p * 2)(act, tanh)
    G.call("gn_graph_compile", g, ins, 3, outs, 2, ctypes.byref(comp))
    rng = np.random.default_rng(73)
    a = rng.standard_normal((300, 256)).astype(np.float32)
    b = (0.1 * rng.standard_normal((520, 256))).astype(np.float32)
    a16, b16 = a.astype(np.float16), b.astype(np.float16)
    ba, bb = G.Buffer(data=a16.view(np.uint16)), G.Buffer(data=b16.view(np.uint16))
    bu, bo1, bo2 = G.Buffer(8 * 8 * 4), G.Buffer(300 * 520 * 4), G.Buffer(300 * 520 * 4)
    G.call("gn_graph_execute", comp.value, None, _ptrs(ba, bb, bu), 3, _ptrs(bo1, bo2), 2)
    pre = a16.astype(np.float64) @ b16.astype(np.float64).T
    e1 = O.rel_frob(bo1.to_array((300, 520)), O.act_f64(G.ACT_GELU, pre))
    e2 = O.rel_frob(bo2.to_array((300, 520)), np.tanh(pre))
    _say("graph fp16 gelu / tanh", e1, e2)
    assert e1 <= 1e-5 and e2 <= 1e-5
    rc, msg = G.call_rc("gn_graph_compile", g, ins, 1, outs, 1, ctypes.byref(comp))
    assert rc == -1 and "needed but not an input" in msg
    L.gn_graph_release(comp.value)
    L.gn_graph_release(g)
