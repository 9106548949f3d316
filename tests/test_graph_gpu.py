"""HIP graph capture of the device-pointer API: the GEMM (fp16 ring and register-staged
kernels, fp32), CSR SpMM and SpMV launch no memset and allocate nothing, so a caller can
capture them once and replay the graph. Each replay is compared with the eager result
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
    w32 = torch.randn(300, 500, device=dev)
    bias = torch.randn(500, device=dev)
    rp, col, val = O.random_csr(2000, 3000, 20.0, seed=3)
    d_rp, d_col, d_val = (torch.from_numpy(v).to(dev) for v in (rp, col, val))
    D = torch.randn(3000, 64, device=dev)
    xv = torch.randn(3000, device=dev)

    c16 = torch.empty(4096, 4096, device=dev)
    y32 = torch.empty(700, 500, device=dev)
    S = torch.empty(2000, 64, device=dev)
    yv = torch.empty(2000, device=dev)

    def work():
        G.gemm(a16, b16, c16)
        G.gemm(x32, w32, y32, bias=bias, act=G.ACT_GELU)
        G.spmm_csr(2000, 64, 3000, val.size, d_rp, d_col, d_val, D, S)
        G.spmv_csr(2000, 3000, val.size, d_rp, d_col, d_val, xv, yv)

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

    outs = (c16, y32, S, yv)
    for rep in range(3):
        # new inputs, eager work and a synchronisation between replays
        with torch.no_grad():
            a16.copy_(torch.randn_like(a16, dtype=torch.float32).half())
            w32.mul_(0.5).add_(0.1)
            D.copy_(torch.randn_like(D))
            xv.mul_(-1.5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        work()  # eager, on the current stream
        torch.cuda.synchronize()
        for name, gt, ref in zip(("gemm f16", "gemm f32", "spmm", "spmv"), got, outs):
            same = torch.equal(gt, ref)
            _say("replay", rep, name, "bit-identical" if same else "DIFFERS")
            assert same, (rep, name)
