"""gn_activation_backward_noalloc (the allocation-free form of gn_activation_backward)
through the C ABI: its outputs equal the allocating entry point's bit for bit, on two
calls in a row (the second smaller, so the shared device scratch holds the first call's
partial sums when it starts), and it allocates nothing from the library pool. Shapes
beyond its scratch are refused with a clear error before any launch."""
import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _backward(entry, dev, dy, pre, act, alpha, scale):
    import torch

    rows, cols = pre.shape
    gi = torch.full((rows, cols), float("nan"), dtype=torch.float32, device=dev)
    gb = torch.full((cols,), float("nan"), dtype=torch.float32, device=dev)
    sp = torch.cuda.current_stream().cuda_stream
    G.call(entry, dy.data_ptr(), pre.data_ptr(), rows, cols, act, alpha, scale, gi.data_ptr(), gb.data_ptr(), sp)
    torch.cuda.current_stream().synchronize()
    return gi.cpu().numpy(), gb.cpu().numpy()


@pytest.mark.parametrize("act", [G.ACT_RELU, G.ACT_GELU])
def test_noalloc_matches_allocating_entry_two_calls(dev, act):
    import torch

    shapes = [(2048, 3000), (333, 517)]  # second call smaller: stale partials in the scratch
    for i, (rows, cols) in enumerate(shapes):
        print("noalloc call", i, "shape", rows, cols, "act", act, flush=True)
        dy = torch.from_numpy(O.normal((rows, cols), 42, 500 + i)).to(dev)
        pre = torch.from_numpy(O.normal((rows, cols), 42, 600 + i)).to(dev)
        torch.cuda.current_stream().synchronize()
        before = G.memory_stats()
        gi_n, gb_n = _backward("gn_activation_backward_noalloc", dev, dy, pre, act, 0.1, 1.25)
        after = G.memory_stats()
        assert after[0] == before[0] and after[2] == before[2], "the no-alloc entry point used the library pool"
        gi_a, gb_a = _backward("gn_activation_backward", dev, dy, pre, act, 0.1, 1.25)
        np.testing.assert_array_equal(gi_n, gi_a)
        np.testing.assert_array_equal(gb_n, gb_a)
        # and against the oracle (float64), as the allocating entry point's own tests do
        ref_gi = O.act_backward_f64(act, dy.cpu().numpy(), pre.cpu().numpy(), 0.1, 1.25)
        assert O.rel_frob(gi_n, ref_gi) <= 1e-5
        assert O.rel_frob(gb_n, ref_gi.sum(axis=0)) <= 1e-5


def test_noalloc_without_bias_and_empty(dev):
    import torch

    dy = torch.from_numpy(O.normal((64, 80), 42, 700)).to(dev)
    pre = torch.from_numpy(O.normal((64, 80), 42, 701)).to(dev)
    gi = torch.empty((64, 80), dtype=torch.float32, device=dev)
    sp = torch.cuda.current_stream().cuda_stream
    G.call("gn_activation_backward_noalloc", dy.data_ptr(), pre.data_ptr(), 64, 80, G.ACT_TANH, 0.0, 1.0,
           gi.data_ptr(), None, sp)
    gb = torch.full((80,), 7.0, dtype=torch.float32, device=dev)
    G.call("gn_activation_backward_noalloc", dy.data_ptr(), pre.data_ptr(), 0, 80, G.ACT_TANH, 0.0, 1.0,
           gi.data_ptr(), gb.data_ptr(), sp)  # zero rows: the column sums are zero
    torch.cuda.current_stream().synchronize()
    ref_gi = O.act_backward_f64(G.ACT_TANH, dy.cpu().numpy(), pre.cpu().numpy(), 0.0, 1.0)
    assert O.rel_frob(gi.cpu().numpy(), ref_gi) <= 1e-5
    assert (gb.cpu().numpy() == 0).all()


def test_noalloc_rejects_beyond_scratch(dev):
    """One row of 2^21 + 1 columns needs 2^21 + 1 partial sums, one more than the scratch
    holds: refused on the host before any launch (real buffers, so nothing could fault)."""
    import torch

    cols = (1 << 21) + 1
    dy = torch.zeros((1, cols), dtype=torch.float32, device=dev)
    pre = torch.zeros((1, cols), dtype=torch.float32, device=dev)
    gi = torch.zeros((1, cols), dtype=torch.float32, device=dev)
    gb = torch.zeros((cols,), dtype=torch.float32, device=dev)
    sp = torch.cuda.current_stream().cuda_stream
    rc, msg = G.call_rc("gn_activation_backward_noalloc", dy.data_ptr(), pre.data_ptr(), 1, cols, G.ACT_RELU, 0.0,
                        1.0, gi.data_ptr(), gb.data_ptr(), sp)
    assert rc == -1 and "scratch" in msg, (rc, msg)
    # the largest accepted width still runs
    G.call("gn_activation_backward_noalloc", dy.data_ptr(), pre.data_ptr(), 1, cols - 1, G.ACT_RELU, 0.0, 1.0,
           gi.data_ptr(), gb.data_ptr(), sp)
    torch.cuda.current_stream().synchronize()
