"""Benchmark of the MI355X GEMM / SpMM backend (one JSON line on stdout).

Headline (value): config C3, fp16-in / fp32-accumulate GEMM, M=N=K=8192, NN,
A ~ N(0,1), B ~ N(0,0.02^2) cast to fp16 on the device before the timed region.
One step = one 8192^3 GEMM launch on operands resident in HBM.

Also reported (secondary): C2 fp32 4096^3 in NN/NT/TN/TT, C4 fused linear
(512x4096 . 11008x4096^T + b, ReLU and GELU), C5 CSR SpMM (65536^2 @ 0.1% x
65536x256) and SpMV, each with its roofline fraction.

Timing: W untimed warm-up steps, then K steps bracketed by device synchronisation,
timed with HIP events recorded on the stream the kernels are launched on.
cpu_baseline: the oracle's float64 GEMM (a restatement of gonum Dense.Mul
semantics) on a bounded row sample of the same problem, on the host cores.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "go-nngpu_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "GEMM TFLOP/s + % MFMA peak (fp32, fp16→fp32); CSR SpMM HBM GB/s, 1 MI355X"
PEAK_F16_TFLOPS = 2516.6   # dense MFMA fp16, 256 CU x 4096 flop/clk x 2.4 GHz
PEAK_F32_TFLOPS = 157.3    # fp32 MFMA
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed(fn, steps, warmup, stream):
    """Average ms per call of fn() over `steps`, events on `stream`."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def load_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE),
    recorded in profiles/traffic.json; None if not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def cpu_baseline_gemm(n, rows):
    """Oracle float64 GEMM on `rows` output rows of the n^3 problem; TFLOP/s."""
    import numpy as np

    from oracle import oracle as O

    A = O.normal((rows, n), 42, 101)
    B = O.normal((n, n), 42, 102, 0.0, 0.02)
    threads = O.threads()
    t0 = time.perf_counter()
    O.gemm_f64(A, B, nthreads=threads)
    dt = time.perf_counter() - t0
    del np
    return {"value": 2.0 * rows * n * n / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"oracle float64 GEMM ({rows}x{n}) . ({n}x{n}): {rows} of the {n} output rows, "
                      f"{dt:.1f} s on {threads} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=512)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (single-GPU build; "
              "see DESIGN.md for how the path shards)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import gonngpu as G
    from gonngpu import synth

    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    G.init()
    dev = torch.device("cuda:0")
    sp = stream.cuda_stream

    # ---------------------------------------------------------------- C3 headline
    n = 8192
    a32 = torch.empty((n, n), dtype=torch.float32, device=dev)
    b32 = torch.empty((n, n), dtype=torch.float32, device=dev)
    G.fill_normal(a32, 42, 1, 0.0, 1.0, stream_ptr=sp)
    G.fill_normal(b32, 42, 2, 0.0, 0.02, stream_ptr=sp)
    a16 = torch.empty((n, n), dtype=torch.float16, device=dev)
    b16 = torch.empty((n, n), dtype=torch.float16, device=dev)
    G.cast_f32_f16(a32, a16, stream_ptr=sp)
    G.cast_f32_f16(b32, b16, stream_ptr=sp)
    del a32, b32
    c = torch.empty((n, n), dtype=torch.float32, device=dev)

    def step():
        G.gemm(a16, b16, c, stream_ptr=sp)

    log(f"C3: {args.warmup} warmup + {args.steps} timed fp16 GEMM 8192^3 steps")
    ms = timed(step, args.steps, args.warmup, stream)
    flop = 2.0 * n * n * n
    tflops = flop / (ms * 1e-3) / 1e12
    assert torch.isfinite(c[:64]).all().item()
    log(f"C3: {ms:.4f} ms/step, {tflops:.1f} TFLOP/s ({100 * tflops / PEAK_F16_TFLOPS:.1f}% of fp16 peak)")
    traffic = load_traffic("gemm_f16_8192_nn")
    roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / PEAK_F16_TFLOPS, 4), "traffic": traffic,
                "kernel": "gemm_f16_kernel<256,256,64,2,4,NN>", "flop_per_launch": flop}
    del a16, b16, c
    torch.cuda.empty_cache()

    secondary = {}
    if not args.no_secondary:
        steps2 = max(5, args.steps // 5)
        # ------------------------------------------------------------ C2 fp32 4096^3
        m = 4096
        A = torch.empty((m, m), dtype=torch.float32, device=dev)
        B = torch.empty((m, m), dtype=torch.float32, device=dev)
        C = torch.empty((m, m), dtype=torch.float32, device=dev)
        G.fill_normal(A, 42, 3, stream_ptr=sp)
        G.fill_normal(B, 42, 4, stream_ptr=sp)
        for ta, tb, name in [(0, 0, "NN"), (0, 1, "NT"), (1, 0, "TN"), (1, 1, "TT")]:
            ms2 = timed(lambda: G.gemm(A, B, C, transA=bool(ta), transB=bool(tb), stream_ptr=sp), steps2, 3, stream)
            tf = 2.0 * m ** 3 / (ms2 * 1e-3) / 1e12
            secondary[f"c2_f32_4096_{name}"] = {"ms": round(ms2, 4), "TFLOP/s": round(tf, 2),
                                                "frac_fp32_peak": round(tf / PEAK_F32_TFLOPS, 4)}
            log(f"C2 {name}: {ms2:.3f} ms, {tf:.1f} TFLOP/s")
        del A, B, C
        # ------------------------------------------------------------ C4 fused linear
        X32 = torch.empty((512, 4096), dtype=torch.float32, device=dev)
        W32 = torch.empty((11008, 4096), dtype=torch.float32, device=dev)
        bias = torch.empty((11008,), dtype=torch.float32, device=dev)
        G.fill_normal(X32, 42, 5, stream_ptr=sp)
        G.fill_normal(W32, 42, 6, 0.0, 0.02, stream_ptr=sp)
        G.fill_normal(bias, 42, 7, 0.0, 0.01, stream_ptr=sp)
        X16 = torch.empty((512, 4096), dtype=torch.float16, device=dev)
        W16 = torch.empty((11008, 4096), dtype=torch.float16, device=dev)
        G.cast_f32_f16(X32, X16, stream_ptr=sp)
        G.cast_f32_f16(W32, W16, stream_ptr=sp)
        Y = torch.empty((512, 11008), dtype=torch.float32, device=dev)
        lin_flop = 2.0 * 512 * 11008 * 4096
        for act, name in [(G.ACT_RELU, "relu"), (G.ACT_GELU, "gelu")]:
            ms4 = timed(lambda: G.gemm(X16, W16, Y, transB=True, bias=bias, act=act, stream_ptr=sp), steps2 * 4, 5,
                        stream)
            tf = lin_flop / (ms4 * 1e-3) / 1e12
            secondary[f"c4_linear_{name}"] = {"ms": round(ms4, 5), "TFLOP/s": round(tf, 2),
                                              "frac_fp16_peak": round(tf / PEAK_F16_TFLOPS, 4)}
            log(f"C4 {name}: {ms4 * 1e3:.1f} us, {tf:.1f} TFLOP/s")
        del X32, W32, X16, W16, Y, bias
        # ------------------------------------------------------------ C5 SpMM / SpMV
        M = K = 65536
        N = 256
        rp, col, val = synth.csr_uniform(M, K, 65.536, seed=42)
        nnz = int(val.size)
        d_rp = torch.from_numpy(rp).to(dev)
        d_col = torch.from_numpy(col).to(dev)
        d_val = torch.from_numpy(val).to(dev)
        D = torch.empty((K, N), dtype=torch.float32, device=dev)
        G.fill_normal(D, 42, 8, stream_ptr=sp)
        Cs = torch.empty((M, N), dtype=torch.float32, device=dev)
        ms5 = timed(lambda: G.spmm_csr(M, N, K, nnz, d_rp, d_col, d_val, D, Cs, stream_ptr=sp), steps2 * 2, 3, stream)
        b_s = 4 * (M + 1) + 8 * nnz + 4 * nnz * N + 4 * M * N
        b_c = 4 * (M + 1) + 8 * nnz + 4 * K * N + 4 * M * N
        gbs = b_s / (ms5 * 1e-3) / 1e9
        secondary["c5_spmm"] = {"ms": round(ms5, 4), "nnz": nnz, "GB/s_streamed": round(gbs, 1),
                                "frac_hbm_streamed": round(gbs / PEAK_HBM_GBS, 4),
                                "GB/s_compulsory": round(b_c / (ms5 * 1e-3) / 1e9, 1),
                                "bytes_streamed": b_s, "bytes_compulsory": b_c,
                                "traffic": load_traffic("spmm_csr_c5")}
        log(f"C5 SpMM: {ms5:.4f} ms, {gbs:.0f} GB/s streamed-model")
        x = torch.empty((K,), dtype=torch.float32, device=dev)
        y = torch.empty((M,), dtype=torch.float32, device=dev)
        G.fill_normal(x, 42, 9, stream_ptr=sp)
        ms6 = timed(lambda: G.spmv_csr(M, K, nnz, d_rp, d_col, d_val, x, y, stream_ptr=sp), steps2 * 4, 5, stream)
        bv_s = 4 * (M + 1) + 12 * nnz + 4 * M
        secondary["c5_spmv"] = {"ms": round(ms6, 5), "GB/s_streamed": round(bv_s / (ms6 * 1e-3) / 1e9, 1),
                                "frac_hbm_streamed": round(bv_s / (ms6 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        log(f"C5 SpMV: {ms6 * 1e3:.1f} us")
        del d_rp, d_col, d_val, D, Cs, x, y

    cpu = None
    if not args.no_cpu:
        log(f"cpu_baseline: oracle float64 GEMM on {args.cpu_rows} rows of the 8192^3 problem")
        cpu = cpu_baseline_gemm(n, args.cpu_rows)
        log(f"cpu_baseline: {cpu['value'] * 1e3:.2f} GFLOP/s")

    out = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "C3: fp16-in/fp32-acc GEMM M=N=K=8192, NN, A~N(0,1), B~N(0,0.02^2) cast to fp16",
                   "M": n, "N": n, "K": n, "layout": "row-major NN", "accumulate": "f32", "output": "f32",
                   "parallelism": "single-gpu"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    del np
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
