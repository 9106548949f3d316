"""Benchmark of the MI355X GEMM / SpMM backend (one JSON line on stdout).

Headline (`value`): fp16-in / fp32-accumulate GEMM, M=N=K=8192, NN, A ~ N(0,1),
B ~ N(0,0.02^2), cast to fp16 on the device before the timed region (the
"headline MFMA-utilisation case" of the benchmark configurations). One step = one
8192^3 GEMM launch on operands resident in HBM.

Also measured (`secondary`): fp32 4096^3 GEMM in NN/NT/TN/TT, the fused linear
layer Y = act(X W^T + b) (X 512x4096, W 11008x4096 fp16, ReLU and GELU-tanh), CSR
SpMM (65536^2 at 0.1% density x 65536x256) and CSR SpMV, each with its roofline
fraction.

Timing: W untimed warm-up launches, then K launches bracketed by device
synchronisation, timed with HIP events recorded on the stream the kernels are
launched on; achieved = algorithmic flop (or bytes) per launch / mean launch time.

`roofline.traffic` is the HBM bytes per launch measured by rocprofv3 --pmc
(FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), read from
profiles/traffic.json when that file holds an entry for the kernel, else null.

cpu_baseline: the oracle's float64 GEMM (a restatement of gonum Dense.Mul
semantics) on a bounded row sample of the headline problem, on the host cores.

`e2e` (in `secondary`, never `value`): the headline GEMM from host memory through the
C ABI, PCIe included: upload fp32 A and B (create_gpu_buffer), cast both to fp16 on
the device, GEMM, download C (retrieve_gpu_buffer_data), wall-clock per step.

`ceiling` (in `secondary`, and `roofline.measured_ceiling_tflops`): the sustained rate of
the GEMM's matrix instruction with register operands and no memory traffic
(go-nngpu_amd/lib/mfma_ceiling, run as a child process right after the headline), on
operands with the headline's distributions and on all-zero operands. Under the board's
power limit the clock, and so this rate, depends on the operand values; the first figure
is the most any GEMM on such data can reach on the box.

`rows` times products of a few rows (a linear layer at batch 1-16: the NN GEMV kernel, the
small-product kernel's skinny NT branch, a small MLP layer) beside torch.mm, for scale.

`--only a,b,...` runs a subset of {c3, ceiling, c2, c1, c4, rows, spmm, spmv, e2e, copy} (used by
the rocprofv3 passes that produce profiles/); `copy` is a 1 GiB device copy used to
calibrate the HBM byte counters.
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
PEAK_F16_TFLOPS = 2516.6  # dense MFMA fp16, 256 CU x 4096 flop/clk x 2.4 GHz
PEAK_F32_TFLOPS = 157.3   # fp32 MFMA
MIN_WARM_MS = 50.0        # least untimed GPU time before each timed leg (see timed())
PEAK_HBM_GBS = 8000.0
ALL = ("c3", "ceiling", "c2", "c1", "c4", "rows", "spmm", "spmv", "e2e", "copy")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed(fn, steps, warmup, stream, min_warm_ms=0.0):
    """Mean ms per call of fn() over `steps` calls, events recorded on `stream`.

    `warmup` untimed calls come first; with min_warm_ms > 0 more untimed calls follow
    until at least that much GPU time has gone into warming up. Every leg uses this, the
    headline and its hipBLASLt line included, so all are timed at the same clock state:
    50 launches of a 50 us kernel are 2.5 ms, and kernels measured 10-25% slow that
    early after a leg change (clock ramp), settling within ~30 ms."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    if min_warm_ms > 0:
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        done = 0.0
        while done < min_warm_ms:
            for _ in range(10):
                fn()
            t1.record(stream)
            t1.synchronize()
            done = t0.elapsed_time(t1)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def load_traffic(name):
    """HBM bytes per launch for kernel `name` from profiles/traffic.json, or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            entry = json.load(f).get("kernels", {}).get(name)
    except (OSError, ValueError):
        return None
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def cpu_baseline_gemm(n, rows):
    """Oracle float64 GEMM on `rows` output rows of the n^3 problem (TFLOP/s)."""
    from oracle import oracle as O

    A = O.normal((rows, n), 42, 101)
    B = O.normal((n, n), 42, 102, 0.0, 0.02)
    threads = O.threads()
    t0 = time.perf_counter()
    O.gemm_f64(A, B, nthreads=threads)
    dt = time.perf_counter() - t0
    return {"value": 2.0 * rows * n * n / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"oracle float64 GEMM ({rows}x{n}) . ({n}x{n}): {rows} of the {n} output rows of the "
                      f"headline problem, {dt:.1f} s on {threads} threads (the GPU box's CPU share is 16)",
            "host": host_info()}


def host_info():
    """The CPU the baselines ran on: logical CPUs of the host, CPUs this process may use,
    the OpenMP thread setting and the model name."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"nproc": os.cpu_count(), "affinity": affinity, "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "cpu_model": model}


def cpu_gemm_1thread(n, rows):
    """The same oracle float64 GEMM restatement on one thread (a smaller row sample)."""
    from oracle import oracle as O

    A = O.normal((rows, n), 42, 101)
    B = O.normal((n, n), 42, 102, 0.0, 0.02)
    t0 = time.perf_counter()
    O.gemm_f64(A, B, nthreads=1)
    dt = time.perf_counter() - t0
    return {"value": round(2.0 * rows * n * n / dt / 1e12, 5), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"oracle float64 GEMM ({rows}x{n}) . ({n}x{n}) on one thread, {dt:.1f} s"}


def cpu_numpy_gemm(n, rows):
    """numpy float64 matmul (OpenBLAS, its own threads) on the same sample: an optimised
    CPU line beside the oracle's plain restatement of gonum's Dense.Mul semantics."""
    import numpy as np

    from oracle import oracle as O

    A = O.normal((rows, n), 42, 101).astype(np.float64)
    B = O.normal((n, n), 42, 102, 0.0, 0.02).astype(np.float64)
    t0 = time.perf_counter()
    np.matmul(A, B)
    dt = time.perf_counter() - t0
    return {"value": round(2.0 * rows * n * n / dt / 1e12, 4), "unit": "TFLOP/s",
            "sample": f"numpy float64 matmul ({rows}x{n}) . ({n}x{n}), {dt:.2f} s"}


class Ctx:
    def __init__(self, args):
        import torch

        import gonngpu as G

        self.G = G
        self.torch = torch
        torch.cuda.set_device(0)
        self.stream = torch.cuda.Stream()
        torch.cuda.set_stream(self.stream)
        G.init()
        self.dev = torch.device("cuda:0")
        self.sp = self.stream.cuda_stream
        self.args = args

    def empty(self, shape, dtype=None):
        return self.torch.empty(shape, dtype=dtype or self.torch.float32, device=self.dev)

    def f16_normal(self, shape, sid, std):
        """N(0, std^2) generated on the device in fp32, cast to fp16 (RNE)."""
        x32 = self.empty(shape)
        self.G.fill_normal(x32, 42, sid, 0.0, std, stream_ptr=self.sp)
        x16 = self.empty(shape, self.torch.float16)
        self.G.cast_f32_f16(x32, x16, stream_ptr=self.sp)
        del x32
        return x16


def run_c3(c, steps, warmup):
    n = 8192
    a16 = c.f16_normal((n, n), 1, 1.0)
    b16 = c.f16_normal((n, n), 2, 0.02)
    out = c.empty((n, n))
    log(f"c3: {warmup} warmup launches (then at least {MIN_WARM_MS:.0f} ms of untimed launches) + {steps} timed "
        f"fp16 GEMM 8192^3 launches")
    ms = timed(lambda: c.G.gemm(a16, b16, out, stream_ptr=c.sp), steps, warmup, c.stream, MIN_WARM_MS)
    flop = 2.0 * n ** 3
    tf = flop / (ms * 1e-3) / 1e12
    assert c.torch.isfinite(out[:64]).all().item()
    log(f"c3: {ms:.4f} ms/launch, {tf:.1f} TFLOP/s ({100 * tf / PEAK_F16_TFLOPS:.1f}% of fp16 dense peak)")
    c.vendor_c3 = reference_or_note(vendor_reference, c, a16, b16, flop, steps, "c3")
    return {"ms": ms, "tflops": tf, "flop": flop}


def vendor_reference(c, a, b, flop, steps, name):
    """The same product through torch.mm (hipBLASLt) on the same box, for scale only, never
    `value`: with fp32 output (out_dtype), the contract of this library's GEMM, and with
    torch's default fp16 output (half the C bytes)."""
    t = c.torch
    ms = timed(lambda: t.mm(a, b, out_dtype=t.float32), steps, 10, c.stream, MIN_WARM_MS)
    ms16 = timed(lambda: t.mm(a, b), steps, 10, c.stream, MIN_WARM_MS)
    tf, tf16 = flop / (ms * 1e-3) / 1e12, flop / (ms16 * 1e-3) / 1e12
    log(f"{name} torch.mm (hipBLASLt): fp32 out {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s; "
        f"fp16 out {ms16 * 1e3:.1f} us, {tf16:.1f} TFLOP/s")
    return {"ms": round(ms, 5), "TFLOP/s": round(tf, 2), "fp16_out_ms": round(ms16, 5),
            "fp16_out_TFLOP/s": round(tf16, 2),
            "what": "torch.mm on the same fp16 operands (hipBLASLt), no epilogue: fp32 output "
                    "(out_dtype=float32, this library's contract); fp16_out_*: torch's default fp16 output"}


def sparse_vendor_reference(c, csr, dense, out, steps, b_streamed, kind):
    """The same C5 product through torch's CSR tensor (hipSPARSE over rocSPARSE) on the same
    device arrays, for scale only: torch.mm for SpMM, torch.mv for SpMV. Its sums run in
    another order, so its result is checked against this library's loosely (relFrob 1e-5)."""
    t = c.torch
    M, K, nnz, d_rp, d_col, d_val = csr
    S = t.sparse_csr_tensor(d_rp, d_col, d_val, size=(M, K))
    op = (lambda: t.mm(S, dense)) if kind == "spmm" else (lambda: t.mv(S, dense))
    ref = op()
    t.cuda.synchronize()
    err = (t.linalg.vector_norm((ref - out).double()) / t.linalg.vector_norm(out.double())).item()
    ms = timed(op, steps, 10, c.stream, MIN_WARM_MS)
    gbs = b_streamed / (ms * 1e-3) / 1e9
    log(f"{kind} torch CSR (hipSPARSE): {ms * 1e3:.1f} us, {gbs:.0f} GB/s streamed-bytes model, "
        f"relFrob {err:.1e} against this library's result")
    return {"ms": round(ms, 5), "GB/s_streamed": round(gbs, 1), "relFrob_vs_this_library": err,
            "what": f"torch.{'mm' if kind == 'spmm' else 'mv'} on a torch.sparse_csr_tensor over the same device "
                    "arrays (hipSPARSE / rocSPARSE), a new output tensor per call"}


def reference_or_note(fn, *args):
    """A vendor line for scale: its failure is recorded, never fatal to the bench."""
    try:
        return fn(*args)
    except Exception as e:  # noqa: BLE001 - any failure of a comparison line is only reported
        log(f"{fn.__name__} failed: {type(e).__name__}: {e}")
        return {"failed": f"{type(e).__name__}: {e}"}


def rocsparse_reference(c, csr, dense, out, steps, b_streamed, kind):
    """The same C5 product through rocSPARSE's generic API (rocsparse_spmm / rocsparse_spmv,
    librocsparse.so through ctypes) on the same device arrays and stream, for scale only: the
    buffer-size and preprocess (analysis) stages run once, then only the compute stage is timed,
    for each CSR algorithm that accepts the problem. Results are checked against this
    library's loosely (relFrob 1e-5; the sums run in another order)."""
    import ctypes

    t = c.torch
    try:
        R = ctypes.CDLL("librocsparse.so")
    except OSError as e:
        return {"skipped": f"librocsparse.so not loadable: {e}"}
    vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    OP_NONE, I32, BASE0, F32, ROW = 111, 2, 0, 151, 0
    M, K, nnz, d_rp, d_col, d_val = csr

    def ok(st, what):
        if st != 0:
            raise RuntimeError(f"{what}: rocsparse status {st}")

    h, A, X, Y = vp(), vp(), vp(), vp()
    ok(R.rocsparse_create_handle(ctypes.byref(h)), "create_handle")
    ok(R.rocsparse_set_stream(h, vp(c.sp)), "set_stream")
    ok(R.rocsparse_create_csr_descr(ctypes.byref(A), i64(M), i64(K), i64(nnz), vp(d_rp.data_ptr()),
                                    vp(d_col.data_ptr()), vp(d_val.data_ptr()), ci(I32), ci(I32), ci(BASE0), ci(F32)),
       "create_csr_descr")
    res = t.empty_like(out)
    alpha, beta = ctypes.c_float(1.0), ctypes.c_float(0.0)
    if kind == "spmm":
        N = dense.shape[1]
        ok(R.rocsparse_create_dnmat_descr(ctypes.byref(X), i64(K), i64(N), i64(N), vp(dense.data_ptr()), ci(F32),
                                          ci(ROW)), "create_dnmat_descr B")
        ok(R.rocsparse_create_dnmat_descr(ctypes.byref(Y), i64(M), i64(N), i64(N), vp(res.data_ptr()), ci(F32),
                                          ci(ROW)), "create_dnmat_descr C")
        algs = {"default": 0, "csr": 1, "csr_row_split": 4, "csr_nnz_split": 5, "csr_merge_path": 9}

        def call(alg, stage, size, buf):
            return R.rocsparse_spmm(h, ci(OP_NONE), ci(OP_NONE), ctypes.byref(alpha), A, X, ctypes.byref(beta), Y,
                                    ci(F32), ci(alg), ci(stage), size, buf)
    else:
        ok(R.rocsparse_create_dnvec_descr(ctypes.byref(X), i64(K), vp(dense.data_ptr()), ci(F32)), "create x")
        ok(R.rocsparse_create_dnvec_descr(ctypes.byref(Y), i64(M), vp(res.data_ptr()), ci(F32)), "create y")
        algs = {"default": 0, "csr_adaptive": 2, "csr_rowsplit": 3, "csr_lrb": 7, "csr_nnzsplit": 8}

        def call(alg, stage, size, buf):
            return R.rocsparse_spmv(h, ci(OP_NONE), ctypes.byref(alpha), A, X, ctypes.byref(beta), Y, ci(F32),
                                    ci(alg), ci(stage), size, buf)
    per_alg = {}
    try:
        for name, alg in algs.items():
            size = ctypes.c_size_t(0)
            if call(alg, 1, ctypes.byref(size), None) != 0:  # buffer size
                per_alg[name] = "not supported"
                continue
            buf = t.empty(max(int(size.value), 256), dtype=t.uint8, device=out.device)
            if call(alg, 2, ctypes.byref(size), vp(buf.data_ptr())) != 0:  # preprocess (analysis), once
                per_alg[name] = "preprocess failed"
                continue
            if call(alg, 3, ctypes.byref(size), vp(buf.data_ptr())) != 0:
                per_alg[name] = "compute failed"
                continue
            t.cuda.synchronize()
            err = (t.linalg.vector_norm((res - out).double()) / t.linalg.vector_norm(out.double())).item()
            # wall clock between device-wide synchronisations: some algorithms launch on a stream
            # of their own, which events recorded on this stream would not see
            for _ in range(10):
                call(alg, 3, ctypes.byref(size), vp(buf.data_ptr()))
            res.zero_()
            t.cuda.synchronize()
            n = max(steps, 50)
            bad = 0
            t0 = time.perf_counter()
            for _ in range(n):
                bad += call(alg, 3, ctypes.byref(size), vp(buf.data_ptr())) != 0
            t.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3 / n
            err2 = (t.linalg.vector_norm((res - out).double()) / t.linalg.vector_norm(out.double())).item()
            if bad or not err2 <= 1e-5:  # the timed calls must each have computed the product
                per_alg[name] = f"repeated compute calls: {bad} of {n} failed, result relFrob {err2:.1e}"
                continue
            per_alg[name] = {"ms": round(ms, 5), "GB/s_streamed": round(b_streamed / (ms * 1e-3) / 1e9, 1),
                             "relFrob_vs_this_library": err}
    finally:
        t.cuda.synchronize()
        destroy_dense = R.rocsparse_destroy_dnmat_descr if kind == "spmm" else R.rocsparse_destroy_dnvec_descr
        destroy_dense(X)
        destroy_dense(Y)
        R.rocsparse_destroy_spmat_descr(A)
        R.rocsparse_destroy_handle(h)
    timed_algs = {k: v for k, v in per_alg.items() if isinstance(v, dict) and v["relFrob_vs_this_library"] <= 1e-5}
    best = min(timed_algs, key=lambda k: timed_algs[k]["ms"]) if timed_algs else None
    if best:
        b = timed_algs[best]
        log(f"{kind} rocSPARSE ({best}, analysis done once): {b['ms'] * 1e3:.1f} us, {b['GB/s_streamed']:.0f} GB/s "
            f"streamed-bytes model, relFrob {b['relFrob_vs_this_library']:.1e} against this library's result")
    else:
        log(f"{kind} rocSPARSE: no algorithm timed ({per_alg})")
    return {"best_alg": best, "ms": timed_algs[best]["ms"] if best else None, "per_alg": per_alg,
            "what": "rocsparse_spmm / rocsparse_spmv compute stage on the same device arrays, after one "
                    "buffer-size and preprocess call per algorithm; wall clock per call over back-to-back calls "
                    "between device-wide synchronisations (includes each call's launch cost)"}


def run_c2(c, steps, warmup):
    m = 4096
    A, B, C = c.empty((m, m)), c.empty((m, m)), c.empty((m, m))
    c.G.fill_normal(A, 42, 3, stream_ptr=c.sp)
    c.G.fill_normal(B, 42, 4, stream_ptr=c.sp)
    res = {}
    for ta, tb, name in [(0, 0, "NN"), (0, 1, "NT"), (1, 0, "TN"), (1, 1, "TT")]:
        ms = timed(lambda: c.G.gemm(A, B, C, transA=bool(ta), transB=bool(tb), stream_ptr=c.sp), steps, warmup,
                   c.stream, MIN_WARM_MS)
        tf = 2.0 * m ** 3 / (ms * 1e-3) / 1e12
        res[f"c2_f32_4096_{name}"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 2),
                                      "frac_fp32_peak": round(tf / PEAK_F32_TFLOPS, 4)}
        log(f"c2 {name}: {ms:.3f} ms, {tf:.1f} TFLOP/s ({100 * tf / PEAK_F32_TFLOPS:.1f}% of fp32 peak)")
    res["c2_torch_matmul_reference"] = reference_or_note(c2_vendor_reference, c, A, B, steps)
    return res


def c2_vendor_reference(c, A, B, steps):
    """The C2 NN product through torch.mm (hipBLASLt, fp32 in and out, TF32 off), for scale only."""
    t = c.torch
    m = A.shape[0]
    prev_tf32 = t.backends.cuda.matmul.allow_tf32
    t.backends.cuda.matmul.allow_tf32 = False  # full fp32, as this library computes
    try:
        ms = timed(lambda: t.mm(A, B), steps, 10, c.stream, MIN_WARM_MS)
    finally:
        t.backends.cuda.matmul.allow_tf32 = prev_tf32
    tf = 2.0 * m ** 3 / (ms * 1e-3) / 1e12
    log(f"c2 torch.mm (hipBLASLt) NN: {ms:.3f} ms, {tf:.1f} TFLOP/s")
    return {"ms": round(ms, 4), "TFLOP/s": round(tf, 2),
            "what": "torch.mm on the same fp32 NN operands (hipBLASLt), TF32 off"}


def run_c1(c, steps, warmup):
    """C1: fp32 256^3, entries U[-1,1]. The kernel time per launch inside a captured HIP graph
    of 20 launches (HIP events around the replays: launched one by one from Python the
    kernel waits on the host), the device API's back-to-back launch rate, and the wall clock
    of the synchronous Part-1 call perform_mps_matrix_multiplication on GPUPtr buffers, as
    the gonum facade's Mul makes it."""
    import numpy as np
    import torch

    from gonngpu import synth

    G, n = c.G, 256
    A, B, C = c.empty((n, n)), c.empty((n, n)), c.empty((n, n))
    c.G.fill_uniform(A, 42, 11, stream_ptr=c.sp)
    c.G.fill_uniform(B, 42, 12, stream_ptr=c.sp)
    eager = timed(lambda: c.G.gemm(A, B, C, stream_ptr=c.sp), steps, warmup, c.stream, MIN_WARM_MS)
    reps = 20
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=c.stream):
        cap = torch.cuda.current_stream().cuda_stream
        for _ in range(reps):
            c.G.gemm(A, B, C, stream_ptr=cap)
    ms = timed(graph.replay, max(10, steps // reps), 5, c.stream, MIN_WARM_MS) / reps
    ha, hb = synth.host_uniform((n, n), 13), synth.host_uniform((n, n), 14)
    ba, bb, bc = G.Buffer.from_array(ha), G.Buffer.from_array(hb), G.Buffer(n * n * 4)
    call = lambda: G.call("perform_mps_matrix_multiplication", ba.handle, n, n, bb.handle, n, n, bc.handle, n, n,
                          None)
    for _ in range(max(3, warmup)):
        call()
    t0 = time.perf_counter()
    for _ in range(steps):
        call()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    out = bc.to_array((n, n))
    assert np.isfinite(out).all()
    for b in (ba, bb, bc):
        b.release()
    tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
    log(f"c1 256^3 fp32: kernel {ms * 1e3:.1f} us ({tf:.2f} TFLOP/s) per launch in a graph, device API "
        f"{eager * 1e3:.1f} us per back-to-back launch, perform_mps_matrix_multiplication {wall * 1e3:.1f} us "
        f"per synchronous call")
    return {"kernel_us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 3), "launch_us": round(eager * 1e3, 2),
            "part1_call_us": round(wall * 1e3, 1),
            "what": "kernel_us: per launch inside a captured HIP graph of 20 launches; launch_us: device API "
                    "launches back to back from Python; part1_call_us: the synchronous Part-1 call's wall clock "
                    "(launch + completion wait) on resident GPUPtr buffers"}


def run_c4(c, steps, warmup):
    X16 = c.f16_normal((512, 4096), 5, 1.0)
    W16 = c.f16_normal((11008, 4096), 6, 0.02)
    bias = c.empty((11008,))
    c.G.fill_normal(bias, 42, 7, 0.0, 0.01, stream_ptr=c.sp)
    Y = c.empty((512, 11008))
    flop = 2.0 * 512 * 11008 * 4096
    res = {}
    for act, name in [(c.G.ACT_RELU, "relu"), (c.G.ACT_GELU, "gelu")]:
        ms = timed(lambda: c.G.gemm(X16, W16, Y, transB=True, bias=bias, act=act, stream_ptr=c.sp), steps, warmup,
                   c.stream, MIN_WARM_MS)
        tf = flop / (ms * 1e-3) / 1e12
        res[f"c4_linear_{name}"] = {"ms": round(ms, 5), "TFLOP/s": round(tf, 2),
                                    "frac_fp16_peak": round(tf / PEAK_F16_TFLOPS, 4)}
        log(f"c4 {name}: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s")
    res["c4_torch_matmul_reference"] = reference_or_note(vendor_reference, c, X16, W16.t(), flop, steps, "c4")
    res["c4_interleaved"] = reference_or_note(c4_interleaved, c, X16, W16, bias, Y, flop, steps)
    return res


def run_rows(c, steps):
    """Products of a few rows beside torch.mm (TF32 off; fp32 output for fp16 inputs), event
    timing of back-to-back launches: X W with W stored K x N (NN, the GEMV kernel), X W^T with W
    stored N x K (NT, the small-product kernel's skinny branch), and a small MLP layer. The rate
    is W's bytes over the time (W is read once; X and C are a few rows)."""
    t = c.torch
    t.backends.cuda.matmul.allow_tf32 = False
    cases = [("f32", "NN", 1, 11008, 4096), ("f32", "NN", 2, 16384, 2048), ("f32", "NT", 1, 11008, 4096),
             ("f16", "NN", 1, 16384, 2048), ("f16", "NT", 2, 11008, 4096), ("f32", "NN", 128, 784, 784)]
    out = {}
    for dt, lay, M, N, K in cases:
        tdt = t.float16 if dt == "f16" else t.float32
        X = t.randn(M, K, device=c.dev).to(tdt)
        W = (0.02 * t.randn(N, K, device=c.dev)).to(tdt) if lay == "NT" else (0.02 * t.randn(K, N, device=c.dev)).to(tdt)
        Y = t.empty(M, N, device=c.dev)
        tb = lay == "NT"
        ours = timed(lambda: c.G.gemm(X, W, Y, transB=tb, stream_ptr=c.sp), steps, 10, c.stream, MIN_WARM_MS / 5)
        Wm = W.t() if tb else W
        ref = (lambda: t.mm(X, Wm, out_dtype=t.float32)) if dt == "f16" else (lambda: t.mm(X, Wm, out=Y))
        theirs = timed(ref, steps, 10, c.stream, MIN_WARM_MS / 5)
        wb = N * K * (2 if dt == "f16" else 4)
        key = f"{dt}_{lay}_{M}x{N}x{K}"
        out[key] = {"us": round(ours * 1e3, 2), "TB/s_of_W": round(wb / (ours * 1e-3) / 1e12, 2),
                    "torch_mm_us": round(theirs * 1e3, 2)}
        log(f"rows {key}: {ours * 1e3:.1f} us ({wb / (ours * 1e-3) / 1e12:.2f} TB/s of W), torch.mm {theirs * 1e3:.1f} us")
    out["what"] = ("kernel time per launch (back-to-back launches, HIP events) of this library's gn_gemm and of "
                   "torch.mm on the same operands; torch.mm's launches from Python cost ~18 us each, so its "
                   "figures below that are its call floor, not its kernel")
    return out


def c4_interleaved(c, X16, W16, bias, Y, flop, steps, rounds=7):
    """The C4 lines again in alternation: each round times ReLU, GELU and torch.mm (hipBLASLt,
    fp32 and fp16 output) back to back on the same operands, and each line reports its median
    over the rounds, so that no line is favoured by its place in the order (the board's power
    limit moves the clock between legs run one after the other)."""
    import statistics

    t = c.torch
    Wt = W16.t()
    fns = {"relu": lambda: c.G.gemm(X16, W16, Y, transB=True, bias=bias, act=c.G.ACT_RELU, stream_ptr=c.sp),
           "gelu": lambda: c.G.gemm(X16, W16, Y, transB=True, bias=bias, act=c.G.ACT_GELU, stream_ptr=c.sp),
           "torch_fp32_out": lambda: t.mm(X16, Wt, out_dtype=t.float32),
           "torch_fp16_out": lambda: t.mm(X16, Wt)}
    n = max(20, steps // rounds)
    per = {k: [] for k in fns}
    for _ in range(rounds):
        for k, fn in fns.items():
            per[k].append(timed(fn, n, 5, c.stream))
    med = {k: statistics.median(v) for k, v in per.items()}
    log("c4 interleaved (median of %d rounds of %d launches): " % (rounds, n) +
        ", ".join(f"{k} {v * 1e3:.1f} us" for k, v in med.items()))
    out = {f"{k}_ms": round(v, 5) for k, v in med.items()}
    out.update({f"{k}_TFLOP/s": round(flop / (v * 1e-3) / 1e12, 2) for k, v in med.items()})
    out["what"] = ("the four C4 lines timed in alternation, %d rounds of %d launches each, median per line "
                   "(this library's ReLU and GELU with bias; torch.mm without an epilogue)" % (rounds, n))
    return out


def csr_workload(c):
    from gonngpu import synth

    M = K = 65536
    rp, col, val = synth.csr_uniform(M, K, 65.536, seed=42)
    t = c.torch
    c.csr_host = (rp, col, val)  # for the CPU baselines
    return M, K, int(val.size), t.from_numpy(rp).to(c.dev), t.from_numpy(col).to(c.dev), t.from_numpy(val).to(c.dev)


def cpu_baseline_sparse(c, kind, rows):
    """The reference's own CPU loop for SpMM (metal_bridge_sparse.m:117-133) or SpMV
    (:325-339), restated in the oracle and run on one thread as the reference runs it, on
    the first `rows` rows of the C5 matrix; reported in the GPU leg's streamed-bytes units."""
    from oracle import oracle as O

    rp, col, val = c.csr_host
    M = rp.size - 1
    rows = min(rows, M)
    end = int(rp[rows])
    srp, scol, sval = rp[:rows + 1], col[:end], val[:end]
    if kind == "spmm":
        N = 256
        D = O.normal((M, N), 42, 108)
        t0 = time.perf_counter()
        O.spmm_f32(srp, scol, sval, D)
        dt = time.perf_counter() - t0
        b_s = 4 * (rows + 1) + 8 * end + 4 * end * N + 4 * rows * N
    else:
        x = O.normal((M,), 42, 109)
        t0 = time.perf_counter()
        O.spmv_f32(srp, scol, sval, x)
        dt = time.perf_counter() - t0
        b_s = 4 * (rows + 1) + 12 * end + 4 * rows
    return {"value": round(b_s / dt / 1e9, 2), "unit": "GB/s (streamed-bytes model)", "cores": 1, "kind": "port",
            "ms_full_matrix": round(dt * 1e3 * M / rows, 2),
            "sample": f"oracle restatement of the reference's single-threaded CSR {kind} loop on rows 0..{rows - 1} "
                      f"of the {M}-row C5 matrix ({end} stored entries), {dt:.2f} s"}


def cpu_parallel_sparse(c, kind):
    """The same CSR loop with its rows split over the host threads (OpenMP; each row as the
    reference computes it, bit-identical), on the whole C5 matrix."""
    from oracle import oracle as O

    rp, col, val = c.csr_host
    M = rp.size - 1
    nnz = int(rp[-1])
    threads = O.threads()
    if kind == "spmm":
        N = 256
        D = O.normal((M, N), 42, 108)
        O.spmm_f32_par(rp[:1025], col[:int(rp[1024])], val[:int(rp[1024])], D, threads)  # page in, spin up
        t0 = time.perf_counter()
        O.spmm_f32_par(rp, col, val, D, threads)
        dt = time.perf_counter() - t0
        b_s = 4 * (M + 1) + 8 * nnz + 4 * nnz * N + 4 * M * N
    else:
        x = O.normal((M,), 42, 109)
        O.spmv_f32_par(rp, col, val, x, threads)
        t0 = time.perf_counter()
        O.spmv_f32_par(rp, col, val, x, threads)
        dt = time.perf_counter() - t0
        b_s = 4 * (M + 1) + 12 * nnz + 4 * M
    return {"value": round(b_s / dt / 1e9, 2), "unit": "GB/s (streamed-bytes model)", "cores": threads,
            "kind": "port", "ms_full_matrix": round(dt * 1e3, 3),
            "sample": f"the reference's CSR {kind} loop split by rows over {threads} OpenMP threads, whole C5 matrix "
                      f"({nnz} stored entries)"}


def run_part1_sparse(c, kind, steps, kernel_ms):
    """C5 through the reference-compatible entry point (perform_sparse_dense_matmul or
    perform_sparse_matvec) as the unchanged Go caller makes it: values in a GPUPtr buffer,
    row pointers and column indices as host arrays on every call. The first call uploads
    and validates the index arrays; later calls reuse the copy kept with the values
    buffer. Wall clock per synchronous call, against the device-API kernel time."""
    import numpy as np

    G = c.G
    rp, col, val = c.csr_host
    M = rp.size - 1
    N = 256 if kind == "spmm" else 1
    from gonngpu import synth

    dense = synth.host_normal((M, N), 110) if kind == "spmm" else synth.host_normal((M,), 111)
    bv, bd, bo = G.Buffer.from_array(val), G.Buffer.from_array(dense), G.Buffer(M * N * 4)
    if kind == "spmm":
        args = lambda: (bv.handle, rp.ctypes.data, rp.size, col.ctypes.data, col.size, M, M, val.size, bd.handle, M,
                        N, bo.handle, M, N, None)
        name = "perform_sparse_dense_matmul"
    else:
        args = lambda: (bv.handle, rp.ctypes.data, rp.size, col.ctypes.data, col.size, M, M, val.size, bd.handle, M,
                        bo.handle, M, None)
        name = "perform_sparse_matvec"
    a = args()  # built once, as a Go caller's arguments are: only the call itself is timed
    t0 = time.perf_counter()
    G.call(name, *a)
    first = (time.perf_counter() - t0) * 1e3
    for _ in range(50):  # the per-call time settles over the first tens of synchronous calls
        G.call(name, *a)
    t0 = time.perf_counter()
    for _ in range(steps):
        G.call(name, *a)
    steady = (time.perf_counter() - t0) * 1e3 / steps
    out = bo.to_array((M, N) if kind == "spmm" else (M,))
    assert np.isfinite(out[:16]).all()
    for b in (bv, bd, bo):
        b.release()
    log(f"{kind} via {name}: first call {first:.2f} ms, steady {steady:.4f} ms (kernel {kernel_ms:.4f} ms)")
    return {"first_call_ms": round(first, 3), "steady_ms": round(steady, 4),
            "steady_over_kernel": round(steady / kernel_ms, 3),
            "what": f"{name} with host index arrays (Go call sequence), wall clock per synchronous call; the first "
                    f"call uploads and validates the indices, later calls reuse them"}


def run_spmm(c, steps, warmup, csr):
    M, K, nnz, d_rp, d_col, d_val = csr
    N = 256
    D = c.empty((K, N))
    c.G.fill_normal(D, 42, 8, stream_ptr=c.sp)
    Cs = c.empty((M, N))
    ms = timed(lambda: c.G.spmm_csr(M, N, K, nnz, d_rp, d_col, d_val, D, Cs, stream_ptr=c.sp), steps, warmup,
               c.stream, MIN_WARM_MS)
    b_s = 4 * (M + 1) + 8 * nnz + 4 * nnz * N + 4 * M * N
    b_c = 4 * (M + 1) + 8 * nnz + 4 * K * N + 4 * M * N
    gbs = b_s / (ms * 1e-3) / 1e9
    traffic = load_traffic("spmm_csr_c5")
    log(f"spmm: {ms:.4f} ms, {gbs:.0f} GB/s effective (streamed-bytes model), nnz {nnz}")
    out = {"ms": round(ms, 5), "nnz": nnz, "GB/s_streamed": round(gbs, 1),
           "frac_hbm_streamed": round(gbs / PEAK_HBM_GBS, 4),
           "GB/s_compulsory": round(b_c / (ms * 1e-3) / 1e9, 1), "bytes_streamed": b_s,
           "bytes_compulsory": b_c, "traffic": traffic,
           "note": "streamed bytes count every D-row gather (an effective bandwidth: the gathers are "
                   "served by L2 and the Infinity Cache, so it can exceed the HBM peak); the measured rate "
                   "is the L2 refill traffic per call (FETCH_SIZE + WRITE_SIZE summed over the call's two "
                   "kernel launches, Infinity Cache hits included) over the call's time"}
    if traffic:
        refill = traffic / (ms * 1e-3) / 1e9
        out["GB/s_l2_refill"] = round(refill, 1)
        out["frac_8TBps_l2_refill"] = round(refill / PEAK_HBM_GBS, 4)
        log(f"spmm: {refill:.0f} GB/s of measured L2 refill traffic ({traffic / 1e9:.2f} GB per call)")
    out["torch_sparse_reference"] = reference_or_note(sparse_vendor_reference, c, csr, D, Cs, steps, b_s, "spmm")
    out["rocsparse_reference"] = reference_or_note(rocsparse_reference, c, csr, D, Cs, steps, b_s, "spmm")
    return out


def run_spmv(c, steps, warmup, csr):
    """C5 SpMV two ways on the same device arrays: the grouped layout (gn_spmv_plan_*, the
    kernel perform_sparse_matvec runs once the indices kept with the values buffer are
    validated) and the flat kernel (gn_spmv_csr, the first, validating call's kernel)."""
    M, K, nnz, d_rp, d_col, d_val = csr
    x, y = c.empty((K,)), c.empty((M,))
    c.G.fill_normal(x, 42, 9, stream_ptr=c.sp)
    c.torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan = c.G.SpmvPlan(M, K, nnz, d_rp, d_col, stream_ptr=c.sp)
    c.torch.cuda.synchronize()
    plan_ms = (time.perf_counter() - t0) * 1e3
    ms = timed(lambda: plan.run(d_val, x, y, stream_ptr=c.sp), steps, warmup, c.stream, MIN_WARM_MS)
    flat_ms = timed(lambda: c.G.spmv_csr(M, K, nnz, d_rp, d_col, d_val, x, y, stream_ptr=c.sp), steps, warmup,
                    c.stream, MIN_WARM_MS)
    plan.run(d_val, x, y, stream_ptr=c.sp)  # y = the grouped kernel's result, for the reference check
    c.torch.cuda.synchronize()
    plan.release(stream_ptr=c.sp)
    # compulsory bytes: row pointers, values, x and y once, and the layout per entry (one
    # 4-byte word of column and CSR position for K <= 65536, else 4 + 2 bytes)
    layout_b = 4 if K <= 65536 else 6
    b_s = 4 * (M + 1) + 4 * nnz + layout_b * nnz + 4 * K + 4 * M
    b_flat = 4 * (M + 1) + 8 * nnz + 4 * K + 4 * M
    # the benchmark's streamed-bytes model (row pointers, columns, values, one x gather per
    # entry, y), the unit of the CPU lines
    b_streamed = 4 * (M + 1) + 12 * nnz + 4 * M
    gbs = b_s / (ms * 1e-3) / 1e9
    gbs_streamed = b_streamed / (ms * 1e-3) / 1e9
    log(f"spmv: grouped {ms * 1e3:.1f} us, {gbs_streamed:.0f} GB/s streamed-bytes model, {gbs:.0f} GB/s of "
        f"compulsory bytes (plan built in {plan_ms:.1f} ms); flat kernel {flat_ms * 1e3:.1f} us")
    res = {"ms": round(ms, 5), "kernel": "spmv_grouped_kernel", "GB/s_streamed": round(gbs_streamed, 1),
            "frac_hbm_streamed": round(gbs_streamed / PEAK_HBM_GBS, 4), "bytes_streamed": b_streamed,
            "GB/s_compulsory": round(gbs, 1),
            "frac_hbm_compulsory": round(gbs / PEAK_HBM_GBS, 4), "bytes_compulsory": b_s,
            "plan_build_ms": round(plan_ms, 3),
            "flat_kernel_ms": round(flat_ms, 5), "flat_GB/s_compulsory": round(b_flat / (flat_ms * 1e-3) / 1e9, 1),
            "what": "grouped layout (gn_spmv_plan_run) on resident device arrays; flat_kernel_*: gn_spmv_csr "
                    "(no layout) on the same arrays"}
    res["torch_sparse_reference"] = reference_or_note(sparse_vendor_reference, c, csr, x, y, steps, b_streamed,
                                                      "spmv")
    res["rocsparse_reference"] = reference_or_note(rocsparse_reference, c, csr, x, y, steps, b_streamed, "spmv")
    return res


def run_e2e(c, steps, warmup):
    """C3 from host fp32 arrays: upload, device fp16 cast, GEMM, download (wall clock)."""
    import numpy as np

    from gonngpu import synth

    G = c.G
    n = 8192
    A = synth.host_normal((n, n), 201)
    B = synth.host_normal((n, n), 202, 0.0, 0.02)
    Cout = np.empty((n, n), dtype=np.float32)

    def step():
        ba, bb = G.Buffer.from_array(A), G.Buffer.from_array(B)
        a16, b16, bc = G.Buffer(n * n * 2), G.Buffer(n * n * 2), G.Buffer(n * n * 4)
        G.call("gn_cast_f32_f16", ba.device_ptr, a16.device_ptr, n * n, G.ROUND_NEAREST_EVEN, None)
        G.call("gn_cast_f32_f16", bb.device_ptr, b16.device_ptr, n * n, G.ROUND_NEAREST_EVEN, None)
        G.call("gn_gemm", G.GN_F16, 0, 0, n, n, n, 1.0, a16.device_ptr, n, 0, b16.device_ptr, n, 0, 0.0,
               bc.device_ptr, n, 0, 1, None, G.ACT_NONE, 0.0, None)
        G.call("retrieve_gpu_buffer_data", bc.handle, Cout.ctypes.data, Cout.nbytes)
        for b in (ba, bb, a16, b16, bc):
            b.release()

    for _ in range(warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
    assert np.isfinite(Cout[:4]).all()
    log(f"e2e: {ms:.2f} ms per host-to-host 8192^3 fp16 GEMM (PCIe included), {tf:.1f} TFLOP/s")
    return {"ms": round(ms, 3), "TFLOP/s": round(tf, 1),
            "steps": f"upload A, B fp32 (256 MiB each), device fp16 cast, GEMM, download C fp32 (256 MiB)"}


def run_ceiling(seconds=3.0):
    """The register-operand MFMA rate (see the module docstring), from the probe executable."""
    import subprocess

    exe = os.path.join(ROOT, "go-nngpu_amd", "lib", "mfma_ceiling")
    if not os.path.exists(exe):
        raise RuntimeError(f"{exe} is missing: build it first (__graft_entry__.build() or make in go-nngpu_amd)")
    r = subprocess.run([exe, str(seconds)], capture_output=True, text=True, timeout=120)
    if r.returncode != 0:
        raise RuntimeError(f"mfma_ceiling exited with {r.returncode}: {r.stderr.strip()}")
    res = json.loads(r.stdout.strip().splitlines()[-1])
    for k in ("gemm_data", "zero_data"):
        res[k]["frac_of_peak"] = round(res[k]["tflops"] / PEAK_F16_TFLOPS, 4)
    log(f"mfma ceiling: {res['gemm_data']['tflops']:.0f} TFLOP/s on the headline's data "
        f"({res['gemm_data']['frac_of_peak']:.3f} of peak), {res['zero_data']['tflops']:.0f} on zeros")
    big = res.get("mfma_32x32x16")
    if big:
        log(f"mfma ceiling, {big['instruction']}: {big['gemm_data']['tflops']:.0f} TFLOP/s on the headline's data, "
            f"{big['zero_data']['tflops']:.0f} on zeros")
    return res


def run_copy(c, steps, warmup):
    """1 GiB device-to-device copy (torch's copy kernel): calibration for the PMC byte counters."""
    n = 1 << 28
    a, b = c.empty((n,)), c.empty((n,))
    a.fill_(1.0)
    ms = timed(lambda: b.copy_(a), steps, warmup, c.stream)
    gbs = 2 * 4 * n / (ms * 1e-3) / 1e9
    log(f"copy: {ms:.3f} ms for 1 GiB read + 1 GiB write, {gbs:.0f} GB/s")
    return {"ms": round(ms, 4), "bytes_read": 4 * n, "bytes_written": 4 * n, "GB/s": round(gbs, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--only", default=None, help="comma list of " + ",".join(ALL))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=6144)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (single-GPU build; the path's "
              "sharding across GPUs is a design note, not a measured configuration)", file=sys.stderr)
        sys.exit(2)
    only = ALL[:-1] if args.only is None else tuple(s for s in args.only.split(",") if s)
    for s in only:
        if s not in ALL:
            ap.error(f"unknown workload {s}")

    c = Ctx(args)
    steps, warmup = args.steps, args.warmup
    steps2 = max(5, steps // 5)
    head, secondary = None, {}
    if "c3" in only:
        head = run_c3(c, steps, warmup)
        secondary["c3_torch_matmul_reference"] = c.vendor_c3
        c.torch.cuda.empty_cache()
    if "ceiling" in only:
        try:
            secondary["mfma_power_ceiling"] = run_ceiling()
        except Exception as exc:  # a side measurement: the headline stands without it
            log(f"mfma ceiling probe failed: {exc}")
            secondary["mfma_power_ceiling_error"] = str(exc)
    if "c2" in only:
        secondary.update(run_c2(c, steps2, 3))
        c.torch.cuda.empty_cache()
    if "c1" in only:
        secondary["c1_f32_256"] = run_c1(c, steps2 * 20, 20)
    if "rows" in only:
        secondary["few_rows"] = reference_or_note(run_rows, c, steps2 * 4)
    if "c4" in only:
        secondary.update(run_c4(c, steps2 * 4, 5))
        c.torch.cuda.empty_cache()
    if "spmm" in only or "spmv" in only:
        csr = csr_workload(c)
        if "spmm" in only:
            secondary["c5_spmm"] = run_spmm(c, steps2 * 2, 3, csr)
            secondary["c5_spmm"]["part1_abi"] = run_part1_sparse(c, "spmm", 50, secondary["c5_spmm"]["ms"])
            if not args.no_cpu:
                secondary["c5_spmm"]["cpu_baseline"] = cpu_baseline_sparse(c, "spmm", 16384)
                log(f"cpu_baseline spmm: {secondary['c5_spmm']['cpu_baseline']['value']} GB/s on 1 thread")
                secondary["c5_spmm"]["cpu_parallel"] = cpu_parallel_sparse(c, "spmm")
                log(f"cpu parallel spmm: {secondary['c5_spmm']['cpu_parallel']['value']} GB/s")
        if "spmv" in only:
            secondary["c5_spmv"] = run_spmv(c, steps2 * 4, 5, csr)
            secondary["c5_spmv"]["part1_abi"] = run_part1_sparse(c, "spmv", 100, secondary["c5_spmv"]["ms"])
            if not args.no_cpu:
                secondary["c5_spmv"]["cpu_baseline"] = cpu_baseline_sparse(c, "spmv", 65536)
                log(f"cpu_baseline spmv: {secondary['c5_spmv']['cpu_baseline']['value']} GB/s on 1 thread")
                secondary["c5_spmv"]["cpu_parallel"] = cpu_parallel_sparse(c, "spmv")
                log(f"cpu parallel spmv: {secondary['c5_spmv']['cpu_parallel']['value']} GB/s")
        del csr
        c.torch.cuda.empty_cache()
    if "e2e" in only:
        secondary["c3_from_host_buffers"] = run_e2e(c, 3, 1)
        c.torch.cuda.empty_cache()
    if "copy" in only:
        secondary["copy_calibration"] = run_copy(c, steps2, 3)

    cpu = None
    if head is not None and not args.no_cpu:
        log(f"cpu_baseline: oracle float64 GEMM on {args.cpu_rows} rows of the 8192^3 problem")
        cpu = cpu_baseline_gemm(8192, args.cpu_rows)
        log(f"cpu_baseline: {cpu['value'] * 1e3:.2f} GFLOP/s")
        secondary["cpu_numpy_gemm"] = cpu_numpy_gemm(8192, args.cpu_rows)
        log(f"numpy float64 matmul: {secondary['cpu_numpy_gemm']['value'] * 1e3:.1f} GFLOP/s")
        secondary["cpu_gemm_1thread"] = cpu_gemm_1thread(8192, 96)
        log(f"cpu_baseline 1 thread: {secondary['cpu_gemm_1thread']['value'] * 1e3:.2f} GFLOP/s")

    roofline = None
    if head is not None:
        roofline = {"bound": "mfma", "achieved": round(head["tflops"], 2), "peak": PEAK_F16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(head["tflops"] / PEAK_F16_TFLOPS, 4),
                    "traffic": load_traffic("gemm_f16_8192_nn"),
                    "kernel": "gemm_f16_ring_kernel<256,256,2,4,NN>", "flop_per_launch": head["flop"]}
        if "mfma_power_ceiling" in secondary:
            ceil = secondary["mfma_power_ceiling"]["gemm_data"]["tflops"]
            roofline["measured_ceiling_tflops"] = ceil
            roofline["frac_of_measured_ceiling"] = round(head["tflops"] / ceil, 4)
    out = {
        "metric": METRIC,
        "value": round(head["tflops"], 2) if head else None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(head["ms"], 5) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (device-generated N(0,1) / N(0,0.02^2), cast to fp16 before timing)",
        "config": {"workload": "fp16-in/fp32-acc GEMM M=N=K=8192, row-major NN, A~N(0,1), B~N(0,0.02^2)",
                   "M": 8192, "N": 8192, "K": 8192, "accumulate": "f32", "output": "f32",
                   "parallelism": "single-gpu"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
