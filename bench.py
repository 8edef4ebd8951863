"""Benchmark of the Ozaki-scheme hot path on one MI355X.

Default workload (the headline metric, configuration C3): FP64 -> INT8 slices,
num_splits = 4, M = N = K = 8192, batch 1, A and B entries N(0,1) * 2^e with e
drawn per row of A / per column of B from Uniform-int[-8, 8]
(torch.Generator seed 2).  A "step" is one ozaki_matmul call (split B, split A,
fused cross-GEMM) on inputs already resident in HBM.

Prints one JSON line:
  value        emulated TFLOP/s = 2*M*N*K*batch / (time per step), whole job
  rel_err      ||C - A@B||_F / ||A@B||_F with A@B in float64 (torch.matmul)
  roofline     the cross-GEMM (dominant kernel): int8 ops / its average
               duration from HIP events recorded on the launch stream inside
               the timed region, against MI355X's dense INT8 MFMA peak
  split        both split kernels: algorithmic HBM bytes / their event time
               against the 8 TB/s HBM peak
  cpu_baseline the CPU oracle (a scalar C port of the reference's algorithm)
               on a bounded block of the same workload, host cores
  cpu_torch_matmul  torch.matmul in the input dtype on the host cores
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "emulated TFLOP/s (2MNK/t) FP64→INT8 split=4 at 8192³; rel err vs FP64"

# MI355X published dense peaks
PEAK_INT8_TOPS = 5000.0       # TOP/s dense INT8 MFMA
PEAK_FP16_TFLOPS = 2500.0     # TFLOP/s dense FP16 MFMA
PEAK_HBM_GBS = 8000.0         # GB/s HBM3E

CONFIGS = {
    # name: (input dtype, slice dtype, L, A shape, B shape, seed, distribution)
    "C1": ("float32", "float16", 2, (256, 256), (256, 256), 0, "normal"),
    "C2": ("float32", "float16", 2, (4096, 4096), (4096, 4096), 1, "uniform"),
    "C3": ("float64", "int8", 4, (8192, 8192), (8192, 8192), 2, "exp8"),
    "C4": ("float64", "float16", 3, (16, 1024, 2048), (2048, 1024), 3, "normal"),
    "C5": ("float32", "int8", 3, (1024, 65536), (65536, 1024), 4, "outliers"),
    # one GPU's share of C3 on a 2 x 2 output-stationary grid (no exchange:
    # this GPU's A row-block and B column-block)
    "C3s": ("float64", "int8", 4, (4096, 8192), (8192, 4096), 2, "exp8"),
}


def make_inputs(cfg):
    import torch
    xdt, _, _, sa, sb, seed, dist = cfg
    g = torch.Generator().manual_seed(seed)
    if dist == "exp8":
        A = torch.randn(*sa, generator=g, dtype=torch.float64)
        B = torch.randn(*sb, generator=g, dtype=torch.float64)
        A *= torch.pow(2.0, torch.randint(-8, 9, (*sa[:-1], 1), generator=g).double())
        B *= torch.pow(2.0, torch.randint(-8, 9, (1, sb[-1]), generator=g).double())
    elif dist == "normal":
        A = torch.randn(*sa, generator=g, dtype=torch.float64)
        B = torch.randn(*sb, generator=g, dtype=torch.float64)
    else:
        A = torch.rand(*sa, generator=g, dtype=torch.float32) * 2 - 1
        B = torch.rand(*sb, generator=g, dtype=torch.float32) * 2 - 1
        if dist == "outliers":
            A[torch.rand(*sa, generator=g) < 0.01] *= 1e4
            B[torch.rand(*sb, generator=g) < 0.01] *= 1e4
    return A.to(getattr(torch, xdt)), B.to(getattr(torch, xdt))


def reference_shapes(reps: int = 30):
    """--reference-shapes: ozaki_matmul at the reference's own published points
    (reference/test_results.csv, extracted to tests/golden/reference_published.json):
    4 shapes (B, M, N, K) x 4 dtype scenarios x num_splits 1-4.  Inputs as
    test.py:104-109 (N(0,1), rows of A and columns of B scaled by 10^U(-2,2);
    seeded here); rel-err against a @ b in the input dtype (test.py:112-128);
    time as triton's do_bench takes it: the GPU time between events around
    one call, after a cache flush, median over reps; the same for the call
    replayed from a HIP graph; and the wall-clock time per call of 100 calls
    (and of 100 graph replays) issued back to back.  One JSON line per point,
    then a summary line.  The reference's figures come from its own NVIDIA
    GPU, so the ratio compares two machines, not two implementations."""
    import statistics
    import torch
    import ozaki_triton_amd as ozk

    with open(os.path.join(ROOT, "tests", "golden", "reference_published.json")) as f:
        rows = json.load(f)["rows"]
    dev = torch.device("cuda:0")
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    inputs = {}
    ratios = {}
    for r in rows:
        Bn, M, N, K = r["shape_bmnk"]
        xdt, sdt, L = getattr(torch, r["input_dtype"]), getattr(torch, r["slice_dtype"]), r["splits"]
        key = (Bn, M, N, K, r["input_dtype"])
        if key not in inputs:
            g = torch.Generator().manual_seed(Bn * 1000003 + M * 1009 + N * 31 + K)
            rs = 10 ** ((torch.rand(M, generator=g, dtype=torch.float64) * 2 - 1) * 2)
            cs = 10 ** ((torch.rand(N, generator=g, dtype=torch.float64) * 2 - 1) * 2)
            a = torch.randn((Bn, M, K), generator=g, dtype=torch.float64) * rs[:, None]
            b = torch.randn((Bn, K, N), generator=g, dtype=torch.float64) * cs
            a, b = a.to(xdt).to(dev), b.to(xdt).to(dev)
            inputs[key] = (a, b, torch.nan_to_num(a @ b).double())
        a, b, c_ref = inputs[key]
        C = ozk.ozaki_matmul(a, b, num_splits=L, slice_dtype=sdt).double()
        rel = float((C - c_ref).norm() / c_ref.norm())
        # warmup as triton.testing.do_bench's default: 25 ms of calls (at
        # least 5), synchronised every 8 calls so that host time tracks the GPU
        tw, nw = time.perf_counter(), 0
        while nw < 5 or time.perf_counter() - tw < 0.025:
            ozk.ozaki_matmul(a, b, num_splits=L, slice_dtype=sdt)
            nw += 1
            if nw % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            flush.zero_()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            ozk.ozaki_matmul(a, b, num_splits=L, slice_dtype=sdt)
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        ms = statistics.median(ts)
        # the same call replayed from a HIP graph (captured once; ozaki_matmul
        # allocates nothing inside the library, torch's graph pool holds C and
        # the workspace): launch and host costs drop out
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                C_graph = ozk.ozaki_matmul(a, b, num_splits=L, slice_dtype=sdt)
        torch.cuda.current_stream().wait_stream(side)
        graph.replay()
        torch.cuda.synchronize()
        same = bool(torch.equal(C_graph.double(), C)) if sdt == torch.int8 else None
        gts = []
        for _ in range(reps):
            flush.zero_()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
            e1.synchronize()
            gts.append(e0.elapsed_time(e1))
        gms = statistics.median(gts)
        # back to back, no flush, wall clock per call: what a caller issuing
        # many small products sees, host costs (Python checks, the workspace,
        # launches) included -- the cost graph replay removes
        def per_call_ms(fn, n=100):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(n):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) / n * 1e3
        eager_b2b = per_call_ms(lambda: ozk.ozaki_matmul(a, b, num_splits=L, slice_dtype=sdt))
        graph_b2b = per_call_ms(graph.replay)
        del graph, C_graph
        ratio = r["ozaki_ms"] / ms
        ratios.setdefault(r["scenario"], []).append(ratio)
        print(json.dumps({
            "shape_bmnk": r["shape_bmnk"], "scenario": r["scenario"], "num_splits": L,
            "ms": round(ms, 4), "graph_replay_ms": round(gms, 4),
            "back_to_back_ms": round(eager_b2b, 4), "graph_back_to_back_ms": round(graph_b2b, 4),
            "graph_equals_eager": same,
            "emulated_tflops": round(2.0 * Bn * M * N * K / (ms * 1e-3) / 1e12, 3),
            "rel_err": rel, "reference_ms": round(r["ozaki_ms"], 4),
            "reference_rel_err": r["rel_error"], "reference_ms_over_ms": round(ratio, 3),
            "csv_line": r["csv_line"]}), flush=True)
    geo = {k: round(statistics.geometric_mean(v), 3) for k, v in ratios.items()}
    print(json.dumps({"reference_shapes_summary": {
        "points": len(rows), "reps": reps,
        "geomean_reference_ms_over_ms": geo,
        "note": "reference times from its own NVIDIA GPU (test_results.csv); this build on "
                "one MI355X"}}), flush=True)


def cpu_oracle_baseline(A_cpu, B_cpu, slice_dtype, L, block, pairs="all"):
    """Time the C oracle on a block x block corner of the output with the full
    K: split `block` rows of A and `block` columns of B, then the L^2 slice
    GEMMs and the ordered epilogue.  Single-threaded."""
    import numpy as np
    import oracle
    a = A_cpu.reshape(-1, A_cpu.shape[-1])[:block].numpy()
    b = B_cpu.reshape(-1, B_cpu.shape[-1])[:, :block].numpy() if B_cpu.dim() == 2 else \
        B_cpu[0][:, :block].numpy()
    K = a.shape[1]
    sd = slice_dtype
    alpha = oracle.compute_split_bits(K, sd, "int32" if sd == "int8" else "float32")
    t0 = time.perf_counter()
    a_sl, a_sc = oracle.split(a, L, alpha, sd)
    b_sl, b_sc = oracle.split(np.ascontiguousarray(b).T, L, alpha, sd)
    oracle.cross_gemm(a_sl, b_sl, a_sc, b_sc, str(a.dtype), pairs=pairs)
    dt = time.perf_counter() - t0
    return 2.0 * block * block * K / dt / 1e12, dt


def cpu_torch_matmul(A_cpu, B_cpu, reps):
    import torch
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        torch.matmul(A_cpu, B_cpu)
        ts.append(time.perf_counter() - t0)
    ts.sort()
    t = ts[len(ts) // 2]
    flops = 2.0 * A_cpu.shape[-2] * A_cpu.shape[-1] * B_cpu.shape[-1]
    if A_cpu.dim() == 3:
        flops *= A_cpu.shape[0]
    return flops / t / 1e12, ncores, torch.get_num_threads()


def planned_gemm_kernel(batch, M, N, K, L, sdt, pairs="all"):
    """Name of the cross-GEMM kernel the library's planner picks for this call
    (ozk_debug_gemm_kernel_pairs), e.g. "wide4"."""
    import ctypes
    from ozaki_triton_amd import _lib
    name = ctypes.c_char_p()
    code = {"int8": _lib.OZK_I8, "float16": _lib.OZK_F16}[sdt]
    pc = {"all": _lib.OZK_PAIRS_ALL, "triangular": _lib.OZK_PAIRS_TRIANGULAR}[pairs]
    _lib.check("ozk_debug_gemm_kernel_pairs",
               _lib.load().ozk_debug_gemm_kernel_pairs(batch, M, N, K, L, code, pc, 0,
                                                       ctypes.byref(name), None))
    return name.value.decode()


def gemm_kernel_symbol(plan, L, sdt):
    """Name of the kernel function a planned cross-GEMM launches: the
    launchers take the 16 x 16 MFMA forms ("...q") of the ring (two slices),
    wide, wide4 and solo configurations for the slice dtypes benchmarked
    here (int8, fp16)."""
    q = plan in ("ring", "wide", "wide4", "solo")
    return f"cross_gemm_{plan}{'q' if q else ''}_kernel"


def planned_split_kernel(X, xdt, sdt, L, columns):
    """Split path the planner picks for A's rows or B's columns (through its
    transposed view), as ozaki_matmul hands them over (ozk_debug_split_kernel)."""
    import ctypes
    from ozaki_triton_amd import _lib
    if X.dim() == 2:
        X = X.unsqueeze(0)
    bsz, r, c = X.shape
    rows, K = (c, r) if columns else (r, c)
    xs = (X.stride(0) if bsz > 1 else 0, X.stride(2), X.stride(1)) if columns else \
        (X.stride(0) if bsz > 1 else 0, X.stride(1), X.stride(2))
    nb = bsz if X.stride(0) != 0 and bsz > 1 else 1
    ss = (L * rows * K, rows * K, K, 1)
    name = ctypes.c_char_p()
    nbytes = ctypes.c_size_t(0)
    xd = {"float64": _lib.OZK_F64, "float32": _lib.OZK_F32}[xdt]
    sd = {"int8": _lib.OZK_I8, "float16": _lib.OZK_F16}[sdt]
    _lib.check("ozk_debug_split_kernel", _lib.load().ozk_debug_split_kernel(
        ctypes.c_void_p(X.data_ptr()), xd, nb, rows, K, _lib.i64arr(xs), L, sd,
        ctypes.c_void_p(256), _lib.i64arr(ss), ctypes.byref(name), ctypes.byref(nbytes)))
    return name.value.decode()


def measured_traffic(config: str, kernel: str):
    """HBM-side bytes per launch of a kernel, from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes summarised in profiles/ (scaled by the copy-kernel
    calibration recorded there), or None when that config was not measured.
    Profiled names are demangled ("ozk::cross_gemm_ring_kernel<...>") or, for
    some template arguments, mangled ("_ZN3ozk22cross_gemm_ring_kernel..."):
    the kernel's base name is matched as a whole identifier in either."""
    path = os.path.join(ROOT, "profiles", "cross_gemm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    pat = re.compile(r"(ozk::|ozk\d+)" + re.escape(kernel) + r"(<|I)")
    for name, rec in data.get("configs", {}).get(config, {}).items():
        if pat.search(name):
            return int(rec["traffic_bytes"])
    return None


def vendor_probes():
    """Calibration points for the two rooflines, timed with events: the HBM
    rate torch's own copy kernel reaches (read + write bytes / time) and the
    rate of the vendor int8 GEMM (hipBLASLt through torch._int_mm) at C3's
    size, i.e. ONE of the L*L slice GEMMs the cross-GEMM fuses."""
    import torch
    dev = torch.device("cuda:0")

    def time_ms(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    out = {}
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = time_ms(lambda: dst.copy_(src), 10)
    out["copy_1GiB_ms"] = round(ms, 4)
    out["copy_GBps_read_plus_write"] = round(2 * n / (ms * 1e-3) / 1e9, 1)
    del src, dst
    m = 8192
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randint(-128, 128, (m, m), dtype=torch.int8, device=dev, generator=g)
    b = torch.randint(-128, 128, (m, m), dtype=torch.int8, device=dev, generator=g)
    ms = time_ms(lambda: torch._int_mm(a, b.t()), 5)
    out["int_mm_8192_ms"] = round(ms, 4)
    out["int_mm_TOPs"] = round(2.0 * m ** 3 / (ms * 1e-3) / 1e12, 1)
    # the same GEMM on zero operands: same instructions, same memory traffic,
    # no operand bits toggling in the multipliers
    z = torch.zeros_like(a)
    ms = time_ms(lambda: torch._int_mm(z, z.t()), 5)
    out["int_mm_zeros_TOPs"] = round(2.0 * m ** 3 / (ms * 1e-3) / 1e12, 1)
    del a, b, z
    # the library's cross-GEMM at C3's size (num_splits 4 and 5, the planner's
    # kernel) on three kinds of int8 slices: those of C3's inputs, uniform
    # random ones and zeros.  A kernel limited by its own schedule runs all
    # three at one rate; a rate that rises as fewer operand bits toggle is set
    # by the chip's power limit (the clock), not by the kernel.
    import ozaki_triton_amd as ozk
    A, B = make_inputs(CONFIGS["C3"])
    A, B = A.to(dev), B.to(dev)
    K = A.shape[-1]
    alpha = ozk.compute_split_bits(K, torch.int8, torch.int32)
    for L in (4, 5):
        a_sl, a_sc = ozk.split_matrix(A.unsqueeze(0), L, alpha, torch.int8)
        b_sl, b_sc = ozk.split_matrix(B.t().unsqueeze(0), L, alpha, torch.int8)
        kinds = {"c3_slices": (a_sl, b_sl),
                 "uniform_random": (torch.randint(-128, 128, a_sl.shape, dtype=torch.int8,
                                                  device=dev, generator=g),
                                    torch.randint(-128, 128, b_sl.shape, dtype=torch.int8,
                                                  device=dev, generator=g)),
                 "zeros": (torch.zeros_like(a_sl), torch.zeros_like(b_sl))}
        res = {"kernel": gemm_kernel_symbol(planned_gemm_kernel(1, m, m, K, L, "int8"), L, "int8")}
        for name, (xa, xb) in kinds.items():
            ms = time_ms(lambda: ozk.cross_gemm(xa, xb.transpose(-1, -2), a_sc, b_sc, L,
                                                torch.float64), 5)
            res[name + "_ms"] = round(ms, 4)
            res[name + "_TOPs"] = round(2.0 * m * m * K * L * L / (ms * 1e-3) / 1e12, 1)
        out[f"cross_gemm_L{L}"] = res
        del a_sl, b_sl, kinds
    del A, B
    # the same for fp16: the vendor fp16 GEMM at 8192^3, and the library's
    # fp16-slice cross-GEMM at C2's and C4's shapes (uniform random slices of
    # C2's value range against zeros)
    a16 = torch.randn(m, m, device=dev, generator=g).half()
    ms = time_ms(lambda: a16 @ a16.t(), 5)
    out["matmul_f16_8192_TFLOPs"] = round(2.0 * m ** 3 / (ms * 1e-3) / 1e12, 1)
    z16 = torch.zeros_like(a16)
    ms = time_ms(lambda: z16 @ z16.t(), 5)
    out["matmul_f16_zeros_TFLOPs"] = round(2.0 * m ** 3 / (ms * 1e-3) / 1e12, 1)
    del a16, z16
    for name, (L, bt, M, N, K) in (("C2", (2, 1, 4096, 4096, 4096)),
                                   ("C4", (3, 16, 1024, 1024, 2048))):
        res = {"kernel": gemm_kernel_symbol(planned_gemm_kernel(bt, M, N, K, L, "float16"), L,
                                            "float16")}
        sa = torch.ones(bt, L, M, device=dev)
        sb = torch.ones(bt, L, N, device=dev)
        for kind in ("uniform_random", "zeros"):
            if kind == "zeros":
                xa = torch.zeros(bt, L, M, K, device=dev, dtype=torch.float16)
                xb = torch.zeros(bt, L, N, K, device=dev, dtype=torch.float16)
            else:
                xa = (torch.rand(bt, L, M, K, device=dev, generator=g) * 2 - 1).half()
                xb = (torch.rand(bt, L, N, K, device=dev, generator=g) * 2 - 1).half()
            ms = time_ms(lambda: ozk.cross_gemm(xa, xb.transpose(-1, -2), sa, sb, L,
                                                torch.float64), 5)
            res[kind + "_ms"] = round(ms, 4)
            res[kind + "_TFLOPs"] = round(2.0 * bt * M * N * K * L * L / (ms * 1e-3) / 1e12, 1)
            del xa, xb
        out[f"cross_gemm_f16_{name}"] = res
    print(json.dumps(out), flush=True)


class TimingEvent:
    """A HIP event for timing only, created with hipEventDisableSystemFence:
    recording it writes back and invalidates no caches, which torch's events
    (a system-scope release each) do, so it perturbs the work around it less.
    Created through the HIP runtime torch has loaded (the library's own), as
    a `cuda_event` handle the library records; `factory()` falls back to
    torch's events where that runtime cannot be found."""
    _hip = None
    DISABLE_SYSTEM_FENCE = 0x20000000

    @classmethod
    def factory(cls):
        import ctypes
        import torch
        if cls._hip is None:
            paths = sorted({ln.split()[-1] for ln in open("/proc/self/maps")
                            if "libamdhip64" in ln and "/" in ln})
            if len(paths) != 1:
                return lambda: torch.cuda.Event(enable_timing=True)
            cls._hip = ctypes.CDLL(paths[0])
        return cls

    def __init__(self):
        import ctypes
        h = ctypes.c_void_p()
        rc = self._hip.hipEventCreateWithFlags(ctypes.byref(h),
                                               ctypes.c_uint(self.DISABLE_SYSTEM_FENCE))
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
        self._h = h
        self.cuda_event = h.value

    def record(self):
        import ctypes
        import torch
        rc = self._hip.hipEventRecord(self._h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end) -> float:
        import ctypes
        ms = ctypes.c_float()
        rc = self._hip.hipEventElapsedTime(ctypes.byref(ms), self._h, end._h)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if self._hip is not None and getattr(self, "_h", None) is not None:
            self._hip.hipEventDestroy(self._h)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps before the timed ones (default: at least 3, and as many as "
                         "take about 0.2 s)")
    ap.add_argument("--config", default="C3", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-block", type=int, default=1024)
    ap.add_argument("--num-splits", type=int, default=0,
                    help="override the configuration's num_splits (e.g. 5 at C3: the slice count "
                         "whose rel-err meets 1e-9); the line is then not the headline metric")
    ap.add_argument("--pairs", default="all", choices=["all", "triangular"],
                    help="slice pairs the cross-GEMM sums: all (the reference's sum, the "
                         "metric) or triangular (i + j <= num_splits - 1; not in the reference)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (3 times): the "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--vendor-probes", action="store_true",
                    help="only time the calibration probes of the rooflines: torch's device "
                         "copy of 1 GiB (practical HBM rate), the vendor int8 and fp16 GEMMs "
                         "at 8192^3 on random and zero operands, and the library's cross-GEMM "
                         "at C3's size (int8) and C2's and C4's (fp16) on random and zero "
                         "slices")
    ap.add_argument("--reference-shapes", action="store_true",
                    help="only time ozaki_matmul at the reference's published points "
                         "(test_results.csv: 4 shapes x 4 dtype scenarios x num_splits 1-4)")
    args = ap.parse_args()
    if args.reference_shapes:
        reference_shapes()
        return
    if args.vendor_probes:
        vendor_probes()
        return
    if args.copy_probe_mib:
        import torch
        n = args.copy_probe_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path (the output shards by blocks of A's rows and B's columns with no "
              "reduction; --config C3s measures one GPU's share of C3 on a 2x2 grid)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd.ozaki import _ozaki_matmul_impl

    cfg = CONFIGS[args.config]
    xdt, sdt, L = cfg[0], cfg[1], cfg[2]
    default_L = L
    if args.num_splits:
        L = args.num_splits
    slice_dtype = getattr(torch, sdt)
    dev = torch.device("cuda:0")
    A_cpu, B_cpu = make_inputs(cfg)
    A, B = A_cpu.to(dev), B_cpu.to(dev)
    M, K = A.shape[-2:]
    N = B.shape[-1]
    batch = A.shape[0] if A.dim() == 3 else 1
    print(f"[bench] {args.config}: {xdt}->{sdt} L={L} A{tuple(A.shape)} B{tuple(B.shape)}",
          file=sys.stderr, flush=True)

    # Timing events, recorded by the library on the launch stream between the
    # phases: before the B split, before the A split, before the cross-GEMM,
    # after it (it skips NULL entries).  Each event costs the stream a few
    # microseconds (four per step added 13-18 us to C2's 0.47 ms step and 20 us
    # to C3's 6.6 ms, one box), so a timed step records only the bounds of one
    # part: even steps the splits' (with the B / A boundary only where the
    # splits are separate launches), odd steps the cross-GEMM's.  The events
    # carry no system-scope fence (TimingEvent).
    phases = ("split_b", "split_a", "cross_gemm", "end")
    mk_event = TimingEvent.factory()
    events = []
    for _ in range(args.steps):
        evs = [mk_event() for _ in phases]
        for e in evs:
            e.record()
        events.append(evs)

    # Untimed warmup.  A new workload's first tens of milliseconds run slower
    # (C2's cross-GEMM took 0.60 ms per call after 3 warmup calls and 0.50 ms
    # after 100, one box), so by default the warmup runs for about 0.2 s: the
    # second call is timed on the host and sets the count (at least 3).
    warmup, done = args.warmup, 0
    if warmup is None:
        for _ in range(2):
            tw = time.perf_counter()
            _ozaki_matmul_impl(A, B, L, slice_dtype, False, None, max_splits=8, pairs=args.pairs)
            torch.cuda.synchronize()
        done = 2
        warmup = max(3, min(5000, int(0.2 / max(time.perf_counter() - tw, 1e-6)) + 1))
    warmup = max(warmup, done + 1)
    for _ in range(warmup - done - 1):
        _ozaki_matmul_impl(A, B, L, slice_dtype, False, None, max_splits=8, pairs=args.pairs)
    # the last warmup step with all four events: are the splits one launch
    # (split_pair_kernel / split_duo_kernel)?  Then the B phase's two events
    # fall at one point
    _ozaki_matmul_impl(A, B, L, slice_dtype, False, events[0], max_splits=8, pairs=args.pairs)
    torch.cuda.synchronize()
    one_launch = events[0][0].elapsed_time(events[0][1]) < 0.02
    step_events = [
        ([e[0], None if one_launch else e[1], e[2], None] if s % 2 == 0 else
         [None, None, e[2], e[3]]) for s, e in enumerate(events)] if args.steps > 1 else events

    t0 = time.perf_counter()
    for s in range(args.steps):
        C = _ozaki_matmul_impl(A, B, L, slice_dtype, False, step_events[s], max_splits=8,
                               pairs=args.pairs)
    torch.cuda.synchronize()
    t = time.perf_counter() - t0
    ms = t / args.steps * 1e3

    def avg_ms(a, b):
        """Mean time between phases a and b over the timed steps that recorded both."""
        ia, ib = phases.index(a), phases.index(b)
        got = [ev[ia].elapsed_time(ev[ib]) for ev in step_events
               if ev[ia] is not None and ev[ib] is not None]
        return sum(got) / len(got)

    # single calls, each after a 512 MiB write that evicts L2 and MALL (as
    # triton.testing.do_bench, which reference test.py:125 times with, clears
    # the cache before each call); the median of 20
    import statistics
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    fts = []
    for _ in range(20):
        flush.zero_()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        _ozaki_matmul_impl(A, B, L, slice_dtype, False, None, max_splits=8, pairs=args.pairs)
        e1.record()
        e1.synchronize()
        fts.append(e0.elapsed_time(e1))
    del flush
    flushed_ms = statistics.median(fts)

    # the HBM rate a plain copy reaches on this box in the same run (torch's
    # own device copy of 1 GiB, read + write bytes; outside the timed region):
    # the practical ceiling the split's bytes are compared with below
    csrc = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    cdst = torch.empty_like(csrc)
    for _ in range(3):
        cdst.copy_(csrc)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        cdst.copy_(csrc)
    e1.record()
    e1.synchronize()
    copy_gbs = 2.0 * csrc.numel() / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9
    del cdst
    # the same with the split's own mix of 2 bytes read per byte written (at
    # C3: 8-byte inputs read, 4 one-byte slices written): torch's elementwise
    # add of two 512 MiB byte arrays into a third
    ca, cb = csrc[: 1 << 29], csrc[1 << 29:]
    cc = torch.empty_like(ca)
    for _ in range(3):
        torch.add(ca, cb, out=cc)
    e0.record()
    for _ in range(10):
        torch.add(ca, cb, out=cc)
    e1.record()
    e1.synchronize()
    copy21_gbs = 3.0 * ca.numel() / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9
    del csrc, ca, cb, cc

    if one_launch:
        t_split_b, t_split_a = 0.0, avg_ms("split_b", "cross_gemm")
    else:
        t_split_b, t_split_a = avg_ms("split_b", "split_a"), avg_ms("split_a", "cross_gemm")
    t_cross = avg_ms("cross_gemm", "end")

    emu_flops = 2.0 * M * N * K * batch
    value = emu_flops / (ms * 1e-3) / 1e12

    # accuracy vs FP64 torch.matmul
    C64 = torch.matmul(A.double(), B.double())
    rel = float((C.double() - C64).norm() / C64.norm())
    del C64

    # dominant kernel: cross-GEMM, one slice GEMM of 2*M*N*K ops per pair
    # (L^2 pairs, or L (L + 1) / 2 in the triangular set)
    n_pairs = L * L if args.pairs == "all" else L * (L + 1) // 2
    cross_ops = n_pairs * 2.0 * M * N * K * batch
    if sdt == "int8":
        peak, unit_c = PEAK_INT8_TOPS, "TOP/s"
    else:
        peak, unit_c = PEAK_FP16_TFLOPS, "TFLOP/s"
    achieved = cross_ops / (t_cross * 1e-3) / 1e12
    # the kernels the library chose, asked from its planner (the test hooks of
    # include/ozaki_amd_debug.h), so the profiled name is the one that ran
    gemm_kernel = gemm_kernel_symbol(planned_gemm_kernel(batch, M, N, K, L, sdt, args.pairs), L, sdt)
    # split: read the unique inputs, write the unique slices and scales
    xsz = 8 if xdt == "float64" else 4
    ssz = 1 if sdt == "int8" else 2
    a_elems = A.numel()
    b_elems = B.numel()
    a_rows = A.numel() // K
    b_cols = (B.numel() // K)
    split_bytes = (a_elems + b_elems) * (xsz + L * ssz) + (a_rows + b_cols) * L * 4
    split_ms = t_split_a + t_split_b
    split_gbs = split_bytes / (split_ms * 1e-3) / 1e9

    rec = {
        "metric": (METRIC if args.config == "C3" and L == default_L and args.pairs == "all" else
                   f"emulated TFLOP/s (2MNK/t) {args.config}" +
                   ("" if L == default_L else f" with num_splits={L}") +
                   ("" if args.pairs == "all" else ", triangular pairs")),
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{'f64' if xdt == 'float64' else 'f32'} via {'i8' if sdt == 'int8' else 'f16'} "
                 "slices",
        "data": "synthetic",
        "config": {
            "workload": {
                "C1": "FP32->FP16 num_splits=2, M=N=K=256 (the reference's CPU-runnable case)",
                "C2": "FP32->FP16 num_splits=2, M=N=K=4096",
                "C3": "FP64->INT8 num_splits=4, M=N=K=8192, batch 1",
                "C4": "FP64->FP16 num_splits=3, A[16,1024,2048] x B[2048,1024] (broadcast)",
                "C5": "FP32->INT8 num_splits=3, M=N=1024, K=65536, 1% outliers x1e4",
                "C3s": "FP64->INT8 num_splits=4, A[4096,8192] x B[8192,4096]: one GPU's share "
                       "of C3 on a 2x2 grid",
            }[args.config] + ("" if L == default_L else f"; num_splits overridden to {L}") +
            ("" if args.pairs == "all" else "; triangular pair set (i + j <= num_splits - 1)"),
            "input_dtype": xdt, "slice_dtype": sdt, "num_splits": L, "pairs": args.pairs,
            "M": M, "N": N, "K": K, "batch": batch, "seed": cfg[5],
        },
        "rel_err": rel,
        "median_flushed": {"ms": round(flushed_ms, 4),
                           "value": round(emu_flops / (flushed_ms * 1e-3) / 1e12, 3),
                           "reps": 20, "flush_bytes": 512 << 20,
                           "note": "median of single calls, each after a 512 MiB write "
                                   "(L2 and MALL evicted); value above is the mean of the "
                                   "timed steps"},
        "roofline": {
            "kernel": gemm_kernel,
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": unit_c,
            "frac": round(achieved / peak, 4),
            "traffic": (measured_traffic(args.config, gemm_kernel)
                        if L == default_L and args.pairs == "all" else None),
            "avg_ms": round(t_cross, 4),
        },
        "split": {
            "kernels": {"A": planned_split_kernel(A, xdt, sdt, L, False),
                        "B": planned_split_kernel(B, xdt, sdt, L, True)},
            # both splits in one launch: ms_a covers both
            "one_launch": one_launch,
            "bound": "hbm",
            "bytes": split_bytes,
            "achieved": round(split_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(split_gbs / PEAK_HBM_GBS, 4),
            "ms_a": round(t_split_a, 4),
            "ms_b": round(t_split_b, 4),
            "device_copy_GBps": round(copy_gbs, 1),
            "of_device_copy": round(split_gbs / copy_gbs, 4),
            "device_2to1_GBps": round(copy21_gbs, 1),
            "of_device_2to1": round(split_gbs / copy21_gbs, 4),
        },
    }
    if not args.no_cpu:
        block = min(args.cpu_block, M, N)
        v, dt = cpu_oracle_baseline(A_cpu, B_cpu, sdt, L, block, args.pairs)
        rec["cpu_baseline"] = {
            "value": round(v, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"oracle (C, scalar) on a {block}x{block} output block with the full "
                      f"K={K}: split {block} rows of A + {block} columns of B + {L * L} slice "
                      f"GEMMs + epilogue, {dt:.1f} s",
        }
        tv, ncores, nthr = cpu_torch_matmul(A_cpu[:1] if A_cpu.dim() == 3 else A_cpu, B_cpu, 3)
        rec["cpu_torch_matmul"] = {"value": round(tv, 4), "unit": "TFLOP/s", "cores": ncores,
                                   "threads": nthr, "dtype": xdt, "cpu": cpu_model(),
                                   "reps": 3, "stat": "median"}
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
