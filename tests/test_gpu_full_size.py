"""Parity at the benchmark configurations' full sizes, on the benchmark's own
inputs (bench.make_inputs, the same seeds).

At these sizes the oracle cannot compute the whole output in seconds, so the
checks use properties that hold at any size:

* sampled blocks: the split works per row of A and per column of B
  (ozaki_triton.py:169-211 on A and on B^T), so the oracle run on a set of
  rows of A and columns of B, with the full K, gives exactly that block of the
  whole product.  int8 slices: bit-exact.  fp16 slices: within the
  fp32-accumulation bound of the GPU's dot products (helpers.fp16_cross_bound);
* the full-size splits of C3 and C5 (the cooperative column kernel, the shared
  row kernel and the transpose path at their real grids): sampled rows of A and
  columns of B bit-exact against the oracle's split of those rows / columns;
* accuracy: rel-err ||C - A@B||_F / ||A@B||_F against the FP64 matmul
  (test.py:128's formula) within the bound stated per configuration.  The
  bounds are about twice the reference algorithm's own error at that
  num_splits, K and input distribution (measured on MI355X: C2 4.08e-7, C3
  2.757e-9, C4 2.88e-7, C5 2.45e-6, the last set by C5's 1e4 outliers, which
  take most of their rows' and columns' slice bits); a dropped slice pair or
  a wrong scale moves rel-err by orders of magnitude.

C1 (FP32 -> FP16, 2 slices, 256^3, N(0,1) seed 0) is small enough for the
whole output to be checked against the oracle.
"""
import numpy as np
import pytest
import torch

from tests.helpers import (NAME_OF, assert_bitwise_equal, check_block_vs_oracle,
                           sample_indices, to_np)

pytestmark = pytest.mark.gpu

# rel-err bound against the FP64 matmul per configuration
REL_ERR_BOUND = {"C2": 1e-6, "C3": 4e-9, "C4": 6e-7, "C5": 5e-6}


@pytest.fixture(scope="module")
def bench_mod():
    import bench
    return bench


def _rel_err(C, A, B):
    ref = torch.matmul(A.double(), B.double())
    return float(torch.linalg.norm(C.double() - ref) / torch.linalg.norm(ref))


@pytest.mark.parametrize("name", ["C3", "C2", "C5"])
def test_full_size_single_gemm(oracle, gpu, bench_mod, name):
    """C2 (FP32 -> FP16, 2 slices, 4096^3), C3 (FP64 -> INT8, 4 slices,
    8192^3, per-row / per-column exponents) and C5 (FP32 -> INT8, 3 slices,
    1024 x 1024 x 65536 with 1% outliers): sampled blocks and rel-err."""
    import ozaki_triton_amd as ozk
    xdt, sdt, L, _, _, seed, _ = bench_mod.CONFIGS[name]
    xdt, sdt = getattr(torch, xdt), getattr(torch, sdt)
    A, B = bench_mod.make_inputs(bench_mod.CONFIGS[name])
    print(f"[full size] {name}: {tuple(A.shape)} x {tuple(B.shape)} {xdt} -> {sdt} L={L}",
          flush=True)
    Ad, Bd = A.to(gpu), B.to(gpu)
    C = ozk.ozaki_matmul(Ad, Bd, L, sdt)
    torch.cuda.synchronize()
    rel = _rel_err(C, Ad, Bd)
    print(f"[full size] {name} rel-err {rel:.3e}", flush=True)
    assert rel <= REL_ERR_BOUND[name], (name, rel)
    C_np, A_np, B_np = to_np(C), to_np(A), to_np(B)
    del C, Ad, Bd
    M, N = C_np.shape
    k = 32 if name == "C5" else 64
    rows, cols = sample_indices(M, k, seed), sample_indices(N, k, seed + 1)
    check_block_vs_oracle(oracle, ozk, C_np, A_np, B_np, rows, cols, L, sdt, xdt, f"{name} block")


def test_full_size_broadcast_batch(oracle, gpu, bench_mod):
    """C4: FP64 -> FP16, 3 slices, A [16, 1024, 2048] x B [2048, 1024] (B
    broadcast over the batch and split once): sampled blocks of three batches
    and rel-err over the whole batch."""
    import ozaki_triton_amd as ozk
    xdt, sdt, L, _, _, seed, _ = bench_mod.CONFIGS["C4"]
    xdt, sdt = getattr(torch, xdt), getattr(torch, sdt)
    A, B = bench_mod.make_inputs(bench_mod.CONFIGS["C4"])
    Ad, Bd = A.to(gpu), B.to(gpu)
    C = ozk.ozaki_matmul(Ad, Bd, L, sdt)
    torch.cuda.synchronize()
    assert C.shape == (16, 1024, 1024)
    rel = _rel_err(C, Ad, Bd)
    print(f"[full size] C4 rel-err {rel:.3e}", flush=True)
    assert rel <= REL_ERR_BOUND["C4"], rel
    C_np, A_np, B_np = to_np(C), to_np(A), to_np(B)
    for b in (0, 7, 15):
        rows, cols = sample_indices(1024, 48, seed + b), sample_indices(1024, 48, seed + 100 + b)
        check_block_vs_oracle(oracle, ozk, C_np[b], A_np[b], B_np, rows, cols, L, sdt, xdt,
                     f"C4 batch {b} block")


def test_c1_whole_output(oracle, gpu):
    """C1: FP32 -> FP16, 2 slices, 256^3, A, B N(0,1) float32 from seed 0; the
    whole output within the fp16 bound of the oracle's."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(0)
    A = torch.randn(256, 256, generator=g, dtype=torch.float32)
    B = torch.randn(256, 256, generator=g, dtype=torch.float32)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), 2, torch.float16)
    torch.cuda.synchronize()
    rows = cols = np.arange(256)
    check_block_vs_oracle(oracle, ozk, to_np(C), to_np(A), to_np(B), rows, cols, 2, torch.float16,
                 torch.float32, "C1")


@pytest.mark.parametrize("name", ["C3", "C5"])
def test_full_size_splits(oracle, gpu, bench_mod, name):
    """The splits of C3 and C5 at full size: A's rows (row kernel; the shared
    row kernel for C5's 65536-long rows) and B's columns through the transposed
    view (the cooperative column kernel at C3: 512 groups of 8 chunks; the
    transpose path at C5), sampled rows / columns bit-exact against the
    oracle; every scale a power of two."""
    import ozaki_triton_amd as ozk
    xdt, sdt, L, _, _, seed, _ = bench_mod.CONFIGS[name]
    sdt = getattr(torch, sdt)
    A, B = bench_mod.make_inputs(bench_mod.CONFIGS[name])
    K = A.shape[-1]
    alpha = ozk.compute_split_bits(K, sdt, ozk._select_dot_accum_dtype(sdt))
    for what, X in (("A", A), ("B^T", B.T)):
        sl, sc = ozk.split_matrix(X.to(gpu)[None] if what == "A" else B.to(gpu).T[None], L, alpha,
                                  sdt)
        torch.cuda.synchronize()
        sc_np = to_np(sc)[0]
        mant, _ = np.frexp(sc_np.astype(np.float64))
        assert np.all(mant == 0.5), f"{name} {what}: a scale is not a power of two"
        rows = sample_indices(X.shape[0], 64, seed + 7)
        idx = torch.as_tensor(rows, device=gpu)
        got_sl = to_np(sl[0][:, idx])
        want_sl, want_sc = oracle.split(np.ascontiguousarray(to_np(X)[rows]), L, alpha,
                                        NAME_OF[sdt])
        assert_bitwise_equal(sc_np[:, rows], want_sc, f"{name} {what} scales")
        assert_bitwise_equal(got_sl, want_sl, f"{name} {what} slices")
        del sl, sc


def test_operand_over_2gib_takes_the_staged_kernel(oracle, gpu):
    """Slice operands the LDS-DMA kernels cannot address (their buffer offsets
    are 31-bit: over 2 GiB per batch) fall back to the VGPR-staged kernel.
    int8 slices A [1, 4, 16448, 32768] (2.06 GiB) made on the device, B
    [1, 4, 64, 32768]: a sampled block bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    L, M, N, K = 4, 16448, 64, 32768
    g = torch.Generator(device=gpu).manual_seed(5)
    As = torch.randint(-128, 128, (1, L, M, K), generator=g, dtype=torch.int8, device=gpu)
    assert As.numel() > 2 ** 31
    Bs = torch.randint(-128, 128, (1, L, N, K), generator=g, dtype=torch.int8, device=gpu)
    sa = torch.pow(2.0, torch.randint(-30, -10, (1, L, M), generator=g, device=gpu).float())
    sb = torch.pow(2.0, torch.randint(-30, -10, (1, L, N), generator=g, device=gpu).float())
    C = ozk.cross_gemm(As, Bs.transpose(-1, -2), sa, sb, L, torch.float64)
    torch.cuda.synchronize()
    rows = sample_indices(M, 24, 1)
    idx = torch.as_tensor(rows, device=gpu)
    a = to_np(As[0][:, idx])
    want = oracle.cross_gemm(a, to_np(Bs[0]), to_np(sa[0][:, idx]), to_np(sb[0]), "float64")
    assert_bitwise_equal(to_np(C[0][idx]), want, "over-2GiB operand")
