"""The triangular pair set (OZK_PAIRS_TRIANGULAR; not in the reference, whose
cross-GEMM sums every slice pair, ozaki_triton.py:403-447): C sums only the
pairs i + j <= L - 1, in the reference's i-major / j-minor order.

Every kernel that takes the set (staged, dma, kstep, wide, wide4, pair, solo) runs it
forced and must equal the oracle's triangular sum bit for bit: int8 slices on
random values, float slices on integer values (exact in fp32 in any order,
tests/helpers.py:int_valued_slices).  The oracle's triangular sum is pinned on
the CPU (tests/test_oracle_pins.py, the triangular section)."""
import numpy as np
import pytest
import torch

from tests.helpers import (assert_bitwise_equal, bits, c3_like, check_block_vs_oracle,
                           int_valued_slices, sample_indices, to_np)

pytestmark = pytest.mark.gpu


def _slices(g, L, M, N, K, sdt):
    if sdt == torch.int8:
        As = torch.randint(-128, 128, (1, L, M, K), generator=g, dtype=torch.int8)
        BsT = torch.randint(-128, 128, (1, L, N, K), generator=g, dtype=torch.int8)
        sa = torch.pow(2.0, torch.randint(-20, 5, (1, L, M), generator=g).float())
        sb = torch.pow(2.0, torch.randint(-20, 5, (1, L, N), generator=g).float())
        return As, BsT, sa, sb
    return int_valued_slices(g, 1, L, M, N, K, sdt)


def _cross(ozk, gpu, As, BsT, sa, sb, L, out, pairs):
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L,
                       out, pairs=pairs)
    torch.cuda.synchronize()
    return to_np(C)[0]


TRI_KERNELS = [("staged", 2), ("staged", 3), ("staged", 4), ("dma", 2), ("dma", 3), ("dma", 4),
               ("kstep", 2), ("kstep", 3), ("kstep", 4),
               ("kstep2", 2), ("kstep2", 3), ("kstep2", 4),
               ("wide", 3), ("wide4", 4), ("pair", 3), ("pair", 4), ("pair", 5), ("solo", 4), ("solo", 5)]


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kernel,L", TRI_KERNELS)
@pytest.mark.parametrize("M,N,K", [(100, 72, 1040), (130, 200, 520)])
def test_triangular_each_kernel_bitexact(oracle, gpu, kernel, L, M, N, K, sdt, force):
    """Forced kernel (the K-step kernel has no fp32-slice form at L = 4, and
    no kernel takes 5 fp32 slices: the planner's kernel runs / the call is
    refused), triangular sum against the oracle, and different from the
    all-pairs sum."""
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd import _lib
    print(f"[pairs] {kernel} L={L} {sdt} {M}x{N}x{K}", flush=True)
    force(gemm=kernel)
    g = torch.Generator().manual_seed(M + 3 * N + K + 11 * L)
    As, BsT, sa, sb = _slices(g, L, M, N, K, sdt)
    if sdt == torch.float32 and L == 5:
        with pytest.raises(_lib.OzakiLibError):
            _cross(ozk, gpu, As, BsT, sa, sb, L, torch.float64, "triangular")
        return
    got = _cross(ozk, gpu, As, BsT, sa, sb, L, torch.float64, "triangular")
    a, b, s_a, s_b = to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0])
    want = oracle.cross_gemm(a, b, s_a, s_b, "float64", pairs="triangular")
    assert_bitwise_equal(got, want, f"{kernel} L{L} {sdt} triangular")
    full = oracle.cross_gemm(a, b, s_a, s_b, "float64")
    assert (bits(got) != bits(full)).mean() > 0.9


@pytest.mark.parametrize("out", [torch.float32, torch.float16, torch.bfloat16, torch.int8])
@pytest.mark.parametrize("kernel,L", [("dma", 4), ("kstep", 3), ("wide", 3), ("wide4", 4),
                                      ("pair", 5), ("solo", 4), ("solo", 5)])
def test_triangular_output_dtypes(oracle, gpu, kernel, L, out, force):
    """The fp32 outer accumulator and C's conversions under the triangular set."""
    import ozaki_triton_amd as ozk
    from tests.helpers import NAME_OF
    force(gemm=kernel)
    g = torch.Generator().manual_seed(5 * L + 1)
    As, BsT, sa, sb = _slices(g, L, 96, 80, 1040, torch.int8)
    # scales near 1 so that C spans the int8 range too
    sa, sb = sa.clamp(min=2.0 ** -12), sb.clamp(min=2.0 ** -12)
    got = _cross(ozk, gpu, As, BsT, sa, sb, L, out, "triangular")
    want = oracle.cross_gemm(to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0]),
                             NAME_OF[out], pairs="triangular")
    assert_bitwise_equal(got, want, f"{kernel} L{L} -> {out}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("ksplit", [2, 4])
def test_triangular_wide_split_k(oracle, gpu, sdt, ksplit, force):
    """The wide kernel's split-K hand-over under the triangular set (the
    dropped pairs are not handed over)."""
    import ozaki_triton_amd as ozk
    force(gemm="wide", ksplit=ksplit)
    g = torch.Generator().manual_seed(ksplit)
    As, BsT, sa, sb = _slices(g, 3, 130, 200, 4096, sdt)
    got = _cross(ozk, gpu, As, BsT, sa, sb, 3, torch.float64, "triangular")
    want = oracle.cross_gemm(to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0]), "float64",
                             pairs="triangular")
    assert_bitwise_equal(got, want, f"wide split-K {ksplit} {sdt}")


@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
@pytest.mark.parametrize("L", [2, 3, 4, 5])
def test_triangular_ozaki_matmul_bitexact(oracle, gpu, xdt, L):
    """ozaki_matmul(pairs="triangular") end to end (splits of A and B, then
    the default plan's kernel) against the oracle's ozaki_matmul with the same
    set, int8 slices; one slice is one pair in either set."""
    import ozaki_triton_amd as ozk
    A, B = c3_like((2, 96, 2048), (2048, 136), 60 + L, dtype=xdt)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), L, torch.int8, max_splits=5, pairs="triangular")
    torch.cuda.synchronize()
    want = oracle.ozaki_matmul(to_np(A), to_np(B), L, "int8", pairs="triangular")
    assert_bitwise_equal(to_np(C), want, f"matmul L{L} {xdt} triangular")
    C1 = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), 1, torch.int8, pairs="triangular")
    assert_bitwise_equal(to_np(C1), oracle.ozaki_matmul(to_np(A), to_np(B), 1, "int8"), "L1")


@pytest.mark.parametrize("L", [3, 4, 5])
def test_triangular_strided_inputs(oracle, gpu, L):
    """ozaki_matmul(pairs="triangular") on strided operands: A stored K-major
    (a transposed view of its transpose) and B a column slice of a wider matrix
    (row stride 200 for N = 136).  The splits read both through their strides;
    C must equal the oracle's result on contiguous copies bit for bit."""
    import ozaki_triton_amd as ozk
    A, Bw = c3_like((2, 96, 1024), (1024, 200), 90 + L, dtype=torch.float64)
    Ag = A.to(gpu).transpose(-1, -2).contiguous().transpose(-1, -2)
    Bg = Bw.to(gpu)[:, 8:144]
    assert Ag.stride()[-2:] == (1, 96) and Bg.stride() == (200, 1)
    C = ozk.ozaki_matmul(Ag, Bg, L, torch.int8, max_splits=5, pairs="triangular")
    torch.cuda.synchronize()
    want = oracle.ozaki_matmul(to_np(A), np.ascontiguousarray(to_np(Bw)[:, 8:144]), L, "int8",
                               pairs="triangular")
    assert_bitwise_equal(to_np(C), want, f"strided matmul L{L} triangular")


def test_triangular_rejected_beyond_five_slices(gpu):
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd import _lib
    A = torch.randn(64, 256, dtype=torch.float64, device=gpu)
    with pytest.raises(_lib.OzakiLibError):
        ozk.ozaki_matmul(A, A.T.contiguous(), 6, torch.int8, max_splits=8, pairs="triangular")
    with pytest.raises(ValueError):
        ozk.ozaki_matmul(A, A.T.contiguous(), 4, torch.int8, pairs="upper")


def test_triangular_c3_five_slices(oracle, gpu):
    """C3's size and inputs (bench.py config C3, seed 2) with 5 int8 slices on
    their 15 triangular pairs: rel-err within 1e-9 against the FP64 matmul
    (measured 4.3e-10, the 25-pair figure), and sampled 64 x 64 blocks
    bit-exact against the oracle's triangular sum."""
    import bench
    import ozaki_triton_amd as ozk
    A, B = bench.make_inputs(bench.CONFIGS["C3"])
    Ad, Bd = A.to(gpu), B.to(gpu)
    C = ozk.ozaki_matmul(Ad, Bd, 5, torch.int8, max_splits=5, pairs="triangular")
    torch.cuda.synchronize()
    ref = torch.matmul(Ad, Bd)
    rel = float(torch.linalg.norm(C - ref) / torch.linalg.norm(ref))
    print(f"[pairs] C3 5 slices triangular rel-err {rel:.3e}", flush=True)
    assert rel <= 1e-9, rel
    C_np, A_np, B_np = to_np(C), to_np(A), to_np(B)
    del C, Ad, Bd, ref
    rows, cols = sample_indices(8192, 64, 21), sample_indices(8192, 64, 22)
    check_block_vs_oracle(oracle, ozk, C_np, A_np, B_np, rows, cols, 5, torch.int8,
                          torch.float64, "C3 triangular block", pairs="triangular")

