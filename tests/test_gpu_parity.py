"""GPU parity of the HIP kernels against the CPU oracle.

* split: slices and scales bit-exact for every path (row-resident,
  column-strip-resident, generic strided) and dtype combination;
* int8 cross-GEMM and the whole int8 ozaki_matmul: bit-exact;
* fp16 cross-GEMM: within the a-priori fp32 accumulation bound (the reference's
  own tl.dot accumulates in fp32 hardware order, which no other machine
  reproduces bitwise).
"""
import numpy as np
import pytest
import torch

from tests.helpers import (NAME_OF, assert_bitwise_equal, c3_like, check_block_vs_oracle,
                           fp16_cross_bound, int_valued_slices, oracle_split_batched,
                           sample_indices, to_np, values)

pytestmark = pytest.mark.gpu

COMBOS = [(torch.float64, torch.int8), (torch.float64, torch.float16),
          (torch.float32, torch.int8), (torch.float32, torch.float16)]


def _alpha(ozk, K, slice_dtype):
    return ozk.compute_split_bits(K, slice_dtype, ozk._select_dot_accum_dtype(slice_dtype))


def _check_split(oracle, ozk, X3_dev, L, slice_dtype, what):
    K = X3_dev.shape[-1]
    alpha = _alpha(ozk, K, slice_dtype)
    sl, sc = ozk.split_matrix(X3_dev, L, alpha, slice_dtype)
    torch.cuda.synchronize()
    X3 = to_np(X3_dev.contiguous())
    osl, osc = oracle_split_batched(oracle, X3, L, alpha, slice_dtype)
    assert_bitwise_equal(to_np(sc), osc, f"{what} scales")
    assert_bitwise_equal(to_np(sl), osl, f"{what} slices")


# --------------------------------------------------------------------------- #
# split
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("xdt,sdt", COMBOS)
@pytest.mark.parametrize("L", [1, 2, 4])
@pytest.mark.parametrize("rows,K", [(5, 256), (64, 1000), (33, 2048), (7, 8192)])
@pytest.mark.parametrize("kernel", ["rows", "rowscoop"])
def test_split_rows_path(oracle, gpu, xdt, sdt, L, rows, K, kernel, force):
    """K-contiguous rows: the one-workgroup row kernel and the shared row
    kernel (here one chunk per row, shorter than the chunk), each forced."""
    import ozaki_triton_amd as ozk
    force(split=kernel)
    g = torch.Generator().manual_seed(rows * K + L)
    X = torch.randn(2, rows, K, generator=g, dtype=torch.float64)
    X = X * torch.pow(10.0, torch.empty(2, rows, 1).uniform_(-3, 3, generator=g).double())
    _check_split(oracle, ozk, X.to(xdt).to(gpu), L, sdt, f"{kernel} {xdt} {sdt} L{L} {rows}x{K}")


@pytest.mark.parametrize("xdt,sdt", COMBOS)
@pytest.mark.parametrize("batch,rows,K,L", [(2, 3, 40000, 3), (1, 5, 65536, 4), (1, 4, 16388, 2)])
def test_split_rows_coop_long(oracle, gpu, xdt, sdt, batch, rows, K, L):
    """Rows longer than 16384 (the default there): 2 to 8 workgroups per row
    exchanging the level maxima, ragged last chunks, a batch, per-row
    exponents and outliers."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(batch * rows * K + L)
    X = torch.randn(batch, rows, K, generator=g, dtype=torch.float64)
    X = X * torch.pow(2.0, torch.randint(-8, 9, (batch, rows, 1), generator=g).double())
    X[torch.rand(batch, rows, K, generator=g) < 0.001] *= 1e4
    X[:, 0, :] = 0.0                                   # a zero row
    _check_split(oracle, ozk, X.to(xdt).to(gpu), L, sdt, f"rowscoop {xdt} {sdt} {rows}x{K}")


def _coop_residency():
    import ctypes
    from ozaki_triton_amd import _lib
    got = ctypes.c_int(0)
    assert _lib.load().ozk_debug_coop_residency(-1, ctypes.byref(got)) == 0
    return got.value


def test_coop_residency_matches_the_host_assumption(gpu):
    """One XCD of an MI355X holds 64 workgroups of every cooperative split
    kernel (2 per CU, the fewest over the kernels, x 32 CUs): the figure the
    planner assumes where it sees no device, so a workspace query on such a
    host plans as the device does.  A build that changes the kernels'
    registers can change it; the library's assumption must follow."""
    torch.zeros(1, device=gpu)
    r = _coop_residency()
    print(f"cooperative split kernels: {r} workgroups per XCD", flush=True)
    assert r == 64


@pytest.mark.parametrize("xdt,sdt", [(torch.float64, torch.int8), (torch.float32, torch.float16)])
def test_split_beyond_the_residency_limit(oracle, gpu, xdt, sdt, force):
    """A device assumed to hold 16 workgroups per XCD (as a small partition
    might): groups of more than 8 members are not planned, so rows of 9
    chunks take the generic kernel and 64 KB+ columns the strip kernel, with
    the oracle's bits."""
    import ozaki_triton_amd as ozk
    force(coop_resident=16)
    assert _coop_residency() == 16
    xsz = torch.empty(0, dtype=xdt).element_size()
    g = torch.Generator().manual_seed(16)
    K = 9 * (8192 if xsz == 8 else 16384)
    X = torch.randn(1, 3, K, generator=g, dtype=torch.float64)
    X = X * torch.pow(2.0, torch.randint(-8, 9, (1, 3, 1), generator=g).double())
    _check_split(oracle, ozk, X.to(xdt).to(gpu), 3, sdt, f"rows beyond residency {xdt} {K}")
    K = 9216 if xsz == 8 else 16384                 # 72 / 64 KB columns: 9 / 32 chunks
    B = torch.randn(1, K, 16, generator=g, dtype=torch.float64)
    B = B * torch.pow(2.0, torch.randint(-8, 9, (1, 1, 16), generator=g).double())
    _check_split(oracle, ozk, B.to(xdt).to(gpu).transpose(-1, -2), 3, sdt,
                 f"columns beyond residency {xdt} {K}")


@pytest.mark.parametrize("xdt,sdt", COMBOS)
@pytest.mark.parametrize("L", [1, 3, 4])
@pytest.mark.parametrize("N,K", [(8, 256), (40, 1000), (96, 2048), (24, 8192), (16, 16000)])
@pytest.mark.parametrize("kernel", ["coop", "strip"])
def test_split_strip_path(oracle, gpu, xdt, sdt, L, N, K, kernel, force):
    """B's columns through the transposed view (rows contiguous): the
    cooperative column-group kernel and the one-load-wide strip kernel, each
    forced (the planner picks by column length)."""
    import ozaki_triton_amd as ozk
    force(split=kernel)
    g = torch.Generator().manual_seed(N * K + L + 1)
    B = torch.randn(2, K, N, generator=g, dtype=torch.float64)
    B = B * torch.pow(2.0, torch.randint(-8, 9, (2, 1, N), generator=g).double())
    Bd = B.to(xdt).to(gpu)
    _check_split(oracle, ozk, Bd.transpose(-1, -2), L, sdt,
                 f"{kernel} {xdt} {sdt} L{L} {N}x{K}")


@pytest.mark.parametrize("xdt,sdt", COMBOS)
@pytest.mark.parametrize("batch,N,K,L", [(2, 264, 8192, 4), (1, 72, 16384, 3), (1, 40, 32768, 2),
                                         (3, 48, 4100, 2), (1, 256, 8192, 4), (2, 128, 2048, 3)])
def test_split_coop_groups(oracle, gpu, xdt, sdt, batch, N, K, L, force):
    """The cooperative column split (forced; the default from 64 KB columns)
    at full length: up to 32 workgroups per column group of 128-byte row
    segments (fp64 to K = 32768, fp32 to K = 16384; fp32 at K = 32768 takes
    32-byte groups), a ragged last group and a ragged last K chunk, batched
    operands, per-column exponents and outliers."""
    import ozaki_triton_amd as ozk
    force(split="coop")
    g = torch.Generator().manual_seed(batch * N * K + L)
    B = torch.randn(batch, K, N, generator=g, dtype=torch.float64)
    B = B * torch.pow(2.0, torch.randint(-8, 9, (batch, 1, N), generator=g).double())
    B[torch.rand(batch, K, N, generator=g) < 0.001] *= 1e4
    B[:, :, 5] = 0.0                                   # a zero column
    Bd = B.to(xdt).to(gpu)
    _check_split(oracle, ozk, Bd.transpose(-1, -2), L, sdt, f"coop {xdt} {sdt} b{batch} {N}x{K}")


@pytest.mark.parametrize("xdt,sdt", COMBOS)
@pytest.mark.parametrize("batch,N,K,L", [(1, 40, 65536, 3), (2, 24, 40000, 2), (1, 12, 65500, 4)])
def test_split_coop_long_columns(oracle, gpu, xdt, sdt, batch, N, K, L, force):
    """Columns too long for 32 chunks of 128-byte groups (config 5's B: fp32,
    K = 65536), with the cooperative kernel forced, take its 32-byte groups,
    whose chunks hold 4x the rows (2048 fp32 / 4096 fp64): ragged groups and
    K chunks, batched operands, outliers; bit-exact against the oracle.  (The
    planner sends such columns to the transpose path, which is faster.)"""
    import ctypes
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd import _lib
    from ozaki_triton_amd.ozaki import _TORCH_TO_OZK
    force(split="coop")
    g = torch.Generator().manual_seed(batch * N * K + L)
    B = torch.randn(batch, K, N, generator=g, dtype=torch.float64)
    B = B * torch.pow(2.0, torch.randint(-8, 9, (batch, 1, N), generator=g).double())
    B[torch.rand(batch, K, N, generator=g) < 0.001] *= 1e4
    Bd = B.to(xdt).to(gpu)
    X = Bd.transpose(-1, -2)
    name, nb = ctypes.c_char_p(), ctypes.c_size_t(0)
    sl_st = _lib.i64arr([L * N * K, N * K, K, 1])
    _lib.check("ozk_debug_split_kernel", _lib.load().ozk_debug_split_kernel(
        ctypes.c_void_p(X.data_ptr()), _TORCH_TO_OZK[xdt], batch, N, K,
        _lib.i64arr([X.stride(0), X.stride(1), X.stride(2)]), L, _TORCH_TO_OZK[sdt],
        ctypes.c_void_p(256), sl_st, ctypes.byref(name), ctypes.byref(nb)))
    assert name.value == b"coop", name.value
    _check_split(oracle, ozk, X, L, sdt, f"coop32 {xdt} {sdt} b{batch} {N}x{K}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("a_shape,b_shape", [((200, 8192), (8192, 2100)),
                                             ((64, 4096), (4096, 2048)),
                                             ((2, 96, 8192), (8192, 136))])
def test_split_pair_one_launch(oracle, gpu, sdt, a_shape, b_shape, force):
    """ozaki_matmul's two splits in one launch (split_pair_kernel: fp64
    input, A's rows by the 4-wave row configuration, B's columns by the
    cooperative kernel; A's row blocks interleaved between B's column
    groups): the library records the B phase's two events at one point; C
    equals the two-launch pipeline's (a forced split kernel turns the single
    launch off) bit for bit, and the oracle's on sampled blocks (int8
    bit-exact, float slices within the fp32 accumulation bound)."""
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd.ozaki import _ozaki_matmul_impl
    A, B = c3_like(a_shape, b_shape, seed=sum(a_shape) + sum(b_shape))
    Ad, Bd = A.to(gpu), B.to(gpu)
    L = 3
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in evs:
        e.record()
    C1 = _ozaki_matmul_impl(Ad, Bd, L, sdt, False, evs)
    torch.cuda.synchronize()
    if b_shape == (8192, 2100):
        # B's columns (64 KB each) take the cooperative kernel; split alone they
        # take tens of microseconds, back-to-back events a few
        assert evs[0].elapsed_time(evs[1]) < 0.02, "two launches where one was expected"
    force(split="coop")
    C2 = ozk.ozaki_matmul(Ad, Bd, L, sdt)
    torch.cuda.synchronize()
    assert_bitwise_equal(to_np(C1), to_np(C2), f"one launch vs two {sdt} {a_shape}")
    C_np, A_np, B_np = to_np(C1), to_np(A), to_np(B)
    M, N = a_shape[-2], b_shape[-1]
    rows, cols = sample_indices(M, 24, 3), sample_indices(N, 24, 4)
    for b in range(C_np.shape[0] if C_np.ndim == 3 else 1):
        Cb = C_np[b] if C_np.ndim == 3 else C_np
        Ab = A_np[b] if A_np.ndim == 3 else A_np
        check_block_vs_oracle(oracle, ozk, Cb, Ab, B_np, rows, cols, L, sdt, torch.float64,
                              f"pair {sdt} {a_shape} b{b}")


@pytest.mark.parametrize("xdt,sdt", COMBOS)
def test_split_generic_path(oracle, gpu, xdt, sdt):
    """Strides no fast path takes (every other column, odd K) and a K beyond
    the resident capacity."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(5)
    X = torch.randn(2, 19, 2 * 301, generator=g, dtype=torch.float64).to(xdt).to(gpu)
    _check_split(oracle, ozk, X[:, :, ::2], 3, sdt, "generic strided")
    big = 40000 if xdt == torch.float64 else 70000
    Y = torch.randn(1, 3, big, generator=g, dtype=torch.float64).to(xdt).to(gpu)
    from ozaki_triton_amd import _lib
    with _lib.forced_kernels(split="generic"):   # long rows otherwise take the shared row kernel
        _check_split(oracle, ozk, Y, 2, sdt, "generic long K")


@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
def test_split_edge_rows(oracle, gpu, xdt):
    """Zero rows, power-of-two maxima, the ceil(log2) band, clamped q,
    subnormal-scale rows and exact ties."""
    import ozaki_triton_amd as ozk
    K = 512
    X = torch.zeros(1, 8, K, dtype=torch.float64)
    X[0, 1, 7] = 1.0                                        # power of two
    X[0, 2] = -(2.0 ** -30)                                 # constant power of two
    k, j = 40, 11                                           # band: J(40) = 11
    mu = float(np.uint32(((k + 127) << 23) | j).view(np.float32))
    X[0, 3, 0] = mu
    X[0, 3, 1:] = torch.linspace(-mu, mu, K - 1, dtype=torch.float64)
    X[0, 4] = torch.arange(K, dtype=torch.float64) * 0.5 - 100.0    # ties at s = 1
    X[0, 5] = torch.randn(K, dtype=torch.float64) * 1e-37          # near fp32 underflow
    X[0, 6, ::3] = 3.0 * 2.0 ** -20
    X[0, 7] = torch.randn(K, dtype=torch.float64) * 1e30
    Xd = X.to(xdt).to(gpu)
    for L in (1, 2, 4):
        for sdt in (torch.int8, torch.float16):
            _check_split(oracle, ozk, Xd, L, sdt, f"edge {xdt} {sdt} L{L}")
            _check_split(oracle, ozk, Xd.transpose(-1, -2).contiguous().transpose(-1, -2), L,
                         sdt, f"edge strip {xdt} {sdt} L{L}")


# --------------------------------------------------------------------------- #
# cross-GEMM
# --------------------------------------------------------------------------- #
def _random_slices(g, B, L, M, N, K, sdt):
    if sdt == torch.int8:
        As = torch.randint(-128, 128, (B, L, M, K), generator=g, dtype=torch.int8)
        BsT = torch.randint(-128, 128, (B, L, N, K), generator=g, dtype=torch.int8)
    else:
        As = (torch.rand(B, L, M, K, generator=g) * 2 - 1).mul(64).to(torch.float16)
        BsT = (torch.rand(B, L, N, K, generator=g) * 2 - 1).mul(64).to(torch.float16)
    sa = torch.pow(2.0, torch.randint(-20, 5, (B, L, M), generator=g).float())
    sb = torch.pow(2.0, torch.randint(-20, 5, (B, L, N), generator=g).float())
    return As, BsT, sa, sb


def _planned(batch, M, N, K, L, sdt):
    """The cross-GEMM kernel the planner picks for K-contiguous slices on this
    device (ozk_debug_gemm_kernel)."""
    import ctypes
    from ozaki_triton_amd import _lib
    from ozaki_triton_amd.ozaki import _TORCH_TO_OZK
    name = ctypes.c_char_p()
    _lib.check("ozk_debug_gemm_kernel", _lib.load().ozk_debug_gemm_kernel(
        batch, M, N, K, L, _TORCH_TO_OZK[sdt], 0, ctypes.byref(name), None))
    return name.value.decode()


def _slices_for(g, B, L, M, N, K, sdt):
    """int8: random slices; float dtypes: integer-valued ones, for which the
    fp32-accumulated kernels are exact and must match the oracle bit for bit."""
    if sdt == torch.int8:
        return _random_slices(g, B, L, M, N, K, sdt)
    return int_valued_slices(g, B, L, M, N, K, sdt)


@pytest.mark.parametrize("L", [1, 2, 3, 4])
@pytest.mark.parametrize("out", [torch.float64, torch.float32])
@pytest.mark.parametrize("M,N,K", [(64, 64, 128), (100, 72, 1040), (256, 192, 512), (1, 130, 16)])
def test_cross_gemm_int8_bitexact(oracle, gpu, L, out, M, N, K):
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K + L)
    As, BsT, sa, sb = _random_slices(g, 2, L, M, N, K, torch.int8)
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L, out)
    torch.cuda.synchronize()
    C = to_np(C)
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 NAME_OF[out])
        assert_bitwise_equal(C[b], want, f"int8 cross L{L} {out} {M}x{N}x{K} b{b}")


@pytest.mark.parametrize("L", [1, 2, 3, 4])
@pytest.mark.parametrize("M,N,K", [(64, 64, 128), (100, 72, 1040), (128, 256, 2048)])
def test_cross_gemm_fp16_within_bound(oracle, gpu, L, M, N, K):
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(M + N + K + L)
    As, BsT, sa, sb = _random_slices(g, 1, L, M, N, K, torch.float16)
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L,
                       torch.float64)
    torch.cuda.synchronize()
    C = to_np(C)[0]
    a, bT, s_a, s_b = to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0])
    want = oracle.cross_gemm(a, bT, s_a, s_b, "float64")
    bound = fp16_cross_bound(oracle, a, bT, s_a, s_b)
    err = np.abs(C - want)
    assert np.all(err <= bound), float((err / np.maximum(bound, 1e-300)).max())


def test_cross_gemm_strided_operands(oracle, gpu):
    """N-contiguous B slices (how tune.py:60-65 calls cross_gemm) and
    non-contiguous A slices go through the pack kernel."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(9)
    L, M, N, K = 3, 70, 50, 200
    As, BsT, sa, sb = _random_slices(g, 1, L, M, N, K, torch.int8)
    Bs_n = BsT.transpose(-1, -2).contiguous()          # [1, L, K, N], N-contiguous
    A_wide = torch.zeros(1, L, M, K + 8, dtype=torch.int8)
    A_wide[..., :K] = As
    C = ozk.cross_gemm(A_wide.to(gpu)[..., :K], Bs_n.to(gpu), sa.to(gpu), sb.to(gpu), L,
                       torch.float64)
    torch.cuda.synchronize()
    want = oracle.cross_gemm(to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0]), "float64")
    assert_bitwise_equal(to_np(C)[0], want, "strided cross")


def test_cross_gemm_zero_splits(gpu):
    import ozaki_triton_amd as ozk
    As = torch.zeros(2, 0, 5, 32, dtype=torch.int8, device=gpu)
    Bs = torch.zeros(2, 0, 32, 7, dtype=torch.int8, device=gpu)
    sa = torch.zeros(2, 0, 5, device=gpu)
    sb = torch.zeros(2, 0, 7, device=gpu)
    C = ozk.cross_gemm(As, Bs, sa, sb, 0, torch.float64)
    assert C.shape == (2, 5, 7) and bool((C == 0).all())


# --------------------------------------------------------------------------- #
# ozaki_matmul end to end
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
@pytest.mark.parametrize("L", [1, 2, 3, 4])
def test_ozaki_matmul_int8_bitexact(oracle, gpu, xdt, L):
    import ozaki_triton_amd as ozk
    A, B = c3_like((2, 96, 320), (2, 320, 136), seed=L, dtype=xdt)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), L, torch.int8)
    torch.cuda.synchronize()
    want = oracle.ozaki_matmul(to_np(A), to_np(B), L, "int8")
    assert_bitwise_equal(to_np(C), want, f"ozaki int8 {xdt} L{L}")


@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
def test_ozaki_matmul_broadcast_batch(oracle, gpu, xdt):
    """torch.matmul batch broadcasting (config 4's pattern, small)."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(4)
    A = torch.randn(3, 1, 40, 128, generator=g, dtype=torch.float64).to(xdt)
    B = torch.randn(2, 128, 24, generator=g, dtype=torch.float64).to(xdt)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), 3, torch.int8)
    torch.cuda.synchronize()
    assert C.shape == (3, 2, 40, 24)
    want = oracle.ozaki_matmul(to_np(A), to_np(B), 3, "int8")
    assert_bitwise_equal(to_np(C), want, "broadcast")
    # matches torch.matmul's shape semantics and value to the scheme's accuracy
    ref = torch.matmul(A.double(), B.double())
    rel = float((C.cpu().double() - ref).norm() / ref.norm())
    assert rel < 1e-5


@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
@pytest.mark.parametrize("L", [2, 3])
def test_ozaki_matmul_fp16(oracle, gpu, xdt, L):
    import ozaki_triton_amd as ozk
    A, B = c3_like((1, 128, 512), (1, 512, 96), seed=10 + L, dtype=xdt)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), L, torch.float16)
    torch.cuda.synchronize()
    A64, B64 = to_np(A)[0], to_np(B)[0]
    alpha = ozk.compute_split_bits(512, torch.float16, torch.float32)
    a_sl, a_sc = oracle.split(A64, L, alpha, "float16")
    b_sl, b_sc = oracle.split(B64.T, L, alpha, "float16")
    want = oracle.cross_gemm(a_sl, b_sl, a_sc, b_sc, NAME_OF[xdt])
    bound = fp16_cross_bound(oracle, a_sl, b_sl, a_sc, b_sc)
    if xdt == torch.float32:
        bound = bound + 2.0 ** -23 * np.abs(want)     # output rounding to fp32
    err = np.abs(to_np(C)[0].astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= bound)


def test_ozaki_matmul_degenerate_shapes(gpu):
    import ozaki_triton_amd as ozk
    A = torch.randn(0, 4, 8, dtype=torch.float64, device=gpu)
    B = torch.randn(8, 3, dtype=torch.float64, device=gpu)
    assert ozk.ozaki_matmul(A, B, 2, torch.int8).shape == (0, 4, 3)
    A = torch.randn(4, 8, dtype=torch.float64, device=gpu)
    C = ozk.ozaki_matmul(A, B, 0, torch.int8)
    assert C.shape == (4, 3) and bool((C == 0).all())
    with pytest.raises(ValueError):
        ozk.ozaki_matmul(torch.randn(4, 0, dtype=torch.float64, device=gpu),
                         torch.randn(0, 3, dtype=torch.float64, device=gpu), 2, torch.int8)


@pytest.mark.parametrize("kernel", ["staged", "dma", "pair", "ring", "wide", "wide4",
                                    "kstep", "kstep2", "solo"])
@pytest.mark.parametrize("L", [1, 2, 3, 4])
def test_cross_gemm_each_kernel_bitexact(oracle, gpu, L, kernel, force):
    """Every cross-GEMM kernel, forced: the VGPR-staged one (taken when an
    operand's extent exceeds the 31-bit buffer offsets of the LDS-DMA kernels),
    the 2 x 2 LDS-DMA kernel, the pair-split kernel, its
    five-slot ring form (L >= 3; for L <= 2 the request falls back to the
    2 x 2 kernel), the wide kernel (L = 3), the 96 x 64 wide kernel (L = 4;
    otherwise the default kernel), the K-step kernel (32 x 32 tiles) and the
    one-wave-per-SIMD kernel (L = 4, all 16 pairs in AGPRs)."""
    import ozaki_triton_amd as ozk
    force(gemm=kernel)
    g = torch.Generator().manual_seed(77 + L)
    As, BsT, sa, sb = _random_slices(g, 1, L, 100, 72, 1040, torch.int8)
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L,
                       torch.float64)
    torch.cuda.synchronize()
    want = oracle.cross_gemm(to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0]), "float64")
    assert_bitwise_equal(to_np(C)[0], want, f"{kernel} L{L}")


@pytest.mark.parametrize("sdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kernel,L,M,N,K", [
    ("ring", 2, 256, 384, 4096),    # config 2's kernel: 128 x 128 tiles, K = 4096
    ("wide", 3, 128, 256, 2048),    # config 4's kernel: 64 x 128 tiles, K = 2048
    ("ring", 4, 128, 192, 8192),    # 64 x 64 tiles, K = 8192
    ("wide4", 4, 192, 128, 8192),   # config 3's kernel: 96 x 64 tiles, K = 8192
    ("wide4", 4, 100, 72, 1040),
    ("ring", 3, 130, 72, 4096),
    ("pair", 3, 100, 72, 1040),
    ("pair", 4, 100, 72, 1040),
    ("dma", 1, 130, 260, 1040),
    ("dma", 2, 130, 136, 1040),
    ("staged", 2, 100, 72, 1040),
    ("staged", 4, 100, 72, 520),
    ("kstep", 4, 100, 72, 1040),    # (fp32 slices at L = 4: the planner's kernel)
    ("kstep", 3, 130, 72, 4096),
    ("kstep", 2, 64, 96, 2064),
    ("kstep", 1, 40, 200, 1040),
    ("kstep2", 4, 100, 72, 1040),
    ("kstep2", 3, 130, 72, 4096),
    ("kstep2", 2, 64, 96, 2064),
    ("solo", 4, 100, 72, 1040),     # (fp32 slices: the planner's kernel)
    ("solo", 4, 130, 200, 4096),
])
def test_float_slice_kernels_bitexact(oracle, gpu, kernel, L, M, N, K, sdt, force):
    """Every cross-GEMM kernel with float slices, at the tile shapes and K of
    the BASELINE configurations it serves: on integer-valued slices the
    fp32-accumulated dot is exact in any order, so C must equal the oracle bit
    for bit.  Unlike a tolerance, this fails for a kernel that drops any one
    slice pair (test_oracle_pins.py:test_int_valued_check_catches_a_dropped_pair)."""
    import ozaki_triton_amd as ozk
    force(gemm=kernel)
    g = torch.Generator().manual_seed(M * 3 + N + K + L)
    As, BsT, sa, sb = int_valued_slices(g, 1, L, M, N, K, sdt)
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L,
                       torch.float64)
    torch.cuda.synchronize()
    want = oracle.cross_gemm(to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0]), "float64")
    assert_bitwise_equal(to_np(C)[0], want, f"{kernel} L{L} {sdt} {M}x{N}x{K}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("L", [2, 3, 4])
@pytest.mark.parametrize("K", [16, 128, 200, 300, 520, 1040, 2064])
def test_ring_kernel_stage_counts(oracle, gpu, L, K, sdt, force):
    """The five-slot ring kernel over 1 to 17 stages of 128 bytes of K (the
    prologue fetches a stage and a half, the loop issues each stage's DMA
    ahead over the K steps of the stages before, and the last stage fetches
    the tile's scales into a free slot), with 64 x 64 tiles (L = 3, 4) and
    128 x 128 tiles (L = 2; M and N cut a tile): int8 and integer-valued fp16
    slices bit-exact against the oracle."""
    kernel = "ring"
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(K * 10 + L)
    M, N = (130, 72) if L >= 3 else (200, 136)
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    args = (As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L, torch.float64)
    force(gemm=kernel)
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 "float64")
        assert_bitwise_equal(C[b], want, f"{kernel} {sdt} L{L} K{K} b{b}")


@pytest.mark.parametrize("out", [torch.float64, torch.float32, torch.float16, torch.bfloat16,
                                 torch.int8])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("L", [1, 3, 4])
@pytest.mark.parametrize("kernel", ["kstep", "kstep2"])
def test_kstep_kernel_dtypes(oracle, gpu, L, sdt, out, kernel, force):
    """The K-step kernel, in its 4-wave and its 8-wave (two pair groups)
    form, for every slice and output dtype, batched, with a broadcast (batch
    stride 0) B: int8 and integer-valued float slices bit-exact against the
    oracle (fp32 slices at L = 4 take the planner's kernel for the 4-wave
    form, and L = 1 the 4-wave form for the 8-wave one)."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(ALL_SLICES.index(sdt) * 11 + len(str(out)) + 40 * L)
    M, N, K = 70, 100, 400
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    if out in (torch.float16, torch.bfloat16, torch.int8):
        sa = sa * 2.0 ** (12 if sdt == torch.int8 else 0)
    Bd = BsT[:1].to(gpu).expand(2, -1, -1, -1).transpose(-1, -2)   # broadcast B
    sbd = sb[:1].to(gpu).expand(2, -1, -1)
    args = (As.to(gpu), Bd, sa.to(gpu), sbd, L, out)
    force(gemm=kernel)
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[0]), to_np(sa[b]), to_np(sb[0]),
                                 NAME_OF[out])
        assert_bitwise_equal(C[b], want, f"{kernel} L{L} {sdt} {out} b{b}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("L", [1, 2, 3, 4])
@pytest.mark.parametrize("K", [16, 128, 200, 520, 1040, 2064])
@pytest.mark.parametrize("kernel", ["kstep", "kstep2"])
def test_kstep_kernel_stage_counts(oracle, gpu, L, K, sdt, kernel, force):
    """The K-step kernel (32 x 32 tiles, wave w on K step w of every stage,
    the waves' accumulators summed through the LDS; with kstep2 two such sets
    of 4 waves, each holding half the slice pairs) over 1 to 17 stages of
    128 bytes of K against a ring of 5 or 6 stage slots (fewer stages than
    the prologue would fetch, and more than the ring holds), M and N cutting
    tiles, batch 2: int8 and integer-valued fp16 slices bit-exact against the
    oracle."""
    import ozaki_triton_amd as ozk
    M, N = 70, 45
    g = torch.Generator().manual_seed(K * 10 + L + 5)
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    args = (As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L, torch.float64)
    force(gemm=kernel)
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 "float64")
        assert_bitwise_equal(C[b], want, f"{kernel} {sdt} L{L} K{K} b{b}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("MN", [(130, 200), (64, 128), (200, 136), (1, 300)])
@pytest.mark.parametrize("K", [16, 128, 200, 300, 520, 1040, 2064])
def test_wide_kernel_stage_counts(oracle, gpu, K, MN, sdt, force):
    """The num_splits 3 wide kernel (64 x 128 tiles, every wave holding all 9
    pairs of its 32 x 32 block, two whole stages in the LDS) over 1 to 17
    stages of 128 bytes of K (the prologue fetches stages 0 and 1, the loop
    fetches stage kb + 2 after the barrier of stage kb, the last stage fetches
    the tile's scales into the free buffer), with M and N cutting tiles, and
    batch 2: int8 and integer-valued fp16 slices bit-exact against the
    oracle."""
    import ozaki_triton_amd as ozk
    L, (M, N) = 3, MN
    g = torch.Generator().manual_seed(K * 10 + M + N)
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    args = (As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L, torch.float64)
    force(gemm="wide")
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 "float64")
        assert_bitwise_equal(C[b], want, f"wide {sdt} K{K} M{M} N{N} b{b}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("MN", [(200, 130), (96, 64), (97, 65), (1, 300), (300, 1)])
@pytest.mark.parametrize("K", [16, 128, 200, 300, 520, 1040, 2064])
def test_wide4_kernel_stage_counts(oracle, gpu, K, MN, sdt, force):
    """The num_splits 4 wide kernel (96 x 64 tiles; waves holding pairs
    i = 0..2 of one 32 x 32 block or pairs i = 3 of three blocks, one partial
    hand-off through the LDS; two whole stages of 80 KB) over 1 to 17 stages
    of 128 bytes of K (prologue, the loop's two DMA parts, the last stage's
    scale fetch), with M and N cutting tiles and batch 2: int8 and
    integer-valued fp16 slices bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    L, (M, N) = 4, MN
    g = torch.Generator().manual_seed(K * 10 + M + 3 * N)
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    args = (As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L, torch.float64)
    force(gemm="wide4")
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 "float64")
        assert_bitwise_equal(C[b], want, f"wide4 {sdt} K{K} M{M} N{N} b{b}")


@pytest.mark.parametrize("out", [torch.float64, torch.float32, torch.float16, torch.bfloat16,
                                 torch.int8])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16, torch.bfloat16, torch.float32])
def test_wide4_kernel_dtypes(oracle, gpu, sdt, out, force):
    """The num_splits 4 wide kernel for every slice and output dtype, batched,
    with a broadcast (batch stride 0) B: int8 and integer-valued float slices
    bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    L = 4
    g = torch.Generator().manual_seed(ALL_SLICES.index(sdt) * 11 + len(str(out)) + 900)
    M, N, K = 150, 100, 400
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    if out in (torch.float16, torch.bfloat16, torch.int8):
        sa = sa * 2.0 ** (12 if sdt == torch.int8 else 0)
    Bd = BsT[:1].to(gpu).expand(2, -1, -1, -1).transpose(-1, -2)   # broadcast B
    sbd = sb[:1].to(gpu).expand(2, -1, -1)
    args = (As.to(gpu), Bd, sa.to(gpu), sbd, L, out)
    force(gemm="wide4")
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[0]), to_np(sa[b]), to_np(sb[0]),
                                 NAME_OF[out])
        assert_bitwise_equal(C[b], want, f"wide4 {sdt} {out} b{b}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("MN", [(130, 200), (64, 64), (65, 63), (1, 300), (300, 1)])
@pytest.mark.parametrize("K", [16, 128, 200, 300, 520, 1040, 2064])
def test_solo5_kernel_stage_counts(oracle, gpu, K, MN, sdt):
    """The num_splits 5 kernel (64 x 64 tiles, one wave per SIMD holding all 25
    pairs of its 32 x 32 block, 16 accumulator tiles in AGPRs and 9 in VGPRs,
    two whole stages of 80 KB) over 1 to 17 stages of 128 bytes of K
    (prologue, the loop's two DMA parts, the last stage's scale fetch), with M
    and N cutting tiles and batch 2, chosen by the planner: int8 and
    integer-valued fp16 slices bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    L, (M, N) = 5, MN
    assert _planned(1, M, N, K, L, sdt) == "solo"
    g = torch.Generator().manual_seed(K * 10 + 7 * M + N)
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    args = (As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L, torch.float64)
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 "float64")
        assert_bitwise_equal(C[b], want, f"solo5 {sdt} K{K} M{M} N{N} b{b}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("MN", [(130, 200), (65, 63), (1, 300)])
@pytest.mark.parametrize("K", [16, 128, 200, 520, 1040, 2064])
def test_solo_kernel_four_slices_triangle(oracle, gpu, K, MN, sdt):
    """The one-wave-per-SIMD kernel at num_splits 4 on the triangular pair set
    (10 pairs of a 32 x 32 block in 160 AGPRs; the planner's kernel off wide4's
    rounds rule), over 1 to 17 stages of 128 bytes of K, with M and N cutting
    tiles and batch 2: int8 and integer-valued fp16 slices bit-exact against
    the oracle."""
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd import _lib
    L, (M, N) = 4, MN
    g = torch.Generator().manual_seed(K * 10 + 7 * M + N + 4)
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    args = (As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L, torch.float64)
    with _lib.forced_kernels(gemm="solo"):
        C = to_np(ozk.cross_gemm(*args, pairs="triangular"))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 "float64", pairs="triangular")
        assert_bitwise_equal(C[b], want, f"solo L4 tri {sdt} K{K} M{M} N{N} b{b}")


@pytest.mark.parametrize("out", [torch.float64, torch.float32, torch.float16, torch.bfloat16,
                                 torch.int8])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16, torch.bfloat16])
def test_solo5_kernel_dtypes(oracle, gpu, sdt, out):
    """The num_splits 5 kernel for every slice dtype it takes and every output
    dtype (an fp32 outer accumulator for all but fp64), batched, with a
    broadcast (batch stride 0) B: int8 and integer-valued float slices
    bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    L = 5
    g = torch.Generator().manual_seed(ALL_SLICES.index(sdt) * 13 + len(str(out)) + 1900)
    M, N, K = 150, 100, 400
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    if out in (torch.float16, torch.bfloat16, torch.int8):
        sa = sa * 2.0 ** (12 if sdt == torch.int8 else 0)
    Bd = BsT[:1].to(gpu).expand(2, -1, -1, -1).transpose(-1, -2)   # broadcast B
    sbd = sb[:1].to(gpu).expand(2, -1, -1)
    C = to_np(ozk.cross_gemm(As.to(gpu), Bd, sa.to(gpu), sbd, L, out))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[0]), to_np(sa[b]), to_np(sb[0]),
                                 NAME_OF[out])
        assert_bitwise_equal(C[b], want, f"solo5 {sdt} {out} b{b}")


@pytest.mark.parametrize("xdt,sdt", [(torch.float64, torch.int8), (torch.float32, torch.int8),
                                     (torch.float64, torch.bfloat16)])
def test_ozaki_matmul_five_splits(oracle, gpu, xdt, sdt):
    """The public ozaki_matmul with max_splits raised to 5 (the reference stops
    at 4, ozaki_triton.py:563): splits and the one-launch num_splits 5
    cross-GEMM, bit-exact against the oracle (int8 slices) or within the fp32
    accumulation bound (bf16 slices); for fp64 inputs with int8 slices the
    result is closer to the exact product than with 4 slices."""
    import ozaki_triton_amd as ozk
    A, B = c3_like((2, 96, 1040), (1040, 80), seed=555, dtype=xdt)
    Ad, Bd = A.to(gpu), B.to(gpu)
    C5 = ozk.ozaki_matmul(Ad, Bd, 5, sdt, max_splits=5)
    torch.cuda.synchronize()
    C_np, A_np, B_np = to_np(C5), to_np(A), to_np(B)
    rows, cols = np.arange(96), np.arange(80)
    for b in range(2):
        check_block_vs_oracle(oracle, ozk, C_np[b], A_np[b], B_np, rows, cols, 5, sdt, xdt,
                              f"L5 {xdt} {sdt} b{b}")
    if xdt == torch.float64 and sdt == torch.int8:
        C4 = ozk.ozaki_matmul(Ad, Bd, 4, sdt)
        ref = A @ B
        rel = lambda C: float((C.cpu() - ref).norm() / ref.norm())
        assert rel(C5) < rel(C4)


def _planned_ksplit(batch, M, N, K, L, sdt):
    import ctypes
    from ozaki_triton_amd import _lib
    from ozaki_triton_amd.ozaki import _TORCH_TO_OZK
    name, ks = ctypes.c_char_p(), ctypes.c_int(0)
    _lib.check("ozk_debug_gemm_kernel", _lib.load().ozk_debug_gemm_kernel(
        batch, M, N, K, L, _TORCH_TO_OZK[sdt], 0, ctypes.byref(name), ctypes.byref(ks)))
    return name.value.decode(), ks.value


@pytest.mark.parametrize("out", [torch.float64, torch.float32])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("kernel,L,ranges,MN,K", [
    ("ring", 4, 2, (130, 72), 1040),    # int8: 9 stages of 128 bytes, ranges of 5 and 4
    ("ring", 4, 4, (64, 64), 2064),     # 17 stages: 5, 5, 5, 2
    ("ring", 3, 3, (65, 200), 520),     # 5 stages: 2, 2, 1
    ("ring", 2, 2, (200, 136), 1040),   # 128 x 128 tiles
    ("ring", 4, 8, (1, 300), 1040),     # 9 stages: 8 ranges asked, 5 of 2 stages run
    ("wide", 3, 2, (130, 200), 1040),
    ("wide", 3, 4, (64, 128), 4096),
])
def test_splitk_bitexact(oracle, gpu, sdt, out, kernel, L, ranges, MN, K, force):
    """Split-K (ring and wide kernels): every tile's K cut into ranges, one
    workgroup each; each range stores its raw accumulators, the last to
    arrive adds all of them in range order and runs the ordered epilogue.
    Forced range counts, ranges of unequal length, M and N cutting tiles,
    batch 2 and both outer accumulators: int8 (exact int32 sums) and
    integer-valued fp16 slices bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    M, N = MN
    force(gemm=kernel, ksplit=ranges)
    es = 1 if sdt == torch.int8 else 2
    nkb = -(-K * es // 128)
    per = -(-nkb // ranges)
    assert _planned_ksplit(2, M, N, K, L, sdt) == (kernel, -(-nkb // per))
    g = torch.Generator().manual_seed(K + 3 * M + N + L + ranges)
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    C = to_np(ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu),
                             L, out))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 NAME_OF[out])
        assert_bitwise_equal(C[b], want, f"{kernel} ksplit {ranges} {sdt} {out} b{b}")


@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kernel,L,ranges,MN,K", [("ring", 4, 3, (100, 72), 1040),
                                                 ("wide", 3, 2, (130, 200), 1040)])
def test_splitk_other_slice_dtypes(oracle, gpu, sdt, kernel, L, ranges, MN, K, force):
    """Split-K with bf16 and fp32 slices (fp32: four MFMAs per fragment),
    integer-valued so that the fp32 sums are exact: bit-exact against the
    oracle."""
    import ozaki_triton_amd as ozk
    M, N = MN
    force(gemm=kernel, ksplit=ranges)
    g = torch.Generator().manual_seed(K + M + N + ranges)
    As, BsT, sa, sb = int_valued_slices(g, 2, L, M, N, K, sdt)
    C = to_np(ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu),
                             L, torch.float64))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 "float64")
        assert_bitwise_equal(C[b], want, f"{kernel} ksplit {ranges} {sdt} b{b}")


def test_splitk_without_workspace_runs_unsplit(oracle, gpu, force):
    """A call whose workspace lacks the split-K buffers (here: none at all)
    runs the same kernel without split-K: same bits."""
    import ctypes
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd import _lib
    L, M, N, K = 4, 64, 128, 2048
    force(gemm="ring", ksplit=4)
    g = torch.Generator().manual_seed(99)
    As, BsT, sa, sb = _random_slices(g, 1, L, M, N, K, torch.int8)
    Ad, Bd, sad, sbd = As.to(gpu), BsT.to(gpu), sa.to(gpu), sb.to(gpu)
    C = torch.empty(1, M, N, dtype=torch.float64, device=gpu)
    a_st = _lib.i64arr([L * M * K, M * K, K, 1])
    b_st = _lib.i64arr([L * N * K, N * K, 1, K])
    st = _lib.load().ozk_cross_gemm(
        ctypes.c_void_p(Ad.data_ptr()), a_st, ctypes.c_void_p(Bd.data_ptr()), b_st,
        ctypes.c_void_p(sad.data_ptr()), _lib.i64arr([L * M, M, 1]),
        ctypes.c_void_p(sbd.data_ptr()), _lib.i64arr([L * N, N, 1]), 1, M, N, K, L,
        _lib.OZK_I8, ctypes.c_void_p(C.data_ptr()), _lib.OZK_F64, _lib.i64arr([M * N, N, 1]),
        ctypes.c_void_p(0), 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, _lib.strerror(st)
    torch.cuda.synchronize()
    want = oracle.cross_gemm(to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0]), "float64")
    assert_bitwise_equal(to_np(C)[0], want, "no workspace")


@pytest.mark.parametrize("gemm", ["", "ring"])
@pytest.mark.parametrize("xdt,sdt", [(torch.float64, torch.int8), (torch.float32, torch.float16),
                                     (torch.float64, torch.float16)])
@pytest.mark.parametrize("L", [1, 2, 3, 4])
def test_reference_point_small_grid(oracle, gpu, xdt, sdt, L, gemm, force):
    """The reference's published point (1, 128, 2048, 4096)
    (reference/test_results.csv): 64 tiles of 64 x 64 on 256 CUs.  The
    planner takes the K-step kernel's 256 tiles of 32 x 32; with the ring
    kernel forced (L >= 3) it cuts K into split-K ranges of at least 16
    stages: 2 for int8 slices (32 stages), 4 for fp16 (64).  ozaki_matmul end
    to end, sampled blocks against the oracle (int8 bit-exact, fp16 within
    the fp32 accumulation bound)."""
    import ozaki_triton_amd as ozk
    M, N, K = 128, 2048, 4096
    if gemm:
        if L < 3:
            pytest.skip("the ring kernel serves 3 and 4 slices here")
        force(gemm=gemm)
    kern, ks = _planned_ksplit(1, M, N, K, L, sdt)
    if torch.cuda.get_device_properties(0).multi_processor_count >= 256:
        if gemm:
            assert (kern, ks) == ("ring", 2 if sdt == torch.int8 else 4)
        else:
            assert (kern, ks) == ("kstep" if L == 1 else "kstep2", 1)
    A, B = c3_like((1, M, K), (1, K, N), seed=L + 17, dtype=xdt)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), L, sdt)
    torch.cuda.synchronize()
    rows, cols = sample_indices(M, 24, 1), sample_indices(N, 24, 2)
    check_block_vs_oracle(oracle, ozk, to_np(C)[0], to_np(A)[0], to_np(B)[0], rows, cols, L, sdt,
                          xdt, f"ref point L{L} {xdt} {sdt} {gemm or 'planned'}")


@pytest.mark.parametrize("out", [torch.float64, torch.float32, torch.float16, torch.bfloat16,
                                 torch.int8])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16, torch.bfloat16, torch.float32])
def test_wide_kernel_dtypes(oracle, gpu, sdt, out, force):
    """The wide kernel for every slice and output dtype, batched, with a
    broadcast (batch stride 0) B: int8 and integer-valued float slices
    bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    L = 3
    g = torch.Generator().manual_seed(ALL_SLICES.index(sdt) * 7 + len(str(out)) + 500)
    M, N, K = 100, 150, 400
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    if out in (torch.float16, torch.bfloat16, torch.int8):
        sa = sa * 2.0 ** (12 if sdt == torch.int8 else 0)
    Bd = BsT[:1].to(gpu).expand(2, -1, -1, -1).transpose(-1, -2)   # broadcast B
    sbd = sb[:1].to(gpu).expand(2, -1, -1)
    args = (As.to(gpu), Bd, sa.to(gpu), sbd, L, out)
    force(gemm="wide")
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[0]), to_np(sa[b]), to_np(sb[0]),
                                 NAME_OF[out])
        assert_bitwise_equal(C[b], want, f"wide {sdt} {out} b{b}")


@pytest.mark.parametrize("out", [torch.float64, torch.float32, torch.float16, torch.bfloat16,
                                 torch.int8])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("L", [2, 3, 4])
def test_ring_kernel_dtypes(oracle, gpu, L, sdt, out, force):
    """The ring kernel for every slice and output dtype, batched, with a
    broadcast (batch stride 0) B: int8 and integer-valued float slices
    bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(L * 41 + ALL_SLICES.index(sdt) * 7 + len(str(out)))
    M, N, K = (100, 72, 400) if L >= 3 else (150, 136, 400)
    As, BsT, sa, sb = _slices_for(g, 2, L, M, N, K, sdt)
    if out in (torch.float16, torch.bfloat16, torch.int8):
        sa = sa * 2.0 ** (12 if sdt == torch.int8 else 0)
    Bd = BsT[:1].to(gpu).expand(2, -1, -1, -1).transpose(-1, -2)   # broadcast B
    sbd = sb[:1].to(gpu).expand(2, -1, -1)
    args = (As.to(gpu), Bd, sa.to(gpu), sbd, L, out)
    force(gemm="ring")
    C = to_np(ozk.cross_gemm(*args))
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[0]), to_np(sa[b]), to_np(sb[0]),
                                 NAME_OF[out])
        assert_bitwise_equal(C[b], want, f"ring L{L} {sdt} {out} b{b}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
@pytest.mark.parametrize("a_shape,b_shape", [((2, 96, 200), (2, 200, 72)),    # strip 0, rows 0
                                             ((40, 400), (400, 136)),         # strip 0, rows 1
                                             ((3, 50, 1000), (1000, 24)),     # strip 0, rows 2
                                             ((64, 2000), (2000, 48)),        # strip 1, rows 3
                                             ((33, 4000), (4000, 40)),        # strip 2, rows 4
                                             ((20, 8000), (8000, 16))])       # strip 3, rows 5
def test_split_duo_one_launch(oracle, gpu, sdt, xdt, a_shape, b_shape, force):
    """ozaki_matmul's two splits in one launch (split_duo_kernel: B's columns
    by the 256-lane strip kernel, A's rows by a 256-lane row configuration,
    the strips first): the library records the B phase's two events at one
    point; C equals the two-launch pipeline's (a forced split kernel turns
    the single launch off) bit for bit, and the oracle's on sampled blocks
    (int8 bit-exact, float slices within the fp32 accumulation bound).  The
    pairs of configurations follow K; the last (K <= 8192) is fp64 only."""
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd.ozaki import _ozaki_matmul_impl
    if xdt == torch.float32 and a_shape[-1] > 4096:
        pytest.skip("fp32 columns over 4096 take the 512-lane strip kernel")
    A, B = c3_like(a_shape, b_shape, seed=sum(a_shape) + sum(b_shape) + 7, dtype=xdt)
    Ad, Bd = A.to(gpu), B.to(gpu)
    L = 3
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in evs:
        e.record()
    C1 = _ozaki_matmul_impl(Ad, Bd, L, sdt, False, evs)
    torch.cuda.synchronize()
    assert evs[0].elapsed_time(evs[1]) < 0.02, "two launches where one was expected"
    force(split="strip")
    C2 = ozk.ozaki_matmul(Ad, Bd, L, sdt)
    torch.cuda.synchronize()
    assert_bitwise_equal(to_np(C1), to_np(C2), f"one launch vs two {xdt} {sdt} {a_shape}")
    C_np, A_np, B_np = to_np(C1), to_np(A), to_np(B)
    M, N = a_shape[-2], b_shape[-1]
    rows, cols = sample_indices(M, 16, 5), sample_indices(N, 16, 6)
    for b in range(C_np.shape[0] if C_np.ndim == 3 else 1):
        Cb = C_np[b] if C_np.ndim == 3 else C_np
        Ab = A_np[b] if A_np.ndim == 3 else A_np
        Bb = B_np[b] if B_np.ndim == 3 else B_np
        check_block_vs_oracle(oracle, ozk, Cb, Ab, Bb, rows, cols, L, sdt, xdt,
                              f"duo {xdt} {sdt} {a_shape} b{b}")


@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
def test_split_coop_wait_timeout(oracle, gpu, xdt, force):
    """The cooperative split's bounded wait: forced from the host to look for a
    tag no member writes and to give up at its first check, every wait runs
    out, the kernel still finishes, every scale of the split comes out NaN
    and the sticky device status reports OZK_ERR_DEVICE_WAIT (once: reading
    clears it).  Through ozaki_matmul the whole C is NaN.  Afterwards the
    normal path gives the oracle's bits again and sets no status."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(21)
    K, N, L = 4096, 64, 3
    B = torch.randn(1, K, N, generator=g, dtype=torch.float64).to(xdt).to(gpu)
    BT = B.transpose(-1, -2)
    alpha = _alpha(ozk, K, torch.int8)
    from ozaki_triton_amd import _lib
    ozk.device_status()                       # clear anything older
    force(split="coop")
    force(coop_timeout=True)
    sl, sc = ozk.split_matrix(BT, L, alpha, torch.int8)
    torch.cuda.synchronize()
    assert torch.isnan(sc).all(), "every scale of the split should be NaN after the timeout"
    with pytest.raises(_lib.OzakiLibError) as e:
        ozk.device_status()
    assert e.value.status == _lib.OZK_ERR_DEVICE_WAIT
    ozk.device_status()                       # cleared by the read above
    # through ozaki_matmul: C is NaN everywhere (B's scales are), and flagged
    A = torch.randn(1, 40, K, dtype=torch.float64).to(xdt).to(gpu)
    C = ozk.ozaki_matmul(A, B, L, torch.int8)
    torch.cuda.synchronize()
    assert torch.isnan(C).all()
    with pytest.raises(_lib.OzakiLibError):
        ozk.device_status()
    force(coop_timeout=False)
    _check_split(oracle, ozk, BT, L, torch.int8, f"coop after timeout {xdt}")
    ozk.device_status()                       # the normal path sets nothing


@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
def test_split_rows_coop_wait_timeout(oracle, gpu, xdt, force):
    """The shared row kernel's bounded wait, forced to run out as above: the
    kernel finishes, the scales come out NaN and the device status is set;
    the normal path is exact again afterwards."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(22)
    X = torch.randn(1, 3, 40000, generator=g, dtype=torch.float64).to(xdt).to(gpu)
    alpha = _alpha(ozk, 40000, torch.int8)
    from ozaki_triton_amd import _lib
    ozk.device_status()
    force(coop_timeout=True)
    sl, sc = ozk.split_matrix(X, 2, alpha, torch.int8)
    torch.cuda.synchronize()
    assert torch.isnan(sc).all(), "every scale of the split should be NaN after the timeout"
    with pytest.raises(_lib.OzakiLibError):
        ozk.device_status()
    force(coop_timeout=False)
    _check_split(oracle, ozk, X, 2, torch.int8, f"rowscoop after timeout {xdt}")
    ozk.device_status()


@pytest.mark.parametrize("xdt,sdt", COMBOS)
@pytest.mark.parametrize("long", [False, True])
def test_split_transpose_path(oracle, gpu, xdt, sdt, long, force):
    """Column splits (B^T view) through the transpose into the workspace and a
    row kernel (the path for columns longer than the cooperative column kernel
    takes): rows up to 16384 go to the one-workgroup row kernel, longer ones
    (config 5's B is 65536 long) to the shared row kernel."""
    import ozaki_triton_amd as ozk
    force(split="transpose")
    g = torch.Generator().manual_seed(11)
    K = (20000 if xdt == torch.float64 else 65536) if long else 12000
    B = torch.randn(1, K, 40, generator=g, dtype=torch.float64)
    B[torch.rand(1, K, 40, generator=g) < 0.01] *= 1e4
    Bd = B.to(xdt).to(gpu)
    _check_split(oracle, ozk, Bd.transpose(-1, -2), 3, sdt, f"transpose {xdt} {sdt}")


# --------------------------------------------------------------------------- #
# the remaining dtypes of the reference's tables (ozaki_triton.py:35-48):
# fp16 / bf16 / int8 inputs (split in fp32 after an exact conversion), bf16 and
# fp32 slices, and C in the input dtype
# --------------------------------------------------------------------------- #
ALL_INPUTS = [torch.float64, torch.float32, torch.float16, torch.bfloat16, torch.int8]
ALL_SLICES = [torch.int8, torch.float16, torch.bfloat16, torch.float32]
NEW_COMBOS = [(x, s) for x in ALL_INPUTS for s in ALL_SLICES if (x, s) not in COMBOS]


def _random_input(g, shape, xdt):
    if xdt == torch.int8:
        return torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)
    X = torch.randn(*shape, generator=g, dtype=torch.float64)
    lo, hi = (-3, 3) if xdt == torch.float16 else (-6, 7)   # keep fp16 products finite
    X = X * torch.pow(2.0, torch.randint(lo, hi, (*shape[:-1], 1), generator=g).double())
    return X.to(xdt)


@pytest.mark.parametrize("xdt,sdt", NEW_COMBOS)
@pytest.mark.parametrize("layout", ["rows", "columns", "strided"])
def test_split_all_dtypes(oracle, gpu, xdt, sdt, layout):
    """Slices and scales bit-exact for every (input, slice) pair the reference
    accepts, on K-contiguous rows, on B's columns (transposed view) and on a
    strided view."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(ALL_INPUTS.index(xdt) * 7 + ALL_SLICES.index(sdt))
    if layout == "rows":
        X = _random_input(g, (2, 33, 1000), xdt).to(gpu)
    elif layout == "columns":
        X = _random_input(g, (2, 1000, 48), xdt).to(gpu).transpose(-1, -2)
    else:
        X = _random_input(g, (2, 33, 2 * 300), xdt).to(gpu)[..., ::2]
    _check_split(oracle, ozk, X, 3, sdt, f"{layout} {xdt} {sdt}")


@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("L", [1, 2, 3, 4])
@pytest.mark.parametrize("M,N,K", [(64, 64, 128), (100, 72, 1040)])
def test_cross_gemm_bf16_fp32_within_bound(oracle, gpu, sdt, L, M, N, K):
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(M + N + K + L + (7 if sdt == torch.float32 else 0))
    As = (torch.rand(1, L, M, K, generator=g) * 2 - 1).mul(64).to(sdt)
    BsT = (torch.rand(1, L, N, K, generator=g) * 2 - 1).mul(64).to(sdt)
    sa = torch.pow(2.0, torch.randint(-20, 5, (1, L, M), generator=g).float())
    sb = torch.pow(2.0, torch.randint(-20, 5, (1, L, N), generator=g).float())
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L,
                       torch.float64)
    torch.cuda.synchronize()
    a, bT, s_a, s_b = to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0])
    want = oracle.cross_gemm(a, bT, s_a, s_b, "float64")
    bound = fp16_cross_bound(oracle, a, bT, s_a, s_b)
    err = np.abs(to_np(C)[0] - want)
    assert np.all(err <= bound), float((err / np.maximum(bound, 1e-300)).max())


@pytest.mark.parametrize("out", [torch.float16, torch.bfloat16, torch.int8])
@pytest.mark.parametrize("L", [2, 4])
def test_cross_gemm_output_dtypes_bitexact(oracle, gpu, out, L):
    """int8 slices make the fp32 outer sum exact to the reference's, so C in
    fp16 / bf16 (round to nearest even) and int8 (truncate, saturate) is too."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(31 + L)
    As, BsT, sa, sb = _random_slices(g, 1, L, 100, 72, 520, torch.int8)
    sa = sa * 2.0 ** 12
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L, out)
    torch.cuda.synchronize()
    want = oracle.cross_gemm(to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0]),
                             NAME_OF[out])
    assert_bitwise_equal(to_np(C)[0], want, f"out {out} L{L}")


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.int8])
@pytest.mark.parametrize("sdt", ALL_SLICES)
def test_ozaki_matmul_narrow_inputs(oracle, gpu, xdt, sdt):
    """End to end for the narrow inputs: int8 slices bit-exact; float slices
    within the fp32 accumulation bound plus one rounding of C's dtype."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(ALL_INPUTS.index(xdt) * 5 + ALL_SLICES.index(sdt))
    A = _random_input(g, (2, 70, 300), xdt)
    B = _random_input(g, (300, 50), xdt)
    L = 2
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), L, sdt)
    torch.cuda.synchronize()
    assert C.dtype == xdt and C.shape == (2, 70, 50)
    want, alpha, parts = oracle.ozaki_matmul(to_np(A), to_np(B), L, NAME_OF[sdt],
                                             return_parts=True)
    got = to_np(C)
    if sdt == torch.int8:
        assert_bitwise_equal(got, want, f"{xdt} {sdt}")
        return
    for b, (a_sl, a_sc, b_sl, b_sc) in enumerate(parts):
        bound = fp16_cross_bound(oracle, a_sl, b_sl, a_sc, b_sc)
        gv, wv = values(got[b]), values(want[b])
        if xdt == torch.int8:
            slack = 1.0                              # truncation may step by one
        else:
            ulp = 2.0 ** -10 if xdt == torch.float16 else 2.0 ** -7
            slack = ulp * np.abs(wv) + 2.0 ** -24
        assert np.all(np.abs(gv - wv) <= bound + slack), f"{xdt} {sdt} batch {b}"


def test_matmul_c_abi_with_caller_workspace_and_events(oracle, gpu):
    """ozk_matmul called directly through the C ABI with a caller workspace
    (no allocation inside) equals the oracle bit for bit, and records the four
    phase events on the stream."""
    import ctypes
    from ozaki_triton_amd import _lib
    A, B = c3_like((96, 520), (520, 72), seed=41)
    Ad, Bd = A.to(gpu), B.to(gpu)
    L = _lib.load()
    nb = ctypes.c_size_t(0)
    a = _lib.i64arr([0, 520, 1])
    b = _lib.i64arr([0, 72, 1])
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, 96, 72, 520, a, b, 3, _lib.OZK_I8,
                                        ctypes.byref(nb)) == 0
    ws = torch.empty(nb.value, dtype=torch.uint8, device=gpu)
    C = torch.empty(96, 72, dtype=torch.float64, device=gpu)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in evs:
        e.record()
    arr = (ctypes.c_void_p * 4)(*[ctypes.c_void_p(e.cuda_event) for e in evs])
    st = L.ozk_matmul(ctypes.c_void_p(Ad.data_ptr()), a, ctypes.c_void_p(Bd.data_ptr()), b,
                      _lib.OZK_F64, 1, 96, 72, 520, 3, _lib.OZK_I8, ctypes.c_void_p(C.data_ptr()),
                      _lib.i64arr([96 * 72, 72, 1]), ctypes.c_void_p(ws.data_ptr()), nb.value,
                      arr, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, _lib.strerror(st)
    torch.cuda.synchronize()
    want = oracle.ozaki_matmul(to_np(A), to_np(B), 3, "int8")
    assert_bitwise_equal(to_np(C), want, "ozk_matmul")
    phases = [evs[i].elapsed_time(evs[i + 1]) for i in range(3)]
    assert all(t >= 0 for t in phases) and sum(phases) > 0


def _int_valued_inputs(shape_a, shape_b, seed):
    """A and B holding integers in [-32, 32], every row of A and column of B
    reaching 32, times 2^e per row of A / column of B.  Their level-0 slices
    are the integers themselves (fp16 or int8, scaled by powers of two), the
    residuals are 0, and every dot is an integer below 2^24: the fp16 path is
    then exact and equals the oracle bit for bit, like the int8 path."""
    g = torch.Generator().manual_seed(seed)
    A = torch.randint(-32, 33, shape_a, generator=g).double()
    B = torch.randint(-32, 33, shape_b, generator=g).double()
    A[..., 0] = 32.0
    B[..., 0, :] = -32.0
    A = A * torch.pow(2.0, torch.randint(-8, 9, (*shape_a[:-1], 1), generator=g).double())
    B = B * torch.pow(2.0, torch.randint(-8, 9, (*shape_b[:-2], 1, shape_b[-1]),
                                         generator=g).double())
    return A, B


@pytest.mark.parametrize("gemm", ["", "kstep", "ring"])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("sa,sb", [((2, 128, 256), (256, 96)), ((1, 64, 8192), (8192, 96))])
def test_ozaki_matmul_graph_capture(oracle, gpu, sdt, sa, sb, gemm, force):
    """ozaki_matmul captured in a HIP graph (torch.cuda.graph): every replay,
    with eager work and synchronisations between replays and the inputs
    changed in place, equals the oracle bit for bit (inputs for which the fp16
    path is exact too) and the eager call.  At K = 8192 the B split is the
    cooperative kernel, whose exchange words a fill kernel clears on every
    replay, and the planner's cross-GEMM is the ring kernel with 4 split-K
    ranges per tile, whose arrival counters a fill kernel clears too; at
    K = 256 it is the K-step kernel (test_api_cpu checks both plans).  Each
    kernel is also forced on both shapes."""
    import ozaki_triton_amd as ozk
    if gemm:
        force(gemm=gemm)
    A, B = _int_valued_inputs(sa, sb, seed=53)
    Ad, Bd = A.to(gpu), B.to(gpu)
    L = 3
    ozk.ozaki_matmul(Ad, Bd, L, sdt)          # warm up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            C_graph = ozk.ozaki_matmul(Ad, Bd, L, sdt)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gen = torch.Generator().manual_seed(7)
    for rep in range(4):
        An, Bn = A * 2.0 ** rep, torch.roll(B, rep, -2)
        if rep:
            Ad.copy_(An.to(gpu))
            Bd.copy_(Bn.to(gpu))
        junk = torch.randn(1000, 1000, generator=gen).to(gpu) @ torch.randn(1000, 1000).to(gpu)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = oracle.ozaki_matmul(to_np(An), to_np(Bn), L, NAME_OF[sdt])
        assert_bitwise_equal(to_np(C_graph), want, f"replay {rep} vs oracle")
        eager = ozk.ozaki_matmul(Ad, Bd, L, sdt)
        torch.cuda.synchronize()
        assert_bitwise_equal(to_np(C_graph), to_np(eager), f"replay {rep} vs eager")
        del junk


# --------------------------------------------------------------------------- #
# more than 4 slices: split_matrix and cross_gemm take up to 8 (the reference
# caps only ozaki_matmul, ozaki_triton.py:563); the cross-GEMM runs over i-row
# ranges that continue the fp64 sum from C
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("kernel", ["", "pair"])
@pytest.mark.parametrize("L", [5, 6, 7, 8])
@pytest.mark.parametrize("M,N,K", [(64, 64, 128), (100, 72, 1040)])
def test_cross_gemm_more_splits_int8_bitexact(oracle, gpu, L, M, N, K, kernel, force):
    """5 to 8 slices, the planner's kernel (one launch for 5) and the
    pair-split kernel forced (launched per i-row range, the fp64 sum carried
    in C)."""
    import ozaki_triton_amd as ozk
    if kernel:
        force(gemm=kernel)
    g = torch.Generator().manual_seed(L * 100 + M)
    As, BsT, sa, sb = _random_slices(g, 2, L, M, N, K, torch.int8)
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L,
                       torch.float64)
    torch.cuda.synchronize()
    for b in range(2):
        want = oracle.cross_gemm(to_np(As[b]), to_np(BsT[b]), to_np(sa[b]), to_np(sb[b]),
                                 "float64")
        assert_bitwise_equal(to_np(C)[b], want, f"L{L} {M}x{N}x{K} b{b}")


@pytest.mark.parametrize("kernel", ["", "pair"])
@pytest.mark.parametrize("sdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("L", [5, 6])
def test_cross_gemm_more_splits_float_bitexact(oracle, gpu, sdt, L, kernel, force):
    """5 and 6 float slices on integer-valued slices, the planner's kernel and
    the pair-split kernel forced: bit-exact against the oracle."""
    import ozaki_triton_amd as ozk
    if kernel:
        force(gemm=kernel)
    g = torch.Generator().manual_seed(L + 17)
    M, N, K = 100, 72, 1040
    As, BsT, sa, sb = int_valued_slices(g, 1, L, M, N, K, sdt)
    C = ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), L,
                       torch.float64)
    torch.cuda.synchronize()
    want = oracle.cross_gemm(to_np(As[0]), to_np(BsT[0]), to_np(sa[0]), to_np(sb[0]), "float64")
    assert_bitwise_equal(to_np(C)[0], want, f"L{L} {sdt}")


def test_six_splits_end_to_end(oracle, gpu):
    """fp64 -> int8 with 6 slices composed from split_matrix and cross_gemm
    (as ozaki_matmul would do it): bit-exact against the oracle, and at least
    as accurate as 4 slices (the fp32 residual buffer bounds the gain)."""
    import ozaki_triton_amd as ozk
    A, B = c3_like((96, 1024), (1024, 80), seed=61)
    Ad, Bd = A.to(gpu), B.to(gpu)
    K = 1024
    alpha = ozk.compute_split_bits(K, torch.int8, torch.int32)
    rel = {}
    for L in (4, 6):
        a_sl, a_sc = ozk.split_matrix(Ad.unsqueeze(0), L, alpha, torch.int8)
        bt_sl, b_sc = ozk.split_matrix(Bd.t().unsqueeze(0), L, alpha, torch.int8)
        C = ozk.cross_gemm(a_sl, bt_sl.transpose(-1, -2), a_sc, b_sc, L, torch.float64)[0]
        torch.cuda.synchronize()
        want = oracle.ozaki_matmul(to_np(A), to_np(B), L, "int8")
        assert_bitwise_equal(to_np(C), want, f"L{L}")
        ref = A @ B
        rel[L] = float((C.cpu() - ref).norm() / ref.norm())
    assert rel[6] <= rel[4]


def test_more_splits_unsupported_combination_raises(gpu):
    """6 to 8 slices need an fp64 C (the pair-split kernel carries its partial
    sums there); 5 fp32 slices have no kernel but the pair-split one."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(3)
    As, BsT, sa, sb = _random_slices(g, 1, 6, 64, 64, 128, torch.int8)
    with pytest.raises(ozk._lib.OzakiLibError):
        ozk.cross_gemm(As.to(gpu), BsT.to(gpu).transpose(-1, -2), sa.to(gpu), sb.to(gpu), 6,
                       torch.float32)
    As32, Bs32 = As[:, :5].float(), BsT[:, :5].float()
    with pytest.raises(ozk._lib.OzakiLibError):
        ozk.cross_gemm(As32.to(gpu), Bs32.to(gpu).transpose(-1, -2), sa[:, :5].to(gpu),
                       sb[:, :5].to(gpu), 5, torch.float32)


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("L,batch,M,N", [
    (1, 1, 4096, 4096),    # 128 x 256 tiles kept (512 of them)
    (1, 1, 2048, 4096),    # shrunk to 128 x 128
    (1, 2, 2048, 1024),    # shrunk to 64 x 128 (the reference's published (2, 2048, 1024, 256))
    (1, 1, 2048, 2048),    # 64 x 128
    (2, 1, 2048, 2048),    # L = 2: the ring kernel's 128 x 128 tiles (256 of them)
    (2, 1, 1024, 1024),    # L = 2: 64 x 64 (LDS-DMA kernel)
    (3, 1, 2048, 2048),    # L = 3: the wide kernel's 64 x 128 tiles (512 of them)
    (3, 1, 1280, 1280),    # L = 3: wide (200 tiles, one round against the ring's two)
    (3, 1, 1536, 1536),    # L = 3: ring (288 wide tiles take two rounds, 576 ring tiles three)
    (3, 2, 1024, 1000),    # L = 3: wide, batch 2, N cutting a tile
])
def test_tile_table_shrink_steps(oracle, gpu, sdt, L, batch, M, N):
    """The tile table (plan_gemm) shrinks 128 x 256 tiles for grids under 512
    workgroups, N first while it is the larger side: every (rows, columns)
    step it can stop at has a kernel.  (An earlier order stopped at 128 x 64,
    which no kernel took: the launch failed.)  At num_splits 3 it takes the
    wide kernel where its rounds of 256 tiles finish sooner than the ring
    kernel's.  Sampled blocks against the oracle, K = 256."""
    import ozaki_triton_amd as ozk
    K = 256
    A, B = c3_like((batch, M, K), (batch, K, N), seed=M + N + L, dtype=torch.float32)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), L, sdt)
    torch.cuda.synchronize()
    C_np, A_np, B_np = to_np(C), to_np(A), to_np(B)
    for b in range(batch):
        rows, cols = sample_indices(M, 40, b + 1), sample_indices(N, 40, b + 2)
        check_block_vs_oracle(oracle, ozk, C_np[b], A_np[b], B_np[b], rows, cols, L, sdt,
                              torch.float32, f"L{L} {sdt} b{b} {M}x{N}")


@pytest.mark.parametrize("L", [2, 4])
@pytest.mark.parametrize("xdt,sdt", COMBOS)
@pytest.mark.parametrize("batch,N,K", [(1, 2048, 4096), (2, 1024, 6000), (1, 1024, 4096)])
def test_split_columns_default_plan(oracle, gpu, xdt, sdt, batch, N, K, L):
    """B's columns through the transposed view with the planner's own choice
    (no kernel forced): fp64 columns from 32 KB into 1 or 2 int8 slices, 2048
    or more of them, take the cooperative kernel; more slices, fewer columns,
    fp32 columns or fp16 slices the strip kernel (test_api_cpu checks the
    plans)."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(batch * N + K)
    B = torch.randn(batch, K, N, generator=g, dtype=torch.float64)
    B = B * torch.pow(2.0, torch.randint(-8, 9, (batch, 1, N), generator=g).double())
    _check_split(oracle, ozk, B.to(xdt).to(gpu).transpose(-1, -2), L, sdt,
                 f"default {xdt} {sdt} b{batch} {N}x{K} L{L}")


@pytest.mark.parametrize("kernel", ["", "dma", "ring", "pair", "staged", "wide", "wide4",
                                    "solo5", "kstep", "kstep2"])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("K", [1, 2, 3, 5, 7, 9, 255, 257, 1003])
def test_packed_rows_last_piece(oracle, gpu, kernel, sdt, K, force):
    """Slice rows that are not whole 16-byte pieces (K * element size) go
    through the pack kernel's zero-padded copy.  The LDS-DMA kernels load
    16-byte pieces; the last piece of the operand's last row (the last slice
    of its last row) crosses the end of the buffer unless the buffer's extent
    runs to that row's 16-byte boundary, and a crossing piece comes back
    zeroed.  Full outputs against the oracle, every kernel forced in turn:
    int8 bit-exact, fp16 within the fp32 accumulation bound."""
    import ozaki_triton_amd as ozk
    if kernel:
        force(gemm=kernel)
    L = (3 if kernel == "wide" else 4 if kernel in ("ring", "pair", "wide4", "kstep", "kstep2")
         else 5 if kernel == "solo5" else 2)
    A, B = c3_like((1, 33, K), (1, K, 20), seed=K + 100)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), L, sdt, max_splits=L)
    torch.cuda.synchronize()
    rows, cols = np.arange(33), np.arange(20)
    check_block_vs_oracle(oracle, ozk, to_np(C)[0], to_np(A)[0], to_np(B)[0], rows, cols, L, sdt,
                          torch.float64, f"K{K} {kernel or 'default'} {sdt}")


@pytest.mark.parametrize("xdt", [torch.float64, torch.float32, torch.float16])
@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
def test_infinite_entries(oracle, gpu, xdt, sdt):
    """Rows of A and columns of B holding +-inf: their level-0 maximum is inf,
    and the reference's scale exp2(ceil(log2(inf)) - alpha) is inf, so exactly
    those rows and columns of C are non-finite, as in the oracle; every other
    entry is computed from finite slices (int8: bit-exact with the oracle)."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(41)
    A = torch.randn(1, 40, 96, generator=g, dtype=torch.float64).to(xdt)
    B = torch.randn(1, 96, 30, generator=g, dtype=torch.float64).to(xdt)
    A[0, 3, 7] = float("inf")
    A[0, 10, 0] = float("-inf")
    B[0, 4, 2] = float("inf")
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), 3, sdt)
    torch.cuda.synchronize()
    got = to_np(C)[0].astype(np.float64)
    want = oracle.ozaki_matmul(to_np(A), to_np(B), 3, NAME_OF[sdt])[0].astype(np.float64)
    bad = ~np.isfinite(got)
    expect = np.zeros_like(bad)
    expect[[3, 10], :] = True
    expect[:, 2] = True
    assert np.array_equal(bad, expect)
    assert np.array_equal(~np.isfinite(want), expect)
    if sdt == torch.int8:
        assert_bitwise_equal(got[~bad], want[~bad], f"finite entries {xdt}")


def test_concurrent_calls_from_threads(gpu):
    """Four host threads call ozaki_matmul at once, each on its own stream
    (default priority) with its own inputs, dtype and slice count; ctypes
    releases the GIL during the C calls.  Every result equals the same call
    made alone."""
    import threading
    import ozaki_triton_amd as ozk
    cfgs = [((2, 200, 300), (300, 150), torch.float64, torch.int8, 4),
            ((1, 256, 4096), (4096, 192), torch.float32, torch.float16, 2),
            ((3, 96, 1000), (1000, 64), torch.float64, torch.bfloat16, 3),
            ((1, 130, 8192), (8192, 70), torch.float64, torch.int8, 3)]
    inputs = []
    for n, (sa, sb, xdt, sdt, L) in enumerate(cfgs):
        A, B = c3_like(sa, sb, seed=300 + n, dtype=xdt)
        inputs.append((A.to(gpu), B.to(gpu), sdt, L))
    alone = [ozk.ozaki_matmul(A, B, L, sdt) for A, B, sdt, L in inputs]
    torch.cuda.synchronize()
    got = [[None] * 8 for _ in inputs]
    errors = []

    def worker(i):
        try:
            A, B, sdt, L = inputs[i]
            s = torch.cuda.Stream(gpu)
            s.wait_stream(torch.cuda.default_stream(gpu))
            with torch.cuda.stream(s):
                for r in range(8):
                    got[i][r] = ozk.ozaki_matmul(A, B, L, sdt)
            s.synchronize()
        except Exception as e:   # reported below, on the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(inputs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i, ref in enumerate(alone):
        for r in range(8):
            assert torch.equal(got[i][r], ref), (i, r)


def test_c_abi_example_program(gpu):
    """The C ABI from plain C++, with no Python or torch in the caller:
    tests/c_abi_example.cpp (built by build()) runs one FP64 -> INT8 product
    through ozk_matmul and through ozk_split x2 + ozk_cross_gemm, checks that
    both agree bit for bit and match a CPU fp64 product, and exits 0."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi_example")
    if not os.path.exists(exe):
        pytest.fail("tests/c_abi_example is not built: run __graft_entry__.build()")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c_abi_example ok" in r.stdout, r.stdout


@pytest.mark.parametrize("xdt,off", [(torch.float64, 1), (torch.float32, 1), (torch.float32, 2)])
@pytest.mark.parametrize("K", [8192, 40000])
def test_unaligned_operands(oracle, gpu, xdt, off, K):
    """Operands whose data pointer is not 16-byte aligned (a view starting
    `off` elements into its storage): the workspace query sees no pointers
    and sizes for aligned ones, so the split plans for these pointers must
    need no more (they take the generic kernel, or the transpose path when
    the aligned plan does too).  C bit-exact against the oracle, for A's rows
    and for B's columns at lengths whose aligned plans take the cooperative
    kernels."""
    import ozaki_triton_amd as ozk
    M, N, L = 48, 40, 3
    A, B = c3_like((M, K), (K, N), seed=K + off, dtype=xdt)
    Ad = torch.empty(off + M * K, dtype=xdt, device=gpu)[off:].view(M, K)
    Bd = torch.empty(off + K * N, dtype=xdt, device=gpu)[off:].view(K, N)
    Ad.copy_(A.to(gpu))
    Bd.copy_(B.to(gpu))
    assert Ad.data_ptr() % 16 != 0 and Bd.data_ptr() % 16 != 0
    C = ozk.ozaki_matmul(Ad, Bd, L, torch.int8)
    torch.cuda.synchronize()
    want = oracle.ozaki_matmul(to_np(A), to_np(B), L, "int8")
    assert_bitwise_equal(to_np(C), want, f"unaligned {xdt} +{off} K{K}")


def test_repeated_call_fast_path(oracle, gpu):
    """A repeated ozaki_matmul with the same shapes, strides and dtypes skips the
    Python checks (ozaki._CALLS): the second call, on other data, is still
    bit-exact; other strides (a transposed B) get their own entry; an operand
    that needs a copy (neither of its last two dims contiguous) is not cached;
    the phase events work on a cached call."""
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd import ozaki as oz
    from tests.helpers import c3_like
    oz._CALLS.clear()
    A1, B1 = c3_like((2, 96, 1040), (1040, 72), 31)
    A2, B2 = c3_like((2, 96, 1040), (1040, 72), 32)
    for A, B in ((A1, B1), (A2, B2)):
        C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), 3, torch.int8)
        assert_bitwise_equal(to_np(C), oracle.ozaki_matmul(to_np(A), to_np(B), 3, "int8"), "cached")
    assert len(oz._CALLS) == 1
    Bt = B2.T.contiguous().to(gpu).T          # column-major B: other strides
    C = ozk.ozaki_matmul(A2.to(gpu), Bt, 3, torch.int8)
    assert_bitwise_equal(to_np(C), oracle.ozaki_matmul(to_np(A2), to_np(B2), 3, "int8"), "B^T")
    assert len(oz._CALLS) == 2
    As = A2.to(gpu).repeat_interleave(2, dim=-1)[..., ::2]   # strided in both last dims
    C = ozk.ozaki_matmul(As, B2.to(gpu), 3, torch.int8)
    assert_bitwise_equal(to_np(C), oracle.ozaki_matmul(to_np(A2), to_np(B2), 3, "int8"), "copy")
    assert len(oz._CALLS) == 2
    from ozaki_triton_amd.ozaki import _ozaki_matmul_impl
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in evs:   # torch creates an event at its first record
        e.record()
    Ad, Bd = A1.to(gpu), B1.to(gpu)
    C = _ozaki_matmul_impl(Ad, Bd, 3, torch.int8, False, evs)
    torch.cuda.synchronize()
    assert evs[0].elapsed_time(evs[3]) > 0
    assert_bitwise_equal(to_np(C), oracle.ozaki_matmul(to_np(A1), to_np(B1), 3, "int8"), "events")


def test_bench_timing_events_partial(oracle, gpu):
    """bench.py's timed steps pass the library two of its four phase events
    (None for the others), created by bench.TimingEvent without the
    system-scope fence: the call records only those, on the launch stream,
    and stays bit-exact, on the cached and the uncached path."""
    from ozaki_triton_amd import ozaki as oz
    from ozaki_triton_amd.ozaki import _ozaki_matmul_impl
    from tests.helpers import c3_like
    import bench
    mk = bench.TimingEvent.factory()
    assert mk is bench.TimingEvent, "HIP runtime of torch not found"
    A, B = c3_like((1, 200, 3000), (3000, 136), 41)
    Ad, Bd = A.to(gpu), B.to(gpu)
    want = oracle.ozaki_matmul(to_np(A), to_np(B), 4, "int8")
    for cached in (False, True):
        if not cached:
            oz._CALLS.clear()
        evs = [mk() for _ in range(4)]
        for e in evs:
            e.record()
        torch.cuda.synchronize()
        for k, part in enumerate(([evs[0], None, evs[2], None], [None, None, evs[2], evs[3]])):
            C = _ozaki_matmul_impl(Ad, Bd, 4, torch.int8, False, part)
            torch.cuda.synchronize()
            assert_bitwise_equal(to_np(C), want, f"partial events cached={cached}")
            # the splits, then the cross-GEMM: both take time
            assert (evs[0].elapsed_time(evs[2]) if k == 0 else evs[2].elapsed_time(evs[3])) > 0


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.int8])
def test_ozaki_matmul_narrow_inputs_long_k(oracle, gpu, xdt):
    """Narrow inputs over a K that takes the long-row paths after the exact
    fp32 conversion: A's rows through the shared row kernel (K > 16384) and
    B's columns through the cooperative column kernel or the transpose, end
    to end with int8 slices, bit-exact against the oracle; broadcast batch."""
    import ozaki_triton_amd as ozk
    g = torch.Generator().manual_seed(71 + ALL_INPUTS.index(xdt))
    K = 20000
    A = _random_input(g, (2, 24, K), xdt)
    B = _random_input(g, (K, 40), xdt)
    print(f"narrow long K {xdt} A{tuple(A.shape)} B{tuple(B.shape)}", flush=True)
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), 3, torch.int8)
    torch.cuda.synchronize()
    assert C.dtype == xdt and C.shape == (2, 24, 40)
    want = oracle.ozaki_matmul(to_np(A), to_np(B), 3, "int8")
    assert_bitwise_equal(to_np(C), want, f"narrow long K {xdt}")
    ozk.device_status()                     # raises if a cooperative wait gave up
