"""Host-side tests (no GPU): the C ABI loads and exports every declared
symbol, its argument checks return the documented codes without touching a
device, and the Python API keeps the reference's assertions and messages."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols(header):
    with open(os.path.join(ROOT, "include", header)) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(ozk_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from ozaki_triton_amd import _lib
    L = _lib.load()
    headers = sorted(f for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h"))
    assert headers == ["ozaki_amd.h", "ozaki_amd_debug.h"]
    assert _declared_symbols("ozaki_amd.h") == sorted(_lib.EXPORTED)
    assert _declared_symbols("ozaki_amd_debug.h") == sorted(_lib.EXPORTED_DEBUG)
    for name in _lib.EXPORTED + _lib.EXPORTED_DEBUG:
        assert hasattr(L, name), name
    assert L.ozk_version() >= 300


def test_strerror_names_every_code():
    from ozaki_triton_amd import _lib
    for code in range(0, -11, -1):
        assert _lib.strerror(code) != "unknown status"
    assert _lib.strerror(-99) == "unknown status"


def test_compute_split_bits_abi_matches_python_formula():
    import math
    from ozaki_triton_amd import _lib
    L = _lib.load()
    out = ctypes.c_int(0)
    for acc, acc_bits in ((_lib.OZK_I32, 31), (_lib.OZK_F32, 23)):
        for sd, sbits in ((_lib.OZK_I8, 7), (_lib.OZK_F16, 10), (_lib.OZK_BF16, 7),
                          (_lib.OZK_F32, 23)):
            for n in [1, 2, 3, 100, 255, 256, 4096, 8192, 65536, 1 << 20, (1 << 21) + 1,
                      1 << 28, 1 << 30]:
                st = L.ozk_compute_split_bits(n, sd, acc, ctypes.byref(out))
                want = min(int((acc_bits - math.log2(n)) / 2), sbits)
                assert out.value == want
                assert st == (_lib.OZK_OK if want >= 1 else _lib.OZK_ERR_ALPHA)
    assert L.ozk_compute_split_bits(8, _lib.OZK_I8, _lib.OZK_F64, ctypes.byref(out)) == \
        _lib.OZK_ERR_ACCUM
    assert L.ozk_compute_split_bits(0, _lib.OZK_I8, _lib.OZK_I32, ctypes.byref(out)) == \
        _lib.OZK_ERR_SHAPE


def test_split_abi_rejects_bad_arguments_on_host():
    from ozaki_triton_amd import _lib
    L = _lib.load()
    s3 = _lib.i64arr([6, 3, 1])
    s4 = _lib.i64arr([12, 6, 3, 1])
    p = ctypes.c_void_p(0x1000)
    null = ctypes.c_void_p(0)

    def call(**kw):
        a = dict(X=p, xd=_lib.OZK_F64, B=1, R=2, K=3, L=2, alpha=7, sd=_lib.OZK_I8, S=p, C=p,
                 ws=null, wsb=0)
        a.update(kw)
        return L.ozk_split(a["X"], a["xd"], a["B"], a["R"], a["K"], s3, a["L"], a["alpha"],
                           a["sd"], a["S"], s4, a["C"], s3, a["ws"], a["wsb"], null)

    assert call(xd=_lib.OZK_I32) == _lib.OZK_ERR_DTYPE     # not an input dtype
    assert call(sd=_lib.OZK_F64) == _lib.OZK_ERR_DTYPE     # not a slice dtype
    assert call(L=9) == _lib.OZK_ERR_SPLITS                # up to 8 slices
    assert call(L=-1) == _lib.OZK_ERR_SPLITS
    assert call(K=-1) == _lib.OZK_ERR_SHAPE
    assert call(alpha=0) == _lib.OZK_ERR_ALPHA
    assert call(X=null) == _lib.OZK_ERR_NULL
    # nothing to do: returns OK without any device call
    assert call(B=0) == _lib.OZK_OK
    assert call(L=0) == _lib.OZK_OK
    # the generic (strided) path recomputes each level's residual from the
    # input: no workspace
    nb = ctypes.c_size_t(123)
    xs_bad = _lib.i64arr([6, 3, 2])
    assert L.ozk_split_workspace_bytes(_lib.OZK_F64, 1, 2, 3, xs_bad, 2, _lib.OZK_I8, s4,
                                       ctypes.byref(nb)) == 0
    assert nb.value == 0
    # the cooperative column path needs its exchange words: refused without
    # them, or with a workspace that is not 16-byte aligned (before anything
    # is enqueued)
    K, N = 8192, 16
    xs_c = _lib.i64arr([K * N, 1, N])
    sl_c = _lib.i64arr([2 * N * K, N * K, K, 1])
    sc_c = _lib.i64arr([2 * N, N, 1])
    assert L.ozk_split_workspace_bytes(_lib.OZK_F64, 1, N, K, xs_c, 2, _lib.OZK_I8, sl_c,
                                       ctypes.byref(nb)) == 0
    assert nb.value == 1 * 2 * 8 * 16 * 8 + 8
    assert L.ozk_split(p, _lib.OZK_F64, 1, N, K, xs_c, 2, 7, _lib.OZK_I8, p, sl_c, p, sc_c, null,
                       0, null) == _lib.OZK_ERR_WORKSPACE
    assert L.ozk_split(p, _lib.OZK_F64, 1, N, K, xs_c, 2, 7, _lib.OZK_I8, p, sl_c, p, sc_c,
                       ctypes.c_void_p(0x2008), 1 << 20, null) == _lib.OZK_ERR_WORKSPACE


def test_split_workspace_narrow_inputs():
    """fp16 / bf16 / int8 inputs are split from an exact fp32 copy in the
    workspace (ozaki_triton.py:188 loads them into the fp32 RES); an odd K
    takes the generic kernel, which needs nothing behind the copy."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    nb = ctypes.c_size_t(0)
    M, K = 96, 512
    sl = _lib.i64arr([3 * M * K, M * K, K, 1])
    for xd in (_lib.OZK_F16, _lib.OZK_BF16, _lib.OZK_I8):
        for sd in (_lib.OZK_I8, _lib.OZK_F16, _lib.OZK_BF16, _lib.OZK_F32):
            assert L.ozk_split_workspace_bytes(xd, 1, M, K, _lib.i64arr([M * K, K, 1]), 3, sd, sl,
                                               ctypes.byref(nb)) == 0
            assert nb.value == M * K * 4
    K2 = 510
    sl2 = _lib.i64arr([3 * M * K2, M * K2, K2, 1])
    assert L.ozk_split_workspace_bytes(_lib.OZK_F16, 1, M, K2, _lib.i64arr([M * K2, K2, 1]), 3,
                                       _lib.OZK_I8, sl2, ctypes.byref(nb)) == 0
    assert nb.value == M * K2 * 4
    # fp32 slices are 4 bytes: the resident paths still need no workspace
    sl4 = _lib.i64arr([2 * M * K, M * K, K, 1])
    assert L.ozk_split_workspace_bytes(_lib.OZK_F64, 1, M, K, _lib.i64arr([M * K, K, 1]), 2,
                                       _lib.OZK_F32, sl4, ctypes.byref(nb)) == 0
    assert nb.value == 0


def test_split_workspace_per_path():
    from ozaki_triton_amd import _lib
    L = _lib.load()
    nb = ctypes.c_size_t(123)
    K, M, N = 8192, 8192, 8192
    sl = _lib.i64arr([4 * M * K, M * K, K, 1])
    # A rows (K-contiguous): row-resident, no workspace
    assert L.ozk_split_workspace_bytes(_lib.OZK_F64, 1, M, K, _lib.i64arr([M * K, K, 1]), 4,
                                       _lib.OZK_I8, sl, ctypes.byref(nb)) == 0
    assert nb.value == 0
    # B^T view (rows contiguous, 64 KB columns): column groups of 16 fp64
    # columns cut into K chunks of 1024 rows exchange one 8-byte maximum per
    # column, level and chunk: 512 groups x 4 levels x 8 chunks x 16 columns x 8 bytes,
    # plus the launch's status word
    assert L.ozk_split_workspace_bytes(_lib.OZK_F64, 1, N, K, _lib.i64arr([K * N, 1, N]), 4,
                                       _lib.OZK_I8, sl, ctypes.byref(nb)) == 0
    assert nb.value == 512 * 4 * 8 * 16 * 8 + 8
    # short columns (under 64 KB) take the strip kernel: no workspace
    Ks = 512
    sls = _lib.i64arr([2 * N * Ks, N * Ks, Ks, 1])
    assert L.ozk_split_workspace_bytes(_lib.OZK_F32, 1, N, Ks, _lib.i64arr([Ks * N, 1, N]), 2,
                                       _lib.OZK_F16, sls, ctypes.byref(nb)) == 0
    assert nb.value == 0
    # a column longer than the cooperative column kernel's 128-byte groups
    # take is transposed into the workspace first (config 5: fp32, K = 65536);
    # its rows, longer than 16384, then go to the row kernel shared by 4
    # workgroups per row, whose exchange words follow the transposed copy:
    # 1024 rows x 3 levels x 4 chunks x 8 bytes, and a status word
    K5, N5 = 65536, 1024
    sl5 = _lib.i64arr([3 * N5 * K5, N5 * K5, K5, 1])
    assert L.ozk_split_workspace_bytes(_lib.OZK_F32, 1, N5, K5, _lib.i64arr([K5 * N5, 1, N5]),
                                       3, _lib.OZK_I8, sl5, ctypes.byref(nb)) == 0
    assert nb.value == N5 * K5 * 4 + N5 * 3 * 4 * 8 + 8
    # and A's rows of config 5 (K-contiguous) need only the exchange words
    assert L.ozk_split_workspace_bytes(_lib.OZK_F32, 1, N5, K5, _lib.i64arr([K5 * N5, K5, 1]),
                                       3, _lib.OZK_I8, sl5, ctypes.byref(nb)) == 0
    assert nb.value == N5 * 3 * 4 * 8 + 8


def test_cross_gemm_abi_checks_and_workspace():
    from ozaki_triton_amd import _lib
    L = _lib.load()
    nb = ctypes.c_size_t(0)
    p = ctypes.c_void_p(0x1000)
    null = ctypes.c_void_p(0)
    M, N, K, Ls = 64, 48, 256, 3
    a = _lib.i64arr([Ls * M * K, M * K, K, 1])
    b_kcontig = _lib.i64arr([Ls * N * K, N * K, 1, K])
    b_ncontig = _lib.i64arr([Ls * N * K, N * K, N, 1])
    assert L.ozk_cross_gemm_workspace_bytes(1, M, N, K, Ls, _lib.OZK_I8, p, a, p, b_kcontig,
                                            ctypes.byref(nb)) == 0
    assert nb.value == 0
    assert L.ozk_cross_gemm_workspace_bytes(1, M, N, K, Ls, _lib.OZK_I8, p, a, p, b_ncontig,
                                            ctypes.byref(nb)) == 0
    assert nb.value == Ls * N * K
    s3 = _lib.i64arr([M * N, N, 1])
    sc = _lib.i64arr([Ls * M, M, 1])

    def call(**kw):
        d = dict(L=Ls, sd=_lib.OZK_I8, od=_lib.OZK_F64, B=1, K=K, C=p, b=b_kcontig, ws=null,
                 wsb=0)
        d.update(kw)
        return L.ozk_cross_gemm(p, a, p, d["b"], p, sc, p, sc, d["B"], M, N, d["K"], d["L"],
                                d["sd"], d["C"], d["od"], s3, d["ws"], d["wsb"], null)

    assert call(sd=_lib.OZK_F64) == _lib.OZK_ERR_DTYPE
    assert call(od=_lib.OZK_I32) == _lib.OZK_ERR_DTYPE
    assert call(L=9) == _lib.OZK_ERR_SPLITS
    # more than 4 slices: int8 / fp16 / bf16 slices only, and beyond 5 an fp64 C
    assert call(L=6, od=_lib.OZK_F32) == _lib.OZK_ERR_SPLITS
    assert call(L=5, sd=_lib.OZK_F32) == _lib.OZK_ERR_SPLITS
    assert call(L=5, od=_lib.OZK_F32, B=0) == _lib.OZK_OK
    assert call(K=-3) == _lib.OZK_ERR_SHAPE
    assert call(C=null) == _lib.OZK_ERR_NULL
    assert call(b=b_ncontig) == _lib.OZK_ERR_WORKSPACE
    assert call(b=b_ncontig, ws=ctypes.c_void_p(0x2004), wsb=1 << 20) == _lib.OZK_ERR_WORKSPACE
    assert call(B=0) == _lib.OZK_OK


def test_splitk_workspace():
    """Grids under half the CUs cut each tile's K into ranges (split-K, planned
    for 256 CUs in the queries).  The workspace queries add the ranges'
    accumulators (tiles x ranges x 8 waves x registers x 64 lanes x 4 bytes)
    and one arrival counter per tile, plus 256 bytes of alignment slack;
    forcing one range (the test hook) takes them away."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    nb = ctypes.c_size_t(0)
    p = ctypes.c_void_p(0x1000)
    M, N, K, Ls = 1024, 1024, 65536, 3
    a = _lib.i64arr([Ls * M * K, M * K, K, 1])
    b = _lib.i64arr([Ls * N * K, N * K, 1, K])
    # config 5's wide kernel, L = 3: 128 tiles of 64 x 128, 2 ranges of 256
    # stages, 9 pairs x 16 registers per wave; 128 counters (512 bytes)
    splitk = 128 * 2 * 8 * 144 * 64 * 4 + 512 + 256
    assert L.ozk_cross_gemm_workspace_bytes(1, M, N, K, Ls, _lib.OZK_I8, p, a, p, b,
                                            ctypes.byref(nb)) == 0
    assert nb.value == splitk
    a3, b3 = _lib.i64arr([M * K, K, 1]), _lib.i64arr([K * N, N, 1])
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, M, N, K, a3, b3, Ls, _lib.OZK_I8,
                                        ctypes.byref(nb)) == 0
    with_splitk = nb.value
    try:
        assert L.ozk_debug_force_gemm_ksplit(1) == 0
        assert L.ozk_cross_gemm_workspace_bytes(1, M, N, K, Ls, _lib.OZK_I8, p, a, p, b,
                                                ctypes.byref(nb)) == 0
        assert nb.value == 0
        assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, M, N, K, a3, b3, Ls, _lib.OZK_I8,
                                            ctypes.byref(nb)) == 0
        assert with_splitk - nb.value == splitk
    finally:
        L.ozk_debug_force_gemm_ksplit(0)
    assert L.ozk_debug_force_gemm_ksplit(-1) == _lib.OZK_ERR_SPLITS


# --------------------------------------------------------------------------- #
# Python API: the reference's checks and messages (ozaki_triton.py:97,560-563)
# --------------------------------------------------------------------------- #
def test_ozaki_matmul_assertions():
    import ozaki_triton_amd as ozk
    a64 = torch.zeros(4, 8, dtype=torch.float64)
    a32 = torch.zeros(8, 4, dtype=torch.float32)
    with pytest.raises(AssertionError, match="A/B dtype mismatch"):
        ozk.ozaki_matmul(a64, a32)
    with pytest.raises(AssertionError, match="unsupported input dtype"):
        ozk.ozaki_matmul(a64.to(torch.int32), a64.to(torch.int32))
    with pytest.raises(AssertionError, match="unsupported slice dtype"):
        ozk.ozaki_matmul(a64, a64.T, slice_dtype=torch.float64)
    with pytest.raises(AssertionError, match="num_splits must be <= 4, got 5"):
        ozk.ozaki_matmul(a64, a64.T, num_splits=5)
    # the keyword-only max_splits raises the limit up to OZK_MAX_SPLITS (8)
    with pytest.raises(AssertionError, match="num_splits must be <= 5, got 6"):
        ozk.ozaki_matmul(a64, a64.T, num_splits=6, max_splits=5)
    with pytest.raises(ValueError, match="max_splits must be <= 8"):
        ozk.ozaki_matmul(a64, a64.T, num_splits=5, max_splits=9)
    with pytest.raises(AssertionError, match="contraction dim mismatch: A K=8, B K=4"):
        ozk.ozaki_matmul(a64, a64)
    # a 1-D operand fails unpacking A.shape[-2:] before any assert, as in the
    # reference (ozaki_triton.py:569)
    with pytest.raises(ValueError):
        ozk.ozaki_matmul(torch.zeros(4, dtype=torch.float64), a64)


def test_ozaki_matmul_refuses_cpu_tensors():
    import ozaki_triton_amd as ozk
    a = torch.zeros(4, 8, dtype=torch.float64)
    with pytest.raises(RuntimeError, match="no CPU path"):
        ozk.ozaki_matmul(a, a.T, 2, torch.int8)


def test_unsupported_combinations_raise():
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd.ozaki import _require_supported
    # every combination of the reference's tables (ozaki_triton.py:35-48) is taken
    for x in (torch.float64, torch.float32, torch.float16, torch.bfloat16, torch.int8):
        for sl in (torch.float32, torch.float16, torch.bfloat16, torch.int8):
            _require_supported(x, sl)
    # an int32 C (cross_gemm's output_dtype outside the input dtypes) is not
    with pytest.raises(NotImplementedError):
        _require_supported(torch.int32, torch.int8)
    assert ozk.compute_split_bits(8192, torch.int8, torch.int32) == 7


def test_compute_split_bits_errors():
    import ozaki_triton_amd as ozk
    with pytest.raises(AssertionError, match=r"n=1073741824 .* \(alpha=-3\)"):
        ozk.compute_split_bits(1 << 30, torch.float16, torch.float32)
    with pytest.raises(ValueError, match="unsupported dot_accum_dtype"):
        ozk.compute_split_bits(16, torch.float16, torch.float64)
    with pytest.raises(ValueError):
        ozk.compute_split_bits(0, torch.int8, torch.int32)
    with pytest.raises(KeyError):
        ozk.compute_split_bits(16, torch.float64, torch.float32)


def test_canonicalize_batch_broadcasts_like_matmul():
    import ozaki_triton_amd as ozk
    A = torch.zeros(16, 1024, 64, dtype=torch.float64)
    B = torch.zeros(64, 32, dtype=torch.float64)
    A3, B3, bs = ozk._canonicalize_batch(A, B)
    assert tuple(bs) == (16,)
    assert A3.shape == (16, 1024, 64) and B3.shape == (1, 64, 32)   # B split once
    A = torch.zeros(2, 1, 5, 6, dtype=torch.float64)
    B = torch.zeros(3, 6, 7, dtype=torch.float64)
    A3, B3, bs = ozk._canonicalize_batch(A, B)
    assert tuple(bs) == (2, 3)
    assert A3.shape == (6, 5, 6) and B3.shape == (6, 6, 7)
    assert torch.matmul(A, B).shape == (*bs, 5, 7)
    # a transposed operand is read in place (no copy)
    Bt = torch.zeros(32, 64, dtype=torch.float64).T
    _, B3, _ = ozk._canonicalize_batch(torch.zeros(4, 64, dtype=torch.float64), Bt)
    assert B3.data_ptr() == Bt.data_ptr()


def test_matmul_abi_layout_and_errors():
    """ozk_matmul (the whole ozaki_matmul below its Python checks): workspace
    layout = 256-byte aligned [A slices][A scales][B slices][B scales][split
    scratch][pack]; errors come back before anything is enqueued."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    nb = ctypes.c_size_t(0)
    M = N = K = 8192
    a = _lib.i64arr([M * K, K, 1])
    b = _lib.i64arr([K * N, N, 1])
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, M, N, K, a, b, 4, _lib.OZK_I8,
                                        ctypes.byref(nb)) == 0
    # the split of B^T exchanges column maxima through the split scratch:
    # 512 column groups x 4 levels x 8 K chunks x 16 columns x 8 bytes and a
    # status word, the region rounded to 256 bytes
    assert nb.value == 2 * (4 * M * K + 4 * M * 4) + 512 * 4 * 8 * 16 * 8 + 256
    # broadcast B over a batch of 16 (stride 0): B is split once
    Mb, Kb, Nb = 1024, 2048, 1024
    a16 = _lib.i64arr([Mb * Kb, Kb, 1])
    b0 = _lib.i64arr([0, Nb, 1])
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 16, Mb, Nb, Kb, a16, b0, 3, _lib.OZK_F16,
                                        ctypes.byref(nb)) == 0
    assert nb.value == 16 * 3 * Mb * Kb * 2 + 16 * 3 * Mb * 4 + 3 * Nb * Kb * 2 + 3 * Nb * 4
    # errors: alpha < 1, K = 0 (log2(0)), too many splits, bad dtype
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F32, 1, 4, 4, 1 << 30, a, b, 2, _lib.OZK_F16,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_ALPHA
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F32, 1, 4, 4, 0, a, b, 2, _lib.OZK_F16,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_SHAPE
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, 4, 4, 8, a, b, 9, _lib.OZK_F16,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_SPLITS
    # 5 slices: int8 / fp16 / bf16 slices, any input; 6..8: fp64 in and out
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F32, 1, 4, 4, 8, a, b, 5, _lib.OZK_F16,
                                        ctypes.byref(nb)) == _lib.OZK_OK
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F32, 1, 4, 4, 8, a, b, 5, _lib.OZK_F32,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_SPLITS
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F32, 1, 4, 4, 8, a, b, 6, _lib.OZK_F16,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_SPLITS
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, 4, 4, 8, a, b, 6, _lib.OZK_F32,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_SPLITS
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, 4, 4, 8, a, b, 6, _lib.OZK_I8,
                                        ctypes.byref(nb)) == _lib.OZK_OK
    # ... and slices within the 31-bit extents of the kernels that take them
    # (5 x 32768 x 32768 int8 slices of A are 5 GiB), refused before any launch
    big = _lib.i64arr([32768 * 32768, 32768, 1])
    for dt in (_lib.OZK_F64, _lib.OZK_F32):
        assert L.ozk_matmul_workspace_bytes(dt, 1, 32768, 64, 32768, big, b, 5, _lib.OZK_I8,
                                            ctypes.byref(nb)) == _lib.OZK_ERR_SPLITS
        assert L.ozk_matmul_workspace_bytes(dt, 1, 8192, 64, 32768, big, b, 5, _lib.OZK_I8,
                                            ctypes.byref(nb)) == _lib.OZK_OK
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_I32, 1, 4, 4, 8, a, b, 2, _lib.OZK_F16,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_DTYPE
    p = ctypes.c_void_p(0x1000)
    null = ctypes.c_void_p(0)
    c = _lib.i64arr([M * N, N, 1])

    def call(ws, wsb):
        return L.ozk_matmul(p, a, p, b, _lib.OZK_F64, 1, M, N, K, 4, _lib.OZK_I8, p, c, ws, wsb,
                            None, null)
    need = 2 * (4 * M * K + 4 * M * 4)
    assert call(null, 0) == _lib.OZK_ERR_WORKSPACE
    assert call(ctypes.c_void_p(0x10000), need - 1) == _lib.OZK_ERR_WORKSPACE
    assert call(ctypes.c_void_p(0x10010), need) == _lib.OZK_ERR_WORKSPACE   # not 256-aligned
    # nothing to do: OK without a device call
    assert L.ozk_matmul(p, a, p, b, _lib.OZK_F64, 0, M, N, K, 4, _lib.OZK_I8, p, c, null, 0,
                        None, null) == _lib.OZK_OK


def test_operands_on_two_devices_are_refused():
    """The wrappers hand raw pointers to the kernels, so operands on two GPUs
    are refused on the host (checked with stand-ins: this container has no
    GPU)."""
    import types
    from ozaki_triton_amd.ozaki import _require_gpu
    a = types.SimpleNamespace(is_cuda=True, device=torch.device("cuda", 0))
    b = types.SimpleNamespace(is_cuda=True, device=torch.device("cuda", 1))
    _require_gpu(a, a)
    with pytest.raises(RuntimeError, match="one device"):
        _require_gpu(a, b)


# --------------------------------------------------------------------------- #
# Workspace sizing does not depend on pointer alignment
# --------------------------------------------------------------------------- #
def _split_plan(L, X, xd, batch, rows, K, xs, nsp, sd, S, ss):
    from ozaki_triton_amd import _lib
    name = ctypes.c_char_p()
    nb = ctypes.c_size_t(0)
    assert L.ozk_debug_split_kernel(ctypes.c_void_p(X), xd, batch, rows, K, _lib.i64arr(xs), nsp,
                                    sd, ctypes.c_void_p(S), _lib.i64arr(ss), ctypes.byref(name),
                                    ctypes.byref(nb)) == 0
    return name.value.decode(), nb.value


@pytest.mark.parametrize("xd", [0, 1])          # OZK_F64, OZK_F32
@pytest.mark.parametrize("sd", [4, 2])          # OZK_I8, OZK_F16
@pytest.mark.parametrize("K,rows", [(8192, 8192), (4096, 2048), (65536, 1024), (1000, 64),
                                    (40000, 3)])
def test_split_plan_for_unaligned_pointers_fits_the_query(xd, sd, K, rows):
    """The *_workspace_bytes queries see no pointers and size for aligned ones.
    An operand whose data pointer is 8 (or 4) mod 16 -- e.g. torch.empty(1 +
    M * K)[1:].view(M, K) -- must get a plan that needs no more scratch: the
    query must cover it for A's rows and for B's columns (the B^T view)."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    nsp = 3
    ss = [nsp * rows * K, rows * K, K, 1]
    for xs in ([rows * K, K, 1], [K * rows, 1, rows]):      # A rows, B^T view
        nb = ctypes.c_size_t(0)
        assert L.ozk_split_workspace_bytes(xd, 1, rows, K, _lib.i64arr(xs), nsp, sd,
                                           _lib.i64arr(ss), ctypes.byref(nb)) == 0
        name_al, need_al = _split_plan(L, 0x10000, xd, 1, rows, K, xs, nsp, sd, 0x20000, ss)
        assert need_al == nb.value, (name_al, need_al, nb.value)
        for off in (8, 4) if xd == 1 else (8,):
            name, need = _split_plan(L, 0x10000 + off, xd, 1, rows, K, xs, nsp, sd, 0x20000, ss)
            assert need <= nb.value, (xs, off, name, need, nb.value)
        # slices at an odd address: the fast paths need aligned slice rows
        name, need = _split_plan(L, 0x10000, xd, 1, rows, K, xs, nsp, sd, 0x20001, ss)
        assert need <= nb.value and name == "generic", (name, need)


def test_column_split_plan_by_length_and_slices():
    """B's columns (the B^T view) by column length: the cooperative kernel from
    64 KB; fp64 columns of 32 KB into 1 or 2 int8 slices, 2048 or more of
    them, too; otherwise (3 or more slices, fewer columns, fp16 slices, fp32)
    the strip kernel, which then shares a launch with A's rows."""
    from ozaki_triton_amd import _lib
    L = _lib.load()

    def plan(xd, sd, N, K, nsp):
        return _split_plan(L, 0x10000, xd, 1, N, K, [K * N, 1, N], nsp, sd, 0x20000,
                           [nsp * N * K, N * K, K, 1])[0]
    F64, F32, I8, F16 = _lib.OZK_F64, _lib.OZK_F32, _lib.OZK_I8, _lib.OZK_F16
    assert plan(F64, I8, 8192, 8192, 4) == "coop"        # config 3: 64 KB columns
    assert plan(F64, I8, 2048, 4096, 1) == "coop"        # 32 KB, 2048 columns, 1-2 slices
    assert plan(F64, I8, 2048, 4096, 2) == "coop"
    assert plan(F64, I8, 2048, 4096, 3) == "strip"       # 3-4 slices: strip + rows, one launch
    assert plan(F64, I8, 2048, 4096, 4) == "strip"
    assert plan(F64, I8, 1024, 4096, 2) == "strip"       # under 2048 columns
    assert plan(F64, F16, 2048, 4096, 2) == "strip"      # fp16 slices
    assert plan(F32, I8, 2048, 4096, 2) == "strip"       # 16 KB fp32 columns
    assert plan(F32, I8, 2048, 16384, 2) == "coop"       # 64 KB fp32 columns


def test_matmul_workspace_covers_unaligned_operands():
    """ozk_matmul carves the split scratch from the size its query returned;
    with unaligned operands the plans still fit (checked again in ozk_matmul,
    which returns OZK_ERR_WORKSPACE rather than write past the region)."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    for xd in (0, 1):
        M = N = K = 8192
        nb = ctypes.c_size_t(0)
        assert L.ozk_matmul_workspace_bytes(xd, 1, M, N, K, _lib.i64arr([M * K, K, 1]),
                                            _lib.i64arr([K * N, N, 1]), 4, 4,
                                            ctypes.byref(nb)) == 0
        slices = 2 * (4 * M * K + 4 * M * 4)
        scratch = nb.value - slices
        for xs in ([M * K, K, 1], [K * N, 1, N]):
            name, need = _split_plan(L, 0x10008, xd, 1, M, K, xs, 4, 4, 0x100000,
                                     [4 * M * K, M * K, K, 1])
            assert need <= scratch, (name, need, scratch)


# --------------------------------------------------------------------------- #
# Error parity: compute_split_bits runs for every num_splits, 0 included
# --------------------------------------------------------------------------- #
def test_zero_splits_still_checks_alpha_like_the_reference():
    """ozaki_triton.py:580 calls compute_split_bits before splitting, whatever
    num_splits is: K = 0 raises ValueError (log2(0)) and alpha < 1 the alpha
    assertion, before any device work (here: before the CPU-tensor check)."""
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd import _lib
    with pytest.raises(ValueError):
        ozk.ozaki_matmul(torch.zeros(4, 0, dtype=torch.float64),
                         torch.zeros(0, 3, dtype=torch.float64), 0, torch.int8)
    big = torch.zeros(2, 1 << 22, dtype=torch.float32)   # fp16 slices: alpha = int(0.5) = 0
    with pytest.raises(AssertionError, match="alpha="):
        ozk.ozaki_matmul(big, big.T, 0, torch.float16)
    L = _lib.load()
    nb = ctypes.c_size_t(0)
    a = _lib.i64arr([0, 1, 1])
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, 4, 3, 0, a, a, 0, _lib.OZK_I8,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_SHAPE
    assert L.ozk_matmul_workspace_bytes(_lib.OZK_F32, 1, 4, 3, 1 << 30, a, a, 0, _lib.OZK_F16,
                                        ctypes.byref(nb)) == _lib.OZK_ERR_ALPHA


# --------------------------------------------------------------------------- #
# Test hooks and the planner's kernel choice
# --------------------------------------------------------------------------- #
def test_debug_hooks_reject_unknown_names():
    from ozaki_triton_amd import _lib
    L = _lib.load()
    assert L.ozk_debug_force_gemm_kernel(b"fastest") == _lib.OZK_ERR_DTYPE
    assert L.ozk_debug_force_split_kernel(b"fastest") == _lib.OZK_ERR_DTYPE
    for k in (b"staged", b"dma", b"pair", b"ring", b"wide", b"wide4", b"solo", b"solo5", b"",
              None):
        assert L.ozk_debug_force_gemm_kernel(k) == 0
    for k in (b"coop", b"strip", b"transpose", b"generic", b"rows", b"rowscoop", None):
        assert L.ozk_debug_force_split_kernel(k) == 0


def _gemm_kernel(L, batch, M, N, K, nsp, sd, cus, with_ksplit=False):
    name = ctypes.c_char_p()
    ks = ctypes.c_int(0)
    assert L.ozk_debug_gemm_kernel(batch, M, N, K, nsp, sd, cus, ctypes.byref(name),
                                   ctypes.byref(ks)) == 0
    return (name.value.decode(), ks.value) if with_ksplit else name.value.decode()


def test_planner_kernel_choice():
    """num_splits 3: the wide kernel where its rounds of one workgroup per CU
    finish no later (16 x 16 forms: 3 * wide rounds <= 2 * ring rounds; the 32
    x 32 forms of fp32 slices: 12 * wide rounds < 7 * ring rounds), measured
    crossovers at 200 / 288 / 384 / 512 wide tiles on 256 CUs; the rule
    follows the device's compute-unit count (a 32-CU partition)."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    I8 = _lib.OZK_I8
    # wide tiles = (M / 64) * (N / 128)
    assert _gemm_kernel(L, 1, 640, 2560, 4096, 3, I8, 256) == "wide"      # 200 tiles
    assert _gemm_kernel(L, 1, 1024, 2304, 4096, 3, I8, 256) == "wide"     # 288: 2 vs 3 rounds
    assert _gemm_kernel(L, 1, 1024, 3072, 4096, 3, I8, 256) == "wide"     # 384
    assert _gemm_kernel(L, 1, 1024, 2304, 4096, 3, _lib.OZK_F32, 256) == "ring"   # 32 x 32 forms
    assert _gemm_kernel(L, 1, 1024, 3840, 4096, 3, I8, 256) == "wide"     # 480
    assert _gemm_kernel(L, 1, 1024, 4096, 4096, 3, I8, 256) == "wide"     # 512
    assert _gemm_kernel(L, 16, 1024, 1024, 2048, 3, _lib.OZK_F16, 256) == "wide"   # config 4
    # config 5: 128 wide tiles with 2 split-K ranges each, one round, against
    # 256 ring tiles in one round (3 * 1 * 1 <= 2 * 1 * 2)
    assert _gemm_kernel(L, 1, 1024, 1024, 65536, 3, I8, 256) == "wide"
    # 200 wide tiles on 32 CUs: 7 rounds against 13 -> 21 <= 26: wide; 288: 9 vs 18 -> wide
    assert _gemm_kernel(L, 1, 640, 2560, 4096, 3, I8, 32) == "wide"
    assert _gemm_kernel(L, 1, 1024, 2304, 4096, 3, I8, 32) == "wide"
    # other slice counts
    # num_splits 4: the 96 x 64 wide kernel where 1.45 x its rounds are fewer
    # than the ring kernel's (29 * wide4 rounds < 20 * ring rounds)
    assert _gemm_kernel(L, 1, 8192, 8192, 8192, 4, I8, 256) == "wide4"    # config 3: 43 vs 64
    assert _gemm_kernel(L, 1, 4096, 4096, 8192, 4, I8, 256) == "wide4"    # 11 vs 16
    assert _gemm_kernel(L, 1, 2048, 2048, 8192, 4, I8, 256) == "ring"     # 3 vs 4
    assert _gemm_kernel(L, 1, 1024, 1024, 65536, 4, I8, 256) == "ring"    # 1 vs 1
    assert _gemm_kernel(L, 1, 4096, 4096, 4096, 2, _lib.OZK_F16, 256) == "ring"   # config 2
    assert _gemm_kernel(L, 1, 256, 256, 256, 2, _lib.OZK_F16, 256) == "kstep2"    # config 1
    assert _gemm_kernel(L, 1, 2048, 2048, 2048, 1, I8, 256) == "dma"
    # grids whose 64 x 64 tiles leave more than half the CUs idle: the K-step
    # kernel's 32 x 32 tiles when they fit one round (the reference's
    # (1, 128, 2048, 4096) point: 256 of them), else split-K of the ring or
    # wide kernel, S = CUs / tiles, at most 4, at least 16 stages of 128 bytes
    # of K per range
    # (two slices or more: its 8-wave form with two pair groups, "kstep2")
    for nsp in (1, 2, 3, 4):
        for sd in (I8, _lib.OZK_F16):
            want = "kstep" if nsp == 1 else "kstep2"
            assert _gemm_kernel(L, 1, 128, 2048, 4096, nsp, sd, 256, True) == (want, 1)
    assert _gemm_kernel(L, 1, 128, 2048, 4096, 4, _lib.OZK_F32, 256) == "ring"     # fp32 slices
    assert _gemm_kernel(L, 1, 128, 2048, 4096, 4, I8, 64, True) == ("ring", 1)       # 64 CUs
    # the shapes of test_ozaki_matmul_graph_capture: the K-step kernel, and at
    # K = 8192 the ring kernel with 4 ranges (6 K-step tiles against 8)
    assert _gemm_kernel(L, 2, 128, 96, 256, 3, I8, 256, True) == ("kstep2", 1)
    assert _gemm_kernel(L, 1, 64, 96, 8192, 3, I8, 256, True) == ("ring", 4)
    assert _gemm_kernel(L, 1, 64, 96, 8192, 3, _lib.OZK_F16, 256, True) == ("ring", 4)
    assert _gemm_kernel(L, 1, 32, 32, 4096, 4, I8, 256, True) == ("kstep2", 1)       # S = 2
    assert _gemm_kernel(L, 1, 512, 2048, 4096, 4, I8, 256, True) == ("ring", 1)      # 256 tiles
    assert _gemm_kernel(L, 1, 640, 640, 4096, 4, I8, 256, True) == ("ring", 2)       # 100 tiles, 400
    assert _gemm_kernel(L, 1, 640, 640, 2048, 4, I8, 256, True) == ("ring", 1)       # 16 stages
    assert _gemm_kernel(L, 1, 640, 640, 8192, 4, I8, 256, True) == ("ring", 2)
    assert _gemm_kernel(L, 1, 320, 320, 8192, 4, I8, 256, True) == ("kstep2", 1)     # 100 = 25 x 4
    assert _gemm_kernel(L, 1, 288, 320, 8192, 4, I8, 256, True) == ("ring", 4)       # 90 < 25 x 4
    with _lib.forced_kernels(gemm="ring"):
        # the reference point with the ring kernel forced: split-K
        assert _gemm_kernel(L, 1, 128, 2048, 4096, 4, I8, 256, True) == ("ring", 2)
        assert _gemm_kernel(L, 1, 128, 2048, 4096, 4, _lib.OZK_F16, 256, True) == ("ring", 4)
        assert _gemm_kernel(L, 1, 128, 2048, 8192, 4, I8, 256, True) == ("ring", 4)
    assert _gemm_kernel(L, 1, 1024, 1024, 65536, 3, I8, 256, True) == ("wide", 2)    # config 5
    assert _gemm_kernel(L, 1, 8192, 8192, 8192, 4, I8, 256, True) == ("wide4", 1)    # config 3
    assert _gemm_kernel(L, 16, 1024, 1024, 2048, 3, _lib.OZK_F16, 256, True) == ("wide", 1)
    # num_splits 5: the one-wave-per-SIMD kernel, in one launch, for int8 /
    # fp16 / bf16 slices; fp32 slices and 6 to 8 slices: the pair-split kernel
    assert _gemm_kernel(L, 1, 1024, 1024, 1024, 5, I8, 256) == "solo"
    assert _gemm_kernel(L, 1, 8192, 8192, 8192, 5, I8, 256) == "solo"
    assert _gemm_kernel(L, 1, 4096, 4096, 4096, 5, _lib.OZK_BF16, 256) == "solo"
    assert _gemm_kernel(L, 1, 1024, 1024, 1024, 5, _lib.OZK_F32, 256) == "pair"
    assert _gemm_kernel(L, 1, 1024, 1024, 1024, 6, I8, 256) == "pair"


def _gemm_kernel_pairs(L, batch, M, N, K, nsp, sd, pairs, cus=256):
    name = ctypes.c_char_p()
    ks = ctypes.c_int(0)
    st = L.ozk_debug_gemm_kernel_pairs(batch, M, N, K, nsp, sd, pairs, cus, ctypes.byref(name),
                                       ctypes.byref(ks))
    return (name.value.decode(), ks.value) if st == 0 else st


def test_triangular_planner():
    """The triangular pair set runs on the kernels that hold every pair of a
    block in one wave: the K-step kernel on small grids as for all pairs, else
    the wide kernel at 3 slices (split-K on small grids), the one-wave-per-SIMD
    kernel at 5 (the pair-split kernel for fp32 slices), the LDS-DMA kernel at
    2, and at 4 wide4 where its rounds rule holds, else the one-wave-per-SIMD
    kernel (the LDS-DMA kernel for one round over a long K, and for fp32
    slices); one slice plans as all pairs."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    I8, F16, F32 = _lib.OZK_I8, _lib.OZK_F16, _lib.OZK_F32
    T, A = _lib.OZK_PAIRS_TRIANGULAR, _lib.OZK_PAIRS_ALL
    c3 = (1, 8192, 8192, 8192)
    assert _gemm_kernel_pairs(L, *c3, 5, I8, T) == ("solo", 1)
    assert _gemm_kernel_pairs(L, *c3, 5, F16, T) == ("solo", 1)
    assert _gemm_kernel_pairs(L, *c3, 5, F32, T) == ("pair", 1)
    assert _gemm_kernel_pairs(L, *c3, 5, I8, A) == ("solo", 1)
    assert _gemm_kernel_pairs(L, *c3, 4, I8, T) == ("wide4", 1)
    assert _gemm_kernel_pairs(L, 1, 2048, 2048, 8192, 4, I8, T) == ("solo", 1)
    assert _gemm_kernel_pairs(L, 1, 1024, 1024, 65536, 4, I8, T) == ("dma", 1)   # one round, long K
    assert _gemm_kernel_pairs(L, 1, 2048, 2048, 8192, 4, F32, T) == ("dma", 1)
    assert _gemm_kernel_pairs(L, *c3, 4, I8, A) == ("wide4", 1)
    assert _gemm_kernel_pairs(L, *c3, 3, I8, T) == ("wide", 1)
    assert _gemm_kernel_pairs(L, *c3, 2, I8, T) == ("dma", 1)
    assert _gemm_kernel_pairs(L, 1, 4096, 4096, 4096, 2, F16, T) == ("dma", 1)
    assert _gemm_kernel_pairs(L, 1, 1024, 1024, 65536, 3, I8, T) == ("wide", 2)
    ref_point = (1, 128, 2048, 4096)
    for nsp in (2, 3, 4):
        assert _gemm_kernel_pairs(L, *ref_point, nsp, I8, T) == ("kstep2", 1)
    assert _gemm_kernel_pairs(L, *ref_point, 4, F32, T) == ("dma", 1)
    assert _gemm_kernel_pairs(L, *c3, 1, I8, T) == _gemm_kernel_pairs(L, *c3, 1, I8, A)
    # no kernel sums the triangle over more than 5 slices; unknown sets
    assert _gemm_kernel_pairs(L, *c3, 6, I8, T) == _lib.OZK_ERR_SPLITS
    assert _gemm_kernel_pairs(L, *c3, 4, I8, 2) == _lib.OZK_ERR_SPLITS
    assert _gemm_kernel_pairs(L, *c3, 4, I8, -1) == _lib.OZK_ERR_SPLITS


def test_pair_set_arguments_rejected_before_enqueue():
    """ozk_matmul_pairs / ozk_cross_gemm_pairs refuse an unknown set and the
    triangular set beyond 5 slices (or 5 fp32 slices) before anything touches
    a device: no pointer is read."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    s3 = _lib.i64arr((0, 256, 1))
    s4 = _lib.i64arr((0, 0, 256, 1))
    for nsp, sd, pairs in [(6, _lib.OZK_I8, 1), (4, _lib.OZK_I8, 3), (5, _lib.OZK_F32, 1)]:
        st = L.ozk_matmul_pairs(None, s3, None, s3, _lib.OZK_F64, 1, 64, 64, 256, nsp, sd, pairs,
                                None, s3, None, 0, None, None)
        assert st == _lib.OZK_ERR_SPLITS, (nsp, sd, pairs, st)
    for nsp, pairs in [(6, 1), (4, 7)]:
        st = L.ozk_cross_gemm_pairs(None, s4, None, s4, None, s3, None, s3, 1, 64, 64, 256, nsp,
                                    _lib.OZK_I8, pairs, None, _lib.OZK_F64, s3, None, 0, None)
        assert st == _lib.OZK_ERR_SPLITS, (nsp, pairs, st)


def test_workspace_covers_both_pair_sets():
    """The workspace queries take no pair set: their split-K part is the larger
    of the two sets' plans.  At 64 x 96 x 8192 with 3 int8 slices all pairs
    take the ring kernel with 4 ranges, the triangle the wide kernel with 4."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    assert _gemm_kernel_pairs(L, 1, 64, 96, 8192, 3, _lib.OZK_I8, 0) == ("ring", 4)
    assert _gemm_kernel_pairs(L, 1, 64, 96, 8192, 3, _lib.OZK_I8, 1) == ("wide", 4)
    nb = ctypes.c_size_t(0)
    st = L.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, 64, 96, 8192, _lib.i64arr((0, 8192, 1)),
                                      _lib.i64arr((0, 96, 1)), 3, _lib.OZK_I8, ctypes.byref(nb))
    assert st == 0
    # wide split-K: 1 tile x 4 ranges x 8 waves x 144 registers x 64 lanes x 4 bytes
    wide = 1 * 4 * 8 * 144 * 64 * 4
    assert nb.value >= wide


def _residency(L, force):
    got = ctypes.c_int(0)
    assert L.ozk_debug_coop_residency(force, ctypes.byref(got)) == 0
    return got.value


@pytest.mark.parametrize("resident,max_rows_members,max_col_members",
                         [(None, 56, 32), (72, 64, 32), (40, 32, 32), (24, 16, 16), (9, 1, 1)])
def test_coop_member_limit_follows_residency(resident, max_rows_members, max_col_members):
    """A cooperative group's members wait on each other, so the planner gives a
    group at most (workgroups one XCD holds - 8) members, and never more than
    the kernel's own maximum (64 row chunks, 32 column chunks).  With no GPU
    the MI355X figure is assumed (2 workgroups per CU x 32 CUs per XCD: at
    most 56 members); the override stands in for other devices (a partition
    whose XCD holds fewer).  Longer operands fall to the kernels that do not
    wait."""
    from ozaki_triton_amd import _lib
    L = _lib.load()
    try:
        if resident is not None:
            assert _residency(L, resident) == resident
        else:
            assert _residency(L, 0) == 64
        nsp, sd, xd = 3, 4, 0                       # fp64 into int8 slices
        rows_chunk, col_chunk = 4 * 8 * 256, 1024   # fp64 elements per member

        def plan(K, xs, rows):
            ss = [nsp * rows * K, rows * K, K, 1]
            return _split_plan(L, 0x10000, xd, 1, rows, K, xs, nsp, sd, 0x20000, ss)

        def row_path(K):
            # the shared row kernel from 16384 elements while its chunks fit the
            # limit; else the plain row kernel (up to 32768 fp64) or the generic one
            if K > 16384 and -(-K // rows_chunk) <= max_rows_members:
                return "rowscoop"
            return "rows" if K <= 32768 else "generic"

        for P in (3, max_rows_members, max_rows_members + 1, 65):
            K = P * rows_chunk
            assert plan(K, [4 * K, K, 1], 4)[0] == row_path(K), P
        # columns of 64 KB and more: the cooperative column kernel while its
        # chunks fit the limit; else the strip kernel (K <= 16384) or a
        # transpose into the row path
        rows = 4096
        for P in (8, 16, max_col_members, max_col_members + 1, 33):
            K = P * col_chunk
            name = plan(K, [K * rows, 1, rows], rows)[0]
            if 8 <= P <= max_col_members:   # 64 KB columns and longer
                want = "coop"
            elif K <= 16384:
                want = "strip"
            else:
                want = {"rowscoop": "transposerowscoop", "rows": "transpose",
                        "generic": "generic"}[row_path(K)]
            assert name == want, (P, name)
    finally:
        _residency(L, 0)
