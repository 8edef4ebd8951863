"""GPU parity on special input values, and the cooperative split's failure
path as ozaki_matmul reports it.

* NaN and signed-zero entries (scattered, whole rows / columns) through every
  split path: int8 slices and the scales bit-exact against the oracle (a NaN
  is ignored by the row maximum and quantises to 0), fp16 slices bit-exact
  outside the NaN positions and NaN at them; the whole int8 ozaki_matmul
  bit-exact.  The reference's own behaviour on NaN is not pinned by its tests
  (parity follows the oracle's restatement of its arithmetic:
  ozaki_triton.py:169-206 with Triton's NaN-ignoring maximum).
* A cooperative split wait that gives up inside ozaki_matmul: the cross-GEMM
  reads the split's status word itself (no poison kernel after that split)
  and stores NaN everywhere (0 in an int8 C) and sets the device status.
"""
import numpy as np
import pytest
import torch

from tests.helpers import NAME_OF, assert_bitwise_equal, bits, oracle_split_batched, to_np

pytestmark = pytest.mark.gpu


def _alpha(ozk, K, sdt):
    return ozk.compute_split_bits(K, sdt, ozk._select_dot_accum_dtype(sdt))


def _special(shape, seed, dtype):
    """N(0,1) entries with NaN, +0 and -0 planted: scattered, one whole row
    (last dim = K) of NaN, one of -0.0 and one mixing the three."""
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(*shape, generator=g, dtype=torch.float64)
    u = torch.rand(*shape, generator=g)
    X[u < 0.02] = float("nan")
    X[(u >= 0.02) & (u < 0.04)] = 0.0
    X[(u >= 0.04) & (u < 0.06)] = -0.0
    X[..., 1, :] = float("nan")
    X[..., 2, :] = -0.0
    X[..., 3, ::3] = float("nan")
    X[..., 3, 1::3] = -0.0
    X[..., 3, 2::3] = 0.0
    return X.to(dtype)


def _assert_equal_nan(got, want, what):
    """Bit-exact outside NaN positions; NaN exactly where the oracle has NaN
    (the payload of a NaN is not compared)."""
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ ({int((gn != wn).sum())})"
    assert np.array_equal(bits(got)[~wn], bits(want)[~wn]), f"{what}: non-NaN entries differ"


def _check(oracle, ozk, X3_dev, L, sdt, what):
    K = X3_dev.shape[-1]
    alpha = _alpha(ozk, K, sdt)
    sl, sc = ozk.split_matrix(X3_dev, L, alpha, sdt)
    torch.cuda.synchronize()
    osl, osc = oracle_split_batched(oracle, to_np(X3_dev.contiguous()), L, alpha, sdt)
    assert_bitwise_equal(to_np(sc), osc, f"{what} scales")
    if sdt == torch.int8:
        assert_bitwise_equal(to_np(sl), osl, f"{what} slices")
    else:
        _assert_equal_nan(to_np(sl), osl, f"{what} slices")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
@pytest.mark.parametrize("path,K", [("", 1000), ("rows", 1000), ("rowscoop", 20000)])
def test_split_rows_nan_and_signed_zero(oracle, gpu, xdt, sdt, path, K, force):
    import ozaki_triton_amd as ozk
    if path:
        force(split=path)
    X = _special((1, 40, K), seed=K + 5, dtype=xdt).to(gpu)
    _check(oracle, ozk, X, 3, sdt, f"rows {path or 'default'} {xdt} {sdt} K{K}")


@pytest.mark.parametrize("sdt", [torch.int8, torch.float16])
@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
@pytest.mark.parametrize("path", ["", "coop", "strip", "transpose", "generic"])
def test_split_columns_nan_and_signed_zero(oracle, gpu, xdt, sdt, path, force):
    import ozaki_triton_amd as ozk
    if path:
        force(split=path)
    K, N = 8192, 64
    # columns of B with the special rows of _special along K
    BT = _special((1, N, K), seed=31, dtype=xdt)
    B = BT.transpose(-1, -2).contiguous().to(gpu)
    _check(oracle, ozk, B.transpose(-1, -2), 3, sdt, f"columns {path or 'default'} {xdt} {sdt}")


@pytest.mark.parametrize("xdt", [torch.float64, torch.float32])
@pytest.mark.parametrize("shape", [((64, 4096), (4096, 48)), ((2, 40, 1000), (1000, 72))])
def test_matmul_nan_and_signed_zero_int8(oracle, gpu, xdt, shape):
    """The whole ozaki_matmul (planner's kernels) on inputs with NaN and
    signed zeros, int8 slices: C bit-exact against the oracle (NaN entries
    contribute 0)."""
    import ozaki_triton_amd as ozk
    sa, sb = shape
    A = _special(sa, seed=7, dtype=xdt)
    B = _special(sb[::-1], seed=8, dtype=xdt).transpose(-1, -2).contiguous()
    L = 4
    C = ozk.ozaki_matmul(A.to(gpu), B.to(gpu), L, torch.int8)
    torch.cuda.synchronize()
    got = to_np(C)
    An, Bn = to_np(A), to_np(B)
    if An.ndim == 2:
        want = oracle.ozaki_matmul(An, Bn, L, "int8")
    else:
        want = np.stack([oracle.ozaki_matmul(An[b], Bn, L, "int8") for b in range(An.shape[0])])
    assert not np.isnan(got).any()
    assert_bitwise_equal(got, want, f"matmul {xdt} {shape}")


@pytest.mark.parametrize("case", ["pair_f64", "coop_f32", "rowscoop_f64", "int8_input",
                                  "int8_poison"])
def test_matmul_wait_timeout_reported_by_cross_gemm(gpu, case, force):
    """Every cooperative wait forced to give up at its first check (a tag no
    member writes): the kernels still finish; C is NaN everywhere (a float
    C) or 0 everywhere (an int8 C: its conversion maps NaN to 0); the device
    status reports OZK_ERR_DEVICE_WAIT once.  The cases take each route:
    B's columns in one launch with A's rows, the cross-GEMM checking B's
    status word (pair_f64); B's cooperative split before A's row kernel
    (coop_f32); B's cooperative split and A's shared row kernel, both words
    checked by the cross-GEMM (rowscoop_f64); narrow inputs converted into
    the workspace, then split by the shared row kernel, both words checked
    by the cross-GEMM (int8_input), or, where A's converted copy covers B's
    status word, B's poison kernel and A's word (int8_poison).  The normal
    path afterwards sets no status."""
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd import _lib
    g = torch.Generator().manual_seed(5)
    if case == "pair_f64":
        # 64 KB columns: the cooperative column kernel, sharing its launch
        A = torch.randn(200, 8192, generator=g, dtype=torch.float64)
        B = torch.randn(8192, 2100, generator=g, dtype=torch.float64)
    elif case == "coop_f32":
        force(split="coop")
        A = torch.randn(40, 4096, generator=g, dtype=torch.float32)
        B = torch.randn(4096, 64, generator=g, dtype=torch.float32)
    elif case == "rowscoop_f64":
        A = torch.randn(8, 20000, generator=g, dtype=torch.float64)
        B = torch.randn(20000, 16, generator=g, dtype=torch.float64)
    else:
        # both converted into K-contiguous fp32 copies, whose 40000-long rows
        # take the shared row kernel (three members per row); with 4 columns
        # B's share of the scratch is smaller than A's
        A = torch.randint(-100, 100, (40, 40000), generator=g, dtype=torch.int8)
        n = 4 if case == "int8_poison" else 64
        B = torch.randint(-100, 100, (40000, n), generator=g, dtype=torch.int8)
    Ad, Bd = A.to(gpu), B.to(gpu)
    ozk.device_status()                       # clear anything older
    force(coop_timeout=True)
    C = ozk.ozaki_matmul(Ad, Bd, 3, torch.int8)
    torch.cuda.synchronize()
    if C.dtype == torch.int8:
        assert (C == 0).all(), "an int8 C should be 0 everywhere after a failed split"
    else:
        assert torch.isnan(C).all(), "C should be NaN everywhere after a failed split"
    with pytest.raises(_lib.OzakiLibError) as e:
        ozk.device_status()
    assert e.value.status == _lib.OZK_ERR_DEVICE_WAIT
    ozk.device_status()                       # cleared by the read above
    force(coop_timeout=False)
    C2 = ozk.ozaki_matmul(Ad, Bd, 3, torch.int8)
    torch.cuda.synchronize()
    if C2.dtype != torch.int8:
        assert not torch.isnan(C2).any()
    ozk.device_status()                       # the normal path sets nothing
