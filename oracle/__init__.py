"""CPU oracle for the Ozaki-scheme hot path (split -> fused cross-GEMM).

TEST INFRASTRUCTURE ONLY.  This package is the checker.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product package ``ozaki_triton_amd`` never imports it and has no
CPU fallback.

The arithmetic lives in ``ozaki_oracle.c`` (plain C, built into
``libozaki_oracle.so`` by ``oracle/Makefile``); this module is a numpy/ctypes
front end that mirrors the reference's Python structure:

* ``compute_split_bits``  <- /root/reference/ozaki_triton.py:76-98
* ``split``               <- ozaki_triton.py:137-211 (kernel) and 214-256 (wrapper)
* ``cross_gemm``          <- ozaki_triton.py:306-452 (kernel) and 455-498 (wrapper)
* ``ozaki_matmul``        <- ozaki_triton.py:504-606 (broadcast + split B via B^T)
* ``cross_gemm(..., pairs="triangular")``: not in the reference; the library's
  OZK_PAIRS_TRIANGULAR, the same sum over the pairs i + j <= L - 1 only

Pins (see tests/test_oracle_*.py): the exponent rule against numpy's float32
log2 and the committed exhaustive band table; fp64->fp16 rounding against
numpy's astype; fp64->bf16 rounding against exact rational rounding and
torch's fp32->bf16; narrow inputs split as their exact fp32 values; fp32
slices; the C casts to fp16 / bf16 / int8; split invariants (powers-of-two scales, int8 range, exact
reconstruction of fp32 inputs, residual bounds); the int8 cross-GEMM against
numpy's exact int64 matmul and against the fp64 product of the reconstructed
operands; the triangular sum against the all-pairs sum minus numpy's dropped
terms and against numpy on exact integer-valued slices; and the end-to-end
relative errors the reference publishes in reference/test_results.csv for the
same input distribution.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libozaki_oracle.so")

F64, F32, F16, BF16, I8, I32 = 0, 1, 2, 3, 4, 5

_lib = None


def build() -> str:
    """Compile the oracle library with oracle/Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        L.ozo_compute_split_bits.argtypes = [i64, i32, i32]
        L.ozo_compute_split_bits.restype = i32
        L.ozo_band_J.argtypes = [i32]
        L.ozo_band_J.restype = i32
        L.ozo_ceil_log2_f32.argtypes = [ctypes.c_float]
        L.ozo_ceil_log2_f32.restype = i32
        L.ozo_pow2f.argtypes = [i32]
        L.ozo_pow2f.restype = ctypes.c_float
        L.ozo_scale_from_max.argtypes = [ctypes.c_float, i32]
        L.ozo_scale_from_max.restype = ctypes.c_float
        L.ozo_split.argtypes = [vp, i32, i64, i64, i64, i64, i32, i32, i32, vp, vp]
        L.ozo_split.restype = i32
        L.ozo_cross_gemm.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32, i32, vp, i32]
        L.ozo_cross_gemm.restype = i32
        L.ozo_cross_gemm_pairs.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32, i32, vp, i32,
                                           i32, i32]
        L.ozo_cross_gemm_pairs.restype = i32
        L.ozo_int8_pair_dots.argtypes = [vp, vp, i64, i64, i64, i32, vp]
        L.ozo_int8_pair_dots.restype = i32
        L.ozo_f64_to_f16_array.argtypes = [vp, vp, i64]
        L.ozo_f64_to_f16_array.restype = None
        L.ozo_ceil_log2_f32_array.argtypes = [vp, vp, i64]
        L.ozo_ceil_log2_f32_array.restype = None
        L.ozo_f64_to_bf16_array.argtypes = [vp, vp, i64]
        L.ozo_f64_to_bf16_array.restype = None
        L.ozo_bf16_to_f64_array.argtypes = [vp, vp, i64]
        L.ozo_bf16_to_f64_array.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def code_of(dtype) -> int:
    """Map a numpy / torch dtype (or its name) to the shared dtype code.  numpy
    has no bfloat16: a uint16 array holds bfloat16 bit patterns."""
    name = str(dtype).replace("torch.", "")
    return {"float64": F64, "float32": F32, "float16": F16, "bfloat16": BF16, "uint16": BF16,
            "int8": I8, "int32": I32}[name]


# numpy storage of each dtype code (bfloat16 as uint16 bit patterns)
_NP_OF = {F64: np.float64, F32: np.float32, F16: np.float16, BF16: np.uint16, I8: np.int8}


# --------------------------------------------------------------------------- #
def compute_split_bits(n: int, slice_dtype, dot_accum_dtype) -> int:
    """alpha = min(int((acc_bits - log2 n)/2), slice_bits) (ozaki_triton.py:76-98)."""
    return int(lib().ozo_compute_split_bits(n, code_of(slice_dtype), code_of(dot_accum_dtype)))


def band_J(k: int) -> int:
    return int(lib().ozo_band_J(k))


def ceil_log2_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.int32)
    lib().ozo_ceil_log2_f32_array(_ptr(x), _ptr(out), x.size)
    return out


def f64_to_f16(x: np.ndarray) -> np.ndarray:
    """Single-rounding binary64 -> binary16; returns float16 values."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ozo_f64_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out.view(np.float16)


def f64_to_bf16(x: np.ndarray) -> np.ndarray:
    """Single-rounding binary64 -> bfloat16; returns the uint16 bit patterns."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ozo_f64_to_bf16_array(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f64(h: np.ndarray) -> np.ndarray:
    """Exact bfloat16 bit patterns -> binary64 values."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float64)
    lib().ozo_bf16_to_f64_array(_ptr(h), _ptr(out), h.size)
    return out


def to_f64(a: np.ndarray) -> np.ndarray:
    """Exact values of an array in any shared dtype (uint16 = bfloat16 bits)."""
    return bf16_to_f64(a) if a.dtype == np.uint16 else a.astype(np.float64)


def scale_from_max(mu: float, alpha: int) -> float:
    return float(lib().ozo_scale_from_max(mu, alpha))


# --------------------------------------------------------------------------- #
def split(X: np.ndarray, num_splits: int, alpha: int, slice_dtype):
    """Split a 2-D operand X [rows, K] (any strides) into slices [L, rows, K] and
    scales [L, rows] fp32, per ozaki_triton.py:157-211."""
    assert X.ndim == 2
    xd = code_of(X.dtype)
    sd = code_of(slice_dtype)
    rows, K = X.shape
    item = X.itemsize
    sr, sk = X.strides[0] // item, X.strides[1] // item
    # hand the C code the base pointer of the (possibly strided) view
    slices = np.empty((num_splits, rows, K), dtype=_NP_OF[sd])
    scales = np.empty((num_splits, rows), dtype=np.float32)
    rc = lib().ozo_split(X.ctypes.data, xd, rows, K, sr, sk, num_splits, alpha, sd,
                         _ptr(slices), _ptr(scales))
    if rc != 0:
        raise RuntimeError(f"ozo_split failed: {rc}")
    return slices, scales


PAIRS = {"all": 0, "triangular": 1}


def cross_gemm(As: np.ndarray, Bs_T: np.ndarray, sa: np.ndarray, sb: np.ndarray,
               out_dtype, skip_pair: int = -1, pairs: str = "all") -> np.ndarray:
    """As [L, M, K], Bs_T [L, N, K] (B slices stored K-contiguous), sa [L, M],
    sb [L, N] -> C [M, N] (ozaki_triton.py:357-452).  pairs = "triangular"
    sums only the pairs i + j <= L - 1 (not in the reference: the library's
    OZK_PAIRS_TRIANGULAR), in the same order.  skip_pair = i * L + j
    leaves that pair's term out: a planted mistake for tests that must show
    their checks catch a dropped pair (never used as a reference)."""
    As = np.ascontiguousarray(As)
    Bs_T = np.ascontiguousarray(Bs_T)
    sa = np.ascontiguousarray(sa, dtype=np.float32)
    sb = np.ascontiguousarray(sb, dtype=np.float32)
    L, M, K = As.shape
    L2, N, K2 = Bs_T.shape
    assert L == L2 and K == K2
    od = code_of(out_dtype)
    C = np.empty((M, N), dtype=_NP_OF[od])
    rc = lib().ozo_cross_gemm_pairs(_ptr(As), _ptr(Bs_T), _ptr(sa), _ptr(sb), M, N, K, L,
                                    code_of(As.dtype), _ptr(C), od, PAIRS[pairs], int(skip_pair))
    if rc != 0:
        raise RuntimeError(f"ozo_cross_gemm failed: {rc}")
    return C


def int8_pair_dots(As: np.ndarray, Bs_T: np.ndarray) -> np.ndarray:
    """Exact int64 acc[i, j, m, n] = As[i, m, :] . Bs_T[j, n, :]."""
    As = np.ascontiguousarray(As, dtype=np.int8)
    Bs_T = np.ascontiguousarray(Bs_T, dtype=np.int8)
    L, M, K = As.shape
    _, N, _ = Bs_T.shape
    out = np.empty((L, L, M, N), dtype=np.int64)
    lib().ozo_int8_pair_dots(_ptr(As), _ptr(Bs_T), M, N, K, L, _ptr(out))
    return out


def _slice_dtype_name(slice_dtype) -> str:
    return str(slice_dtype).replace("torch.", "")


def ozaki_matmul(A: np.ndarray, B: np.ndarray, num_splits: int, slice_dtype,
                 return_parts: bool = False, pairs: str = "all"):
    """numpy restatement of ozaki_matmul (ozaki_triton.py:534-606): broadcast the
    batch dims (504-531), split A rows and B columns (through B^T, 593-595),
    cross-GEMM per batch, output in the input dtype (bfloat16 as uint16 bits)."""
    assert A.dtype == B.dtype and code_of(A.dtype) in (F64, F32, F16, BF16, I8)
    M, K = A.shape[-2:]
    K2, N = B.shape[-2:]
    assert K == K2
    batch = np.broadcast_shapes(A.shape[:-2], B.shape[:-2])
    BN = int(math.prod(batch))
    A3 = np.broadcast_to(A, (*batch, M, K)).reshape(BN, M, K)
    B3 = np.broadcast_to(B, (*batch, K, N)).reshape(BN, K, N)
    sdn = _slice_dtype_name(slice_dtype)
    acc = "int32" if sdn == "int8" else "float32"
    alpha = compute_split_bits(K, sdn, acc)
    if alpha < 1:
        raise AssertionError(f"n={K} alpha={alpha}")
    C = np.empty((BN, M, N), dtype=A.dtype)
    parts = []
    for b in range(BN):
        a_sl, a_sc = split(A3[b], num_splits, alpha, sdn)
        b_sl, b_sc = split(B3[b].T, num_splits, alpha, sdn)
        C[b] = cross_gemm(a_sl, b_sl, a_sc, b_sc, A.dtype, pairs=pairs)
        if return_parts:
            parts.append((a_sl, a_sc, b_sl, b_sc))
    C = C.reshape(*batch, M, N)
    if return_parts:
        return C, alpha, parts
    return C
