"""ctypes binding of libozaki_amd.so (declarations: include/ozaki_amd.h).

The library is the only compute path of this package.  If it is missing the
import of the product API fails loudly; there is no CPU or eager fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libozaki_amd.so")

# dtype and status codes (include/ozaki_amd.h)
OZK_F64, OZK_F32, OZK_F16, OZK_BF16, OZK_I8, OZK_I32 = 0, 1, 2, 3, 4, 5
OZK_OK = 0
OZK_ERR_NULL = -1
OZK_ERR_DTYPE = -2
OZK_ERR_SPLITS = -3
OZK_ERR_SHAPE = -4
OZK_ERR_ALPHA = -5
OZK_ERR_WORKSPACE = -6
OZK_ERR_LAUNCH = -7
OZK_ERR_ACCUM = -8
OZK_ERR_DEVICE_WAIT = -9
OZK_ERR_TOO_LARGE = -10
OZK_STATIC_SCRATCH_BYTES = 64 << 20
OZK_MAX_SPLITS = 8
OZK_PAIRS_ALL, OZK_PAIRS_TRIANGULAR = 0, 1

# every symbol include/ozaki_amd.h declares
EXPORTED = (
    "ozk_strerror",
    "ozk_version",
    "ozk_device_status",
    "ozk_compute_split_bits",
    "ozk_split_workspace_bytes",
    "ozk_split",
    "ozk_cross_gemm_workspace_bytes",
    "ozk_cross_gemm",
    "ozk_matmul_workspace_bytes",
    "ozk_matmul",
    "ozk_matmul_static",
    "ozk_cross_gemm_pairs",
    "ozk_matmul_pairs",
)

# the test hooks of include/ozaki_amd_debug.h
EXPORTED_DEBUG = (
    "ozk_debug_force_gemm_kernel",
    "ozk_debug_force_gemm_ksplit",
    "ozk_debug_force_split_kernel",
    "ozk_debug_force_coop_timeout",
    "ozk_debug_coop_residency",
    "ozk_debug_gemm_kernel",
    "ozk_debug_gemm_kernel_pairs",
    "ozk_debug_split_kernel",
)

_lib = None


class OzakiLibError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, status: int):
        self.status = status
        super().__init__(f"{fn} failed: {strerror(status)} (status {status})")


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(ozaki_triton_amd has no fallback path)")
    L = ctypes.CDLL(LIB_PATH)
    i64, i32, vp, sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
    p64 = ctypes.POINTER(ctypes.c_int64)
    L.ozk_strerror.argtypes = [i32]
    L.ozk_strerror.restype = ctypes.c_char_p
    L.ozk_version.argtypes = []
    L.ozk_version.restype = i32
    L.ozk_device_status.argtypes = [i32, ctypes.POINTER(ctypes.c_int), vp]
    L.ozk_device_status.restype = i32
    L.ozk_compute_split_bits.argtypes = [i64, i32, i32, ctypes.POINTER(ctypes.c_int)]
    L.ozk_compute_split_bits.restype = i32
    L.ozk_split_workspace_bytes.argtypes = [i32, i64, i64, i64, p64, i32, i32, p64,
                                            ctypes.POINTER(sz)]
    L.ozk_split_workspace_bytes.restype = i32
    L.ozk_split.argtypes = [vp, i32, i64, i64, i64, p64, i32, i32, i32, vp, p64, vp, p64,
                            vp, sz, vp]
    L.ozk_split.restype = i32
    L.ozk_cross_gemm_workspace_bytes.argtypes = [i64, i64, i64, i64, i32, i32, vp, p64, vp,
                                                 p64, ctypes.POINTER(sz)]
    L.ozk_cross_gemm_workspace_bytes.restype = i32
    L.ozk_cross_gemm.argtypes = [vp, p64, vp, p64, vp, p64, vp, p64, i64, i64, i64, i64, i32,
                                 i32, vp, i32, p64, vp, sz, vp]
    L.ozk_cross_gemm.restype = i32
    L.ozk_matmul_workspace_bytes.argtypes = [i32, i64, i64, i64, i64, p64, p64, i32, i32,
                                             ctypes.POINTER(ctypes.c_size_t)]
    L.ozk_matmul_workspace_bytes.restype = i32
    L.ozk_matmul.argtypes = [vp, p64, vp, p64, i32, i64, i64, i64, i64, i32, i32, vp, p64, vp,
                             sz, ctypes.POINTER(ctypes.c_void_p), vp]
    L.ozk_matmul.restype = i32
    L.ozk_matmul_static.argtypes = [vp, p64, vp, p64, i32, i64, i64, i64, i64, i32, i32, vp,
                                    p64, ctypes.POINTER(ctypes.c_void_p), vp]
    L.ozk_matmul_static.restype = i32
    L.ozk_cross_gemm_pairs.argtypes = [vp, p64, vp, p64, vp, p64, vp, p64, i64, i64, i64, i64,
                                       i32, i32, i32, vp, i32, p64, vp, sz, vp]
    L.ozk_cross_gemm_pairs.restype = i32
    L.ozk_matmul_pairs.argtypes = [vp, p64, vp, p64, i32, i64, i64, i64, i64, i32, i32, i32, vp,
                                   p64, vp, sz, ctypes.POINTER(ctypes.c_void_p), vp]
    L.ozk_matmul_pairs.restype = i32
    cp = ctypes.c_char_p
    L.ozk_debug_force_gemm_kernel.argtypes = [cp]
    L.ozk_debug_force_gemm_kernel.restype = i32
    L.ozk_debug_force_split_kernel.argtypes = [cp]
    L.ozk_debug_force_split_kernel.restype = i32
    L.ozk_debug_force_coop_timeout.argtypes = [i32]
    L.ozk_debug_force_coop_timeout.restype = i32
    L.ozk_debug_coop_residency.argtypes = [i32, ctypes.POINTER(ctypes.c_int)]
    L.ozk_debug_coop_residency.restype = i32
    L.ozk_debug_force_gemm_ksplit.argtypes = [i32]
    L.ozk_debug_force_gemm_ksplit.restype = i32
    L.ozk_debug_gemm_kernel.argtypes = [i64, i64, i64, i64, i32, i32, i32,
                                        ctypes.POINTER(ctypes.c_char_p),
                                        ctypes.POINTER(ctypes.c_int)]
    L.ozk_debug_gemm_kernel.restype = i32
    L.ozk_debug_gemm_kernel_pairs.argtypes = [i64, i64, i64, i64, i32, i32, i32, i32,
                                              ctypes.POINTER(ctypes.c_char_p),
                                              ctypes.POINTER(ctypes.c_int)]
    L.ozk_debug_gemm_kernel_pairs.restype = i32
    L.ozk_debug_split_kernel.argtypes = [vp, i32, i64, i64, i64, p64, i32, i32, vp, p64,
                                         ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(sz)]
    L.ozk_debug_split_kernel.restype = i32
    _lib = L
    return L


def strerror(status: int) -> str:
    return load().ozk_strerror(int(status)).decode()


def i64arr(vals) -> ctypes.Array:
    vals = [int(v) for v in vals]
    return (ctypes.c_int64 * len(vals))(*vals)


def check(fn: str, status: int) -> None:
    if status != OZK_OK:
        raise OzakiLibError(fn, status)


def device_status(clear: bool = True, stream=None) -> int:
    """Wait for `stream` (a hipStream_t as int, or None for the null stream)
    and return the sticky device status of the current device: OZK_OK, or
    OZK_ERR_DEVICE_WAIT if a cooperative split wait gave up since the last
    clear (the scales of that split, and the C computed from them, are NaN)."""
    st = ctypes.c_int(0)
    check("ozk_device_status", load().ozk_device_status(int(bool(clear)), ctypes.byref(st),
                                                         ctypes.c_void_p(stream or 0)))
    return int(st.value)


class forced_kernels:
    """Context manager for tests: force the cross-GEMM kernel (`gemm`: "staged",
    "dma", "pair", "ring", "wide", "wide4", "solo"), its split-K ranges
    (`ksplit`, ring and wide kernels; 1: none) and / or the split kernel
    (`split`: "coop", "strip", "transpose", "generic", "rows", "rowscoop") of
    the calls this host thread makes inside it, and optionally make every
    cooperative split wait give up at once (`coop_timeout`).  Restores the
    defaults on exit."""

    def __init__(self, gemm=None, split=None, coop_timeout=False, ksplit=None):
        self.gemm, self.split, self.coop_timeout = gemm, split, coop_timeout
        self.ksplit = ksplit

    def __enter__(self):
        L = load()
        if self.gemm is not None:
            check("ozk_debug_force_gemm_kernel", L.ozk_debug_force_gemm_kernel(self.gemm.encode()))
        if self.ksplit is not None:
            check("ozk_debug_force_gemm_ksplit", L.ozk_debug_force_gemm_ksplit(int(self.ksplit)))
        if self.split is not None:
            check("ozk_debug_force_split_kernel",
                  L.ozk_debug_force_split_kernel(self.split.encode()))
        if self.coop_timeout:
            L.ozk_debug_force_coop_timeout(1)
        return self

    def __exit__(self, *exc):
        L = load()
        L.ozk_debug_force_gemm_kernel(None)
        L.ozk_debug_force_gemm_ksplit(0)
        L.ozk_debug_force_split_kernel(None)
        L.ozk_debug_force_coop_timeout(0)
        return False
