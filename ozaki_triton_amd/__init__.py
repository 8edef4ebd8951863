"""ozaki_triton_amd -- MI355X-native Ozaki-scheme emulated matmul.

Drop-in for the hot path of WhFanatic/Ozaki_triton (ozaki_triton.py): the same
``ozaki_matmul`` / ``split_matrix`` / ``cross_gemm`` / ``compute_split_bits``
API, computed by hand-written gfx950 HIP kernels (libozaki_amd.so, C ABI in
include/ozaki_amd.h).
"""
from .ozaki import (  # noqa: F401
    _INPUT_DTYPES,
    _SLICE_DTYPE_INFO,
    _canonicalize_batch,
    _select_dot_accum_dtype,
    _select_out_accum_dtype,
    compute_split_bits,
    cross_gemm,
    device_status,
    ozaki_matmul,
    split_matrix,
)

__all__ = ["ozaki_matmul", "split_matrix", "cross_gemm", "compute_split_bits"]
