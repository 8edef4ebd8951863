import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def oracle():
    import oracle as _oracle
    _oracle.lib()   # builds libozaki_oracle.so with gcc if it is missing
    return _oracle


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but torch.cuda.is_available() is False")
    return torch.device("cuda:0")


@pytest.fixture
def force():
    """force(gemm=..., split=..., coop_timeout=..., ksplit=..., coop_resident=...) forces kernels
    through the library's thread-local test hooks (include/ozaki_amd_debug.h)
    for the rest of the test; the defaults come back at teardown."""
    from ozaki_triton_amd import _lib
    L = _lib.load()

    def set_(gemm=None, split=None, coop_timeout=None, ksplit=None, coop_resident=None):
        if gemm is not None:
            _lib.check("ozk_debug_force_gemm_kernel", L.ozk_debug_force_gemm_kernel(gemm.encode()))
        if ksplit is not None:
            _lib.check("ozk_debug_force_gemm_ksplit", L.ozk_debug_force_gemm_ksplit(int(ksplit)))
        if split is not None:
            _lib.check("ozk_debug_force_split_kernel",
                       L.ozk_debug_force_split_kernel(split.encode()))
        if coop_timeout is not None:
            L.ozk_debug_force_coop_timeout(1 if coop_timeout else 0)
        if coop_resident is not None:
            L.ozk_debug_coop_residency(int(coop_resident), None)

    yield set_
    L.ozk_debug_force_gemm_kernel(None)
    L.ozk_debug_force_gemm_ksplit(0)
    L.ozk_debug_force_split_kernel(None)
    L.ozk_debug_force_coop_timeout(0)
    L.ozk_debug_coop_residency(0, None)
