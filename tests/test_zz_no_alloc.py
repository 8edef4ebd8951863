"""ozk_matmul_static: ozk_matmul on the library's own device scratch array, for
callers that cannot allocate.  Checked through the C ABI against the
workspace entry point ozk_matmul on the same inputs, bit for bit, on calls in
a row (a smaller one after a larger one, then the larger one again), and
against the OZK_STATIC_SCRATCH_BYTES limit."""
import ctypes
import gc

import pytest
import torch

from tests.helpers import assert_bitwise_equal, c3_like, to_np

pytestmark = pytest.mark.gpu


def _strides3(t):
    return (t.stride(0) if t.dim() == 3 and t.shape[0] > 1 else 0, t.stride(-2), t.stride(-1))


def _matmul(static, A, B, L, xd, sd, batch):
    from ozaki_triton_amd import _lib
    lib = _lib.load()
    M, K = A.shape[-2:]
    N = B.shape[-1]
    a_st, b_st = _lib.i64arr(_strides3(A)), _lib.i64arr(_strides3(B))
    C = torch.full((batch, M, N), float("nan"), dtype=A.dtype, device=A.device)
    c_st = _lib.i64arr(C.stride())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if static:
        # nothing allocated: neither through torch's caching allocator nor on
        # the device at all (free device memory; the runtime places the
        # library's scratch array, like the kernels' code, in device memory
        # when the module is first used on the device, so _warm_up runs a
        # call first).  Python's cycle collector is held off meanwhile: a
        # collection could free other tests' tensors inside the window.
        gc.collect()
        gc.disable()
        try:
            torch.cuda.synchronize()
            before = torch.cuda.memory_allocated()
            free0 = torch.cuda.mem_get_info()[0]
            st = lib.ozk_matmul_static(ctypes.c_void_p(A.data_ptr()), a_st,
                                       ctypes.c_void_p(B.data_ptr()), b_st, xd, batch, M, N, K,
                                       L, sd, ctypes.c_void_p(C.data_ptr()), c_st, None, stream)
            torch.cuda.synchronize()
            allocated, free1 = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]
        finally:
            gc.enable()
        assert allocated <= before, (allocated, before)
        assert free1 >= free0, ("device memory was allocated", free0, free1)
        return st, C
    nb = ctypes.c_size_t(0)
    assert lib.ozk_matmul_workspace_bytes(xd, batch, M, N, K, a_st, b_st, L, sd,
                                          ctypes.byref(nb)) == 0
    ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=A.device)
    st = lib.ozk_matmul(ctypes.c_void_p(A.data_ptr()), a_st, ctypes.c_void_p(B.data_ptr()), b_st,
                        xd, batch, M, N, K, L, sd, ctypes.c_void_p(C.data_ptr()), c_st,
                        ctypes.c_void_p(ws.data_ptr()), nb.value, None, stream)
    torch.cuda.synchronize()
    return st, C


def _warm_up(gpu):
    """One static call: the device's copy of the scratch array and the
    kernels' code are in place afterwards."""
    from ozaki_triton_amd import _lib
    lib = _lib.load()
    A = torch.randn(64, 256, dtype=torch.float64, device=gpu)
    B = torch.randn(256, 64, dtype=torch.float64, device=gpu)
    C = torch.empty(1, 64, 64, dtype=torch.float64, device=gpu)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = lib.ozk_matmul_static(ctypes.c_void_p(A.data_ptr()), _lib.i64arr([0, 256, 1]),
                               ctypes.c_void_p(B.data_ptr()), _lib.i64arr([0, 64, 1]),
                               _lib.OZK_F64, 1, 64, 64, 256, 2, _lib.OZK_I8,
                               ctypes.c_void_p(C.data_ptr()), _lib.i64arr(C.stride()), None,
                               stream)
    assert st == 0, _lib.strerror(st)
    torch.cuda.synchronize()


def test_static_entry_matches_workspace_entry(gpu):
    from ozaki_triton_amd import _lib
    _warm_up(gpu)
    # 1: FP64 -> INT8, 4 slices, K = 8192: B's columns take the cooperative
    #    split, whose exchange words live in the scratch (about 25 MB in all)
    A1, B1 = c3_like((256, 8192), (8192, 512), seed=71)
    # 2: smaller, FP32 -> FP16, 3 slices, A batched against a broadcast B
    A2, B2 = c3_like((2, 96, 1000), (1000, 72), seed=72, dtype=torch.float32)
    cases = [(A1, B1, 4, _lib.OZK_F64, _lib.OZK_I8, 1),
             (A2, B2, 3, _lib.OZK_F32, _lib.OZK_F16, 2),
             (A1 * 3.0, B1, 4, _lib.OZK_F64, _lib.OZK_I8, 1)]   # the larger one again
    for i, (A, B, L, xd, sd, batch) in enumerate(cases):
        Ad, Bd = A.to(gpu), B.to(gpu)
        st, C_ws = _matmul(False, Ad, Bd, L, xd, sd, batch)
        assert st == 0, _lib.strerror(st)
        st, C_st = _matmul(True, Ad, Bd, L, xd, sd, batch)
        assert st == 0, _lib.strerror(st)
        torch.cuda.synchronize()
        assert_bitwise_equal(to_np(C_st), to_np(C_ws), f"static vs workspace, call {i}")


def test_static_entry_refuses_calls_beyond_its_scratch(gpu):
    """A call needing more than OZK_STATIC_SCRATCH_BYTES is refused before
    anything is enqueued: C keeps its contents."""
    from ozaki_triton_amd import _lib
    _warm_up(gpu)
    lib = _lib.load()
    M = N = K = 4096                      # 4 int8 slices of A and B: 64 MiB each
    a = _lib.i64arr([0, K, 1])
    b = _lib.i64arr([0, N, 1])
    nb = ctypes.c_size_t(0)
    assert lib.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, M, N, K, a, b, 4, _lib.OZK_I8,
                                          ctypes.byref(nb)) == 0
    assert nb.value > _lib.OZK_STATIC_SCRATCH_BYTES
    A = torch.randn(M, K, dtype=torch.float64, device=gpu)
    B = torch.randn(K, N, dtype=torch.float64, device=gpu)
    st, C = _matmul(True, A, B, 4, _lib.OZK_F64, _lib.OZK_I8, 1)
    assert st == _lib.OZK_ERR_TOO_LARGE
    torch.cuda.synchronize()
    assert torch.isnan(C).all()
    # the same with 1 slice fits (32 MiB of slices) and matches ozk_matmul
    st, C_st = _matmul(True, A, B, 1, _lib.OZK_F64, _lib.OZK_I8, 1)
    assert st == 0, _lib.strerror(st)
    st, C_ws = _matmul(False, A, B, 1, _lib.OZK_F64, _lib.OZK_I8, 1)
    assert st == 0
    torch.cuda.synchronize()
    assert_bitwise_equal(to_np(C_st), to_np(C_ws), "static vs workspace, 1 slice")


def test_static_entry_without_split_k_buffers(gpu):
    """A call whose workspace query exceeds OZK_STATIC_SCRATCH_BYTES only
    through its optional split-K buffers runs, without them, and gives
    ozk_matmul's bits (int8 slice products are exact in any order)."""
    from ozaki_triton_amd import _lib
    _warm_up(gpu)
    lib = _lib.load()
    M = N = 1024
    K = 8192                              # 3 int8 slices: 48 MiB; split-K buffers: 72 MiB
    a = _lib.i64arr([0, K, 1])
    b = _lib.i64arr([0, N, 1])
    nb = ctypes.c_size_t(0)
    assert lib.ozk_matmul_workspace_bytes(_lib.OZK_F64, 1, M, N, K, a, b, 3, _lib.OZK_I8,
                                          ctypes.byref(nb)) == 0
    assert nb.value > _lib.OZK_STATIC_SCRATCH_BYTES
    A, B = c3_like((M, K), (K, N), seed=73)
    Ad, Bd = A.to(gpu), B.to(gpu)
    st, C_ws = _matmul(False, Ad, Bd, 3, _lib.OZK_F64, _lib.OZK_I8, 1)
    assert st == 0, _lib.strerror(st)
    st, C_st = _matmul(True, Ad, Bd, 3, _lib.OZK_F64, _lib.OZK_I8, 1)
    assert st == 0, _lib.strerror(st)
    torch.cuda.synchronize()
    assert_bitwise_equal(to_np(C_st), to_np(C_ws), "static without split-K vs workspace")
