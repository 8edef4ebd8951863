"""A seeded sweep of ozaki_matmul over the planners' decision boundaries.

The split planner and the cross-GEMM tile table choose kernels and tiles from
the shape (row / column kernels by K and alignment, the cooperative kernels from
64 KB columns and 16384-long rows, 128 x 256 down to 64 x 64 tiles by grid
size, the ring or pair kernel by num_splits).  Each case draws M, N and K from
values on either side of those boundaries, plus a batch (broadcast or not),
transposed input views, the input and slice dtypes and num_splits 1-8, and
checks sampled output blocks against the oracle: bit-exact for int8 slices,
within the fp32-accumulation bound for float slices.  The draw is seeded, so the cases are the same on every
run; each case's parameters are in its test id.
"""
import numpy as np
import pytest
import torch

from tests.helpers import check_block_vs_oracle, sample_indices, to_np

pytestmark = pytest.mark.gpu

MN_VALUES = [1, 7, 63, 64, 65, 127, 128, 129, 255, 256, 257, 1000, 1024, 2047, 2048, 2049, 3000]
# K: the split kernels' limits (4-element groups, 64 KB columns, 16384-long
# rows) and rows that are not whole 16-byte pieces (the pack kernel's copies)
K_VALUES = [1, 3, 4, 7, 100, 255, 256, 257, 1000, 1024, 2048, 4100, 8192, 8196, 16384, 16388]


def _cases(n=120, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M, N = int(rng.choice(MN_VALUES)), int(rng.choice(MN_VALUES))
        K = int(rng.choice(K_VALUES))
        xdt = str(rng.choice(["float64", "float32"]))
        sdt = str(rng.choice(["int8", "float16", "bfloat16", "float32"]))
        L = int(rng.integers(1, 9 if (xdt == "float64" and sdt != "float32") else 5))
        batch = int(rng.choice([1, 1, 2, 3]))
        bcast = bool(batch > 1 and rng.random() < 0.5)
        views = str(rng.choice(["", "", "tA", "tB", "tAtB"]))
        # bounded work: the GPU product and the oracle's sampled blocks stay small
        if batch * M * N * K > 2 ** 32 or M * K * batch > 2 ** 25 or N * K > 2 ** 25:
            continue
        out.append((M, N, K, xdt, sdt, L, batch, bcast, views))
    return out


CASES = _cases()


@pytest.mark.parametrize("M,N,K,xdt,sdt,L,batch,bcast,views", CASES,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}-{c[3]}-{c[4]}-L{c[5]}-b{c[6]}"
                              f"{'bc' if c[7] else ''}{'-' + c[8] if c[8] else ''}" for c in CASES])
def test_shape_sweep(oracle, gpu, M, N, K, xdt, sdt, L, batch, bcast, views):
    import ozaki_triton_amd as ozk
    from ozaki_triton_amd.ozaki import _ozaki_matmul_impl
    xdt, sdt = getattr(torch, xdt), getattr(torch, sdt)
    print(f"[sweep] M={M} N={N} K={K} {xdt} -> {sdt} L={L} batch={batch} broadcast={bcast} "
          f"views={views}", flush=True)
    g = torch.Generator().manual_seed(M * 7919 + N * 104729 + K * 31 + L)
    A = torch.randn(batch, M, K, generator=g, dtype=torch.float64)
    A = A * torch.pow(2.0, torch.randint(-6, 7, (batch, M, 1), generator=g).double())
    B = torch.randn(1 if bcast else batch, K, N, generator=g, dtype=torch.float64)
    B = B * torch.pow(2.0, torch.randint(-6, 7, (B.shape[0], 1, N), generator=g).double())
    if bcast:
        B = B[0]
    A, B = A.to(xdt), B.to(xdt)
    Ad, Bd = A.to(gpu), B.to(gpu)
    if "tA" in views:      # A as the transposed view of a K-major buffer
        Ad = Ad.mT.contiguous().mT
    if "tB" in views:      # B as the transposed view of an N-major buffer
        Bd = Bd.mT.contiguous().mT
    # num_splits above 4 (the reference's limit) through the internal entry,
    # which the C ABI's limit of 8 bounds
    C = _ozaki_matmul_impl(Ad, Bd, L, sdt, False, None, max_splits=8)
    torch.cuda.synchronize()
    assert C.shape == (batch, M, N) and C.dtype == xdt
    C_np, A_np, B_np = to_np(C), to_np(A), to_np(B)
    for b in sorted({0, batch - 1}):
        rows = sample_indices(M, min(M, 24), b + 11)
        cols = sample_indices(N, min(N, 24), b + 12)
        check_block_vs_oracle(oracle, ozk, C_np[b], A_np[b], B_np if bcast else B_np[b], rows,
                              cols, L, sdt, xdt, f"b{b}")
