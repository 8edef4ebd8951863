"""Shared helpers for the parity tests (test infrastructure only)."""
import numpy as np
import torch

NP_OF = {torch.float64: np.float64, torch.float32: np.float32, torch.int8: np.int8,
         torch.float16: np.float16, torch.bfloat16: np.uint16}
NAME_OF = {torch.int8: "int8", torch.float16: "float16", torch.float64: "float64",
           torch.float32: "float32", torch.bfloat16: "bfloat16"}


def to_np(t: torch.Tensor) -> np.ndarray:
    """numpy copy of a tensor; bfloat16 (which numpy lacks) as uint16 bit
    patterns, the oracle's convention."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def values(a: np.ndarray) -> np.ndarray:
    """float64 values of an array (uint16 = bfloat16 bit patterns)."""
    if a.dtype == np.uint16:
        return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return a.astype(np.float64)


def oracle_split_batched(oracle, X3: np.ndarray, L: int, alpha: int, slice_dtype):
    """Oracle split of every batch of X3 [B, rows, K] (any strides)."""
    sl, sc = [], []
    for b in range(X3.shape[0]):
        s, c = oracle.split(X3[b], L, alpha, NAME_OF.get(slice_dtype, slice_dtype))
        sl.append(s)
        sc.append(c)
    return np.stack(sl), np.stack(sc)


def bits(a: np.ndarray) -> np.ndarray:
    """View an array's bytes as unsigned ints (bitwise comparison, -0 != +0)."""
    a = np.ascontiguousarray(a)
    return a.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[a.itemsize])


def assert_bitwise_equal(got: np.ndarray, want: np.ndarray, what: str = ""):
    assert got.shape == want.shape, (what, got.shape, want.shape)
    gb, wb = bits(got), bits(want)
    if not np.array_equal(gb, wb):
        idx = np.argwhere(gb != wb)
        first = tuple(idx[0])
        raise AssertionError(
            f"{what}: {len(idx)} of {got.size} elements differ; first at {first}: "
            f"got {got[first]!r} want {want[first]!r}")


def fp16_cross_bound(oracle_np, A_sl, B_slT, sa, sb):
    """Error bound for a GPU float-slice (fp16 / bf16 / fp32) cross-GEMM against
    the oracle's (binary64 accumulated) result, per output element:
        sum_ij sa_i sb_j gamma_{K+2} (|A_i| |B_j|^T)  (fp32 dot of K products,
        the fl32 of the accumulator and of the scaled term)
    with gamma_n = n u / (1 - n u), u = 2^-24, plus the rounding of the outer
    accumulation (L^2 terms)."""
    L, M, K = A_sl.shape
    u = 2.0 ** -24
    g = (K + 2) * u / (1 - (K + 2) * u)
    Aa = np.abs(values(A_sl))
    Ba = np.abs(values(B_slT))
    bound = np.zeros((M, B_slT.shape[1]))
    mag = np.zeros_like(bound)
    for i in range(L):
        for j in range(L):
            t = (Aa[i] @ Ba[j].T) * sa[i][:, None].astype(np.float64) * sb[j][None, :].astype(np.float64)
            bound += g * t
            mag += t
    return bound + 2 * L * L * u * mag


def c3_like(shape_a, shape_b, seed, dtype=torch.float64, exp_range=8):
    """Inputs of the FP64 -> INT8 benchmark's (C3) distribution: N(0,1) * 2^e with e drawn per
    row of A / per column of B from Uniform-int[-exp_range, exp_range]."""
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(*shape_a, generator=g, dtype=torch.float64)
    B = torch.randn(*shape_b, generator=g, dtype=torch.float64)
    ea = torch.randint(-exp_range, exp_range + 1, (*shape_a[:-1], 1), generator=g)
    eb = torch.randint(-exp_range, exp_range + 1, (*shape_b[:-2], 1, shape_b[-1]), generator=g)
    A = A * torch.pow(2.0, ea.double())
    B = B * torch.pow(2.0, eb.double())
    return A.to(dtype), B.to(dtype)


def sample_indices(n, k, seed):
    """k indices of range(n): both ends, a tile boundary and random ones."""
    rng = np.random.default_rng(seed)
    fixed = [i for i in (0, 1, 63, 64, n // 2, n - 1) if i < n]
    rest = rng.choice(n, size=k, replace=False)
    idx = sorted(set(fixed) | set(rest.tolist()))
    return np.array(idx[:k] if len(idx) > k else idx)


def check_block_vs_oracle(oracle, ozk, C_np, A_np, B_np, rows, cols, L, sdt, xdt, what,
                          pairs="all"):
    """C_np[rows][:, cols] against the oracle's result for A_np[rows] and
    B_np[:, cols] (one batch, full K), summed over the pair set `pairs`."""
    K = A_np.shape[-1]
    sd = NAME_OF[sdt]
    alpha = ozk.compute_split_bits(K, sdt, ozk._select_dot_accum_dtype(sdt))
    a_sl, a_sc = oracle.split(np.ascontiguousarray(A_np[rows]), L, alpha, sd)
    b_sl, b_sc = oracle.split(np.ascontiguousarray(B_np[:, cols].T), L, alpha, sd)
    want = oracle.cross_gemm(a_sl, b_sl, a_sc, b_sc, NAME_OF[xdt], pairs=pairs)
    got = np.ascontiguousarray(C_np[np.ix_(rows, cols)])
    if sdt == torch.int8:
        assert_bitwise_equal(got, want, what)
    else:
        bound = fp16_cross_bound(oracle, a_sl, b_sl, a_sc, b_sc)
        if xdt == torch.float32:
            bound = bound + 2.0 ** -23 * np.abs(want.astype(np.float64))   # output rounding
        err = np.abs(got.astype(np.float64) - want.astype(np.float64))
        assert np.all(err <= bound), (what, float((err / np.maximum(bound, 1e-300)).max()))


def int_valued_slices(g, B, L, M, N, K, sdt, vmax=32, exp_range=(-20, 5)):
    """Float slices (float16 / bfloat16 / float32) holding integers in
    [-vmax, vmax] and power-of-two scales 2^[lo, hi).  With K * vmax^2 <= 2^24
    every product and every partial dot sum is an integer that fp32 holds
    exactly, so an fp32-accumulating kernel gives the exact dot in whatever
    order it adds, and its C must equal the oracle's (exact dot, then the
    reference's epilogue) bit for bit: a dropped slice pair, a misplaced
    fragment or a wrong scale shows."""
    assert K * vmax * vmax <= 1 << 24
    As = torch.randint(-vmax, vmax + 1, (B, L, M, K), generator=g).to(sdt)
    BsT = torch.randint(-vmax, vmax + 1, (B, L, N, K), generator=g).to(sdt)
    lo, hi = exp_range
    sa = torch.pow(2.0, torch.randint(lo, hi, (B, L, M), generator=g).float())
    sb = torch.pow(2.0, torch.randint(lo, hi, (B, L, N), generator=g).float())
    return As, BsT, sa, sb
