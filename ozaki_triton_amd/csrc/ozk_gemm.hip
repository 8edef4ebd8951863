// ozk_gemm.hip -- cross-GEMM planner (the tile table that replaces the
// reference's autotuner, ozaki_triton.py:263-304), split-K set-up, the pack
// and zero kernels, and the dispatch to the per-slice-dtype kernel units.
#include "ozk_gemm_kernels.h"

namespace ozk {

// ---------------------------------------------------------------------------
// Pack kernel: any-stride slices -> K-contiguous, 16-byte padded rows.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_kernel(PackParams p) {
    const int64_t total = p.batch * p.L * p.rows * p.Kp;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t k = idx % p.Kp;
        int64_t rest = idx / p.Kp;
        const int64_t r = rest % p.rows;
        rest /= p.rows;
        const int64_t l = rest % p.L;
        const int64_t b = rest / p.L;
        const int64_t so = b * p.s_b + l * p.s_l + r * p.s_r + k * p.s_k;
        if (p.esize == 1) {
            ((int8_t *)p.dst)[idx] = (k < p.K) ? ((const int8_t *)p.src)[so] : (int8_t)0;
        } else if (p.esize == 2) {
            ((uint16_t *)p.dst)[idx] = (k < p.K) ? ((const uint16_t *)p.src)[so] : (uint16_t)0;
        } else {
            ((uint32_t *)p.dst)[idx] = (k < p.K) ? ((const uint32_t *)p.src)[so] : 0u;
        }
    }
}

// num_splits == 0: the reference's kernel stores its zero-initialised outer
// accumulator (ozaki_triton.py:426,452), so C is all zeros.
__global__ __launch_bounds__(256) void zero_c_kernel(GemmParams p) {
    const int64_t total = p.batch * p.M * p.N;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t n = idx % p.N;
        const int64_t m = (idx / p.N) % p.M;
        const int64_t b = idx / (p.N * p.M);
        const int64_t o = b * p.cs_b + m * p.cs_m + n * p.cs_n;
        if (p.out_dtype == 0) store_c(p, o, 0.0);
        else store_c(p, o, 0.0f);
    }
}

hipError_t launch_zero_c(const GemmParams &p, hipStream_t st) {
    const int64_t total = p.batch * p.M * p.N;
    if (total == 0) return hipSuccess;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(zero_c_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_pack(const PackParams &p, hipStream_t st) {
    const int64_t total = p.batch * p.L * p.rows * p.Kp;
    if (total == 0) return hipSuccess;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Tile table (replaces the reference's Optuna search, ozaki_triton.py:263-304):
// the wave tile is the largest whose L*L accumulators fit the register file
// (L*L*MI*NI*16 <= 256 per lane), shrunk when the grid would leave CUs idle.
// ---------------------------------------------------------------------------
// Compute units of the current device, asked once per device (256 on MI355X;
// fewer on a partitioned device).
static int device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
        c = 256;
    cached[dev].store(c, std::memory_order_relaxed);
    return c;
}

GemmPlan plan_gemm(const GemmParams &p, int L, int slice_dtype, int cus) {
    GemmPlan plan{1, 1, 8, kGemmStaged, 1, 0};
    int mi = 1, ni = 1;
    if (L <= 1) { mi = 2; ni = 4; }
    else if (L == 2) { mi = 2; ni = 2; }
    auto nt = [&](int a, int c) {
        return p.batch * ((p.M + 64 * a - 1) / (64 * a)) * ((p.N + 64 * c - 1) / (64 * c));
    };
    // a grid smaller than two waves of 256 CUs loses more to idle CUs than the
    // larger tile gains in reuse.  Shrinks N while it is the larger, then M:
    // (2,4) -> (2,2) -> (1,2) -> (1,1), the (mi, ni) pairs launch_L instantiates.
    // num_splits 2 keeps the ring kernel's 128 x 128 tiles from one wave of
    // tiles on (256 or more: 0.75-0.86x the LDS-DMA kernel's 64 x 128 tiles at
    // 256, 0.94-0.97x at 384; 1.8-1.9x slower at 64)
    const bool ring2 = L == 2 && nt(2, 2) >= 256;
    while (!ring2 && (mi > 1 || ni > 1) && nt(mi, ni) < 512) {
        if (ni > mi) ni /= 2;
        else mi /= 2;
    }
    plan.mi = mi;
    plan.ni = ni;
    plan.group_m = 8;
    const int es = slice_dtype == 4 ? 1 : slice_dtype == 1 ? 4 : 2;
    // The test hooks (include/ozaki_amd_debug.h) force a kernel (tests cover
    // every one at small sizes).  By default, when both operands fit the
    // 31-bit buffer offsets of the LDS-DMA kernels: for L = 3 the wide kernel
    // where it finishes its grid sooner (below), the ring kernel for L = 3, 4
    // (64 x 64 tiles) and for L = 2 on grids of 256 or more 128 x 128 tiles,
    // the pair-split kernel for L > 5, the 2 x 2 LDS-DMA kernel with its larger
    // wave tiles otherwise; for L = 5 the one-wave-per-SIMD kernel; else the
    // VGPR-staged kernel.
    const bool fits = dma_extent(p.as_l, p.as_m, L, p.M, p.K, es) >= 0 &&
                      dma_extent(p.bs_l, p.bs_n, L, p.N, p.K, es) >= 0;
    // Both L = 3 kernels run one workgroup per CU (144 KB of LDS each), so a
    // grid takes ceil(tiles / 256) rounds.  A wide tile (64 x 128) does twice
    // a ring tile's (64 x 64) work at 1.11-1.24x its rate: about 12/7 of its
    // time.  Measured (cross-GEMM alone, int8 K = 8192 and fp16 K = 4096),
    // wide / ring rate by wide tiles: 32: 0.65, 128: 0.78, 200: 1.20,
    // 256: 1.14, 288: 0.95, 384: 1.01-1.03, 480: 1.16-1.18, 512 to 8192:
    // 1.11-1.24; the rule below picks the faster one at each of these except
    // 384 (within 3%).
    const int64_t kCUs = cus > 0 ? cus : device_cus();
    // Split-K (ring and wide kernels): a grid of fewer tiles than half the
    // CUs cuts each tile's K stages into S ranges, one workgroup each: S =
    // CUs / tiles, at most 4 (the last range reads all S ranges'
    // accumulators back) and at least 16 stages (2 KB of K) per range: the
    // hand-over costs about as much as 8 to 16 stages of int8 MFMA work
    // (measured at (1, 128, 2048, 4096), cross-GEMM alone: int8 num_splits 4
    // 66.7 us unsplit, 61.0 with 2 ranges of 16 stages, 63.4 with 4 of 8;
    // num_splits 3 47.7 against 54.7 with 4 of 8; fp16 num_splits 4 106.1,
    // 81.2 with 2 of 32, 73.5 with 4 of 16; C5 wide 899 us unsplit, 572 with
    // 2 ranges of 256 against the ring kernel's 592).  Sized for at most 256
    // CUs, so the workspace queries (which plan for 256) cover any gfx950
    // device.
    const int nkb_all = (int)((p.K * es + kDmaRB - 1) / kDmaRB);
    const int64_t cus_k = kCUs < 256 ? kCUs : 256;
    auto ksplit_for = [&](int64_t ntiles) -> int {
        if (ntiles <= 0 || 2 * ntiles > cus_k) return 1;
        int64_t sk = cus_k / ntiles;
        if (sk > 4) sk = 4;
        if (sk > nkb_all / 16) sk = nkb_all / 16;
        return sk >= 2 ? (int)sk : 1;
    };
    const int64_t wide_tiles = p.batch * ((p.M + 63) / 64) * ((p.N + 127) / 128);
    const int sr = ksplit_for(nt(1, 1)), sw = ksplit_for(wide_tiles);
    const int64_t wide_rounds = (wide_tiles * sw + kCUs - 1) / kCUs;
    const int64_t ring_rounds = (nt(1, 1) * sr + kCUs - 1) / kCUs;
    // with split-K a round of S ranges takes 1 / S of a tile's time.  The 16
    // x 16 forms (int8 / fp16 / bf16 slices): a wide round takes 1.42-1.56
    // ring rounds (cross-GEMM alone, wide / ring time: rounds 2 / 3 at 1024 x
    // 2304 x 4096 0.961, 1024 x 3072 x 4096 0.944, 1536^2 x 8192 0.982 (fp16
    // 1.017); 2 / 4 at 2048^2 x 4096 0.771; 1 / 2 at 1280^2 x 8192 0.725; 8 /
    // 16 at 4096^3 0.782), so the wide kernel takes ties at 3 : 2; the 32 x
    // 32 forms (fp32 slices) about 12 : 7
    const bool wide3 = L == 3 && (slice_dtype == 1 ? 12 * wide_rounds * sr < 7 * ring_rounds * sw
                                                   : 3 * wide_rounds * sr <= 2 * ring_rounds * sw);
    // L = 4: the 96 x 64 wide kernel (one workgroup per CU, like the ring
    // kernel) does 1.5 ring tiles of work per tile in about 1.45 ring tiles'
    // time (measured, 16 x 16 forms, wide4 / ring time: 8192^3 43 rounds
    // against 64, 0.966; 4096^2 x 8192 11 / 16, 0.957; 3072^2 x 8192 6 / 9,
    // 0.949; 1536^2 x 8192 2 / 3, 0.929 (fp16 0.928); 2048^2 x 8192 3 / 4,
    // 1.133 (fp16 1.184); 1024^2 x 65536 1 / 1, 1.219 (fp16 1.328))
    const int64_t wide4_rounds = (p.batch * ((p.M + 95) / 96) * ((p.N + 63) / 64) + kCUs - 1) / kCUs;
    const bool wide4 = L == 4 && 29 * wide4_rounds < 20 * ring_rounds;
    // L = 5: the one-wave-per-SIMD kernel (one launch; int8 / fp16 / bf16
    // slices); L = 6..8 and fp32 slices: the pair-split kernel per i-row range
    const bool solo5 = L == 5 && slice_dtype != 1;
    // L = 1..4 on grids whose 64 x 64 tiles leave more than half the CUs idle
    // and whose 32 x 32 tiles fit one round: the K-step kernel.  A workgroup
    // of it does 1/4 of a 64 x 64 tile over all of K; one of the ring
    // kernel's S split-K ranges does 1/S of a whole tile, so with S < 4 the
    // K-step kernel wins, and with S = 4 only when it has as many workgroups.
    // Measured (kernel trace, int8 unless noted), K-step against the kernel
    // the planner would take otherwise: (1, 128, 2048, 4096) L = 4 28.9 us
    // vs 39.4 (ring, S = 2), L = 3 22.5 vs 26.2, L = 2 15.9 vs 23.9 (LDS-DMA),
    // L = 1 10.6 vs 16.3, fp16 L = 4 48.7 vs 55.5 (S = 4), L = 3 36.3 vs 36.7,
    // L = 2 25.8 vs 43.8, L = 1 16.9 vs 25.9; 256^2 x 4096 L = 4 25.9 vs 34.0
    // (S = 2); config 1 (fp16, L = 2) 7.1 vs 9.6; 320^2 x 8192 L = 4 42.8 vs
    // 41.1 (S = 4, 100 workgroups each); 64 x 96 x 8192 L = 3 33.2 vs 28.2
    // (S = 4, 6 workgroups against 8); 640^2 x 4096 L = 4, 400 tiles in two
    // rounds, 53.7 vs 45.0 (S = 2)
    const int64_t kstep_tiles = p.batch * ((p.M + 31) / 32) * ((p.N + 31) / 32);
    const int s_ring = L >= 3 ? ksplit_for(nt(1, 1)) : 1;
    const bool kstep = L <= 4 && !(L == 4 && slice_dtype == 1) && 2 * nt(1, 1) <= kCUs &&
                       kstep_tiles <= kCUs &&
                       (s_ring < 4 || kstep_tiles >= nt(1, 1) * s_ring);
    plan.kind = !fits              ? kGemmStaged
                : kstep            ? kGemmKStep
                : L <= 1           ? kGemmDMA
                : L == 2           ? ((mi == 2 && ni == 2) ? kGemmRing : kGemmDMA)
                : wide3            ? kGemmWide
                : wide4            ? kGemmWide4
                : L <= 4           ? kGemmRing
                : solo5            ? kGemmSolo
                                   : kGemmPair;
    // two slices or more: the K-step kernel's 8-wave form, two pair groups
    // whose waves share the SIMDs (the same bits; cross-GEMM alone at
    // (1, 128, 2048, 4096) and 256^2 x 4096, int8 and fp16, 2-4 slices:
    // 3-9% faster)
    if (plan.kind == kGemmKStep && L >= 2) plan.kind = kGemmKStep2;
    const int force = debug_overrides().gemm;
    auto forced = [&](int kind) { return force == kind; };
    if (p.tri && L >= 2) {
        // The triangular pair set: the K-step kernel where it runs by
        // default, else the wide kernel at L = 3 (with split-K on small
        // grids), wide4 at L = 4 where its rounds rule holds, the LDS-DMA
        // kernel at L = 2, the one-wave-per-SIMD kernel otherwise at L = 4
        // (below) and at L = 5 (int8 / fp16 / bf16; fp32 slices: the LDS-DMA
        // kernel at L = 4, the pair-split kernel over all i-rows at L = 5).
        // Measured, cross-GEMM alone, full-range random int8 slices, pair /
        // solo at L = 5: 8192^3 8.12 / 6.99 ms,
        // 4096^2 x 8192 2.04 / 1.75, 2048^2 x 8192 0.487 / 0.399, 1024^2 x
        // 65536 1.16 / 1.04, 1024^2 x 8192 0.127 / 0.101 (all 25 pairs: 14.05
        // / 9.29, 3.52 / 2.26, 0.816 / 0.562, 1.77 / 1.12, 0.209 / 0.142).
        // At L = 4 wide4 against the LDS-DMA kernel: 8192^3
        // 5.88 / 6.54 ms, 4096^2 x 8192 1.47-1.64 / 1.66-1.81, 2048^2 x 8192
        // 0.382 / 0.391, 1024^2 x 65536 1.05 / 0.80.  L > 5 has no kernel
        // (the caller rejects it).
        // At L = 4 off wide4's rounds rule: the one-wave-per-SIMD kernel,
        // except a single round over a long K (cross-GEMM alone, int8, solo /
        // LDS-DMA: 2048^2 x 8192 0.277 / 0.349 ms, 2048^2 x 4096 0.148 /
        // 0.188, 1024^2 x 8192 0.075 / 0.094, 1024^2 x 65536 0.910 / 0.782).
        // Where the rules hold, wide4 keeps the triangle (solo / wide4, one
        // box: 8192^3 5.36 / 5.41 ms, 4096 x 8192 x 8192 2.64 / 2.63, 4096^2
        // x 8192 1.33 / 1.30, 8192^2 x 4096 2.88 / 2.64)
        const bool solo4 = L == 4 && slice_dtype != 1 && !(nt(1, 1) <= kCUs && nkb_all >= 256);
        plan.kind = !fits     ? kGemmStaged
                    : kstep   ? kGemmKStep2
                    : L == 3  ? kGemmWide
                    : wide4   ? kGemmWide4
                    : solo4   ? kGemmSolo
                    : L <= 4  ? kGemmDMA
                    : solo5   ? kGemmSolo
                              : kGemmPair;
        if (L <= 4) {
            if (forced(kGemmStaged)) plan.kind = kGemmStaged;
            else if (fits && forced(kGemmDMA)) plan.kind = kGemmDMA;
            else if (fits && forced(kGemmPair) && L >= 3) plan.kind = kGemmPair;
            else if (fits && forced(kGemmWide) && L == 3) plan.kind = kGemmWide;
            else if (fits && forced(kGemmWide4) && L == 4) plan.kind = kGemmWide4;
            else if (fits && forced(kGemmKStep) && !(L == 4 && slice_dtype == 1))
                plan.kind = kGemmKStep;
            else if (fits && forced(kGemmKStep2) && L >= 2) plan.kind = kGemmKStep2;
            else if (fits && forced(kGemmSolo) && L == 4 && slice_dtype != 1) plan.kind = kGemmSolo;
        } else if (fits && forced(kGemmSolo) && solo5) {
            plan.kind = kGemmSolo;
        } else if (fits && forced(kGemmPair)) {
            plan.kind = kGemmPair;
        }
        if (plan.kind == kGemmWide4) plan.group_m = 4;
        plan.kb_per_split = nkb_all;
        if (plan.kind == kGemmWide) {
            const int fk = debug_overrides().ksplit;
            int sk = fk > 0 ? fk : ksplit_for(wide_tiles);
            if (sk > nkb_all) sk = nkb_all;
            if (sk > 1) {
                plan.kb_per_split = (nkb_all + sk - 1) / sk;
                plan.ksplit = (nkb_all + plan.kb_per_split - 1) / plan.kb_per_split;
            }
        }
        return plan;
    }
    if (L > 4) {
        // the pair-split kernel keeps its partial sums in an fp64 C
        if (fits && forced(kGemmPair) && p.out_dtype == 0 && slice_dtype != 1)
            plan.kind = kGemmPair;
        return plan;
    }
    if (forced(kGemmStaged)) plan.kind = kGemmStaged;
    else if (fits && forced(kGemmDMA)) plan.kind = kGemmDMA;
    else if (fits && forced(kGemmPair)) plan.kind = L >= 3 ? kGemmPair : kGemmDMA;
    else if (fits && forced(kGemmRing)) plan.kind = L >= 2 ? kGemmRing : kGemmDMA;
    else if (fits && forced(kGemmWide)) plan.kind = L == 3 ? kGemmWide : plan.kind;
    else if (fits && forced(kGemmWide4)) plan.kind = L == 4 ? kGemmWide4 : plan.kind;
    else if (fits && forced(kGemmKStep)) plan.kind = (L == 4 && slice_dtype == 1) ? plan.kind : kGemmKStep;
    else if (fits && forced(kGemmKStep2) && L >= 2) plan.kind = kGemmKStep2;
    else if (fits && forced(kGemmSolo) && L == 4 && slice_dtype != 1) plan.kind = kGemmSolo;
    // 96 x 64 tiles: groups of 4 tile rows (C3: 7.12-7.16 ms against 7.21-7.23
    // with 8, 7.33-7.35 with 16; cross-GEMM alone, one box)
    if (plan.kind == kGemmWide4) plan.group_m = 4;
    plan.kb_per_split = nkb_all;
    if (plan.kind == kGemmRing || plan.kind == kGemmWide) {
        const int64_t tiles_k = plan.kind == kGemmWide ? wide_tiles : L <= 2 ? nt(2, 2) : nt(1, 1);
        const int fk = debug_overrides().ksplit;
        int sk = fk > 0 ? fk : ksplit_for(tiles_k);
        if (sk > nkb_all) sk = nkb_all;
        if (sk > 1) {
            // every range holds at least one stage
            plan.kb_per_split = (nkb_all + sk - 1) / sk;
            plan.ksplit = (nkb_all + plan.kb_per_split - 1) / plan.kb_per_split;
        }
    }
    return plan;
}

// tiles of a kind's launch and 32-bit accumulator registers per wave that a
// split-K range hands over
static void splitk_shape(const GemmParams &p, const GemmPlan &plan, int L, int64_t *tiles,
                         int *regs) {
    const int bm = plan.kind == kGemmWide ? 64 : L <= 2 ? 128 : 64;
    const int bn = plan.kind == kGemmWide ? 128 : L <= 2 ? 128 : 64;
    *tiles = p.batch * ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
    if (plan.kind == kGemmWide) {
        *regs = 3 * 3 * 16;
    } else {
        const int P = L * L, P0 = (L == 3) ? 6 : (P + 1) / 2;   // PairSplit<L, L>
        const int w = L <= 2 ? 2 : 1;
        *regs = (P0 > P - P0 ? P0 : P - P0) * w * w * 16;
    }
}

static size_t round256(size_t x) { return (x + 255) / 256 * 256; }

size_t splitk_bytes(const GemmParams &p, const GemmPlan &plan, int L) {
    if (plan.ksplit <= 1) return 0;
    int64_t tiles;
    int regs;
    splitk_shape(p, plan, L, &tiles, &regs);
    const size_t part = (size_t)(tiles * plan.ksplit * kSplitKWaves * regs) * 64 * 4;
    return round256(part) + round256((size_t)tiles * 4);
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t *p, int64_t n) {
    for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

hipError_t setup_splitk(GemmParams &p, const GemmPlan &plan, int L, void *ws, hipStream_t st) {
    p.ksplit = plan.ksplit;
    p.kb_per_split = plan.kb_per_split;
    p.kpart = nullptr;
    p.kcount = nullptr;
    if (plan.ksplit <= 1) return hipSuccess;
    int64_t tiles;
    int regs;
    splitk_shape(p, plan, L, &tiles, &regs);
    const size_t part = (size_t)(tiles * plan.ksplit * kSplitKWaves * regs) * 64 * 4;
    p.kpart = (uint32_t *)ws;
    p.kcount = (uint32_t *)((char *)ws + round256(part));
    const int64_t blocks = (tiles + 255) / 256 < 1024 ? (tiles + 255) / 256 : 1024;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p.kcount, tiles);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmParams &p, const GemmPlan &plan, int L, int slice_dtype,
                       hipStream_t st) {
    switch (slice_dtype) {
    case 4: return launch_gemm_i8(p, plan, L, st);
    case 2: return launch_gemm_f16(p, plan, L, st);
    case 3: return launch_gemm_bf16(p, plan, L, st);
    case 1: return launch_gemm_f32(p, plan, L, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace ozk
