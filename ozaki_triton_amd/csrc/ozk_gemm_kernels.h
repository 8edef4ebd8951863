#pragma once
// ozk_gemm_kernels.h -- the cross-GEMM kernels and their launch templates.
//
// Included by one translation unit per slice dtype (ozk_gemm_i8.hip, _f16,
// _bf16, _f32), each of which instantiates its own kernels, so the four
// compile in parallel; the planner and the untyped kernels live in
// ozk_gemm.hip.
//
// The fused cross-GEMM of ozaki_triton.py:306-452 as LDS-staged MFMA kernels
// for gfx950.
//
//   C[m, n] = sum_{i<L} sum_{j<L} fl32(fl32(fl32(acc_ij[m, n]) * sa_i[m]) * sb_j[n])
//   acc_ij  = A_i[m, :] . B_j[:, n]        (int8: exact int32, fp16: fp32 MFMA)
//   the outer sum runs i-major, j-minor from +0 in the output's accumulator
//   dtype (fp64 for fp64 output, fp32 for every other output dtype), exactly as
//   the reference; kernels are templated on the slice type (int8, fp16, bf16,
//   fp32), that accumulator type and the pair set (all pairs, or with TRI the
//   triangle i + j <= L - 1: Pairs below), and store_c converts to C's dtype.
//
// Design (one workgroup = 256 lanes = 4 waves in a 2 x 2 grid):
//   * Every wave owns a (32*MI) x (32*NI) block of C and ALL L*L slice pairs
//     for it, so each output element's L*L accumulators live in one lane and
//     the ordered epilogue needs no cross-wave traffic.
//   * v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_f16 / _bf16: 32 bytes of K
//     per row per instruction, 16 accumulator registers per lane (fp32 slices:
//     four v_mfma_f32_32x32x2_f32 per 32 bytes).
//   * Both operands are K-contiguous ([L, M, K] and B^T = [L, N, K]); a stage
//     holds 128 bytes of K for all L*(BM+BN) rows, staged global -> VGPR ->
//     LDS with the next stage's loads in flight during the current MFMAs
//     (double-buffered LDS, one barrier per stage).  16-byte chunks are
//     XOR-swizzled by row so ds_read_b128 / ds_write_b128 are bank-conflict
//     free.
//   * int8 products are exact integers, so the order in which K is fed to
//     the MFMA cannot change acc_ij: the int8 result is bit-identical to the
//     reference for any tiling.
//   * Workgroups are remapped so each XCD (own L2) processes a contiguous
//     range of tiles, grouped GROUP_M tile-rows at a time.
#include <atomic>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "ozk_common.h"
#include "ozk_internal.h"

namespace ozk {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <typename ST> struct Mfma;
template <> struct Mfma<int8_t> {
    using Acc = i32x16;
    using Elem = int;
    static constexpr bool kExactAcc = true;    // int32 sums: exact in any order
    OZK_DEV static Acc zero() { return Acc{0}; }
    OZK_DEV static Acc run(i32x4 a, i32x4 b, Acc c) {
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
    }
    OZK_DEV static float to_f32(int x) { return (float)x; }   // RNE int32 -> fp32
};
template <> struct Mfma<_Float16> {
    using Acc = f32x16;
    using Elem = float;
    static constexpr bool kExactAcc = false;
    OZK_DEV static Acc zero() { return Acc{0.0f}; }
    OZK_DEV static Acc run(i32x4 a, i32x4 b, Acc c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    OZK_DEV static float to_f32(float x) { return x; }
};

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
template <> struct Mfma<__bf16> {
    using Acc = f32x16;
    using Elem = float;
    static constexpr bool kExactAcc = false;
    OZK_DEV static Acc zero() { return Acc{0.0f}; }
    OZK_DEV static Acc run(i32x4 a, i32x4 b, Acc c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    OZK_DEV static float to_f32(float x) { return x; }
};
// fp32 slices: a 16-byte fragment is 4 floats; lane (row, h) of the 32x32x2
// MFMA supplies k = h of that instruction, so MFMA q contracts component q of
// both operands' fragments (the same k on A and B), 4 MFMAs per fragment.
// The fragment is bit-cast as a whole: with this compiler, bit-casting the
// int vector's elements one by one made all four MFMAs read component 0.
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <> struct Mfma<float> {
    using Acc = f32x16;
    using Elem = float;
    static constexpr bool kExactAcc = false;
    OZK_DEV static Acc zero() { return Acc{0.0f}; }
    OZK_DEV static Acc run(i32x4 a, i32x4 b, Acc c) {
        const f32x4 fa = __builtin_bit_cast(f32x4, a), fb = __builtin_bit_cast(f32x4, b);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.x, fb.x, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.y, fb.y, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.z, fb.z, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa.w, fb.w, c, 0, 0, 0);
        return c;
    }
    OZK_DEV static float to_f32(float x) { return x; }
};

// Final store of the outer accumulator (ozaki_triton.py:452): fp64 output is
// the fp64 accumulator itself; otherwise the fp32 accumulator is stored as
// fp32, rounded to nearest even for fp16 / bf16, or truncated toward zero and
// saturated for int8 (NVIDIA's float-to-integer conversion; NaN -> 0).
// A failed split before the launch (p.failed) makes every entry NaN.
OZK_DEV void store_c(const GemmParams &p, int64_t idx, double v) {
    ((double *)p.C)[idx] = p.failed ? __longlong_as_double(0x7ff8000000000000ll) : v;
}
// partial of an earlier launch (num_splits > 4 runs with an fp64 or fp32 C)
OZK_DEV double load_c(const GemmParams &p, int64_t idx, double) { return ((const double *)p.C)[idx]; }
OZK_DEV float load_c(const GemmParams &p, int64_t idx, float) { return ((const float *)p.C)[idx]; }
OZK_DEV void store_c(const GemmParams &p, int64_t idx, float v) {
    if (p.failed) v = __int_as_float(0x7fc00000);
    switch (p.out_dtype) {
    case 1: ((float *)p.C)[idx] = v; break;
    case 2: ((_Float16 *)p.C)[idx] = (_Float16)v; break;
    case 3: ((uint16_t *)p.C)[idx] = (uint16_t)((v != v) ? 0x7FC0u : f32_to_bf16_bits(v)); break;
    default: {
        const float t = (v != v) ? 0.0f : fminf(fmaxf(truncf(v), -128.0f), 127.0f);
        ((int8_t *)p.C)[idx] = (int8_t)(int)t;
    }
    }
}

// Kernel entry: reads the status words of the cooperative splits that ran
// before on the same stream (complete when the kernel starts) into p.failed,
// and records a failure in the device's sticky status (one lane).
OZK_DEV void resolve_split_fail(GemmParams &p) {
    p.failed = 0;
    // scalar loads (the constant address space): the words do not change
    // while the kernel runs, and the value stays in a scalar register
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (p.split_fail[i] &&
            *(const __attribute__((address_space(4))) uint32_t *)(uintptr_t)p.split_fail[i] != 0)
            p.failed = 1;
    if (!p.failed) return;
    if (blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_fetch_or(p.dev_status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

OZK_DEV int64_t xcd_remap_gemm(int64_t g, int64_t n) {
    const int64_t q = n / 8;
    if (g >= q * 8) return g;
    return (g % 8) * q + g / 8;
}

template <int N, typename F> OZK_DEV void static_for(F &&f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

// ---------------------------------------------------------------------------
// Pair sets.  The reference sums all L x L slice pairs (i, j).  With TRI a
// kernel sums only the triangle i + j <= L - 1, L (L + 1) / 2 pairs: the
// terms it drops are of the order of the split's own truncation error (pair
// (i, j) carries about 2^(-alpha (i + j)) of C's magnitude).  Pair n of a set
// is its n-th pair in i-major, j-minor order, the order of the outer sum, so
// a kernel that walks n in order sums the reference's terms in the
// reference's order and only leaves the others out.
// ---------------------------------------------------------------------------
template <int L, bool TRI> struct Pairs {
    static constexpr int N = TRI ? L * (L + 1) / 2 : L * L;
    __host__ __device__ static constexpr bool kept(int i, int j) { return !TRI || i + j < L; }
    // index of pair (i, 0)
    __host__ __device__ static constexpr int first(int i) {
        return TRI ? i * L - i * (i - 1) / 2 : i * L;
    }
    __host__ __device__ static constexpr int i_of(int n) {
        int i = 0;
        while (i + 1 < L && first(i + 1) <= n) ++i;
        return i;
    }
    __host__ __device__ static constexpr int j_of(int n) { return n - first(i_of(n)); }
};
static_assert(Pairs<5, true>::N == 15 && Pairs<5, true>::i_of(14) == 4 &&
                  Pairs<5, true>::j_of(14) == 0 && Pairs<5, true>::j_of(4) == 4 &&
                  Pairs<5, true>::i_of(5) == 1 && Pairs<4, false>::j_of(6) == 2,
              "pair table");

constexpr int kRowBytes = 128;   // bytes of K per row per stage
constexpr int kChunks = kRowBytes / 16;

template <int L, int MI, int NI> struct GemmShape {
    static constexpr int BM = 64 * MI;
    static constexpr int BN = 64 * NI;
    static constexpr int A_ROWS = L * BM;
    static constexpr int B_ROWS = L * BN;
    static constexpr int ROWS = A_ROWS + B_ROWS;
    static constexpr int STAGE = ROWS * kRowBytes;
    static constexpr int LOADS = ROWS * kChunks / 256;   // 16-byte chunks per lane per stage
    static constexpr int A_LOADS = A_ROWS * kChunks / 256;
    static constexpr int LDS_BYTES = 2 * STAGE;
    static_assert((ROWS * kChunks) % 256 == 0, "stage must split evenly over 256 lanes");
};

// gfx950's LDS serves a ds_read_b128 16 lanes (256 bytes, all 64 banks) per
// cycle.  For 128-byte rows, rows r and r + 2 share banks, so the 16-byte
// chunk is XORed with (r >> 1) & 7: the 16 rows one pass reads land on 16
// distinct chunk columns.
OZK_DEV int swz(int row, int chunk) {
    return row * kRowBytes + ((chunk ^ ((row >> 1) & 7)) << 4);
}

template <typename ST, int L, int MI, int NI, typename AccT, bool TRI>
__global__ __launch_bounds__(256, 1) void cross_gemm_kernel(GemmParams p, int group_m) {
    resolve_split_fail(p);
    using PS = Pairs<L, TRI>;
    using Sh = GemmShape<L, MI, NI>;
    using MF = Mfma<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;   // outer accumulator: fp64 for fp64 output, else fp32 (store_c)
    constexpr int BM = Sh::BM, BN = Sh::BN;
    constexpr int ES = (int)sizeof(ST);
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5, lr = lane & 31;

    // ---- tile coordinates ----
    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    const int64_t g = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const int64_t kbytes = p.K * ES;
    const int nkb = (int)((kbytes + kRowBytes - 1) / kRowBytes);

    // ---- per-lane load descriptors: lane loads chunk (tid % 8) of rows
    //      tid/8 + 32*u, u < LOADS ----
    const int lch = tid & 7;
    const int lrow = tid >> 3;
    const char *Ab = (const char *)p.A + (bidx * p.as_b) * ES;
    const char *Bb = (const char *)p.B + (bidx * p.bs_b) * ES;

    auto load_stage = [&](int kb, i32x4 *stg) {
        const int64_t kofs = (int64_t)kb * kRowBytes + lch * 16;
        const bool kok = kofs < kbytes;
#pragma unroll
        for (int u = 0; u < Sh::LOADS; ++u) {
            const char *ptr;
            bool ok;
            if (u < Sh::A_LOADS) {
                constexpr int per = BM / 32;
                const int i = u / per;
                const int64_t m = m0 + lrow + 32 * (u % per);
                ok = kok && (m < p.M);
                ptr = Ab + ((int64_t)i * p.as_l + m * p.as_m) * ES + kofs;
            } else {
                constexpr int per = BN / 32;
                const int ub = u - Sh::A_LOADS;
                const int j = ub / per;
                const int64_t n = n0 + lrow + 32 * (ub % per);
                ok = kok && (n < p.N);
                ptr = Bb + ((int64_t)j * p.bs_l + n * p.bs_n) * ES + kofs;
            }
            stg[u] = ok ? *(const i32x4 *)ptr : i32x4{0, 0, 0, 0};
        }
    };
    auto store_stage = [&](char *buf, const i32x4 *stg) {
#pragma unroll
        for (int u = 0; u < Sh::LOADS; ++u) {
            const int row = lrow + 32 * u;
            *(i32x4 *)(buf + swz(row, lch)) = stg[u];
        }
    };

    Acc acc[L][L][MI][NI];
#pragma unroll
    for (int i = 0; i < L; ++i)
#pragma unroll
        for (int j = 0; j < L; ++j)
#pragma unroll
            for (int a = 0; a < MI; ++a)
#pragma unroll
                for (int c = 0; c < NI; ++c) acc[i][j][a][c] = MF::zero();

    i32x4 stg[Sh::LOADS];
    if (nkb > 0) {
        load_stage(0, stg);
        store_stage(smem, stg);
    }
    __syncthreads();

    for (int kb = 0; kb < nkb; ++kb) {
        const bool more = kb + 1 < nkb;
        if (more) load_stage(kb + 1, stg);
        const char *buf = smem + (kb & 1) * Sh::STAGE;
#pragma unroll
        for (int kk = 0; kk < kChunks / 2; ++kk) {
            const int ch = 2 * kk + h;
            i32x4 af[L][MI], bf[L][NI];
#pragma unroll
            for (int i = 0; i < L; ++i)
#pragma unroll
                for (int a = 0; a < MI; ++a) {
                    const int row = i * BM + wm * 32 * MI + a * 32 + lr;
                    af[i][a] = *(const i32x4 *)(buf + swz(row, ch));
                }
#pragma unroll
            for (int j = 0; j < L; ++j)
#pragma unroll
                for (int c = 0; c < NI; ++c) {
                    const int row = Sh::A_ROWS + j * BN + wn * 32 * NI + c * 32 + lr;
                    bf[j][c] = *(const i32x4 *)(buf + swz(row, ch));
                }
#pragma unroll
            for (int i = 0; i < L; ++i)
#pragma unroll
                for (int j = 0; j < L; ++j)
#pragma unroll
                    for (int a = 0; a < MI; ++a)
#pragma unroll
                        for (int c = 0; c < NI; ++c)
                            if (PS::kept(i, j))
                                acc[i][j][a][c] = MF::run(af[i][a], bf[j][c], acc[i][j][a][c]);
        }
        if (more) store_stage(smem + ((kb + 1) & 1) * Sh::STAGE, stg);
        __syncthreads();
    }

    // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
    const float *sab = p.sa + bidx * p.sas_b;
    const float *sbb = p.sb + bidx * p.sbs_b;
    const int64_t cbase = bidx * p.cs_b;
#pragma unroll
    for (int c = 0; c < NI; ++c) {
        const int64_t col = n0 + wn * 32 * NI + c * 32 + lr;
        const bool cok = col < p.N;
        float sbv[L];
#pragma unroll
        for (int j = 0; j < L; ++j) sbv[j] = cok ? sbb[j * p.sbs_l + col * p.sbs_n] : 0.0f;
#pragma unroll
        for (int a = 0; a < MI; ++a) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * 32 * MI + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (cok && row < p.M) {
                    OA out = (OA)0;
#pragma unroll
                    for (int i = 0; i < L; ++i) {
                        const float sai = sab[i * p.sas_l + row * p.sas_m];
#pragma unroll
                        for (int j = 0; j < L; ++j) {
                            if (!PS::kept(i, j)) continue;
                            const float x = MF::to_f32(acc[i][j][a][c][r]);
                            const float t1 = x * sai;
                            const float t2 = t1 * sbv[j];
                            out = out + (OA)t2;
                        }
                    }
                    store_c(p, cbase + row * p.cs_m + col * p.cs_n, out);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Pipelined variant: global -> LDS by buffer_load ... lds (no VGPR staging),
// a ring of DMA_STAGES LDS stages of 64 bytes of K per row, loads issued
// DMA_STAGES-1 stages ahead.  Lane i of a DMA instruction writes LDS bytes
// [16 i, 16 i + 16) of that instruction's 1 KB window, so the XOR swizzle is
// applied by choosing which 16-byte chunk of global memory each lane fetches.
// Out-of-range rows and K tails are fetched from a buffer offset beyond
// num_records, which the hardware returns as zeros.
// ---------------------------------------------------------------------------
constexpr int kDmaRB = 128;          // 2 x 2 DMA kernel stage rows (bytes of K; 64 also works)
constexpr int kDmaStages = (kDmaRB == 64) ? 4 : 2;   // LDS ring slots

template <int L, int MI, int NI> struct DmaShape {
    static constexpr int BM = 64 * MI;
    static constexpr int BN = 64 * NI;
    static constexpr int A_ROWS = L * BM;
    static constexpr int ROWS = L * (BM + BN);
    static constexpr int STAGE = ROWS * kDmaRB;
    static constexpr int LPS = STAGE / (4 * 1024);      // DMA instructions per wave per stage
    static constexpr int LDS_BYTES = kDmaStages * STAGE;
    static_assert(STAGE % 4096 == 0, "stage must be a whole number of 1 KB wave windows");
};

// LDS byte offset of logical 16-byte chunk c of row r inside one stage.
// gfx950 serves a ds_read_b128 16 lanes (256 bytes = all 64 banks) per pass;
// the XOR spreads the 16 consecutive rows of one pass over all banks
// (64-byte rows repeat banks every 4 rows, 128-byte rows every 2).
template <int RB> OZK_DEV int rswz(int r, int c) {
    if constexpr (RB == 64) return r * 64 + ((c ^ ((r >> 2) & 3)) << 4);
    else return r * 128 + ((c ^ ((r >> 1) & 7)) << 4);
}

// s_waitcnt with only the vector-memory counter limited to n
template <int N> OZK_DEV void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Workgroup execution barrier without the release fence of __syncthreads()
// (which would wait for every outstanding global load, i.e. drain the DMA
// prefetch ring).  Callers make their own DMA writes complete with
// wait_vmcnt first; the memory clobber keeps the compiler from moving LDS
// accesses across the barrier.
OZK_DEV void exec_barrier() { asm volatile("s_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------
// Split-K hand-off (ring and wide kernels on grids too small to fill the
// chip).  A tile's 128-byte K stages are cut into p.ksplit ranges of
// p.kb_per_split stages, one workgroup each (consecutive workgroup ids).
// Every range stores its raw accumulators (for int8 slices the exact int32
// dot products) to p.kpart, lane-contiguous per register, and counts itself
// in the tile's arrival counter; the range that arrives last reads all
// ranges' accumulators back, adds them in range order (from zero) and goes
// on to the epilogue, the others exit.  No workgroup waits for another, and
// C does not depend on which range arrives last.
// ---------------------------------------------------------------------------
constexpr int kSplitKWaves = 8;   // both kernels run 8 waves
// The lane index read where it is used (an opaque read the compiler cannot
// hoist), so no split-K address is held in registers through the K loop.
OZK_DEV int lane_here() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}
OZK_DEV uint32_t *splitk_slot(const GemmParams &p, int64_t tile, int range, int wave, int regs,
                              int lane) {
    return p.kpart + (((tile * p.ksplit + range) * kSplitKWaves + wave) * regs) * 64 + lane;
}
// The accumulators go through agent-scope stores and loads, which write
// through to, and read from, the level every XCD shares: once a store has
// completed (vmcnt), every later agent-scope load sees it, with no L2
// write-back or invalidation (a fence here costs a write-back of the whole
// L2 per wave).
OZK_DEV void splitk_put(uint32_t *dst, uint32_t v) {
    __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
OZK_DEV uint32_t splitk_get(const uint32_t *src) {
    return __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// one accumulator tile (16 registers, 64 words apart): all 16 loads are
// issued before the first is used
template <typename Acc> OZK_DEV Acc splitk_get16(const uint32_t *src) {
    i32x16 u;
#pragma unroll
    for (int r = 0; r < 16; ++r) u[r] = (int)splitk_get(src + r * 64);
    return __builtin_bit_cast(Acc, u);
}
// Called by every wave after it stored its accumulators: true in the
// workgroup that arrived last.  Every wave's stores complete before the
// barrier, and the counter is incremented after it, so the range that reads
// ksplit - 1 from the counter finds every range's accumulators in place.
OZK_DEV bool splitk_arrive(const GemmParams &p, int64_t tile, int *flag) {
    wait_vmcnt<0>();
    exec_barrier();
    if (threadIdx.x == 0)
        *flag = (int)__hip_atomic_fetch_add(p.kcount + tile, 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // the flag's LDS write
    exec_barrier();
    return *flag == p.ksplit - 1;
}

template <typename ST, int L, int MI, int NI, typename AccT, bool TRI>
__global__ __launch_bounds__(256, 1) void cross_gemm_dma_kernel(GemmParams p, int group_m,
                                                                uint32_t a_records,
                                                                uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = DmaShape<L, MI, NI>;
    using MF = Mfma<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;   // outer accumulator: fp64 for fp64 output, else fp32 (store_c)
    constexpr int BM = Sh::BM, BN = Sh::BN;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave index is uniform across the wave; saying so keeps the LDS-DMA
    // destination (M0) and the A/B choice per instruction scalar
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5, lr = lane & 31;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    const int64_t g = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb = (int)((kbytes + kDmaRB - 1) / kDmaRB);
    constexpr int CH = kDmaRB / 16;       // 16-byte chunks per row
    constexpr int STEPS = kDmaRB / 32;    // 32-byte MFMA K steps per stage

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // Per-lane source offsets (bytes, excluding the stage's K offset) for the
    // LPS DMA instructions of this wave; kOOB marks rows outside the matrix.
    // A 1 KB DMA window covers whole rows and A_ROWS is a multiple of 64,
    // so each instruction reads only A or only B (uniform per wave).
    uint32_t src[Sh::LPS];
    int chunk[Sh::LPS];
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) {
        const int pos = (wave * Sh::LPS + q) * 64 + lane;   // 16-byte unit in the stage
        const int r = pos / CH;
        const int pc = pos % CH;
        chunk[q] = (kDmaRB == 64) ? (pc ^ ((r >> 2) & 3)) : (pc ^ ((r >> 1) & 7));
        if (r < Sh::A_ROWS) {
            const int i = r / BM;
            const int64_t m = m0 + r % BM;
            src[q] = (m < p.M) ? (uint32_t)(((int64_t)i * p.as_l + m * p.as_m) * ES) : kOOB;
        } else {
            const int rb = r - Sh::A_ROWS;
            const int j = rb / BN;
            const int64_t n = n0 + rb % BN;
            src[q] = (n < p.N) ? (uint32_t)(((int64_t)j * p.bs_l + n * p.bs_n) * ES) : kOOB;
        }
    }

    auto issue_one = [&](int kb, int q) {
        char *dst = smem + (kb % kDmaStages) * Sh::STAGE + wave * Sh::LPS * 1024;
        const uint32_t kofs = (uint32_t)kb * kDmaRB + chunk[q] * 16;
        const uint32_t vo = (src[q] == kOOB || kofs >= kbytes) ? kOOB : src[q] + kofs;
        auto *ldsp = (__attribute__((address_space(3))) void *)(dst + q * 1024);
        const bool isA = (wave * Sh::LPS + q) * (1024 / kDmaRB) < Sh::A_ROWS;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(isA ? rA : rB, ldsp, 16, vo, 0, 0, 0);
    };
    auto issue_stage = [&](int kb) {
#pragma unroll
        for (int q = 0; q < Sh::LPS; ++q) issue_one(kb, q);
    };

    Acc acc[L][L][MI][NI];
#pragma unroll
    for (int i = 0; i < L; ++i)
#pragma unroll
        for (int j = 0; j < L; ++j)
#pragma unroll
            for (int a = 0; a < MI; ++a)
#pragma unroll
                for (int c = 0; c < NI; ++c) acc[i][j][a][c] = MF::zero();

#pragma unroll
    for (int s = 0; s < kDmaStages - 1; ++s)
        if (s < nkb) issue_stage(s);

    // Fragments of one 32-byte K step: this wave's A rows for every slice i
    // and B rows for every slice j.  Read r (r < L*MI: A, else B) of step kk.
    struct Frags {
        i32x4 a[L][MI];
        i32x4 b[L][NI];
    };
    using PS = Pairs<L, TRI>;
    constexpr int kReads = L * (MI + NI);
    constexpr int kMfmas = PS::N * MI * NI;
    auto read_one = [&](const char *buf, int kk, int r, Frags &f) {
        const int ch = 2 * kk + h;
        if (r < L * MI) {
            const int i = r / MI, a = r % MI;
            f.a[i][a] = *(const i32x4 *)(buf + rswz<kDmaRB>(i * BM + wm * 32 * MI + a * 32 + lr, ch));
        } else {
            const int j = (r - L * MI) / NI, c = (r - L * MI) % NI;
            f.b[j][c] = *(const i32x4 *)(buf + rswz<kDmaRB>(Sh::A_ROWS + j * BN + wn * 32 * NI +
                                                            c * 32 + lr, ch));
        }
    };
    // MFMAs of `cur`, with the reads of the next step's fragments into `nxt`
    // interleaved one per MFMA, so no MFMA waits on a read issued after the
    // reads of its own operands and the LDS latency hides under the MFMAs.
    auto step = [&](const Frags &cur, Frags &nxt, const char *nbuf, int nkk) {
        static_for<kMfmas>([&](auto q_) {
            constexpr int q = decltype(q_)::value;
            constexpr int i = PS::i_of(q / (MI * NI)), j = PS::j_of(q / (MI * NI));
            constexpr int a = (q / NI) % MI, c = q % NI;
            acc[i][j][a][c] = MF::run(cur.a[i][a], cur.b[j][c], acc[i][j][a][c]);
            if constexpr (q < kReads) read_one(nbuf, nkk, q, nxt);
            __builtin_amdgcn_sched_barrier(0);   // keep this order
        });
#pragma unroll
        for (int q = kMfmas; q < kReads; ++q) read_one(nbuf, nkk, q, nxt);
    };
    // stage kb has landed once at most the loads of the stages issued after it
    // are outstanding; then the barrier publishes every wave's DMA writes
    // When stage kb is awaited, stages up to kb + DMA_STAGES - 2 have been
    // issued (each LPS loads per lane).
    auto stage_ready = [&](int kb) {
        const int after = min(kDmaStages - 2, nkb - 1 - kb);
        static_assert(kDmaStages >= 2 && kDmaStages <= 6, "wait table");
        // only counts that can occur (after <= DMA_STAGES - 2) are instantiated
        if constexpr (kDmaStages - 2 >= 4) { if (after == 4) { wait_vmcnt<4 * Sh::LPS>(); goto waited; } }
        if constexpr (kDmaStages - 2 >= 3) { if (after == 3) { wait_vmcnt<3 * Sh::LPS>(); goto waited; } }
        if constexpr (kDmaStages - 2 >= 2) { if (after == 2) { wait_vmcnt<2 * Sh::LPS>(); goto waited; } }
        if constexpr (kDmaStages - 2 >= 1) { if (after == 1) { wait_vmcnt<Sh::LPS>(); goto waited; } }
        wait_vmcnt<0>();
    waited:
        // this wave's reads of the slot refilled after the barrier must have
        // completed, not only been issued
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0) only
        exec_barrier();
    };

    // Software pipeline over 32-byte K steps (two per stage).
    Frags f0, f1;
    if (nkb > 0) {
        stage_ready(0);
        if (kDmaStages - 1 < nkb) issue_stage(kDmaStages - 1);
#pragma unroll
        for (int q = 0; q < kReads; ++q) read_one(smem, 0, q, f0);
    }
    for (int kb = 0; kb < nkb; ++kb) {
        const char *buf = smem + (kb % kDmaStages) * Sh::STAGE;
        // steps 0 .. STEPS-2 of this stage, each reading the next step's
        // fragments; f0 / f1 alternate
#pragma unroll
        for (int kk = 0; kk + 1 < STEPS; ++kk) {
            if (kk % 2 == 0) step(f0, f1, buf, kk + 1);
            else step(f1, f0, buf, kk + 1);
        }
        if (kb + 1 < nkb) {
            stage_ready(kb + 1);
            // the ring slot of stage kb + DMA_STAGES is the one of stage kb,
            // whose reads every wave completed before this barrier
            if (kb + kDmaStages < nkb) issue_stage(kb + kDmaStages);
        }
        // last step: reads the next stage's step-0 fragments (on the last
        // stage, unused data from a slot that is not being written)
        if ((STEPS - 1) % 2 == 0) step(f0, f1, smem + ((kb + 1) % kDmaStages) * Sh::STAGE, 0);
        else step(f1, f0, smem + ((kb + 1) % kDmaStages) * Sh::STAGE, 0);
        if ((STEPS - 1) % 2 == 0) {   // next stage's step 0 expects its fragments in f0
#pragma unroll
            for (int i = 0; i < L; ++i)
#pragma unroll
                for (int a = 0; a < MI; ++a) f0.a[i][a] = f1.a[i][a];
#pragma unroll
            for (int j = 0; j < L; ++j)
#pragma unroll
                for (int c = 0; c < NI; ++c) f0.b[j][c] = f1.b[j][c];
        }
    }

    // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
    const float *sab = p.sa + bidx * p.sas_b;
    const float *sbb = p.sb + bidx * p.sbs_b;
    const int64_t cbase = bidx * p.cs_b;
#pragma unroll
    for (int c = 0; c < NI; ++c) {
        const int64_t col = n0 + wn * 32 * NI + c * 32 + lr;
        const bool cok = col < p.N;
        float sbv[L];
#pragma unroll
        for (int j = 0; j < L; ++j) sbv[j] = cok ? sbb[j * p.sbs_l + col * p.sbs_n] : 0.0f;
#pragma unroll
        for (int a = 0; a < MI; ++a) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * 32 * MI + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (cok && row < p.M) {
                    OA out = (OA)0;
#pragma unroll
                    for (int i = 0; i < L; ++i) {
                        const float sai = sab[i * p.sas_l + row * p.sas_m];
#pragma unroll
                        for (int j = 0; j < L; ++j) {
                            if (!PS::kept(i, j)) continue;
                            const float x = MF::to_f32(acc[i][j][a][c][r]);
                            const float t1 = x * sai;
                            const float t2 = t1 * sbv[j];
                            out = out + (OA)t2;
                        }
                    }
                    store_c(p, cbase + row * p.cs_m + col * p.cs_n, out);
                }
            }
        }
    }
}

// one MFMA with its accumulator in AGPRs (AG) or VGPRs
template <typename ST, bool AG> struct HandMfma;
template <bool AG> struct HandMfma<int8_t, AG> {
    OZK_DEV static void run(i32x16 &c, i32x4 a, i32x4 b) {
        if constexpr (AG) asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
        else asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    }
};
template <bool AG> struct HandMfma<_Float16, AG> {
    OZK_DEV static void run(f32x16 &c, i32x4 a, i32x4 b) {
        if constexpr (AG) asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
        else asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    }
};
template <bool AG> struct HandMfma<__bf16, AG> {
    OZK_DEV static void run(f32x16 &c, i32x4 a, i32x4 b) {
        if constexpr (AG) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
        else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    }
};

// ---------------------------------------------------------------------------
// K-step kernel for grids too small to fill the chip with 64 x 64 tiles (tall
// or skinny C, large K).  32 x 32 tiles, 4 waves (one per SIMD).  Wave w
// takes the 32-byte K step w of every 128-byte stage and all L x L slice
// pairs on it, so per stage it reads L A and L B fragments for L^2 MFMAs (8
// reads for 16 MFMAs at L = 4) and no tile's K is split across workgroups.
//   * Stages of 2L x 32 rows x 128 bytes are fetched by LDS-DMA into a ring
//     of NST slots; stage kb + NST reuses the slot of stage kb after the
//     barrier that follows every wave's reads of it.  The fragments of stage
//     kb + 1 are read while the MFMAs of stage kb run, with stage kb + NST's
//     DMA instructions spread between those MFMAs.
//   * Epilogue: the four waves' accumulators of each pair are summed through
//     the LDS in wave order (int32: exact; fp32: the same order every call),
//     in 16-byte pieces, groups of up to 4 pairs at a time, one pair per
//     wave; that wave turns the sum into t_ij = fl32(fl32(fl32(acc) * sa_i) *
//     sb_j) in the LDS.  Then each wave sums, for a quarter of the tile, the
//     t values of the pairs (all L^2, or the triangular set) in the i-major /
//     j-minor order from +0 (ozaki_triton.py:420-452) and stores C.  The
//     tile's scales are loaded at kernel start.
// ---------------------------------------------------------------------------
template <int L, bool TRI, int G = 1> struct KStepShape {
    static constexpr int BM = 32, BN = 32;
    static constexpr int NW = 4 * G;                          // waves: K step (w & 3), pair group (w >> 2)
    static constexpr int ROWS = 2 * L * 32;                   // A rows then B rows
    static constexpr int STAGE = ROWS * kDmaRB;
    static constexpr int LPS = STAGE / (NW * 1024);           // DMA instructions per wave per stage
    static constexpr int NST = (160 * 1024 / STAGE) < 6 ? (160 * 1024 / STAGE) : 6;
    static constexpr int NP = Pairs<L, TRI>::N;               // slice pairs summed
    static constexpr int P0 = (NP + G - 1) / G;               // pairs of group 0
    static constexpr int first(int g) { return g ? P0 : 0; }
    static constexpr int count(int g) { return g ? NP - P0 : P0; }
    static constexpr int PR = G == 1 ? (NP < 4 ? NP : 4) : 2; // pairs per epilogue round and group
    static constexpr int NG = (P0 + PR - 1) / PR;             // epilogue rounds
    static constexpr int T_BYTES = NP * 16 * 64 * 4;          // t values [pair][reg / 4][lane][4]
    static constexpr int R_BYTES = NW * PR * 16 * 64 * 4;     // [wave][pair][reg / 4][lane][4]
    static constexpr int S_BYTES = 2 * L * 32 * 4;            // sa [L][32], sb [L][32]
    static constexpr int EPI_BYTES = T_BYTES + R_BYTES + S_BYTES;
    static constexpr int LDS_BYTES = NST * STAGE > EPI_BYTES ? NST * STAGE : EPI_BYTES;
    static constexpr bool kHand = L == 4 && G == 1;   // accumulators in AGPRs, hand-placed MFMAs
    static_assert(G == 1 || (G == 2 && NP >= 2), "two pair groups need two pairs");
    static_assert(STAGE % (NW * 1024) == 0, "a stage is whole 1 KB windows per wave");
    static_assert(NST >= 3, "stages in flight");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
    static_assert(kDmaRB == 128 && L * 32 <= 128, "four K steps per stage; scales one per lane");
};
// The slices a K-step pair group reads: A slices [ilo, ilo + na), B slices
// [jlo, jlo + nb) of its pairs [f, f + c) of the pair order.
template <int L, bool TRI> struct KStepGroup {
    using PS = Pairs<L, TRI>;
    static constexpr int ilo(int f, int c) { return PS::i_of(f); }
    static constexpr int na(int f, int c) { return PS::i_of(f + c - 1) - PS::i_of(f) + 1; }
    static constexpr int jlo(int f, int c) {
        int m = L;
        for (int n = f; n < f + c; ++n) m = PS::j_of(n) < m ? PS::j_of(n) : m;
        return m;
    }
    static constexpr int nb(int f, int c) {
        int m = 0;
        for (int n = f; n < f + c; ++n) m = PS::j_of(n) > m ? PS::j_of(n) : m;
        return m - jlo(f, c) + 1;
    }
};

template <typename ST, int L, typename AccT, bool TRI, int G>
__global__ __launch_bounds__(256 * G, 1) void cross_gemm_kstep_kernel(GemmParams p, int group_m,
                                                                      uint32_t a_records,
                                                                      uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = KStepShape<L, TRI, G>;
    using KG = KStepGroup<L, TRI>;
    using PS = Pairs<L, TRI>;
    using MF = Mfma<ST>;
    using Acc = typename MF::Acc;
    using Elem = typename MF::Elem;
    using OA = AccT;
    constexpr int BM = Sh::BM, BN = Sh::BN, LPS = Sh::LPS, NST = Sh::NST;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = wave & 3, grp = wave >> 2;   // K step of every stage, pair group
    const int h = lane >> 5, lr = lane & 31;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    const int64_t g = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb = (int)((kbytes + kDmaRB - 1) / kDmaRB);

    // this lane's scale of the tile (lanes 0..32L-1: sa [L][32], lanes
    // 128..128+32L-1: sb [L][32]), loaded first so that its latency passes
    // under the K loop; the epilogue stores it in the LDS
    float scl = 0.0f;
    {
        const int e = tid & 127, s = e / 32, o = e % 32;
        if (e < L * 32 && tid < 256) {
            if (tid < 128) {
                if (m0 + o < p.M) scl = p.sa[bidx * p.sas_b + s * p.sas_l + (m0 + o) * p.sas_m];
            } else if (n0 + o < p.N) {
                scl = p.sb[bidx * p.sbs_b + s * p.sbs_l + (n0 + o) * p.sbs_n];
            }
        }
    }

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // per-lane source offsets of this wave's LPS instructions of a stage (a
    // 1 KB window is 8 whole 128-byte rows, all of A or all of B)
    uint32_t src[LPS];
    int chunk[LPS];
#pragma unroll
    for (int q = 0; q < LPS; ++q) {
        const int pos = (wave * LPS + q) * 64 + lane;
        const int r = pos / 8, pc = pos % 8;
        chunk[q] = pc ^ ((r >> 1) & 7);
        if (r < L * BM) {
            const int64_t m = m0 + r % BM;
            src[q] = (m < p.M) ? (uint32_t)(((int64_t)(r / BM) * p.as_l + m * p.as_m) * ES) : kOOB;
        } else {
            const int rb = r - L * BM;
            const int64_t n = n0 + rb % BN;
            src[q] = (n < p.N) ? (uint32_t)(((int64_t)(rb / BN) * p.bs_l + n * p.bs_n) * ES) : kOOB;
        }
    }
    auto issue_one = [&](int kb, int q) {
        const uint32_t kofs = (uint32_t)kb * kDmaRB + chunk[q] * 16;
        const uint32_t vo = (src[q] == kOOB || kofs >= kbytes) ? kOOB : src[q] + kofs;
        auto *ldsp = (__attribute__((address_space(3))) void *)(smem + (kb % NST) * Sh::STAGE +
                                                              (wave * LPS + q) * 1024);
        const bool isA = (wave * LPS + q) * 8 < L * BM;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(isA ? rA : rB, ldsp, 16, vo, 0, 0, 0);
    };
    auto issue_stage = [&](int kb) {
#pragma unroll
        for (int q = 0; q < LPS; ++q) issue_one(kb, q);
    };
    // stage s has landed once at most the instructions of the stages issued
    // after it are outstanding (stages up to s + NST - 2 are issued when s is
    // awaited); the lgkmcnt wait completes this wave's reads of the slot the
    // next issue refills, and the barrier publishes every wave's DMA writes
    auto stage_ready = [&](int s) {
        const int after = min(NST - 2, nkb - 1 - s);
        static_assert(NST - 2 <= 4, "wait table");
        if constexpr (NST - 2 >= 4) { if (after == 4) { wait_vmcnt<4 * LPS>(); goto waited; } }
        if constexpr (NST - 2 >= 3) { if (after == 3) { wait_vmcnt<3 * LPS>(); goto waited; } }
        if constexpr (NST - 2 >= 2) { if (after == 2) { wait_vmcnt<2 * LPS>(); goto waited; } }
        if (after == 1) { wait_vmcnt<LPS>(); goto waited; }
        wait_vmcnt<0>();
    waited:
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0) only
        exec_barrier();
    };

    // The main loop and the first part of the epilogue of pair group GI
    // (compile-time pair range; G = 1: every pair).
    f32x4 *T = (f32x4 *)smem;
    using E4 = Elem __attribute__((ext_vector_type(4)));
    E4 *R = (E4 *)(smem + Sh::T_BYTES);
    float *S = (float *)(smem + Sh::T_BYTES + Sh::R_BYTES);
    auto body = [&](auto GI_) {
        constexpr int GI = decltype(GI_)::value;
        constexpr int F = Sh::first(GI), NPG = Sh::count(GI);
        constexpr int ILO = KG::ilo(F, NPG), NA = KG::na(F, NPG);
        constexpr int JLO = KG::jlo(F, NPG), NB = KG::nb(F, NPG);
        Acc acc[NPG];
#pragma unroll
        for (int n = 0; n < NPG; ++n) acc[n] = MF::zero();
        // At L = 4 with one pair group the 16 accumulator tiles (256
        // registers) live in the AGPRs, through hand-placed MFMAs (left to the
        // compiler, the K loop spills).  The compiler's hazard recogniser does
        // not see into inline assembly: the zeroed tiles are pinned here, 8
        // wait states before any MFMA reads them.
        constexpr bool kHand = Sh::kHand;
        if constexpr (kHand) {
            static_for<NPG>([&](auto n_) {
                constexpr int n = decltype(n_)::value;
                (void)acc;   // an ordinary use, so that the capture does not hinge on the asm operand
                asm volatile("" : "+a"(acc[n]));
            });
            asm volatile("s_nop 7" ::: "memory");
        }

        struct Frags {
            i32x4 a[NA];
            i32x4 b[NB];
        };
        const int ch = 2 * ks + h;   // this wave's 16-byte chunk of a stage row
        auto read_frags = [&](int kb, Frags &f) {
            const char *buf = smem + (kb % NST) * Sh::STAGE;
#pragma unroll
            for (int i = 0; i < NA; ++i)
                f.a[i] = *(const i32x4 *)(buf + rswz<kDmaRB>((ILO + i) * BM + lr, ch));
#pragma unroll
            for (int j = 0; j < NB; ++j)
                f.b[j] = *(const i32x4 *)(buf + rswz<kDmaRB>(L * BM + (JLO + j) * BN + lr, ch));
        };
        // the group's MFMAs of one stage, with the DMA instructions of stage
        // dkb (if dkb >= 0) spread between them: issued in a burst, the
        // waves' instructions fill the vector-memory queue and stall each
        // wave at issue
        auto mfmas = [&](const Frags &f, int dkb) {
            static_for<NPG>([&](auto n_) {
                constexpr int n = decltype(n_)::value;
                constexpr int i = PS::i_of(F + n) - ILO, j = PS::j_of(F + n) - JLO;
                if constexpr (kHand) HandMfma<ST, true>::run(acc[n], f.a[i], f.b[j]);
                else acc[n] = MF::run(f.a[i], f.b[j], acc[n]);
                static_for<LPS>([&](auto d_) {
                    constexpr int d = decltype(d_)::value;
                    // instruction d goes after MFMA (d * NPG) / LPS
                    if constexpr ((d * NPG) / LPS == n) {
                        if (dkb >= 0) issue_one(dkb, d);
                    }
                });
                __builtin_amdgcn_sched_barrier(0);
            });
        };
        // stage kb: the next stage's fragments into `nxt` (after its barrier,
        // which also frees stage kb's slot for stage kb + NST), then the MFMAs
        // of `cur` with stage kb + NST's DMA between them
        auto stage = [&](int kb, const Frags &cur, Frags &nxt) {
            int dkb = -1;
            if (kb + 1 < nkb) {
                stage_ready(kb + 1);
                if (kb + NST < nkb) dkb = kb + NST;
                read_frags(kb + 1, nxt);
            }
            mfmas(cur, dkb);
        };

        if (nkb > 0) {
#pragma unroll
            for (int s = 0; s < NST - 1; ++s)
                if (s < nkb) issue_stage(s);
            stage_ready(0);
            if (NST - 1 < nkb) issue_stage(NST - 1);
            Frags f0, f1;
            read_frags(0, f0);
            int kb = 0;
            for (; kb + 1 < nkb; kb += 2) {
                stage(kb, f0, f1);
                stage(kb + 1, f1, f0);
            }
            if (kb < nkb) stage(kb, f0, f1);
        }

        // the hand-placed MFMAs' results are read below: 64 wait states first
        if constexpr (kHand) asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");

        // ---- epilogue ----
        wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);
        exec_barrier();   // every wave is past its last read of the ring
        // LDS: T [pair][4][lane] x 4 t values, R [wave][pair][4][lane] x 4
        // accumulator values, S the scales; 16-byte pieces, a wave's 64
        // pieces contiguous.  Round gi takes the group's pairs gi PR .. gi PR
        // + PR - 1: every wave stores its accumulators of them, then wave
        // (group, pp) sums pair pp over the group's four K-step waves in
        // K-step order and turns the sum into t_ij.  Both groups run all
        // rounds (their barriers are shared).
        if ((tid & 127) < L * 32 && tid < 256) S[(tid < 128 ? 0 : L * 32) + (tid & 127)] = scl;
        static_for<Sh::NG>([&](auto gi_) {
            constexpr int gi = decltype(gi_)::value;
            static_for<Sh::PR>([&](auto pp_) {
                constexpr int pp = decltype(pp_)::value;
                constexpr int n = gi * Sh::PR + pp;
                if constexpr (n < NPG) {
                    const Acc v = acc[n];
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        R[((wave * Sh::PR + pp) * 4 + c) * 64 + lane] =
                            E4{v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]};
                }
            });
            __builtin_amdgcn_s_waitcnt(0xC07F);
            exec_barrier();
            const int n = gi * Sh::PR + ks;   // this wave's pair of the round
            if (ks < Sh::PR && n < NPG) {
                const int pr = F + n;
                const int i = PS::i_of(pr), j = PS::j_of(pr);
                const float sbj = S[L * 32 + j * 32 + lr];
                const int w0 = GI * 4;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    E4 v = R[(((w0 + 0) * Sh::PR + ks) * 4 + c) * 64 + lane];
                    v = v + R[(((w0 + 1) * Sh::PR + ks) * 4 + c) * 64 + lane];
                    v = v + R[(((w0 + 2) * Sh::PR + ks) * 4 + c) * 64 + lane];
                    v = v + R[(((w0 + 3) * Sh::PR + ks) * 4 + c) * 64 + lane];
                    // registers 4c .. 4c + 3: rows 8c + 4h + 0..3 of the tile
                    f32x4 tv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float t1 = MF::to_f32(v[e]) * S[i * 32 + 8 * c + 4 * h + e];
                        tv[e] = t1 * sbj;
                    }
                    T[(pr * 4 + c) * 64 + lane] = tv;
                }
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);
            exec_barrier();
        });
    };
    if constexpr (G == 1) {
        body(std::integral_constant<int, 0>{});
    } else {
        if (grp == 0) body(std::integral_constant<int, 0>{});
        else body(std::integral_constant<int, 1>{});
    }
    // waves 0..3: accumulator registers 4w .. 4w + 3 of every lane, rows
    // 8w + 4h + 0..3, summed over every pair in order
    if (wave >= 4) return;
    const int64_t col = n0 + lr;
    const int64_t cbase = bidx * p.cs_b;
    OA out[4] = {(OA)0, (OA)0, (OA)0, (OA)0};
#pragma unroll
    for (int q = 0; q < Sh::NP; ++q) {
        const f32x4 tv = T[(q * 4 + wave) * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = out[e] + (OA)tv[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t row = m0 + 8 * wave + 4 * h + e;
        if (col < p.N && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, out[e]);
    }
}

// Pair-split variant: 8 waves, two per SIMD.  The 2 x 2 grid of 32 x 32 wave
// blocks is covered twice: wave group g (0 or 1) accumulates the slice pairs
// [g*P0, ...) of the i-major / j-minor pair order, P0 = ceil(L*L/2) (6 at
// L = 3), so a wave holds about half the accumulators (128 registers at
// L = 4) and two waves share a SIMD.  While one waits on its DMA issue, an LDS read or the stage barrier,
// the other's MFMAs run.  The epilogue keeps the reference's ordered sum:
// group 0 sums its pairs from +0 and hands the partial to group 1 through
// LDS; group 1 adds its pairs, in order, and stores C.
// ---------------------------------------------------------------------------
// The kernel covers the pairs of R consecutive i-rows [i0, i0 + R) of the
// order (R = L: all of them).  num_splits > 4 runs as several such launches in
// i-major order, each continuing the sum from C, which holds the partial in
// the fp64 outer accumulator between launches.
// At num_splits 3 group 0 takes the pairs of i-rows 0 and 1 (6 MFMAs from 5
// fragment reads per K step) and group 1 those of row 2 (3 MFMAs from 4
// reads): about 6% faster on the fp16 broadcast-batch shape than the 5 / 4
// split, whose group 1 needs A fragments of two i-rows for 4 MFMAs.
// With the triangular pair set (TRI, all i-rows in one launch: R = L) the
// order is that of the kept pairs; at num_splits 5 group 0 takes (0, 0..4)
// and (1, 0..2), group 1 the other 7.
template <int L, int R, bool TRI = false> struct PairSplit {
    static_assert(!TRI || R == L, "the triangular set runs all i-rows in one launch");
    static constexpr int P = TRI ? Pairs<L, true>::N : R * L;
    static constexpr int P0 = (L == 3 && R == 3 && !TRI) ? 6 : (P + 1) / 2;
    static constexpr int first(int g) { return g ? P0 : 0; }
    static constexpr int count(int g) { return g ? P - P0 : P0; }
    // slice pair n of the launch's order (i relative to its first i-row)
    static constexpr int i_of(int n) { return TRI ? Pairs<L, true>::i_of(n) : n / L; }
    static constexpr int j_of(int n) { return TRI ? Pairs<L, true>::j_of(n) : n % L; }
    static constexpr int ilo(int g) { return i_of(first(g)); }
    static constexpr int na(int g) { return i_of(first(g) + count(g) - 1) - ilo(g) + 1; }
};

template <int L, int R> struct PairShape {
    static constexpr int BM = 64, BN = 64;
    static constexpr int A_ROWS = R * BM;
    static constexpr int ROWS = (R + L) * BM;
    static constexpr int STAGE = ROWS * kDmaRB;
    static constexpr int LPS = STAGE / (8 * 1024);   // DMA instructions per wave per stage
    static constexpr int LDS_BYTES = kDmaStages * STAGE;
    static_assert(STAGE % 8192 == 0, "stage must be a whole number of 1 KB windows per wave");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
};

template <typename ST, int L, typename AccT, int R, bool TRI>
__global__ __launch_bounds__(512, 1) void cross_gemm_pair_kernel(GemmParams p, int group_m,
                                                                 uint32_t a_records,
                                                                 uint32_t b_records, int i0,
                                                                 int cont) {
    resolve_split_fail(p);
    using Sh = PairShape<L, R>;
    using PS = PairSplit<L, R, TRI>;
    using MF = Mfma<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;   // outer accumulator: fp64 for fp64 output, else fp32 (store_c)
    constexpr int BM = Sh::BM, BN = Sh::BN;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int blk = wave & 3, grp = wave >> 2;
    const int wm = blk >> 1, wn = blk & 1;
    const int h = lane >> 5, lr = lane & 31;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    const int64_t g = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb = (int)((kbytes + kDmaRB - 1) / kDmaRB);
    constexpr int CH = kDmaRB / 16;
    constexpr int STEPS = kDmaRB / 32;

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // Per-lane source offsets of this wave's LPS DMA instructions (a 1 KB
    // window covers 8 whole rows; A_ROWS is a multiple of 8, so each
    // instruction reads only A or only B).
    uint32_t src[Sh::LPS];
    int chunk[Sh::LPS];
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) {
        const int pos = (wave * Sh::LPS + q) * 64 + lane;
        const int r = pos / CH;
        const int pc = pos % CH;
        chunk[q] = (kDmaRB == 64) ? (pc ^ ((r >> 2) & 3)) : (pc ^ ((r >> 1) & 7));
        if (r < Sh::A_ROWS) {
            const int i = i0 + r / BM;
            const int64_t m = m0 + r % BM;
            src[q] = (m < p.M) ? (uint32_t)(((int64_t)i * p.as_l + m * p.as_m) * ES) : kOOB;
        } else {
            const int rb = r - Sh::A_ROWS;
            const int j = rb / BN;
            const int64_t n = n0 + rb % BN;
            src[q] = (n < p.N) ? (uint32_t)(((int64_t)j * p.bs_l + n * p.bs_n) * ES) : kOOB;
        }
    }
    auto issue_one = [&](int kb, int q) {
        char *dst = smem + (kb % kDmaStages) * Sh::STAGE + wave * Sh::LPS * 1024;
        const uint32_t kofs = (uint32_t)kb * kDmaRB + chunk[q] * 16;
        const uint32_t vo = (src[q] == kOOB || kofs >= kbytes) ? kOOB : src[q] + kofs;
        auto *ldsp = (__attribute__((address_space(3))) void *)(dst + q * 1024);
        const bool isA = (wave * Sh::LPS + q) * (1024 / kDmaRB) < Sh::A_ROWS;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(isA ? rA : rB, ldsp, 16, vo, 0, 0, 0);
    };
    auto issue_stage = [&](int kb) {
#pragma unroll
        for (int q = 0; q < Sh::LPS; ++q) issue_one(kb, q);
    };
    // stage kb has landed once at most the loads of the stages issued after
    // it are outstanding; the barrier then publishes every wave's DMA writes,
    // and the lgkmcnt wait makes this wave's reads of the slot about to be
    // refilled complete first
    auto stage_ready = [&](int kb) {
        const int after = min(kDmaStages - 2, nkb - 1 - kb);
        static_assert(kDmaStages >= 2 && kDmaStages <= 6, "wait table");
        if constexpr (kDmaStages - 2 >= 4) { if (after == 4) { wait_vmcnt<4 * Sh::LPS>(); goto waited; } }
        if constexpr (kDmaStages - 2 >= 3) { if (after == 3) { wait_vmcnt<3 * Sh::LPS>(); goto waited; } }
        if constexpr (kDmaStages - 2 >= 2) { if (after == 2) { wait_vmcnt<2 * Sh::LPS>(); goto waited; } }
        if constexpr (kDmaStages - 2 >= 1) { if (after == 1) { wait_vmcnt<Sh::LPS>(); goto waited; } }
        wait_vmcnt<0>();
    waited:
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0) only
        exec_barrier();
    };

#pragma unroll
    for (int s = 0; s < kDmaStages - 1; ++s)
        if (s < nkb) issue_stage(s);

    const float *sab = p.sa + bidx * p.sas_b;
    const float *sbb = p.sb + bidx * p.sbs_b;
    const int64_t cbase = bidx * p.cs_b;
    OA *part = (OA *)smem;   // epilogue hand-off [4 blocks][16][64 lanes]
    const int64_t col = n0 + wn * 32 + lr;
    const bool cok = col < p.N;

    // The main loop and epilogue of wave group G (compile-time pair range).
    auto body = [&](auto G_) {
        constexpr int G = decltype(G_)::value;
        constexpr int F = PS::first(G), NP = PS::count(G), ILO = PS::ilo(G), NA = PS::na(G);
        constexpr int kReads = NA + L;
        struct Frags {
            i32x4 a[NA];
            i32x4 b[L];
        };
        Acc acc[NP];
#pragma unroll
        for (int q = 0; q < NP; ++q) acc[q] = MF::zero();

        auto read_one = [&](const char *buf, int kk, int r, Frags &f) {
            const int ch = 2 * kk + h;
            if (r < NA) {
                f.a[r] = *(const i32x4 *)(buf + rswz<kDmaRB>((ILO + r) * BM + wm * 32 + lr, ch));
            } else {
                const int j = r - NA;
                f.b[j] = *(const i32x4 *)(buf + rswz<kDmaRB>(Sh::A_ROWS + j * BN + wn * 32 + lr, ch));
            }
        };
        // MFMAs of `cur` with the next step's reads into `nxt` interleaved
        auto step = [&](const Frags &cur, Frags &nxt, const char *nbuf, int nkk) {
            static_for<NP>([&](auto q_) {
                constexpr int q = decltype(q_)::value;
                constexpr int i = PS::i_of(F + q), j = PS::j_of(F + q);
                acc[q] = MF::run(cur.a[i - ILO], cur.b[j], acc[q]);
                if constexpr (q < kReads) read_one(nbuf, nkk, q, nxt);
                __builtin_amdgcn_sched_barrier(0);
            });
#pragma unroll
            for (int q = NP; q < kReads; ++q) read_one(nbuf, nkk, q, nxt);
        };

        // A stage's DMA is issued in three parts: the first right after its
        // ring slot is released (stage_ready of the stage before it), the
        // others before the first two K steps of that stage.  Issued at once,
        // the 8 waves' instructions overfill the vector-memory queue and each
        // wave stalls at issue for hundreds of cycles.
        static_assert(kDmaStages == 2, "the DMA issue schedule assumes a ring of two stages");
        constexpr int DP1 = (Sh::LPS + 2) / 3, DP2 = (2 * DP1 < Sh::LPS) ? 2 * DP1 : Sh::LPS;
        auto issue_part = [&](int kb, int part) {
            const int lo = part == 0 ? 0 : part == 1 ? DP1 : DP2;
            const int hi = part == 0 ? DP1 : part == 1 ? DP2 : Sh::LPS;
#pragma unroll
            for (int q = 0; q < Sh::LPS; ++q)
                if (q >= lo && q < hi) issue_one(kb, q);
        };
        Frags f0, f1;
        if (nkb > 0) {
            stage_ready(0);
            if (1 < nkb) issue_part(1, 0);
#pragma unroll
            for (int q = 0; q < kReads; ++q) read_one(smem, 0, q, f0);
        }
        for (int kb = 0; kb < nkb; ++kb) {
            const char *buf = smem + (kb % kDmaStages) * Sh::STAGE;
#pragma unroll
            for (int kk = 0; kk + 1 < STEPS; ++kk) {
                if (kk < 2 && kb + 1 < nkb) issue_part(kb + 1, kk + 1);
                if (kk % 2 == 0) step(f0, f1, buf, kk + 1);
                else step(f1, f0, buf, kk + 1);
            }
            if (kb + 1 < nkb) {
                stage_ready(kb + 1);
                if (kb + 2 < nkb) issue_part(kb + 2, 0);
            }
            if ((STEPS - 1) % 2 == 0) step(f0, f1, smem + ((kb + 1) % kDmaStages) * Sh::STAGE, 0);
            else step(f1, f0, smem + ((kb + 1) % kDmaStages) * Sh::STAGE, 0);
            if ((STEPS - 1) % 2 == 0) {
#pragma unroll
                for (int i = 0; i < NA; ++i) f0.a[i] = f1.a[i];
#pragma unroll
                for (int j = 0; j < L; ++j) f0.b[j] = f1.b[j];
            }
        }
        // every wave is past its last ring read before the ring holds partials
        __builtin_amdgcn_s_waitcnt(0xC07F);
        exec_barrier();

        // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
        float sbv[L];
#pragma unroll
        for (int j = 0; j < L; ++j) sbv[j] = cok ? sbb[j * p.sbs_l + col * p.sbs_n] : 0.0f;
        // t values of this group's pairs: fl32(fl32(fl32(acc) * sa_i) * sb_j)
        float tv[NP][16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + wm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            const bool ok = cok && row < p.M;
            float sai[NA];
#pragma unroll
            for (int i = 0; i < NA; ++i)
                sai[i] = ok ? sab[(int64_t)(i0 + ILO + i) * p.sas_l + row * p.sas_m] : 0.0f;
            static_for<NP>([&](auto q_) {
                constexpr int q = decltype(q_)::value;
                constexpr int i = PS::i_of(F + q), j = PS::j_of(F + q);
                const float x = MF::to_f32(acc[q][r]);
                const float t1 = x * sai[i - ILO];
                tv[q][r] = t1 * sbv[j];
            });
        }
        if constexpr (G == 0) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                // from +0, or from the partial an earlier launch left in C
                OA out = (OA)0;
                if (cont) {
                    const int64_t row = m0 + wm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (cok && row < p.M) out = load_c(p, cbase + row * p.cs_m + col * p.cs_n, out);
                }
#pragma unroll
                for (int q = 0; q < NP; ++q) out = out + (OA)tv[q][r];
                part[(blk * 16 + r) * 64 + lane] = out;
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);
            exec_barrier();
        } else {
            exec_barrier();
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                OA out = part[(blk * 16 + r) * 64 + lane];
#pragma unroll
                for (int q = 0; q < NP; ++q) out = out + (OA)tv[q][r];
                if (cok && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, out);
            }
        }
    };
    if (grp == 0) body(std::integral_constant<int, 0>{});
    else body(std::integral_constant<int, 1>{});
}

// ---------------------------------------------------------------------------
// Ring variant of the pair-split kernel, for num_splits 3 and 4 (all i-rows in
// one launch).  Same 8 waves, wave blocks and pair split; what changes is how
// operands reach the LDS.
//   * The ring has five slots of half a stage: half stage 2kb holds the A
//     rows and 2kb + 1 the B rows of stage kb (128 bytes of K), in slot
//     h % 5.  A(kb + 2) reuses the slot of B(kb - 1), which is free from the
//     start of stage kb, so it can be fetched two stages ahead; B(kb + 1)
//     reuses the slot of A(kb - 1) and is fetched one stage ahead.
//   * The DMA of stage kb's time window (B(kb + 1), then A(kb + 2)) is spread
//     one instruction at a time between this wave's MFMAs.  The LDS-DMA path
//     accepts about one 1 KB instruction per 13 cycles per CU; issued in
//     bursts, the 8 waves' instructions fill the vector-memory queue and each
//     wave stalls at issue for hundreds of cycles.
//   * A K step issues all reads of the next step before its MFMAs: under
//     load an LDS read takes several hundred cycles to return.
// Per stage each wave issues LPH instructions of B(kb + 1) in K steps 0 and 1
// and LPH of A(kb + 2) in steps 2 and 3 (the part in step 3 after the stage
// barrier); the barrier before stage kb + 1 waits for everything but the
// step-2 part of A(kb + 2).
// ---------------------------------------------------------------------------
// W = 1 for num_splits 3 and 4: 32 x 32 wave blocks, 64 x 64 tiles.  W = 2
// for num_splits 2: 64 x 64 wave blocks, 128 x 128 tiles; a wave then holds
// 2 pairs x 4 blocks, again 128 accumulator registers, and the slot is again
// 32 KB.
template <int L, int W> struct RingShape {
    static constexpr int NW = 8;                       // waves
    static constexpr int BM = 64 * W, BN = 64 * W;
    static constexpr int SLOT = L * BM * kDmaRB;       // one half stage (A rows or B rows)
    // six slots where they fit (L = 3: 144 KB): then whole stages are fetched
    // two ahead, B as well as A
    static constexpr int NSLOT = 6 * SLOT <= 160 * 1024 ? 6 : 5;
    static constexpr int LPH = SLOT / (NW * 1024);     // DMA instructions per wave per half stage
    static constexpr int LDS_BYTES = NSLOT * SLOT;
    static constexpr int B0 = (LPH + 1) / 2;           // B(kb + 1) instructions in step 0
    static constexpr int A2 = (LPH + 1) / 2;           // A(kb + 2) instructions in step 2
    static_assert(SLOT % (NW * 1024) == 0, "a half stage must be whole 1 KB windows per wave");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
    static_assert(L * BM <= 256, "the scales of a tile: one dword per lane of four waves");
    static_assert(kDmaRB == 128, "the ring assumes 128-byte stage rows");
};

template <typename ST, int L, typename AccT, int W>
__global__ __launch_bounds__(512, 1) void cross_gemm_ring_kernel(GemmParams p, int group_m,
                                                                 uint32_t a_records,
                                                                 uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = RingShape<L, W>;
    using PS = PairSplit<L, L>;
    using MF = Mfma<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;
    constexpr int BM = Sh::BM, BN = Sh::BN;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    constexpr int LPH = Sh::LPH;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int blk = wave & 3, grp = wave >> 2;
    const int wm = blk >> 1, wn = blk & 1;
    const int h = lane >> 5, lr = lane & 31;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    // split-K: workgroup g0 is K range g0 % S of tile g0 / S
    const int S = p.ksplit > 1 ? p.ksplit : 1;
    const int64_t g0 = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int krange = (int)(g0 % S);
    const int64_t g = g0 / S;
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb_all = (int)((kbytes + kDmaRB - 1) / kDmaRB);
    const int kb0 = S > 1 ? krange * p.kb_per_split : 0;   // this range's first stage
    const int nkb = S > 1 ? min(p.kb_per_split, nkb_all - kb0) : nkb_all;
    const uint32_t kbyte0 = (uint32_t)kb0 * kDmaRB;
    constexpr int STEPS = kDmaRB / 32;

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // Per-lane source offsets of this wave's LPH instructions of an A half
    // and of a B half (a 1 KB window is 8 whole 128-byte rows).
    uint32_t srcA[LPH], srcB[LPH];
    int chA[LPH], chB[LPH];
#pragma unroll
    for (int q = 0; q < LPH; ++q) {
        const int pos = (wave * LPH + q) * 64 + lane;
        const int r = pos / 8, pc = pos % 8;
        const int c = pc ^ ((r >> 1) & 7);
        chA[q] = chB[q] = c;
        const int64_t m = m0 + r % BM, n = n0 + r % BN;
        srcA[q] = (m < p.M) ? (uint32_t)(((int64_t)(r / BM) * p.as_l + m * p.as_m) * ES) : kOOB;
        srcB[q] = (n < p.N) ? (uint32_t)(((int64_t)(r / BN) * p.bs_l + n * p.bs_n) * ES) : kOOB;
    }
    auto slot = [&](int hs) { return smem + (hs % Sh::NSLOT) * Sh::SLOT; };
    auto issue_a = [&](int kb, int q) {
        const uint32_t kofs = kbyte0 + (uint32_t)kb * kDmaRB + chA[q] * 16;
        const uint32_t vo = (srcA[q] == kOOB || kofs >= kbytes) ? kOOB : srcA[q] + kofs;
        auto *ldsp = (__attribute__((address_space(3))) void *)(slot(2 * kb) + (wave * LPH + q) * 1024);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, vo, 0, 0, 0);
    };
    auto issue_b = [&](int kb, int q) {
        const uint32_t kofs = kbyte0 + (uint32_t)kb * kDmaRB + chB[q] * 16;
        const uint32_t vo = (srcB[q] == kOOB || kofs >= kbytes) ? kOOB : srcB[q] + kofs;
        auto *ldsp = (__attribute__((address_space(3))) void *)(slot(2 * kb + 1) + (wave * LPH + q) * 1024);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, vo, 0, 0, 0);
    };

    // The scales of the tile (L x BM of A's rows and L x BN of B's columns,
    // at most 2 KB) are fetched into a free ring slot by one dword DMA
    // instruction per wave at the start of the last stage, so the epilogue
    // reads them from the LDS instead of waiting on global loads.  The slot is
    // the one of A(nkb), which is never fetched.  Waves 0-3 fetch A's scales
    // [L][BM] (entry 64 wave + lane), waves 4-7 B's [L][BN].
    char *const scl = slot(2 * nkb);
    auto issue_scales = [&]() {
        const bool isa = wave < 4;
        const int e = (isa ? wave : wave - 4) * 64 + lane;
        const int s = e / BM;                              // slice
        const int64_t rc = (isa ? m0 : n0) + e % BM;       // row of A / column of B
        const int64_t ext = isa ? ((int64_t)(L - 1) * p.sas_l + (p.M - 1) * p.sas_m + 1)
                                : ((int64_t)(L - 1) * p.sbs_l + (p.N - 1) * p.sbs_n + 1);
        const bool ok = s < L && rc < (isa ? p.M : p.N);
        const uint32_t vo = ok ? (uint32_t)(((int64_t)s * (isa ? p.sas_l : p.sbs_l) +
                                             rc * (isa ? p.sas_m : p.sbs_n)) * 4)
                               : kOOB;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(isa ? p.sa + bidx * p.sas_b : p.sb + bidx * p.sbs_b), (short)0,
            (int)(ext * 4 < 0x7FFFFFFF ? ext * 4 : 0x7FFFFFFF), 0x00020000);
        auto *ldsp = (__attribute__((address_space(3))) void *)(scl + (isa ? 0 : 1024) +
                                                              (isa ? wave : wave - 4) * 256);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, ldsp, 4, vo, 0, 0, 0);
    };
    const float *sa_lds = (const float *)scl, *sb_lds = (const float *)(scl + 1024);

    // prologue: stage 0 and A(1) (six slots: all of stage 1); stage 0 must
    // land before the first reads
#pragma unroll
    for (int q = 0; q < LPH; ++q) issue_a(0, q);
#pragma unroll
    for (int q = 0; q < LPH; ++q) issue_b(0, q);
    if (nkb > 1) {
#pragma unroll
        for (int q = 0; q < LPH; ++q) issue_a(1, q);
        if constexpr (Sh::NSLOT == 6) {
#pragma unroll
            for (int q = 0; q < LPH; ++q) issue_b(1, q);
            wait_vmcnt<2 * LPH>();
        } else {
            wait_vmcnt<LPH>();
        }
    } else {
        wait_vmcnt<0>();
    }
    exec_barrier();

    const int64_t cbase = bidx * p.cs_b;
    OA *part = (OA *)smem;   // epilogue hand-off [4 blocks][W * W][16][64 lanes]

    auto body = [&](auto G_) {
        constexpr int G = decltype(G_)::value;
        constexpr int F = PS::first(G), NP = PS::count(G), ILO = PS::ilo(G), NA = PS::na(G);
        constexpr int kReads = (NA + L) * W;
        constexpr int NMF = NP * W * W;   // MFMAs per K step
        struct Frags {
            i32x4 a[NA][W];
            i32x4 b[L][W];
        };
        Acc acc[NP][W][W];
#pragma unroll
        for (int q = 0; q < NP; ++q)
#pragma unroll
            for (int x = 0; x < W * W; ++x) acc[q][x / W][x % W] = MF::zero();

        auto read_one = [&](int kb, int kk, int r, Frags &f) {
            const int ch = 2 * kk + h;
            if (r < NA * W) {
                const int i = r / W, x = r % W;
                f.a[i][x] = *(const i32x4 *)(slot(2 * kb) +
                                             rswz<kDmaRB>((ILO + i) * BM + wm * 32 * W + 32 * x + lr, ch));
            } else {
                const int j = (r - NA * W) / W, x = (r - NA * W) % W;
                f.b[j][x] = *(const i32x4 *)(slot(2 * kb + 1) +
                                             rswz<kDmaRB>(j * BN + wn * 32 * W + 32 * x + lr, ch));
            }
        };
        // One K step: the reads of the next K step (stage rkb, step nkk) into
        // `nxt`, issued first, then the MFMAs of `cur` with this step's DMA
        // instructions [lo, hi) of half stage kind (0: none, 1: A, 2: B) of
        // stage dkb spread between them.
        auto step = [&](const Frags &cur, Frags &nxt, int rkb, int nkk, int kind, int dkb, int lo,
                        int hi) {
            const int cnt = hi - lo;
#pragma unroll
            for (int q = 0; q < kReads; ++q) read_one(rkb, nkk, q, nxt);
#pragma unroll
            for (int n = 0; n < NMF; ++n) {
                const int q = n / (W * W), x = (n / W) % W, y = n % W;
                const int i = (F + q) / L, j = (F + q) % L;
                acc[q][x][y] = MF::run(cur.a[i - ILO][x], cur.b[j][y], acc[q][x][y]);
#pragma unroll
                for (int d = 0; d < LPH; ++d) {
                    // instruction lo + d goes after MFMA (d * NMF) / cnt
                    if (d < cnt && (d * NMF) / cnt == n) {
                        if (kind == 1) issue_a(dkb, lo + d);
                        else if (kind == 2) issue_b(dkb, lo + d);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        Frags f0, f1;
        if (nkb > 0) {
#pragma unroll
            for (int q = 0; q < kReads; ++q) read_one(0, 0, q, f0);
        }
        static_assert(STEPS == 4, "four 32-byte K steps per stage");
        if (nkb == 0) issue_scales();
        for (int kb = 0; kb < nkb; ++kb) {
            const bool nb = kb + 1 < nkb, na = kb + 2 < nkb;
            // no DMA is outstanding in the last stage: its waits are unaffected
            if (!nb) issue_scales();
            if constexpr (Sh::NSLOT == 6) {
                // A(kb + 2) and B(kb + 2) take the slots of A(kb - 1) and
                // B(kb - 1), released by the barrier of stage kb - 1
                step(f0, f1, kb, 1, na ? 1 : 0, kb + 2, 0, Sh::A2);
                step(f1, f0, kb, 2, na ? 1 : 0, kb + 2, Sh::A2, LPH);
                step(f0, f1, kb, 3, na ? 2 : 0, kb + 2, 0, Sh::B0);
                if (nb) {
                    // stage kb + 1 has landed once only stage kb + 2's
                    // instructions issued so far may be outstanding
                    if (na) wait_vmcnt<LPH + Sh::B0>();
                    else wait_vmcnt<0>();
                    __builtin_amdgcn_s_waitcnt(0xC07F);
                    exec_barrier();
                }
                step(f1, f0, kb + 1, 0, na ? 2 : 0, kb + 2, Sh::B0, LPH);
            } else {
                step(f0, f1, kb, 1, nb ? 2 : 0, kb + 1, 0, Sh::B0);
                step(f1, f0, kb, 2, nb ? 2 : 0, kb + 1, Sh::B0, LPH);
                step(f0, f1, kb, 3, na ? 1 : 0, kb + 2, 0, Sh::A2);
                if (nb) {
                    // stage kb + 1 has landed once only this wave's first part
                    // of A(kb + 2) may be outstanding; the barrier publishes
                    // every wave's DMA writes, and the lgkmcnt wait makes this
                    // wave's reads of stage kb complete before slots are refilled
                    if (na) wait_vmcnt<Sh::A2>();
                    else wait_vmcnt<0>();
                    __builtin_amdgcn_s_waitcnt(0xC07F);
                    exec_barrier();
                }
                // the last step reads stage kb + 1's step 0 (unused past the end)
                step(f1, f0, kb + 1, 0, na ? 1 : 0, kb + 2, Sh::A2, LPH);
            }
        }

        // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
        // every wave's scale DMA has landed and every wave is past its last
        // ring read
        wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);
        exec_barrier();
        if (S > 1) {
            // split-K: the ranges' accumulators into the last range's
            // registers (the flag word sits in a ring slot no stage used)
            constexpr int RW = (PS::count(0) > PS::count(1) ? PS::count(0) : PS::count(1)) * W * W * 16;
            const int ln = lane_here();
            uint32_t *mine = splitk_slot(p, g, krange, wave, RW, ln);
#pragma unroll
            for (int q = 0; q < NP; ++q)
#pragma unroll
                for (int x = 0; x < W * W; ++x) {
                    const i32x16 u = __builtin_bit_cast(i32x16, acc[q][x / W][x % W]);
#pragma unroll
                    for (int r = 0; r < 16; ++r) splitk_put(mine + ((q * W * W + x) * 16 + r) * 64, (uint32_t)u[r]);
                }
            if (!splitk_arrive(p, g, (int *)slot(2 * nkb + 1))) return;
            if constexpr (MF::kExactAcc) {
                // int32 sums are exact in any order: this range's
                // accumulators stay, the other ranges are added
                for (int s2 = 0; s2 < S; ++s2) {
                    if (s2 == krange) continue;
                    const uint32_t *src = splitk_slot(p, g, s2, wave, RW, ln);
#pragma unroll
                    for (int q = 0; q < NP; ++q)
#pragma unroll
                        for (int x = 0; x < W * W; ++x)
                            acc[q][x / W][x % W] += splitk_get16<Acc>(src + (q * W * W + x) * 16 * 64);
                }
            } else {
            // every range read back in range order: range 0 straight into
            // the accumulators, then the others added one tile at a time
            {
                const uint32_t *src = splitk_slot(p, g, 0, wave, RW, ln);
#pragma unroll
                for (int q = 0; q < NP; ++q)
#pragma unroll
                    for (int x = 0; x < W * W; ++x)
                        acc[q][x / W][x % W] = splitk_get16<Acc>(src + (q * W * W + x) * 16 * 64);
            }
            for (int s2 = 1; s2 < S; ++s2) {
                const uint32_t *src = splitk_slot(p, g, s2, wave, RW, ln);
#pragma unroll
                for (int q = 0; q < NP; ++q)
#pragma unroll
                    for (int x = 0; x < W * W; ++x)
                        acc[q][x / W][x % W] += splitk_get16<Acc>(src + (q * W * W + x) * 16 * 64);
            }
            }
        }
        // this wave's scales into registers: sa of its rows, sb of its columns
        float sbv[W][L], sav[W][16][NA];
#pragma unroll
        for (int y = 0; y < W; ++y) {
            const int ct = wn * 32 * W + 32 * y + lr;
#pragma unroll
            for (int j = 0; j < L; ++j) sbv[y][j] = sb_lds[j * BN + ct];
        }
#pragma unroll
        for (int x = 0; x < W; ++x)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rt = wm * 32 * W + 32 * x + 8 * (r >> 2) + 4 * h + (r & 3);
#pragma unroll
                for (int i = 0; i < NA; ++i) sav[x][r][i] = sa_lds[(ILO + i) * BM + rt];
            }
        // t value of pair q, block (x, y), accumulator row r:
        // fl32(fl32(fl32(acc) * sa_i) * sb_j)
        auto tval = [&](int q, int x, int y, int r) {
            const int i = (F + q) / L, j = (F + q) % L;
            const float t1 = MF::to_f32(acc[q][x][y][r]) * sav[x][r][i - ILO];
            return t1 * sbv[y][j];
        };
        // the partial sums overwrite the scales: every wave has read them
        __builtin_amdgcn_s_waitcnt(0xC07F);
        exec_barrier();
        if constexpr (G == 0) {
#pragma unroll
            for (int x = 0; x < W; ++x)
#pragma unroll
                for (int y = 0; y < W; ++y)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        OA out = (OA)0;
#pragma unroll
                        for (int q = 0; q < NP; ++q) out = out + (OA)tval(q, x, y, r);
                        part[(((blk * W + x) * W + y) * 16 + r) * 64 + lane] = out;
                    }
            __builtin_amdgcn_s_waitcnt(0xC07F);
            exec_barrier();
        } else {
            exec_barrier();
#pragma unroll
            for (int x = 0; x < W; ++x)
#pragma unroll
                for (int y = 0; y < W; ++y) {
                    const int64_t col = n0 + wn * 32 * W + 32 * y + lr;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t row = m0 + wm * 32 * W + 32 * x + 8 * (r >> 2) + 4 * h + (r & 3);
                        OA out = part[(((blk * W + x) * W + y) * 16 + r) * 64 + lane];
#pragma unroll
                        for (int q = 0; q < NP; ++q) out = out + (OA)tval(q, x, y, r);
                        if (col < p.N && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, out);
                    }
                }
        }
    };
    if (grp == 0) body(std::integral_constant<int, 0>{});
    else body(std::integral_constant<int, 1>{});
}

// ---------------------------------------------------------------------------
// Wide kernel for num_splits 3: 64 x 128 tiles, 8 waves in a 2 x 4 grid of
// 32 x 32 blocks, each wave holding all 9 slice pairs of its block (144
// accumulator registers).  Per 32-byte K step a wave reads 3 A and 3 B
// fragments for 9 MFMAs (the ring kernel's wave groups read 9 fragments for
// the 9 MFMAs of two waves), and a stage of 128 bytes of K (24 KB of A rows,
// 48 KB of B rows) feeds 288 MFMAs (the ring kernel's 48 KB: 144).  Each wave
// sums its own pairs in the reference's i-major / j-minor order, so the
// epilogue hands nothing between waves.
// The LDS holds two whole stages (144 KB; the A and B halves differ in size,
// so they do not form a ring of equal slots).  Stage kb + 2 is fetched into
// stage kb's buffer, released by the barrier of stage kb: P1 instructions per
// wave in the K step after that barrier, the rest in the next K step, and the
// barrier of stage kb + 1 waits for all of them.
// ---------------------------------------------------------------------------
struct WideShape {
    static constexpr int L = 3;
    static constexpr int NW = 8;                         // waves
    static constexpr int BM = 64, BN = 128;
    static constexpr int A_BYTES = L * BM * kDmaRB;      // 24 KB
    static constexpr int B_BYTES = L * BN * kDmaRB;      // 48 KB
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int LA = A_BYTES / (NW * 1024);     // A instructions per wave per stage
    static constexpr int LB = B_BYTES / (NW * 1024);     // B instructions per wave per stage
    static constexpr int LPS = LA + LB;
    static constexpr int P1 = 5;                         // issued in the K step after the barrier
    static constexpr int LDS_BYTES = 2 * STAGE;
    static_assert(A_BYTES % (NW * 1024) == 0 && B_BYTES % (NW * 1024) == 0,
                  "a half stage must be whole 1 KB windows per wave");
    static_assert(P1 >= LPS - P1 && P1 <= LPS, "the larger part goes first");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
    static_assert(L * (BM + BN) * 4 <= STAGE, "the tile's scales fit a stage buffer");
    static_assert(kDmaRB == 128, "128-byte stage rows");
};

template <typename ST, typename AccT, bool TRI>
__global__ __launch_bounds__(512, 1) void cross_gemm_wide_kernel(GemmParams p, int group_m,
                                                                 uint32_t a_records,
                                                                 uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = WideShape;
    using MF = Mfma<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;
    constexpr int L = Sh::L, BM = Sh::BM, BN = Sh::BN;
    using PS = Pairs<L, TRI>;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const int h = lane >> 5, lr = lane & 31;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    // split-K: workgroup g0 is K range g0 % S of tile g0 / S
    const int S = p.ksplit > 1 ? p.ksplit : 1;
    const int64_t g0 = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int krange = (int)(g0 % S);
    const int64_t g = g0 / S;
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb_all = (int)((kbytes + kDmaRB - 1) / kDmaRB);
    const int kb0 = S > 1 ? krange * p.kb_per_split : 0;   // this range's first stage
    const int nkb = S > 1 ? min(p.kb_per_split, nkb_all - kb0) : nkb_all;
    const uint32_t kbyte0 = (uint32_t)kb0 * kDmaRB;

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // This wave's LPS DMA instructions of a stage: q < LA fetch window
    // wave * LA + q of the A half, the others window wave * LB + q - LA of the
    // B half (a 1 KB window is 8 whole 128-byte rows; lane -> row lane / 8,
    // physical chunk lane % 8, which holds logical chunk pc ^ ((r >> 1) & 7);
    // with r = 8 window + lane / 8 that is c0, or c0 ^ 4 in an odd window).
    auto window = [&](int q) { return q < Sh::LA ? wave * Sh::LA + q : wave * Sh::LB + q - Sh::LA; };
    const int c0 = (lane & 7) ^ (lane >> 4);
    uint32_t src[Sh::LPS];
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) {
        const int r = window(q) * 8 + lane / 8;
        if (q < Sh::LA) {
            const int64_t m = m0 + r % BM;
            src[q] = (m < p.M) ? (uint32_t)(((int64_t)(r / BM) * p.as_l + m * p.as_m) * ES) : kOOB;
        } else {
            const int64_t n = n0 + r % BN;
            src[q] = (n < p.N) ? (uint32_t)(((int64_t)(r / BN) * p.bs_l + n * p.bs_n) * ES) : kOOB;
        }
    }
    auto buf = [&](int kb) { return smem + (kb & 1) * Sh::STAGE; };
    auto issue = [&](int kb, int q) {
        const int ch = c0 ^ ((window(q) & 1) << 2);
        const uint32_t kofs = kbyte0 + (uint32_t)kb * kDmaRB + ch * 16;
        const uint32_t vo = (src[q] == kOOB || kofs >= kbytes) ? kOOB : src[q] + kofs;
        auto *ldsp = (__attribute__((address_space(3))) void *)(
            buf(kb) + (q < Sh::LA ? 0 : Sh::A_BYTES) + window(q) * 1024);
        if (q < Sh::LA) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, vo, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, vo, 0, 0, 0);
    };

    // The tile's scales (A's [L][BM], then B's [L][BN]: 2304 bytes) are
    // fetched by dword DMA into the buffer of stage nkb, which holds no stage
    // the tile still reads, at the start of the last stage: instruction
    // u < 9 (wave u and wave u - 8) fetches entries 64 u .. 64 u + 63, the
    // first 3 of A's scales, the next 6 of B's.
    char *const scl = buf(nkb);
    auto issue_scales = [&]() {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int u = q * Sh::NW + wave;
            if (u >= L * (BM + BN) / 64) break;
            const bool isa = u < L * BM / 64;
            const int e = (isa ? u : u - L * BM / 64) * 64 + lane;
            const int s = isa ? e / BM : e / BN;                 // slice
            const int64_t rc = isa ? m0 + e % BM : n0 + e % BN;  // row of A / column of B
            const int64_t ext = isa ? ((int64_t)(L - 1) * p.sas_l + (p.M - 1) * p.sas_m + 1)
                                    : ((int64_t)(L - 1) * p.sbs_l + (p.N - 1) * p.sbs_n + 1);
            const bool ok = rc < (isa ? p.M : p.N);
            const uint32_t vo = ok ? (uint32_t)(((int64_t)s * (isa ? p.sas_l : p.sbs_l) +
                                                 rc * (isa ? p.sas_m : p.sbs_n)) * 4)
                                   : kOOB;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(isa ? p.sa + bidx * p.sas_b : p.sb + bidx * p.sbs_b), (short)0,
                (int)(ext * 4 < 0x7FFFFFFF ? ext * 4 : 0x7FFFFFFF), 0x00020000);
            auto *ldsp = (__attribute__((address_space(3))) void *)(scl + u * 256);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, ldsp, 4, vo, 0, 0, 0);
        }
    };
    const float *sa_lds = (const float *)scl, *sb_lds = (const float *)(scl + L * BM * 4);

    // prologue: stages 0 and 1; stage 0 must land before the first reads
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) issue(0, q);
    if (nkb > 1) {
#pragma unroll
        for (int q = 0; q < Sh::LPS; ++q) issue(1, q);
        wait_vmcnt<Sh::LPS>();
    } else {
        wait_vmcnt<0>();
    }
    exec_barrier();

    struct Frags {
        i32x4 a[L];
        i32x4 b[L];
    };
    Acc acc[L][L];
#pragma unroll
    for (int i = 0; i < L; ++i)
#pragma unroll
        for (int j = 0; j < L; ++j) acc[i][j] = MF::zero();

    auto read_one = [&](int kb, int kk, int r, Frags &f) {
        const int c = 2 * kk + h;
        if (r < L) f.a[r] = *(const i32x4 *)(buf(kb) + rswz<kDmaRB>(r * BM + wm * 32 + lr, c));
        else
            f.b[r - L] = *(const i32x4 *)(buf(kb) + Sh::A_BYTES +
                                          rswz<kDmaRB>((r - L) * BN + wn * 32 + lr, c));
    };
    // One K step: the reads of the next K step (stage rkb, step nkk) into
    // `nxt`, issued first, then the 9 MFMAs of `cur` with, if `on`, DMA
    // instructions [lo, hi) of stage dkb spread between them (lo and hi are
    // constants at every call, so the spread folds at compile time).
    auto step = [&](const Frags &cur, Frags &nxt, int rkb, int nkk, int dkb, bool on, int lo,
                    int hi) {
        const int cnt = hi - lo;
#pragma unroll
        for (int q = 0; q < 2 * L; ++q) read_one(rkb, nkk, q, nxt);
        constexpr int NMF = PS::N;
        static_for<NMF>([&](auto n_) {
            constexpr int n = decltype(n_)::value;
            constexpr int i = PS::i_of(n), j = PS::j_of(n);
            acc[i][j] = MF::run(cur.a[i], cur.b[j], acc[i][j]);
#pragma unroll
            for (int d = 0; d < Sh::P1; ++d) {
                // instruction lo + d goes after MFMA (d * NMF) / cnt
                if (d < cnt && (d * NMF) / cnt == n && on) issue(dkb, lo + d);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    Frags f0, f1;
    if (nkb > 0) {
#pragma unroll
        for (int q = 0; q < 2 * L; ++q) read_one(0, 0, q, f0);
    }
    static_assert(kDmaRB / 32 == 4, "four 32-byte K steps per stage");
    if (nkb == 0) issue_scales();
    for (int kb = 0; kb < nkb; ++kb) {
        const bool nb = kb + 1 < nkb, n2 = kb + 2 < nkb;
        // no DMA is outstanding in the last stage: its waits are unaffected
        if (!nb) issue_scales();
        // the rest of stage kb + 1 (stage 1 went out whole in the prologue)
        step(f0, f1, kb, 1, kb + 1, nb && kb >= 1, Sh::P1, Sh::LPS);
        step(f1, f0, kb, 2, kb + 1, false, 0, 0);
        step(f0, f1, kb, 3, kb + 1, false, 0, 0);
        if (nb) {
            // stage kb + 1 is the only DMA outstanding; the barrier publishes
            // every wave's DMA writes, and the lgkmcnt wait makes this wave's
            // reads of stage kb complete before its buffer is refilled
            wait_vmcnt<0>();
            __builtin_amdgcn_s_waitcnt(0xC07F);
            exec_barrier();
        }
        // the last step reads stage kb + 1's step 0 (unused past the end)
        step(f1, f0, kb + 1, 0, kb + 2, n2, 0, Sh::P1);
    }

    // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    exec_barrier();
    if (S > 1) {
        // split-K: the ranges' accumulators into the last range's registers
        // (the flag word sits in the stage buffer the scales did not use)
        constexpr int RW = L * L * 16;
        const int ln = lane_here();
        uint32_t *mine = splitk_slot(p, g, krange, wave, RW, ln);
#pragma unroll
        for (int n = 0; n < L * L; ++n) {
            if (!PS::kept(n / L, n % L)) continue;
            const i32x16 u = __builtin_bit_cast(i32x16, acc[n / L][n % L]);
#pragma unroll
            for (int r = 0; r < 16; ++r) splitk_put(mine + (n * 16 + r) * 64, (uint32_t)u[r]);
        }
        if (!splitk_arrive(p, g, (int *)buf(nkb + 1))) return;
        if constexpr (MF::kExactAcc) {
            // int32 sums are exact in any order: this range's accumulators
            // stay, the other ranges are added one tile (16 loads in
            // flight) at a time
            for (int s2 = 0; s2 < S; ++s2) {
                if (s2 == krange) continue;
                const uint32_t *src = splitk_slot(p, g, s2, wave, RW, ln);
#pragma unroll
                for (int n = 0; n < L * L; ++n)
                    if (PS::kept(n / L, n % L)) acc[n / L][n % L] += splitk_get16<Acc>(src + n * 16 * 64);
            }
        } else {
            // every range read back, this one's too, in range order: range
            // 0 straight into the accumulators, then the others added
            {
                const uint32_t *src = splitk_slot(p, g, 0, wave, RW, ln);
#pragma unroll
                for (int n = 0; n < L * L; ++n)
                    if (PS::kept(n / L, n % L)) acc[n / L][n % L] = splitk_get16<Acc>(src + n * 16 * 64);
            }
            for (int s2 = 1; s2 < S; ++s2) {
                const uint32_t *src = splitk_slot(p, g, s2, wave, RW, ln);
#pragma unroll
                for (int n = 0; n < L * L; ++n)
                    if (PS::kept(n / L, n % L)) acc[n / L][n % L] += splitk_get16<Acc>(src + n * 16 * 64);
            }
        }
    }
    const int ct = wn * 32 + lr;
    const int64_t col = n0 + ct;
    const int64_t cbase = bidx * p.cs_b;
    float sbv[L];
#pragma unroll
    for (int j = 0; j < L; ++j) sbv[j] = sb_lds[j * BN + ct];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int rt = wm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        const int64_t row = m0 + rt;
        OA out = (OA)0;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const float sai = sa_lds[i * BM + rt];
#pragma unroll
            for (int j = 0; j < L; ++j) {
                if (!PS::kept(i, j)) continue;
                // fl32(fl32(fl32(acc) * sa_i) * sb_j), summed i-major, j-minor
                const float t1 = MF::to_f32(acc[i][j][r]) * sai;
                out = out + (OA)(t1 * sbv[j]);
            }
        }
        if (col < p.N && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, out);
    }
}

// ---------------------------------------------------------------------------
// Wide kernel for num_splits 4: 96 x 64 tiles (row blocks x = 0..2, column
// blocks y = 0..1 of 32 x 32), 8 waves of 12 accumulator tiles each, so that
// every wave reads 3 A and 4 B fragments per 32-byte K step for 12 MFMAs
// (0.58 fragment reads per MFMA; the ring kernel's 64 x 64 tiles: 0.75) and a
// stage of 128 bytes of K (48 KB of A rows, 32 KB of B rows) feeds 384 MFMAs
// (0.21 KB of DMA per MFMA; ring: 0.25).
//   * waves 0..5 (x = wave / 2, y = wave % 2) hold the pairs i = 0..2, j = 0..3
//     of block (x, y): A fragments (slice u, rows of x), u = 0..2;
//   * waves 6, 7 (y = wave - 6) hold the pairs i = 3, j = 0..3 of the blocks
//     (0..2, y): A fragments (slice 3, rows of block u), u = 0..2;
//   * every wave: B fragments (slice j, columns of y), j = 0..3, and
//     acc[u][j] += A_u . B_j.
// The reference's sum runs i-major, so the i = 3 pairs come last: a wave of
// the first kind sums its 12 pairs in order from +0 and hands the partial to
// the wave of its y through the LDS, which adds its 4 pairs in order and
// stores C.  The second kind converts its accumulators to the fp32 t values
// before the hand-off barrier, so only the additions follow it.
// 12 accumulator tiles are 192 registers of the 256 a wave has at two waves
// per SIMD, so only the A fragments are double-buffered: the B fragments of
// the next K step are read one by one as the MFMAs of the current step
// release them (j-outer order), 9 MFMAs before their first use.
// The LDS holds two whole stages (160 KB); stage kb + 2 is fetched into stage
// kb's buffer after the barrier of stage kb, P1 instructions per wave in the
// K step after that barrier and the rest in the next.
// With the triangular pair set (TRI: i + j <= 3) a wave of the first kind
// keeps 9 of its 12 pairs and one of the second kind the pair (3, 0) of its 3
// blocks; the others' MFMAs and terms are left out (a wave-uniform branch on
// the wave's kind where the two kinds differ).
// ---------------------------------------------------------------------------
struct Wide4Shape {
    static constexpr int L = 4;
    static constexpr int NW = 8;                         // waves
    static constexpr int BM = 96, BN = 64;
    static constexpr int A_BYTES = L * BM * kDmaRB;      // 48 KB
    static constexpr int B_BYTES = L * BN * kDmaRB;      // 32 KB
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int LA = A_BYTES / (NW * 1024);     // A instructions per wave per stage
    static constexpr int LB = B_BYTES / (NW * 1024);     // B instructions per wave per stage
    static constexpr int LPS = LA + LB;
    static constexpr int P1 = 6;                         // issued in the K step after the barrier
    static constexpr int LDS_BYTES = 2 * STAGE;
    static constexpr int NSC = L * (BM + BN) / 64;       // scale instructions (64 entries each)
    static_assert(A_BYTES % (NW * 1024) == 0 && B_BYTES % (NW * 1024) == 0,
                  "a half stage must be whole 1 KB windows per wave");
    static_assert(P1 >= LPS - P1 && P1 <= LPS, "the larger part goes first");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
    static_assert(NSC <= 2 * NW, "two scale instructions per wave at most");
    static_assert(kDmaRB == 128, "128-byte stage rows");
};

template <typename ST, typename AccT, bool TRI>
__global__ __launch_bounds__(512, 1) void cross_gemm_wide4_kernel(GemmParams p, int group_m,
                                                                  uint32_t a_records,
                                                                  uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = Wide4Shape;
    using MF = Mfma<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;
    constexpr int L = Sh::L, BM = Sh::BM, BN = Sh::BN;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool last_i = wave >= 6;                 // holds the pairs i = 3
    const int wy = last_i ? wave - 6 : (wave & 1);
    const int wx = last_i ? 0 : (wave >> 1);
    // A fragment u: LDS row a_row0 + u * a_rstep (+ lane row)
    const int a_row0 = last_i ? 3 * BM : wx * 32;
    const int a_rstep = last_i ? 32 : BM;
    const int h = lane >> 5, lr = lane & 31;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    const int64_t g = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb = (int)((kbytes + kDmaRB - 1) / kDmaRB);

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // This wave's LPS DMA instructions of a stage: q < LA fetch window
    // wave * LA + q of the A half, the others window wave * LB + q - LA of the
    // B half (a 1 KB window is 8 whole 128-byte rows; lane -> row lane / 8,
    // physical chunk lane % 8, which holds logical chunk pc ^ ((r >> 1) & 7);
    // with r = 8 window + lane / 8 that is c0, or c0 ^ 4 in an odd window).
    // A window (8 rows) never straddles a slice (96 or 64 rows = 12 or 8
    // windows), so an instruction's source offset is a wave-uniform part (slice,
    // first row of the window, K block) plus one of four per-lane parts (lane
    // row lane / 8 and chunk, for A or B and even or odd windows).  The uniform
    // part goes through readfirstlane at each use, so the compiler keeps just
    // the four lane parts in registers instead of one sum per instruction.
    auto window = [&](int q) { return q < Sh::LA ? wave * Sh::LA + q : wave * Sh::LB + q - Sh::LA; };
    const int lrow = lane >> 3;
    const int c0 = (lane & 7) ^ (lane >> 4);
    const uint32_t ch16[2] = {(uint32_t)c0 * 16, (uint32_t)(c0 ^ 4) * 16};
    const uint32_t a_lp[2] = {(uint32_t)(lrow * p.as_m * ES) + ch16[0],
                              (uint32_t)(lrow * p.as_m * ES) + ch16[1]};
    const uint32_t b_lp[2] = {(uint32_t)(lrow * p.bs_n * ES) + ch16[0],
                              (uint32_t)(lrow * p.bs_n * ES) + ch16[1]};
    auto buf = [&](int kb) { return smem + (kb & 1) * Sh::STAGE; };
    auto issue = [&](int kb, int q) {
        const int w = window(q);
        const int par = w & 1;
        int64_t first, rows;
        int64_t ubase;
        if (q < Sh::LA) {
            first = m0 + (w % (BM / 8)) * 8;
            rows = p.M;
            ubase = ((int64_t)(w / (BM / 8)) * p.as_l + first * p.as_m) * ES;
        } else {
            first = n0 + (w % (BN / 8)) * 8;
            rows = p.N;
            ubase = ((int64_t)(w / (BN / 8)) * p.bs_l + first * p.bs_n) * ES;
        }
        const int rows_left = (int)(rows - first < 8 ? rows - first : 8);   // may be <= 0
        const int kleft = (int)kbytes - kb * kDmaRB;                       // > 0
        const uint32_t ub = (uint32_t)__builtin_amdgcn_readfirstlane((int)(ubase + kb * kDmaRB));
        const bool ok = lrow < rows_left && (int)ch16[par] < kleft;
        const uint32_t vo = ok ? (q < Sh::LA ? a_lp[par] : b_lp[par]) + ub : kOOB;
        auto *ldsp = (__attribute__((address_space(3))) void *)(
            buf(kb) + (q < Sh::LA ? 0 : Sh::A_BYTES) + w * 1024);
        if (q < Sh::LA) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, vo, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, vo, 0, 0, 0);
    };

    // The tile's scales (A's [L][BM], then B's [L][BN]: 2560 bytes) are
    // fetched by dword DMA into the buffer of stage nkb, which holds no stage
    // the tile still reads, at the start of the last stage: instruction
    // u < NSC (wave u and wave u - 8) fetches entries 64 u .. 64 u + 63.
    // The lane is read where the scales are fetched (lane_here), so that
    // their offsets are not computed before the K loop and held through it.
    char *const scl = buf(nkb);
    auto issue_scales = [&]() {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int u = q * Sh::NW + wave;
            if (u >= Sh::NSC) break;
            const bool isa = u < L * BM / 64;
            const int e = (isa ? u : u - L * BM / 64) * 64 + lane_here();
            const int s = isa ? e / BM : e / BN;                 // slice
            const int64_t rc = isa ? m0 + e % BM : n0 + e % BN;  // row of A / column of B
            const int64_t ext = isa ? ((int64_t)(L - 1) * p.sas_l + (p.M - 1) * p.sas_m + 1)
                                    : ((int64_t)(L - 1) * p.sbs_l + (p.N - 1) * p.sbs_n + 1);
            const bool ok = rc < (isa ? p.M : p.N);
            const uint32_t vo = ok ? (uint32_t)(((int64_t)s * (isa ? p.sas_l : p.sbs_l) +
                                                 rc * (isa ? p.sas_m : p.sbs_n)) * 4)
                                   : kOOB;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(isa ? p.sa + bidx * p.sas_b : p.sb + bidx * p.sbs_b), (short)0,
                (int)(ext * 4 < 0x7FFFFFFF ? ext * 4 : 0x7FFFFFFF), 0x00020000);
            auto *ldsp = (__attribute__((address_space(3))) void *)(scl + u * 256);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, ldsp, 4, vo, 0, 0, 0);
        }
    };
    const float *sa_lds = (const float *)scl, *sb_lds = (const float *)(scl + L * BM * 4);

    // prologue: stages 0 and 1; stage 0 must land before the first reads
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) issue(0, q);
    if (nkb > 1) {
#pragma unroll
        for (int q = 0; q < Sh::LPS; ++q) issue(1, q);
        wait_vmcnt<Sh::LPS>();
    } else {
        wait_vmcnt<0>();
    }
    exec_barrier();

    struct FragsA {
        i32x4 a[3];
    };
    i32x4 fb[L];   // B fragments, single-buffered
    Acc acc[3][L];
#pragma unroll
    for (int u = 0; u < 3; ++u)
#pragma unroll
        for (int j = 0; j < L; ++j) acc[u][j] = MF::zero();

    // Fragment rows start at multiples of 32, so the swizzle key of a lane's
    // row, ((row >> 1) & 7), is that of lr for every fragment: the address is
    // a wave-uniform row offset plus one of four per-lane offsets (one per
    // K step of a stage), rswz<kDmaRB> with its terms regrouped.
    // The uniform part (buffer, first row) goes through readfirstlane at each
    // use, so only the four per-lane offsets stay in registers.
    const int key = (lr >> 1) & 7;
    int lane_rd[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) lane_rd[kk] = lr * kDmaRB + (((2 * kk + h) ^ key) << 4);
    const int smem_base = (int)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
    auto lds_at = [&](int uniform, int kk) {
        const int u = __builtin_amdgcn_readfirstlane(uniform);
        return (const __attribute__((address_space(3))) i32x4 *)(uintptr_t)(u + lane_rd[kk]);
    };
    auto read_a = [&](int kb, int kk, int u, FragsA &f) {
        f.a[u] = *lds_at(smem_base + (kb & 1) * Sh::STAGE + (a_row0 + u * a_rstep) * kDmaRB, kk);
    };
    auto read_b = [&](int kb, int kk, int j) {
        fb[j] = *lds_at(smem_base + (kb & 1) * Sh::STAGE + Sh::A_BYTES + (j * BN + wy * 32) * kDmaRB, kk);
    };
    // One K step: the A reads of the next K step (stage rkb, step nkk) into
    // `nxt`, issued first; then the 12 MFMAs of `cur` and the current B
    // fragments, j-outer, each B fragment re-read for the next step after its
    // last MFMA; with, if `on`, DMA instructions [lo, hi) of stage dkb spread
    // between them (lo and hi are constants at every call, so the spread
    // folds at compile time).
    auto step = [&](const FragsA &cur, FragsA &nxt, int rkb, int nkk, int dkb, bool on, int lo,
                    int hi) {
        const int cnt = hi - lo;
#pragma unroll
        for (int u = 0; u < 3; ++u) read_a(rkb, nkk, u, nxt);
#pragma unroll
        for (int n = 0; n < 3 * L; ++n) {
            const int j = n / 3, u = n % 3;
            // the pair (u, j) in a wave of the first kind, (3, j) in one of the second
            const bool first = !TRI || u + j <= L - 1, second = !TRI || j == 0;
            if (first && second) acc[u][j] = MF::run(cur.a[u], fb[j], acc[u][j]);
            else if (first || second) {
                if (first != last_i) acc[u][j] = MF::run(cur.a[u], fb[j], acc[u][j]);
            }
            if (u == 2) read_b(rkb, nkk, j);
#pragma unroll
            for (int d = 0; d < Sh::P1; ++d) {
                // instruction lo + d goes after MFMA (d * 12) / cnt
                if (d < cnt && (d * 3 * L) / cnt == n && on) issue(dkb, lo + d);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    FragsA f0, f1;
    if (nkb > 0) {
#pragma unroll
        for (int u = 0; u < 3; ++u) read_a(0, 0, u, f0);
#pragma unroll
        for (int j = 0; j < L; ++j) read_b(0, 0, j);
    }
    static_assert(kDmaRB / 32 == 4, "four 32-byte K steps per stage");
    if (nkb == 0) issue_scales();
    for (int kb = 0; kb < nkb; ++kb) {
        const bool nb = kb + 1 < nkb, n2 = kb + 2 < nkb;
        // no DMA is outstanding in the last stage: its waits are unaffected
        if (!nb) issue_scales();
        // the rest of stage kb + 1 (stage 1 went out whole in the prologue)
        step(f0, f1, kb, 1, kb + 1, nb && kb >= 1, Sh::P1, Sh::LPS);
        step(f1, f0, kb, 2, kb + 1, false, 0, 0);
        step(f0, f1, kb, 3, kb + 1, false, 0, 0);
        if (nb) {
            // stage kb + 1 is the only DMA outstanding; the barrier publishes
            // every wave's DMA writes, and the lgkmcnt wait makes this wave's
            // reads of stage kb complete before its buffer is refilled
            wait_vmcnt<0>();
            __builtin_amdgcn_s_waitcnt(0xC07F);
            exec_barrier();
        }
        // the last step reads stage kb + 1's step 0 (unused past the end)
        step(f1, f0, kb + 1, 0, kb + 2, n2, 0, Sh::P1);
    }

    // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    exec_barrier();
    // the epilogue's lane values are read afresh (lane_here), so that none is
    // held through the K loop, where the registers are all taken and such
    // values were spilled to scratch
    const int elane = lane_here();
    const int eh = elane >> 5;
    const int ct = wy * 32 + (elane & 31);
    const int64_t col = n0 + ct;
    const int64_t cbase = bidx * p.cs_b;
    float sbv[L];
#pragma unroll
    for (int j = 0; j < L; ++j) sbv[j] = sb_lds[j * BN + ct];
    // rows of accumulator registers 4 q .. 4 q + 3 of A fragment u, inside the
    // tile, start at row4(u, q): their 4 scales are one 16-byte LDS read
    auto row4 = [&](int u, int q) { return (last_i ? u * 32 : wx * 32) + 8 * q + 4 * eh; };
    auto sa4 = [&](int i, int u, int q) {
        return *(const f32x4 *)(sa_lds + i * BM + row4(u, q));
    };
    // the i = 3 waves: t values fl32(fl32(fl32(acc) * sa_3) * sb_j) in place
    // of their accumulators, before the hand-off (one block at a time, each
    // behind a scheduling barrier: the scale reads are not hoisted).  The
    // accumulator vectors are bit-cast whole: with this compiler a bit-cast of
    // single elements of a vector reads element 0.
    if (last_i) {
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            f32x4 s4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) s4[q] = sa4(3, u, q);
#pragma unroll
            for (int j = 0; j < (TRI ? 1 : L); ++j) {
                f32x16 tv;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    tv[r] = (MF::to_f32(acc[u][j][r]) * s4[r >> 2][r & 3]) * sbv[j];
                acc[u][j] = __builtin_bit_cast(Acc, tv);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // the partial sums go to the buffer of the last stage, which every wave
    // has finished reading (the scales sit in the other one)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    exec_barrier();
    OA *part = (OA *)buf(nkb + 1);   // [6 blocks][16][64 lanes]
    static_assert(6 * 16 * 64 * sizeof(OA) <= Sh::STAGE, "the partials fit a stage buffer");
    if (!last_i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            f32x4 s4[3];
#pragma unroll
            for (int i = 0; i < 3; ++i) s4[i] = sa4(i, 0, q);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * q + e;
                OA out = (OA)0;
#pragma unroll
                for (int i = 0; i < 3; ++i)
#pragma unroll
                    for (int j = 0; j < L; ++j) {
                        if (TRI && i + j > L - 1) continue;
                        // fl32(fl32(fl32(acc) * sa_i) * sb_j), summed i-major, j-minor
                        const float t1 = MF::to_f32(acc[i][j][r]) * s4[i][e];
                        out = out + (OA)(t1 * sbv[j]);
                    }
                part[(wave * 16 + r) * 64 + elane] = out;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        exec_barrier();
    } else {
        exec_barrier();
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            f32x16 tv[L];
#pragma unroll
            for (int j = 0; j < L; ++j) tv[j] = __builtin_bit_cast(f32x16, acc[u][j]);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + row4(u, r >> 2) + (r & 3);
                OA out = part[((u * 2 + wy) * 16 + r) * 64 + elane];
#pragma unroll
                for (int j = 0; j < (TRI ? 1 : L); ++j) out = out + (OA)tv[j][r];
                if (col < p.N && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, out);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// The num_splits 4 wide kernel on 16 x 16 x 64 MFMAs (int8 slices:
// v_mfma_i32_16x16x64_i8).  At the chip's power limit the rate is set by the
// energy of each MFMA's operands, and one 16 x 16 x 64 instruction moves a
// quarter of the accumulator registers of a 32 x 32 x 32 one for half its
// work: on random int8 data with wide4's LDS reads and DMA per MFMA, a probe
// of the two streams ran 0.58 against 0.53 of the dense peak.
// Tile, waves, pair assignment, LDS stages and DMA are wide4's.  A K step is
// 64 bytes (two per 128-byte stage).  Lane l of a fragment reads row l % 16 of
// 16 rows, bytes 16 (l / 16) .. + 15 of the step; the instruction pairs the
// same bytes of A and B, so the int32 dot products are wide4's exactly.  A
// wave's 12 accumulator tiles of 32 x 32 become 48 of 16 x 16,
// acc[u][j][rh][ch] (row half rh, column half ch of its 32 x 32 blocks), whose
// register e of lane l holds row 16 rh + 4 (l / 16) + e, column 16 ch + l % 16.
// Per K step a wave reads 6 A fragments p = (u, rh) and 8 B fragments g =
// (j, ch) and runs 48 MFMAs, B-outer: the A fragments stay in registers and
// each is re-read for the next step right after its last MFMA (6 MFMAs before
// its next use); B fragment g + 1 is read while g's 6 MFMAs run.  So the
// step's own B fragments come from the LDS during the step, and the stage
// barrier sits before the last B fragment's group of the stage's second step:
// every wave has then read the stage, whose buffer the DMA of stage kb + 2
// refills from that group on, and stage kb + 1 has landed for the next step's
// reads.  Registers: 192 accumulators, 24 for A, 8 for B (wide4: 192, 24, 16).
// ---------------------------------------------------------------------------
// At two waves per SIMD a wave has 256 registers, which the compiler splits
// into 128 VGPRs and 128 AGPRs once AGPRs are used; left to itself it keeps
// all 192 accumulator registers in VGPRs beside the fragments, and the K loop
// spills.  So the MFMAs are placed by hand: the accumulators of u = 1, 2 (128
// registers) in the AGPRs, those of u = 0 (64) in VGPRs, which the epilogue
// reads first.  Hazards the
// compiler's recogniser cannot see into the inline assembly: an accumulator
// is first read as srcC after its zero fill and 8 wait states, accumulated
// again only 48 MFMAs later, and read by other instructions only in the
// epilogue, after 64 wait states.  The fragment registers an MFMA reads as
// srcA / srcB may be rewritten by the next LDS read right after it (srcA /
// srcB are read as the instruction issues).
template <typename ST> struct Mfma16;
template <> struct Mfma16<int8_t> {
    using Acc = i32x4;
    static constexpr bool kExactAcc = true;    // int32 sums: exact in any order
    OZK_DEV static Acc zero() { return Acc{0}; }
    template <bool AG> OZK_DEV static void run(Acc &c, i32x4 a, i32x4 b) {
        if constexpr (AG) asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
        else asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    }
    // the compiler's own form (it places the accumulator and sees the hazards)
    OZK_DEV static Acc mfma(i32x4 a, i32x4 b, Acc c) {
        return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
    }
    OZK_DEV static float to_f32(int x) { return (float)x; }
};
// fp16 / bf16 slices: 16 x 16 x 32, 16 bytes of K per lane as for int8
template <> struct Mfma16<_Float16> {
    using Acc = f32x4;
    static constexpr bool kExactAcc = false;
    OZK_DEV static Acc zero() { return Acc{0.0f}; }
    template <bool AG> OZK_DEV static void run(Acc &c, i32x4 a, i32x4 b) {
        if constexpr (AG) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
        else asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    }
    OZK_DEV static Acc mfma(i32x4 a, i32x4 b, Acc c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    OZK_DEV static float to_f32(float x) { return x; }
};
template <> struct Mfma16<__bf16> {
    using Acc = f32x4;
    static constexpr bool kExactAcc = false;
    OZK_DEV static Acc zero() { return Acc{0.0f}; }
    template <bool AG> OZK_DEV static void run(Acc &c, i32x4 a, i32x4 b) {
        if constexpr (AG) asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
        else asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    }
    OZK_DEV static Acc mfma(i32x4 a, i32x4 b, Acc c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    OZK_DEV static float to_f32(float x) { return x; }
};

template <typename ST, typename AccT, bool TRI>
__global__ __launch_bounds__(512, 1) void cross_gemm_wide4q_kernel(GemmParams p, int group_m,
                                                                   uint32_t a_records,
                                                                   uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = Wide4Shape;
    using MF = Mfma16<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;
    constexpr int L = Sh::L, BM = Sh::BM, BN = Sh::BN;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    // DMA of stage kb + 2: P1 instructions in the groups after stage kb's
    // barrier, the rest in groups 0 .. G0 - 1 of stage kb + 1's first step
    // (C3, cross-GEMM ms, four paired runs on two boxes: G0 = 4 6.09-6.27
    // against 6.23-6.33 with the rest spread over all 8 groups; P1 = 6 or 8
    // slower)
    constexpr int P1 = 4, G0 = 4;
    static_assert(Sh::NW == 8 && Sh::LA == 6 && Sh::LB == 4 && BM == 96 && BN == 64,
                  "the window arithmetic below is written for this shape");
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool last_i = wave >= 6;                 // holds the pairs i = 3
    const int wy = last_i ? wave - 6 : (wave & 1);
    const int wx = last_i ? 0 : (wave >> 1);

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    const int64_t g = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb = (int)((kbytes + kDmaRB - 1) / kDmaRB);

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // Stage DMA, wide4's windows: a 1 KB window is 8 whole 128-byte rows
    // (lane -> row lane / 8, physical chunk lane % 8, which holds logical
    // chunk c0 = (lane % 8) ^ (lane / 16) in an even window and c0 ^ 4 in an
    // odd one).  Wave w fetches A windows 6 w .. 6 w + 5 (slice w / 2, rows
    // m0 + 48 (w % 2) + 8 q) and B windows 4 w .. 4 w + 3 (slice w / 2, rows
    // n0 + 32 (w % 2) + 8 q), so a window's parity is that of q.  The source
    // offset of window q of stage kb is base + q step + 128 kb, plus the
    // lane's part (4 registers: A / B, parity); the bounds are tested per lane
    // only where a window has fewer than 8 rows in the operand or the stage
    // runs past K.
    const int half = wave & 1, wsl = wave >> 1;
    const int64_t a_first = m0 + 48 * half, b_first = n0 + 32 * half;
    const uint32_t a_base = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(((int64_t)wsl * p.as_l + a_first * p.as_m) * ES));
    const uint32_t b_base = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(((int64_t)wsl * p.bs_l + b_first * p.bs_n) * ES));
    const uint32_t a_step = (uint32_t)__builtin_amdgcn_readfirstlane((int)(8 * p.as_m * ES));
    const uint32_t b_step = (uint32_t)__builtin_amdgcn_readfirstlane((int)(8 * p.bs_n * ES));
    // windows whose 8 rows are all inside the operand, and stages whose 128
    // bytes are all inside K
    const int a_full = (int)(p.M - a_first <= 0 ? 0 : ((p.M - a_first) / 8 < 6 ? (p.M - a_first) / 8 : 6));
    const int b_full = (int)(p.N - b_first <= 0 ? 0 : ((p.N - b_first) / 8 < 4 ? (p.N - b_first) / 8 : 4));
    const int nkb_full = (int)(kbytes / kDmaRB);
    uint32_t lane_src[2][2];   // [A, B][window parity]
    {
        const int lrow = lane >> 3;
        const int c0 = (lane & 7) ^ (lane >> 4);
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            const uint32_t chb = (uint32_t)(par ? (c0 ^ 4) : c0) * 16;
            lane_src[0][par] = (uint32_t)(lrow * p.as_m * ES) + chb;
            lane_src[1][par] = (uint32_t)(lrow * p.bs_n * ES) + chb;
        }
    }
    auto buf = [&](int kb) { return smem + (kb & 1) * Sh::STAGE; };
    // DMA instruction q (< LA: A window q of this wave; else B window q - LA)
    // of stage kb; q is a constant at every call.  FAST: the window's rows
    // and the stage are known to lie inside the operand, and the uniform part
    // of the source is the instruction's scalar offset.
    auto issue = [&](int kb, int q, auto FAST) {
        const bool isa = q < Sh::LA;
        const int qq = isa ? q : q - Sh::LA;
        const uint32_t ub = (isa ? a_base + (uint32_t)qq * a_step : b_base + (uint32_t)qq * b_step) +
                            (uint32_t)kb * kDmaRB;
        const uint32_t lsrc = lane_src[isa ? 0 : 1][qq & 1];
        if constexpr (decltype(FAST)::value) {
            auto *ldsp = (__attribute__((address_space(3))) void *)(
                buf(kb) + (isa ? 0 : Sh::A_BYTES) + (wave * (isa ? Sh::LA : Sh::LB) + qq) * 1024);
            if (isa) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, lsrc, (int)ub, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, lsrc, (int)ub, 0, 0);
            return;
        }
        uint32_t vo;
        if (qq < (isa ? a_full : b_full) && kb < nkb_full) {
            vo = lsrc + ub;
        } else {
            const int64_t first = (isa ? a_first : b_first) + 8 * qq;
            const int64_t rl = (isa ? p.M : p.N) - first;
            const int rows_left = (int)(rl < 8 ? rl : 8);               // may be <= 0
            const int kleft = (int)kbytes - kb * kDmaRB;                // > 0
            const int ln = lane_here();
            const int c0 = (ln & 7) ^ (ln >> 4);
            const int chb = ((qq & 1) ? (c0 ^ 4) : c0) * 16;
            vo = ((ln >> 3) < rows_left && chb < kleft) ? lsrc + ub : kOOB;
        }
        auto *ldsp = (__attribute__((address_space(3))) void *)(
            buf(kb) + (isa ? 0 : Sh::A_BYTES) + (wave * (isa ? Sh::LA : Sh::LB) + qq) * 1024);
        if (isa) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, vo, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, vo, 0, 0, 0);
    };
    // the tile's scales, as in wide4: into the buffer of stage nkb during the
    // last stage (the lane read where they are fetched), at the start of the
    // LDS (nkb even) or at its end (nkb odd), so that the rest of it is one
    // free range for the epilogue
    char *const scl = (nkb & 1) ? smem + 2 * Sh::STAGE - Sh::NSC * 256 : smem;
    auto issue_scales = [&]() {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int u = q * Sh::NW + wave;
            if (u >= Sh::NSC) break;
            const bool isa = u < L * BM / 64;
            const int e = (isa ? u : u - L * BM / 64) * 64 + lane_here();
            const int s = isa ? e / BM : e / BN;                 // slice
            const int64_t rc = isa ? m0 + e % BM : n0 + e % BN;  // row of A / column of B
            const int64_t ext = isa ? ((int64_t)(L - 1) * p.sas_l + (p.M - 1) * p.sas_m + 1)
                                    : ((int64_t)(L - 1) * p.sbs_l + (p.N - 1) * p.sbs_n + 1);
            const bool ok = rc < (isa ? p.M : p.N);
            const uint32_t vo = ok ? (uint32_t)(((int64_t)s * (isa ? p.sas_l : p.sbs_l) +
                                                 rc * (isa ? p.sas_m : p.sbs_n)) * 4)
                                   : kOOB;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(isa ? p.sa + bidx * p.sas_b : p.sb + bidx * p.sbs_b), (short)0,
                (int)(ext * 4 < 0x7FFFFFFF ? ext * 4 : 0x7FFFFFFF), 0x00020000);
            auto *ldsp = (__attribute__((address_space(3))) void *)(scl + u * 256);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, ldsp, 4, vo, 0, 0, 0);
        }
    };
    const float *sa_lds = (const float *)scl, *sb_lds = (const float *)(scl + L * BM * 4);

    // prologue: stages 0 and 1; stage 0 must land before the first reads
    constexpr std::false_type kChecked{};
    constexpr std::true_type kFast{};
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) issue(0, q, kChecked);
    if (nkb > 1) {
#pragma unroll
        for (int q = 0; q < Sh::LPS; ++q) issue(1, q, kChecked);
        wait_vmcnt<Sh::LPS>();
    } else {
        wait_vmcnt<0>();
    }
    exec_barrier();

    // Fragment rows start at multiples of 16, so the swizzle key of a lane's
    // row, ((row >> 1) & 7), is that of lane % 16 for every fragment.  Per K
    // step a wave computes the address of its A region's and B region's row
    // 0 for its lane once; each fragment is a constant offset from it (the
    // LDS read's immediate).
    const int qrow = lane & 15;
    const int key = (qrow >> 1) & 7;
    int lane_rd[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) lane_rd[kk] = qrow * kDmaRB + (((4 * kk + (lane >> 4)) ^ key) << 4);
    const int smem_base = (int)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
    using lds_cptr = const __attribute__((address_space(3))) char *;
    const int a_org = (last_i ? 3 * BM : wx * 32) * kDmaRB;
    const int b_org = Sh::A_BYTES + wy * 32 * kDmaRB;
    auto region = [&](int kb, int kk, int org) {
        const int u = __builtin_amdgcn_readfirstlane(smem_base + (kb & 1) * Sh::STAGE + org);
        return (lds_cptr)(uintptr_t)(u + lane_rd[kk]);
    };

    i32x4 fa[6];   // A fragments (u, rh), resident through a K step
    i32x4 fb[4];   // B fragments g .. g + 3 (g mod 4)
    Acc acc[3][L][2][2];
#pragma unroll
    for (int u = 0; u < 3; ++u)
#pragma unroll
        for (int j = 0; j < L; ++j)
#pragma unroll
            for (int rh = 0; rh < 2; ++rh)
#pragma unroll
                for (int ch = 0; ch < 2; ++ch) {
                    acc[u][j][rh][ch] = MF::zero();
                    // pinned where the hand-placed MFMAs keep it
                    if (u > 0) asm volatile("" : "+a"(acc[u][j][rh][ch]));
                    else asm volatile("" : "+v"(acc[u][j][rh][ch]));
                }
    asm volatile("s_nop 7" ::: "memory");

    // A fragment (u, rh) of a K step: row 16 rh of the step's A region for u
    // (a_org + u * a_rstep rows), B fragment (j, ch): row j * BN + 16 ch of
    // its B region; 16 rh and j * BN + 16 ch are the LDS reads' immediates
    const int a_rstep = (last_i ? 32 : BM) * kDmaRB;   // bytes between A fragments u and u + 1
    auto read_a = [&](lds_cptr ra, int rh) {
        return *(const __attribute__((address_space(3))) i32x4 *)(ra + 16 * rh * kDmaRB);
    };
    auto read_b = [&](lds_cptr rb, int gb) {   // B fragment gb = (j, ch)
        return *(const __attribute__((address_space(3))) i32x4 *)(
            rb + ((gb >> 1) * BN + 16 * (gb & 1)) * kDmaRB);
    };
    // One K step on the fragments of stage ckb, step ckk (fa and fb hold its
    // A fragments and B fragments 0, 1 on entry).  Group gb runs the 6 MFMAs
    // of B fragment gb and first reads B fragment gb + 2 (groups 6, 7: B
    // fragments 0, 1 of the next step, stage nkb_, step nkk); in group 7, each
    // A fragment of the next step is read right after its last MFMA.  With
    // `bar`, group 6 starts behind the stage barrier.  DMA instructions [lo,
    // hi) of stage dkb are spread over the MFMAs of groups dg0 .. 7 (lo, hi
    // and dg0 are constants at every call; FAST: as issue's).
    auto stepq = [&](int ckb, int ckk, int nkb_, int nkk, bool bar, int dkb, bool on, int lo,
                     int hi, int dg0, auto FAST) __attribute__((always_inline)) {
        const int cnt = hi - lo;
        const int span = ((dg0 == 0 ? G0 : 8) - dg0) * 6;   // the slots the instructions spread over
        const lds_cptr rb_cur = region(ckb, ckk, b_org);
#pragma unroll
        for (int gb = 0; gb < 8; ++gb) {
            if (gb < 6) {
                fb[(gb + 2) & 3] = read_b(rb_cur, gb + 2);
            } else {
                if (gb == 6 && bar) {
                    // stage nkb_ has landed (this wave's DMA, then every
                    // wave's through the barrier), and every wave's reads of
                    // stage ckb are complete before its buffer is refilled
                    wait_vmcnt<0>();
                    __builtin_amdgcn_s_waitcnt(0xC07F);
                    exec_barrier();
                }
                fb[(gb + 2) & 3] = read_b(region(nkb_, nkk, b_org), gb - 6);
            }
            const int j = gb >> 1, ch = gb & 1;
#pragma unroll
            for (int pa = 0; pa < 6; ++pa) {
                const int u = pa >> 1, rh = pa & 1;
                // the pair (u, j) in a wave of the first kind, (3, j) in one of the second
                const bool first = !TRI || u + j <= L - 1, second = !TRI || j == 0;
                auto mfma = [&]() {
                    if (u > 0) MF::template run<true>(acc[u][j][rh][ch], fa[pa], fb[gb & 3]);
                    else MF::template run<false>(acc[u][j][rh][ch], fa[pa], fb[gb & 3]);
                };
                if (first && second) {
                    mfma();
                } else if (first || second) {
                    if (first != last_i) mfma();
                }
                if (gb == 7) fa[pa] = read_a(region(nkb_, nkk, a_org + u * a_rstep), rh);
                const int n = (gb - dg0) * 6 + pa;
#pragma unroll
                for (int d = 0; d < Sh::LPS; ++d) {
                    // instruction lo + d goes after MFMA (d * span) / cnt of the span
                    if (gb >= dg0 && d < cnt && (d * span) / cnt == n && on) issue(dkb, lo + d, FAST);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    if (nkb > 0) {
#pragma unroll
        for (int pa = 0; pa < 6; ++pa) fa[pa] = read_a(region(0, 0, a_org + (pa >> 1) * a_rstep), pa & 1);
        const lds_cptr rb0 = region(0, 0, b_org);
        fb[0] = read_b(rb0, 0);
        fb[1] = read_b(rb0, 1);
    }
    static_assert(kDmaRB / 64 == 2, "two 64-byte K steps per stage");
    if (nkb == 0) issue_scales();
    auto stage = [&](int kb, auto FAST) __attribute__((always_inline)) {
        // FAST stages are 1 .. nkb - 3: the tests below hold
        constexpr bool F = decltype(FAST)::value;
        const bool nb = F || kb + 1 < nkb, n2 = F || kb + 2 < nkb;
        // no DMA is outstanding in the last stage: its waits are unaffected
        if (!nb) issue_scales();
        // the rest of stage kb + 1 (stage 1 went out whole in the prologue)
        stepq(kb, 0, kb, 1, false, kb + 1, nb && (F || kb >= 1), P1, Sh::LPS, 0, FAST);
        // groups 6, 7 read stage kb + 1's step 0 (unused past the end) and
        // start stage kb + 2 in stage kb's buffer
        stepq(kb, 1, kb + 1, 0, nb, kb + 2, n2, 0, P1, 6, FAST);
    };
    // Stages 1 .. kfast - 1 of a tile whose windows all lie inside M and N
    // issue all their DMA (stages kb + 1 and kb + 2 exist and lie inside K)
    // with no tests; the others test each instruction.
    const bool tile_full = a_full == Sh::LA && b_full == Sh::LB;
    const int kfast = min(nkb - 2, nkb_full - 2);
    {
        int kb = 0;
        if (nkb > 0) stage(kb++, kChecked);
        if (tile_full)
            for (; kb < kfast; ++kb) stage(kb, kFast);
        for (; kb < nkb; ++kb) stage(kb, kChecked);
    }

    // the hand-placed MFMAs' results are read below: 64 wait states first
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");

    // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    exec_barrier();
    // the epilogue's lane values are read afresh (lane_here), not held
    // through the K loop
    const int elane = lane_here();
    const int eq = elane & 15, eg = elane >> 4;
    float sbv[L][2];
#pragma unroll
    for (int j = 0; j < L; ++j)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) sbv[j][ch] = sb_lds[j * BN + wy * 32 + 16 * ch + eq];
    // rows of registers 0..3 of row half rh of A fragment u, inside the tile,
    // start at row4(u, rh): their 4 scales are one 16-byte LDS read
    auto row4 = [&](int u, int rh) { return (last_i ? u * 32 : wx * 32) + 16 * rh + 4 * eg; };
    auto sa4 = [&](int i, int u, int rh) {
        return *(const f32x4 *)(sa_lds + i * BM + row4(u, rh));
    };
    // Every wave turns its accumulator tiles into t = fl32(fl32(fl32(acc) *
    // sa_i) * sb_j), tile by tile in one order (u, j, rh, ch), each tile dead
    // after it: a wave of the first kind adds them to the running sums of its
    // 16 elements (the pairs i = u = 0..2, j = 0..3 of its block: i-major,
    // j-minor), one of the second kind (the pairs (3, j) of block u) stores
    // them to the LDS.  After the barrier the first kind adds the (3, j) terms
    // of its block in order and stores C.  T: [wave - 6][u][j][rh, ch][lane]
    // x 4 floats, 96 KB in the free range of the LDS.
    float *const tsm = (float *)(smem + ((nkb & 1) ? 0 : 4096));
    static_assert(4096 + 2 * 3 * L * 4 * 64 * 16 <= 2 * Sh::STAGE - Sh::NSC * 256 &&
                      Sh::NSC * 256 <= 4096,
                  "the t values fit beside the scales");
    auto tslot = [&](int w6, int u, int j, int q) {
        return (f32x4 *)(tsm + ((((w6 * 3 + u) * L + j) * 4 + q) * 64 + elane) * 4);
    };
    OA out[2][2][4];
#pragma unroll
    for (int rh = 0; rh < 2; ++rh)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
            for (int e = 0; e < 4; ++e) out[rh][ch][e] = (OA)0;
#pragma unroll
    for (int u = 0; u < 3; ++u) {
        f32x4 s4[2];
#pragma unroll
        for (int rh = 0; rh < 2; ++rh) s4[rh] = sa4(last_i ? 3 : u, u, rh);
#pragma unroll
        for (int j = 0; j < L; ++j) {
            // the kept pairs: (u, j) in the first kind, (3, j) in the second
            const bool keep = last_i ? (!TRI || j == 0) : (!TRI || u + j <= L - 1);
            if (keep) {
#pragma unroll
                for (int rh = 0; rh < 2; ++rh)
#pragma unroll
                    for (int ch = 0; ch < 2; ++ch) {
                        f32x4 tv;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            tv[e] = (MF::to_f32(acc[u][j][rh][ch][e]) * s4[rh][e]) * sbv[j][ch];
                        if (last_i) {
                            *tslot(wave - 6, u, j, rh * 2 + ch) = tv;
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e) out[rh][ch][e] = out[rh][ch][e] + (OA)tv[e];
                        }
                    }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    exec_barrier();
    if (!last_i) {
        const int64_t cbase = bidx * p.cs_b;
#pragma unroll
        for (int rh = 0; rh < 2; ++rh)
#pragma unroll
            for (int ch = 0; ch < 2; ++ch) {
                const int64_t col = n0 + wy * 32 + 16 * ch + eq;
                f32x4 t3[TRI ? 1 : L];
#pragma unroll
                for (int j = 0; j < (TRI ? 1 : L); ++j) t3[j] = *tslot(wy, wx, j, rh * 2 + ch);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t row = m0 + row4(0, rh) + e;
                    OA o = out[rh][ch][e];
#pragma unroll
                    for (int j = 0; j < (TRI ? 1 : L); ++j) o = o + (OA)t3[j][e];
                    if (col < p.N && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, o);
                }
            }
    }
}

// ---------------------------------------------------------------------------
// The num_splits 3 wide kernel on 16 x 16 MFMAs (int8: v_mfma_i32_16x16x64_i8,
// fp16 / bf16: v_mfma_f32_16x16x32_f16 / _bf16): the same tile (64 x 128, 8
// waves in a 2 x 4 grid of 32 x 32 blocks, each wave all 9 pairs of its
// block), stages, DMA and split-K as cross_gemm_wide_kernel, with a K step of
// 64 bytes (two per stage) as in cross_gemm_wide4q_kernel (there: why).  A
// wave's 9 accumulator tiles of 32 x 32 become 36 of 16 x 16,
// acc[i][j][rh][ch]; register e of lane l holds row 16 rh + 4 (l / 16) + e,
// column 16 ch + l % 16 of the block.  Per K step a wave reads 6 A fragments
// (i, rh) and 6 B fragments (j, ch) and runs 36 MFMAs, B-outer: the A
// fragments stay in registers, each re-read for the next step right after its
// last MFMA; B fragment g + 2 is read while g's 6 MFMAs run (a ring of 3).
// The stage barrier sits before the last two B groups of the stage's second
// step, whose reads are the next stage's.  144 accumulator registers, 24 for
// A, 12 for B: the compiler places them.  The epilogue sums each element's pairs tile by
// tile (i-major, j-minor), so each tile is dead after it.
// ---------------------------------------------------------------------------
template <typename ST, typename AccT, bool TRI>
__global__ __launch_bounds__(512, 1) void cross_gemm_wideq_kernel(GemmParams p, int group_m,
                                                                  uint32_t a_records,
                                                                  uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = WideShape;
    using MF = Mfma16<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;
    constexpr int L = Sh::L, BM = Sh::BM, BN = Sh::BN;
    using PS = Pairs<L, TRI>;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    constexpr int P1 = 4;   // DMA instructions of stage kb + 2 in the groups after the barrier
    static_assert(Sh::NW == 8 && Sh::LA == 3 && Sh::LB == 6 && BM == 64 && BN == 128,
                  "the window arithmetic below is written for this shape");
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    // split-K: workgroup g0 is K range g0 % S of tile g0 / S
    const int S = p.ksplit > 1 ? p.ksplit : 1;
    const int64_t g0 = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int krange = (int)(g0 % S);
    const int64_t g = g0 / S;
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb_all = (int)((kbytes + kDmaRB - 1) / kDmaRB);
    const int kb0 = S > 1 ? krange * p.kb_per_split : 0;   // this range's first stage
    const int nkb = S > 1 ? min(p.kb_per_split, nkb_all - kb0) : nkb_all;
    const uint32_t kbyte0 = (uint32_t)kb0 * kDmaRB;

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // Stage DMA: a 1 KB window is 8 whole 128-byte rows (lane -> row lane /
    // 8, physical chunk lane % 8, which holds logical chunk c0 = (lane % 8) ^
    // (lane / 16) in an even window and c0 ^ 4 in an odd one); the stage's A
    // windows r = 8 s + x (slice s, rows m0 + 8 x) and B windows r = 16 s + x
    // (rows n0 + 8 x) sit at r KB of their regions.  Wave w fetches the A
    // windows w + 8 q (q < 3: slice q, row window w) and the B windows w + 8 q
    // (q < 6: slice q / 2, row window w + 8 (q % 2)), so its windows share
    // its parity and their sources are a base plus multiples of a slice
    // stride: all uniform values fixed before the loop.  The lane's part of
    // the source is held (2 registers); the bounds are tested per lane only
    // where a window has fewer than 8 rows in the operand or the stage runs
    // past K.
    const int64_t a_first = m0 + 8 * wave, b_first = n0 + 8 * wave;
    const uint32_t a_base = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)((a_first * p.as_m) * ES + kbyte0));
    const uint32_t b_base = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)((b_first * p.bs_n) * ES + kbyte0));
    const uint32_t a_sstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(p.as_l * ES));
    const uint32_t b_sstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(p.bs_l * ES));
    const uint32_t b_hstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(64 * p.bs_n * ES));
    // rows of this wave's windows inside the operand (may be <= 0)
    const int a_rows = (int)(p.M - a_first < 8 ? p.M - a_first : 8);
    const int b_rows0 = (int)(p.N - b_first < 8 ? p.N - b_first : 8);
    const int b_rows1 = (int)(p.N - b_first - 64 < 8 ? p.N - b_first - 64 : 8);
    uint32_t lane_src[2];   // [A, B]
    {
        const int c0 = (lane & 7) ^ (lane >> 4);
        const uint32_t chb = (uint32_t)((wave & 1) ? (c0 ^ 4) : c0) * 16;
        lane_src[0] = (uint32_t)((lane >> 3) * p.as_m * ES) + chb;
        lane_src[1] = (uint32_t)((lane >> 3) * p.bs_n * ES) + chb;
    }
    const int nkb_full = (int)(kbytes / kDmaRB);   // stages (counted from K = 0) inside K
    auto buf = [&](int kb) { return smem + (kb & 1) * Sh::STAGE; };
    // DMA instruction q (< LA: A window q of this wave; else B window q - LA)
    // of stage kb (of this range); q is a constant at every call.  FAST: the
    // window's rows and the stage are known to lie inside the operand, and
    // the uniform part of the source is the instruction's scalar offset.
    auto issue = [&](int kb, int q, auto FAST) {
        const bool isa = q < Sh::LA;
        const int qq = isa ? q : q - Sh::LA;
        const uint32_t ub = (isa ? a_base + (uint32_t)qq * a_sstep
                                 : b_base + (uint32_t)(qq >> 1) * b_sstep + ((qq & 1) ? b_hstep : 0u)) +
                            (uint32_t)kb * kDmaRB;
        const uint32_t lsrc = lane_src[isa ? 0 : 1];
        auto *ldsp = (__attribute__((address_space(3))) void *)(
            buf(kb) + (isa ? 0 : Sh::A_BYTES) + (wave + 8 * qq) * 1024);
        if constexpr (decltype(FAST)::value) {
            if (isa) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, lsrc, (int)ub, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, lsrc, (int)ub, 0, 0);
            return;
        }
        const int rows = isa ? a_rows : ((qq & 1) ? b_rows1 : b_rows0);
        uint32_t vo;
        if (rows == 8 && kb0 + kb < nkb_full) {
            vo = lsrc + ub;
        } else {
            const int kleft = (int)kbytes - (int)kbyte0 - kb * kDmaRB;   // > 0
            const int ln = lane_here();
            const int c0 = (ln & 7) ^ (ln >> 4);
            const int chb = ((wave & 1) ? (c0 ^ 4) : c0) * 16;
            vo = ((ln >> 3) < rows && chb < kleft) ? lsrc + ub : kOOB;
        }
        if (isa) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, vo, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, vo, 0, 0, 0);
    };

    // The tile's scales (A's [L][BM], then B's [L][BN]: 2304 bytes), as in
    // the wide kernel: into the buffer of stage nkb at the start of the last
    // stage (the lane read where they are fetched).
    char *const scl = buf(nkb);
    auto issue_scales = [&]() {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int u = q * Sh::NW + wave;
            if (u >= L * (BM + BN) / 64) break;
            const bool isa = u < L * BM / 64;
            const int e = (isa ? u : u - L * BM / 64) * 64 + lane_here();
            const int s = isa ? e / BM : e / BN;                 // slice
            const int64_t rc = isa ? m0 + e % BM : n0 + e % BN;  // row of A / column of B
            const int64_t ext = isa ? ((int64_t)(L - 1) * p.sas_l + (p.M - 1) * p.sas_m + 1)
                                    : ((int64_t)(L - 1) * p.sbs_l + (p.N - 1) * p.sbs_n + 1);
            const bool ok = rc < (isa ? p.M : p.N);
            const uint32_t vo = ok ? (uint32_t)(((int64_t)s * (isa ? p.sas_l : p.sbs_l) +
                                                 rc * (isa ? p.sas_m : p.sbs_n)) * 4)
                                   : kOOB;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(isa ? p.sa + bidx * p.sas_b : p.sb + bidx * p.sbs_b), (short)0,
                (int)(ext * 4 < 0x7FFFFFFF ? ext * 4 : 0x7FFFFFFF), 0x00020000);
            auto *ldsp = (__attribute__((address_space(3))) void *)(scl + u * 256);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, ldsp, 4, vo, 0, 0, 0);
        }
    };
    const float *sa_lds = (const float *)scl, *sb_lds = (const float *)(scl + L * BM * 4);

    // prologue: stages 0 and 1; stage 0 must land before the first reads
    constexpr std::false_type kChecked{};
    constexpr std::true_type kFast{};
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) issue(0, q, kChecked);
    if (nkb > 1) {
#pragma unroll
        for (int q = 0; q < Sh::LPS; ++q) issue(1, q, kChecked);
        wait_vmcnt<Sh::LPS>();
    } else {
        wait_vmcnt<0>();
    }
    exec_barrier();

    // fragments: as in cross_gemm_wide4q_kernel, one lane address per region
    // and K step, the fragment's row its LDS read's immediate
    const int qrow = lane & 15;
    const int key = (qrow >> 1) & 7;
    int lane_rd[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) lane_rd[kk] = qrow * kDmaRB + (((4 * kk + (lane >> 4)) ^ key) << 4);
    const int smem_base = (int)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
    using lds_cptr = const __attribute__((address_space(3))) char *;
    const int a_org = wm * 32 * kDmaRB;
    const int b_org = Sh::A_BYTES + wn * 32 * kDmaRB;
    auto region = [&](int kb, int kk, int org) {
        const int u = __builtin_amdgcn_readfirstlane(smem_base + (kb & 1) * Sh::STAGE + org);
        return (lds_cptr)(uintptr_t)(u + lane_rd[kk]);
    };
    auto read_a = [&](lds_cptr ra, int pa) {   // A fragment pa = (i, rh)
        return *(const __attribute__((address_space(3))) i32x4 *)(
            ra + ((pa >> 1) * BM + 16 * (pa & 1)) * kDmaRB);
    };
    auto read_b = [&](lds_cptr rb, int gb) {   // B fragment gb = (j, ch)
        return *(const __attribute__((address_space(3))) i32x4 *)(
            rb + ((gb >> 1) * BN + 16 * (gb & 1)) * kDmaRB);
    };

    i32x4 fa[2 * L];   // A fragments (i, rh), resident through a K step
    i32x4 fb[3];       // B fragments g .. g + 2 (g mod 3: 6 groups a step close the ring)
    Acc acc[L][L][2][2];
#pragma unroll
    for (int i = 0; i < L; ++i)
#pragma unroll
        for (int j = 0; j < L; ++j)
#pragma unroll
            for (int rh = 0; rh < 2; ++rh)
#pragma unroll
                for (int ch = 0; ch < 2; ++ch) acc[i][j][rh][ch] = MF::zero();

    // One K step (as in cross_gemm_wide4q_kernel): group gb runs the MFMAs
    // of B fragment gb (the kept pairs) and first reads B fragment gb + 2
    // (groups 4, 5: fragments 0, 1 of the next step, stage nkb_, step nkk);
    // in group 5 each A fragment of the next step is read right after its
    // last MFMA.  With `bar`, group 4 starts behind the stage barrier.  DMA
    // instructions [lo, hi) of stage dkb go between the MFMAs of groups
    // dg0 .. 5 (lo, hi and dg0 are constants at every call; FAST: as issue's).
    constexpr int NG = 2 * L, NPA = 2 * L;
    auto stepq = [&](int ckb, int ckk, int nkb_, int nkk, bool bar, int dkb, bool on, int lo,
                     int hi, int dg0, auto FAST) __attribute__((always_inline)) {
        const int cnt = hi - lo;
        const int span = (NG - dg0) * NPA;
        const lds_cptr rb_cur = region(ckb, ckk, b_org);
#pragma unroll
        for (int gb = 0; gb < NG; ++gb) {
            if (gb < NG - 2) {
                fb[(gb + 2) % 3] = read_b(rb_cur, gb + 2);
            } else {
                if (gb == NG - 2 && bar) {
                    // stage nkb_ has landed (this wave's DMA, then every
                    // wave's through the barrier), and every wave's reads of
                    // stage ckb are complete before its buffer is refilled
                    wait_vmcnt<0>();
                    __builtin_amdgcn_s_waitcnt(0xC07F);
                    exec_barrier();
                }
                fb[(gb + 2) % 3] = read_b(region(nkb_, nkk, b_org), gb - (NG - 2));
            }
            const int j = gb >> 1, ch = gb & 1;
            const lds_cptr ra_next = region(nkb_, nkk, a_org);
#pragma unroll
            for (int pa = 0; pa < NPA; ++pa) {
                const int i = pa >> 1, rh = pa & 1;
                if (PS::kept(i, j))
                    acc[i][j][rh][ch] = MF::mfma(fa[pa], fb[gb % 3], acc[i][j][rh][ch]);
                if (gb == NG - 1) fa[pa] = read_a(ra_next, pa);
                const int n = (gb - dg0) * NPA + pa;
#pragma unroll
                for (int d = 0; d < Sh::LPS; ++d) {
                    // instruction lo + d goes after MFMA (d * span) / cnt of the span
                    if (gb >= dg0 && d < cnt && (d * span) / cnt == n && on) issue(dkb, lo + d, FAST);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    if (nkb > 0) {
        const lds_cptr ra0 = region(0, 0, a_org), rb0 = region(0, 0, b_org);
#pragma unroll
        for (int pa = 0; pa < NPA; ++pa) fa[pa] = read_a(ra0, pa);
        fb[0] = read_b(rb0, 0);
        fb[1] = read_b(rb0, 1);
    }
    static_assert(kDmaRB / 64 == 2 && NG % 3 == 0, "two 64-byte K steps per stage; the B ring closes");
    if (nkb == 0) issue_scales();
    auto stage = [&](int kb, auto FAST) __attribute__((always_inline)) {
        // FAST stages are 1 .. nkb - 3: the tests below hold
        constexpr bool F = decltype(FAST)::value;
        const bool nb = F || kb + 1 < nkb, n2 = F || kb + 2 < nkb;
        // no DMA is outstanding in the last stage: its waits are unaffected
        if (!nb) issue_scales();
        // the rest of stage kb + 1 (stage 1 went out whole in the prologue)
        stepq(kb, 0, kb, 1, false, kb + 1, nb && (F || kb >= 1), P1, Sh::LPS, 0, FAST);
        // the last two groups read stage kb + 1's step 0 (unused past the
        // end) and start stage kb + 2 in stage kb's buffer
        stepq(kb, 1, kb + 1, 0, nb, kb + 2, n2, 0, P1, NG - 2, FAST);
    };
    // Stages 1 .. kfast - 1 of a tile whose windows all lie inside M and N
    // issue all their DMA (stages kb + 1 and kb + 2 exist and lie inside K)
    // with no tests; the others test each instruction.
    const bool tile_full = a_rows == 8 && b_rows0 == 8 && b_rows1 == 8;
    const int kfast = min(nkb - 2, nkb_full - kb0 - 2);
    {
        int kb = 0;
        if (nkb > 0) stage(kb++, kChecked);
        if (tile_full)
            for (; kb < kfast; ++kb) stage(kb, kFast);
        for (; kb < nkb; ++kb) stage(kb, kChecked);
    }

    // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    exec_barrier();
    if (S > 1) {
        // split-K, as in the wide kernel: each range stores its raw
        // accumulators (register (rh, ch, e) of pair n at (n * 16 + (2 rh +
        // ch) * 4 + e) * 64 + lane); the last range to arrive adds the others
        constexpr int RW = L * L * 16;
        const int ln = lane_here();
        uint32_t *mine = splitk_slot(p, g, krange, wave, RW, ln);
#pragma unroll
        for (int n = 0; n < L * L; ++n) {
            if (!PS::kept(n / L, n % L)) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const i32x4 u = __builtin_bit_cast(i32x4, acc[n / L][n % L][q >> 1][q & 1]);
#pragma unroll
                for (int e = 0; e < 4; ++e) splitk_put(mine + (n * 16 + q * 4 + e) * 64, (uint32_t)u[e]);
            }
        }
        if (!splitk_arrive(p, g, (int *)buf(nkb + 1))) return;
        auto get4 = [&](const uint32_t *src) {
            i32x4 u;
#pragma unroll
            for (int e = 0; e < 4; ++e) u[e] = (int)splitk_get(src + e * 64);
            return __builtin_bit_cast(Acc, u);
        };
        // int32 sums are exact in any order: this range's accumulators stay
        // and the others are added; float sums: every range read back, this
        // one's too, in range order from range 0
        for (int s2 = 0; s2 < S; ++s2) {
            if (MF::kExactAcc && s2 == krange) continue;
            const uint32_t *src = splitk_slot(p, g, s2, wave, RW, ln);
#pragma unroll
            for (int n = 0; n < L * L; ++n) {
                if (!PS::kept(n / L, n % L)) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const Acc v = get4(src + (n * 16 + q * 4) * 64);
                    Acc &a = acc[n / L][n % L][q >> 1][q & 1];
                    a = (!MF::kExactAcc && s2 == 0) ? v : a + v;
                }
            }
        }
    }
    const int elane = lane_here();
    const int eq = elane & 15, eg = elane >> 4;
    const int64_t cbase = bidx * p.cs_b;
    float sbv[L][2];
#pragma unroll
    for (int j = 0; j < L; ++j)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) sbv[j][ch] = sb_lds[j * BN + wn * 32 + 16 * ch + eq];
    OA out[2][2][4];
#pragma unroll
    for (int rh = 0; rh < 2; ++rh)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
            for (int e = 0; e < 4; ++e) out[rh][ch][e] = (OA)0;
#pragma unroll
    for (int i = 0; i < L; ++i) {
        f32x4 s4[2];
#pragma unroll
        for (int rh = 0; rh < 2; ++rh)
            s4[rh] = *(const f32x4 *)(sa_lds + i * BM + wm * 32 + 16 * rh + 4 * eg);
#pragma unroll
        for (int j = 0; j < L; ++j) {
            if (!PS::kept(i, j)) continue;
#pragma unroll
            for (int rh = 0; rh < 2; ++rh)
#pragma unroll
                for (int ch = 0; ch < 2; ++ch)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        // fl32(fl32(fl32(acc) * sa_i) * sb_j), summed i-major, j-minor
                        const float t1 = MF::to_f32(acc[i][j][rh][ch][e]) * s4[rh][e];
                        out[rh][ch][e] = out[rh][ch][e] + (OA)(t1 * sbv[j][ch]);
                    }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int rh = 0; rh < 2; ++rh)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
            const int64_t col = n0 + wn * 32 + 16 * ch + eq;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t row = m0 + wm * 32 + 16 * rh + 4 * eg + e;
                if (col < p.N && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, out[rh][ch][e]);
            }
        }
}

// ---------------------------------------------------------------------------
// The ring configuration on 16 x 16 MFMAs (int8, fp16, bf16 slices): 64 W x
// 64 W tiles (W = 2 for num_splits 2, 1 for 3 and 4), 8 waves; wave w holds
// block w % 4 (32 W x 32 W) for the pairs (i, j) of its group's A slices
// (group 0: i < IA, group 1 the rest; IA = L / 2 rounded up, the pair
// split's i-row), every j, as 4 W^2 tiles of 16 x 16 per pair.  The stages
// are double-buffered whole (two fit the LDS where the 32 x 32 ring kernel
// needs a ring of half stages).  Per 64-byte K step a wave reads its A
// fragments (i, rh) once and its B fragments (j, ch) through a ring, B group
// g + 2 read while group g's MFMAs run; the next step's A fragments are read
// in the last group, each after its MFMA.  The epilogue hands group 0's
// partial sums to group 1 through the LDS, which adds its own pairs in the
// reference's order.  Interior stages of interior tiles issue their DMA
// unchecked, as in cross_gemm_wideq_kernel.
// ---------------------------------------------------------------------------
template <int L_, int W_> struct RingQShape {
    static constexpr int L = L_, W = W_;
    static constexpr int NW = 8;                         // waves
    static constexpr int BM = 64 * W, BN = 64 * W;
    static constexpr int A_BYTES = L * BM * kDmaRB;
    static constexpr int B_BYTES = L * BN * kDmaRB;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int LA = A_BYTES / (NW * 1024);     // A instructions per wave per stage
    static constexpr int LB = B_BYTES / (NW * 1024);     // B instructions per wave per stage
    static constexpr int LPS = LA + LB;
    static constexpr int LDS_BYTES = 2 * STAGE;          // also the fp64 hand-off: 4 blocks x (32 W)^2 x 8
    static constexpr int IA = PairSplit<L, L>::P0 / L;   // A slices of group 0
    static constexpr int NSC = L * (BM + BN) / 64;       // the tile's scales: 256-byte units
    static_assert(PairSplit<L, L>::P0 % L == 0, "the pair groups split at an i-row");
    static_assert(A_BYTES % (NW * 1024) == 0 && LA == LB, "whole 1 KB windows per wave");
    static_assert(LDS_BYTES <= 160 * 1024 && BM * BN * 8 <= LDS_BYTES, "LDS");
    static_assert(NSC <= NW, "one scale unit per wave");
    static_assert(kDmaRB == 128, "128-byte stage rows");
};

template <typename ST, int L, int W, typename AccT>
__global__ __launch_bounds__(512, 1) void cross_gemm_ringq_kernel(GemmParams p, int group_m,
                                                                  uint32_t a_records,
                                                                  uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = RingQShape<L, W>;
    using MF = Mfma16<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;
    constexpr int BM = Sh::BM, BN = Sh::BN, IA = Sh::IA;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    // DMA of stage kb + 2: P1 instructions in the groups after stage kb's
    // barrier, the rest in the first half of stage kb + 1's first step (C2,
    // cross-GEMM, three paired runs: 0.409 against 0.412 ms spread over the
    // whole step; 4 after the barrier: 0.414)
    constexpr int P1 = 2;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int blk = wave & 3, grp = wave >> 2;   // block; pair group
    const int wm = blk >> 1, wn = blk & 1;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    // split-K: workgroup g0 is K range g0 % S of tile g0 / S
    const int S = p.ksplit > 1 ? p.ksplit : 1;
    const int64_t g0 = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int krange = (int)(g0 % S);
    const int64_t g = g0 / S;
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb_all = (int)((kbytes + kDmaRB - 1) / kDmaRB);
    const int kb0 = S > 1 ? krange * p.kb_per_split : 0;   // this range's first stage
    const int nkb = S > 1 ? min(p.kb_per_split, nkb_all - kb0) : nkb_all;
    const uint32_t kbyte0 = (uint32_t)kb0 * kDmaRB;

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // Stage DMA: 1 KB windows of 8 whole 128-byte rows (lane -> row lane / 8,
    // physical chunk lane % 8, which holds logical chunk c0 = (lane % 8) ^
    // (lane / 16) in an even window and c0 ^ 4 in an odd one); the stage's
    // windows r = 8 W s + x (slice s, rows 8 x of the tile) sit at r KB of the
    // A and B regions.  Wave w fetches windows w + 8 q of each (q < LA: slice
    // q / W, row window w + 8 (q % W)): its windows share its parity, and
    // their sources are a base, plus a slice stride, plus 64 rows.  The lane's
    // part of the source is held; the bounds are tested per lane only where a
    // window has fewer than 8 rows in the operand or the stage runs past K.
    const int64_t a_first = m0 + 8 * wave, b_first = n0 + 8 * wave;
    const uint32_t a_base = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)((a_first * p.as_m) * ES + kbyte0));
    const uint32_t b_base = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)((b_first * p.bs_n) * ES + kbyte0));
    const uint32_t a_sstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(p.as_l * ES));
    const uint32_t b_sstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(p.bs_l * ES));
    const uint32_t a_hstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(64 * p.as_m * ES));
    const uint32_t b_hstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(64 * p.bs_n * ES));
    // rows of this wave's windows inside the operand (may be <= 0)
    const int a_rows0 = (int)(p.M - a_first < 8 ? p.M - a_first : 8);
    const int a_rows1 = (int)(p.M - a_first - 64 < 8 ? p.M - a_first - 64 : 8);
    const int b_rows0 = (int)(p.N - b_first < 8 ? p.N - b_first : 8);
    const int b_rows1 = (int)(p.N - b_first - 64 < 8 ? p.N - b_first - 64 : 8);
    uint32_t lane_src[2];   // [A, B]
    {
        const int c0 = (lane & 7) ^ (lane >> 4);
        const uint32_t chb = (uint32_t)((wave & 1) ? (c0 ^ 4) : c0) * 16;
        lane_src[0] = (uint32_t)((lane >> 3) * p.as_m * ES) + chb;
        lane_src[1] = (uint32_t)((lane >> 3) * p.bs_n * ES) + chb;
    }
    const int nkb_full = (int)(kbytes / kDmaRB);   // stages (counted from K = 0) inside K
    auto buf = [&](int kb) { return smem + (kb & 1) * Sh::STAGE; };
    // DMA instruction q (< LA: A window q of this wave; else B window q - LA)
    // of stage kb (of this range); q is a constant at every call.  FAST: the
    // window's rows and the stage are known to lie inside the operand, and
    // the uniform part of the source is the instruction's scalar offset.
    auto issue = [&](int kb, int q, auto FAST) {
        const bool isa = q < Sh::LA;
        const int qq = isa ? q : q - Sh::LA;
        const bool hi = (qq % W) != 0;
        const uint32_t ub = (isa ? a_base + (uint32_t)(qq / W) * a_sstep + (hi ? a_hstep : 0u)
                                 : b_base + (uint32_t)(qq / W) * b_sstep + (hi ? b_hstep : 0u)) +
                            (uint32_t)kb * kDmaRB;
        const uint32_t lsrc = lane_src[isa ? 0 : 1];
        auto *ldsp = (__attribute__((address_space(3))) void *)(
            buf(kb) + (isa ? 0 : Sh::A_BYTES) + (wave + 8 * qq) * 1024);
        if constexpr (decltype(FAST)::value) {
            if (isa) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, lsrc, (int)ub, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, lsrc, (int)ub, 0, 0);
            return;
        }
        const int rows = isa ? (hi ? a_rows1 : a_rows0) : (hi ? b_rows1 : b_rows0);
        uint32_t vo;
        if (rows == 8 && kb0 + kb < nkb_full) {
            vo = lsrc + ub;
        } else {
            const int kleft = (int)kbytes - (int)kbyte0 - kb * kDmaRB;   // > 0
            const int ln = lane_here();
            const int c0 = (ln & 7) ^ (ln >> 4);
            const int chb = ((wave & 1) ? (c0 ^ 4) : c0) * 16;
            vo = ((ln >> 3) < rows && chb < kleft) ? lsrc + ub : kOOB;
        }
        if (isa) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, vo, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, vo, 0, 0, 0);
    };

    // The tile's scales (A's [L][BM], then B's [L][BN]: NSC 256-byte units,
    // one per wave) into the buffer of stage nkb at the start of the last
    // stage (the lane read where they are fetched).
    char *const scl = buf(nkb);
    auto issue_scales = [&]() {
        if (wave >= Sh::NSC) return;
        const bool isa = wave < L * BM / 64;
        const int e = (isa ? wave : wave - L * BM / 64) * 64 + lane_here();
        const int s = isa ? e / BM : e / BN;                 // slice
        const int64_t rc = isa ? m0 + e % BM : n0 + e % BN;  // row of A / column of B
        const int64_t ext = isa ? ((int64_t)(L - 1) * p.sas_l + (p.M - 1) * p.sas_m + 1)
                                : ((int64_t)(L - 1) * p.sbs_l + (p.N - 1) * p.sbs_n + 1);
        const bool ok = rc < (isa ? p.M : p.N);
        const uint32_t vo = ok ? (uint32_t)(((int64_t)s * (isa ? p.sas_l : p.sbs_l) +
                                             rc * (isa ? p.sas_m : p.sbs_n)) * 4)
                               : kOOB;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(isa ? p.sa + bidx * p.sas_b : p.sb + bidx * p.sbs_b), (short)0,
            (int)(ext * 4 < 0x7FFFFFFF ? ext * 4 : 0x7FFFFFFF), 0x00020000);
        auto *ldsp = (__attribute__((address_space(3))) void *)(scl + wave * 256);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, ldsp, 4, vo, 0, 0, 0);
    };
    const float *sa_lds = (const float *)scl, *sb_lds = (const float *)(scl + L * BM * 4);

    // prologue: stages 0 and 1; stage 0 must land before the first reads
    constexpr std::false_type kChecked{};
    constexpr std::true_type kFast{};
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) issue(0, q, kChecked);
    if (nkb > 1) {
#pragma unroll
        for (int q = 0; q < Sh::LPS; ++q) issue(1, q, kChecked);
        wait_vmcnt<Sh::LPS>();
    } else {
        wait_vmcnt<0>();
    }
    exec_barrier();

    // fragments: as in cross_gemm_wide4q_kernel, one lane address per region
    // and K step, the fragment's row its LDS read's immediate
    const int qrow = lane & 15;
    const int key = (qrow >> 1) & 7;
    int lane_rd[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) lane_rd[kk] = qrow * kDmaRB + (((4 * kk + (lane >> 4)) ^ key) << 4);
    const int smem_base = (int)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
    using lds_cptr = const __attribute__((address_space(3))) char *;
    const int b_org = Sh::A_BYTES + wn * 32 * W * kDmaRB;
    auto region = [&](int kb, int kk, int org) {
        const int u = __builtin_amdgcn_readfirstlane(smem_base + (kb & 1) * Sh::STAGE + org);
        return (lds_cptr)(uintptr_t)(u + lane_rd[kk]);
    };
    constexpr int NR = 2 * W;   // 16-row (16-column) fragments of a 32 W block
    auto read_b = [&](lds_cptr rb, int gb) {   // B fragment gb = (j, ch)
        return *(const __attribute__((address_space(3))) i32x4 *)(
            rb + ((gb / NR) * BN + 16 * (gb % NR)) * kDmaRB);
    };
    const int cbase_row = wm * 32 * W, cbase_col = wn * 32 * W;
    const int64_t cbase = bidx * p.cs_b;
    OA *part = (OA *)smem;   // the hand-off: [4 blocks][rh][ch][e][64 lanes]
    auto pslot = [&](int rh, int ch, int e, int ln) {
        return part + (((blk * NR + rh) * NR + ch) * 4 + e) * 64 + ln;
    };

    auto body = [&](auto G_) __attribute__((always_inline)) {
        constexpr int G = decltype(G_)::value;
        constexpr int ILO = G ? IA : 0, NI = G ? L - IA : IA;   // A slices of this group
        constexpr int NG = L * NR, NPA = NI * NR;               // B groups (j, ch); A fragments (i, rh)
        constexpr int R = NG % 4 == 0 ? 4 : 3;                  // B ring slots
        static_assert(NG % R == 0 && R >= 3, "the B ring closes at the end of a step");
        const int a_org = (ILO * BM + cbase_row) * kDmaRB;
        auto read_a = [&](lds_cptr ra, int pa) {   // A fragment pa = (i - ILO, rh)
            return *(const __attribute__((address_space(3))) i32x4 *)(
                ra + ((pa / NR) * BM + 16 * (pa % NR)) * kDmaRB);
        };
        i32x4 fa[NPA];   // A fragments, resident through a K step
        i32x4 fb[R];     // B groups g .. g + R - 1 (g mod R)
        Acc acc[NI][L][NR][NR];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < L; ++j)
#pragma unroll
                for (int rh = 0; rh < NR; ++rh)
#pragma unroll
                    for (int ch = 0; ch < NR; ++ch) acc[i][j][rh][ch] = MF::zero();

        // One K step: group gb runs the MFMAs of B fragment gb with every A
        // fragment and first reads B fragment gb + 2 (the last two groups:
        // fragments 0, 1 of the next step, stage nkb_, step nkk); in the last
        // group each A fragment of the next step is read right after its MFMA.
        // With `bar`, group NG - 2 starts behind the stage barrier.  DMA
        // instructions [lo, hi) of stage dkb go between the MFMAs of groups
        // dg0 .. NG - 1 (FAST: as issue's).
        auto stepq = [&](int ckb, int ckk, int nkb_, int nkk, bool bar, int dkb, bool on, int lo,
                         int hi, int dg0, auto FAST) __attribute__((always_inline)) {
            const int cnt = hi - lo;
            const int span = ((dg0 == 0 ? NG / 2 : NG) - dg0) * NPA;   // the slots they spread over
            const lds_cptr rb_cur = region(ckb, ckk, b_org);
#pragma unroll
            for (int gb = 0; gb < NG; ++gb) {
                if (gb < NG - 2) {
                    fb[(gb + 2) % R] = read_b(rb_cur, gb + 2);
                } else {
                    if (gb == NG - 2 && bar) {
                        // stage nkb_ has landed (this wave's DMA, then every
                        // wave's through the barrier), and every wave's reads
                        // of stage ckb are complete before its buffer is refilled
                        wait_vmcnt<0>();
                        __builtin_amdgcn_s_waitcnt(0xC07F);
                        exec_barrier();
                    }
                    fb[(gb + 2) % R] = read_b(region(nkb_, nkk, b_org), gb - (NG - 2));
                }
                const int j = gb / NR, ch = gb % NR;
                const lds_cptr ra_next = region(nkb_, nkk, a_org);
#pragma unroll
                for (int pa = 0; pa < NPA; ++pa) {
                    const int i = pa / NR, rh = pa % NR;
                    acc[i][j][rh][ch] = MF::mfma(fa[pa], fb[gb % R], acc[i][j][rh][ch]);
                    if (gb == NG - 1) fa[pa] = read_a(ra_next, pa);
                    const int n = (gb - dg0) * NPA + pa;
#pragma unroll
                    for (int d = 0; d < Sh::LPS; ++d) {
                        // instruction lo + d goes after MFMA (d * span) / cnt of the span
                        if (gb >= dg0 && d < cnt && (d * span) / cnt == n && on) issue(dkb, lo + d, FAST);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };

        if (nkb > 0) {
            const lds_cptr ra0 = region(0, 0, a_org), rb0 = region(0, 0, b_org);
#pragma unroll
            for (int pa = 0; pa < NPA; ++pa) fa[pa] = read_a(ra0, pa);
            fb[0] = read_b(rb0, 0);
            fb[1] = read_b(rb0, 1);
        }
        static_assert(kDmaRB / 64 == 2, "two 64-byte K steps per stage");
        if (nkb == 0) issue_scales();
        auto stage = [&](int kb, auto FAST) __attribute__((always_inline)) {
            // FAST stages are 1 .. nkb - 3: the tests below hold
            constexpr bool F = decltype(FAST)::value;
            const bool nb = F || kb + 1 < nkb, n2 = F || kb + 2 < nkb;
            // no DMA is outstanding in the last stage: its waits are unaffected
            if (!nb) issue_scales();
            // the rest of stage kb + 1 (stage 1 went out whole in the prologue)
            stepq(kb, 0, kb, 1, false, kb + 1, nb && (F || kb >= 1), P1, Sh::LPS, 0, FAST);
            // the last two groups read stage kb + 1's step 0 (unused past the
            // end) and start stage kb + 2 in stage kb's buffer
            stepq(kb, 1, kb + 1, 0, nb, kb + 2, n2, 0, P1, NG - 2, FAST);
        };
        // Stages 1 .. kfast - 1 of a tile whose windows all lie inside M and
        // N issue all their DMA (stages kb + 1 and kb + 2 exist and lie inside
        // K) with no tests; the others test each instruction.
        const bool tile_full = a_rows0 == 8 && b_rows0 == 8 && (W == 1 || (a_rows1 == 8 && b_rows1 == 8));
        const int kfast = min(nkb - 2, nkb_full - kb0 - 2);
        {
            int kb = 0;
            if (nkb > 0) stage(kb++, kChecked);
            if (tile_full)
                for (; kb < kfast; ++kb) stage(kb, kFast);
            for (; kb < nkb; ++kb) stage(kb, kChecked);
        }

        // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
        wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);
        exec_barrier();
        if (S > 1) {
            // split-K, as in the ring kernel: each range stores its raw
            // accumulators (register e of tile n = (i, j, rh, ch) at (n * 4 + e)
            // * 64 + lane); the last range to arrive adds the others
            constexpr int NT = NI * L * NR * NR;
            constexpr int P0 = PairSplit<L, L>::P0, P = L * L;
            constexpr int RW = (P0 > P - P0 ? P0 : P - P0) * W * W * 16;
            static_assert(NT * 4 <= RW, "the hand-over slot holds the wave's tiles");
            const int ln = lane_here();
            uint32_t *mine = splitk_slot(p, g, krange, wave, RW, ln);
            auto tile = [&](int n) -> Acc & {
                return acc[n / (L * NR * NR)][(n / (NR * NR)) % L][(n / NR) % NR][n % NR];
            };
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const i32x4 u = __builtin_bit_cast(i32x4, tile(n));
#pragma unroll
                for (int e = 0; e < 4; ++e) splitk_put(mine + (n * 4 + e) * 64, (uint32_t)u[e]);
            }
            if (!splitk_arrive(p, g, (int *)buf(nkb + 1))) return;
            auto get4 = [&](const uint32_t *src) {
                i32x4 u;
#pragma unroll
                for (int e = 0; e < 4; ++e) u[e] = (int)splitk_get(src + e * 64);
                return __builtin_bit_cast(Acc, u);
            };
            // int32 sums are exact in any order: this range's accumulators
            // stay and the others are added; float sums: every range read
            // back, this one's too, in range order from range 0
            for (int s2 = 0; s2 < S; ++s2) {
                if (MF::kExactAcc && s2 == krange) continue;
                const uint32_t *src = splitk_slot(p, g, s2, wave, RW, ln);
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    const Acc v = get4(src + n * 4 * 64);
                    Acc &a = tile(n);
                    a = (!MF::kExactAcc && s2 == 0) ? v : a + v;
                }
            }
        }
        const int elane = lane_here();
        const int eq = elane & 15, eg = elane >> 4;
        // this wave's scales into registers: sa of its rows (its group's
        // slices), sb of its columns
        f32x4 sav[NI][NR];
        float sbv[L][NR];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int rh = 0; rh < NR; ++rh)
                sav[i][rh] = *(const f32x4 *)(sa_lds + (ILO + i) * BM + cbase_row + 16 * rh + 4 * eg);
#pragma unroll
        for (int j = 0; j < L; ++j)
#pragma unroll
            for (int ch = 0; ch < NR; ++ch) sbv[j][ch] = sb_lds[j * BN + cbase_col + 16 * ch + eq];
        // the partial sums overwrite the scales: every wave has read them
        __builtin_amdgcn_s_waitcnt(0xC07F);
        exec_barrier();
        // fl32(fl32(fl32(acc) * sa_i) * sb_j) of pair (i, j), summed i-major,
        // j-minor: group 0 from zero, group 1 onto group 0's sums
        auto sum_pairs = [&](OA out, int rh, int ch, int e) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < L; ++j) {
                    const float t1 = MF::to_f32(acc[i][j][rh][ch][e]) * sav[i][rh][e];
                    out = out + (OA)(t1 * sbv[j][ch]);
                }
            return out;
        };
        if constexpr (G == 0) {
#pragma unroll
            for (int rh = 0; rh < NR; ++rh)
#pragma unroll
                for (int ch = 0; ch < NR; ++ch)
#pragma unroll
                    for (int e = 0; e < 4; ++e) *pslot(rh, ch, e, elane) = sum_pairs((OA)0, rh, ch, e);
            __builtin_amdgcn_s_waitcnt(0xC07F);
            exec_barrier();
        } else {
            exec_barrier();
#pragma unroll
            for (int rh = 0; rh < NR; ++rh)
#pragma unroll
                for (int ch = 0; ch < NR; ++ch) {
                    const int64_t col = n0 + cbase_col + 16 * ch + eq;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int64_t row = m0 + cbase_row + 16 * rh + 4 * eg + e;
                        const OA out = sum_pairs(*pslot(rh, ch, e, elane), rh, ch, e);
                        if (col < p.N && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, out);
                    }
                }
        }
    };
    if (grp == 0) body(std::integral_constant<int, 0>{});
    else body(std::integral_constant<int, 1>{});
}

// ---------------------------------------------------------------------------
// The tile and stage of the one-wave-per-SIMD ("solo") kernel below, for
// num_splits L = 4, 5: 64 x 64 tiles, 4 waves, two whole stages of 128 bytes
// of K (2 x 16 L KB of LDS).
// ---------------------------------------------------------------------------
template <int L_> struct SoloShape {
    static constexpr int L = L_, BM = 64, BN = 64;
    static constexpr int NW = 4;                         // waves
    static constexpr int A_BYTES = L * BM * kDmaRB;      // 40 KB
    static constexpr int B_BYTES = L * BN * kDmaRB;      // 40 KB
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int LA = A_BYTES / (NW * 1024);     // A instructions per wave per stage
    static constexpr int LB = B_BYTES / (NW * 1024);
    static constexpr int LPS = LA + LB;
    static constexpr int LDS_BYTES = 2 * STAGE;
    static constexpr int NSC = L * (BM + BN) / 64;       // scale instructions (64 entries each)
    static constexpr int SCQ = (NSC + NW - 1) / NW;
    static_assert(A_BYTES % (NW * 1024) == 0 && B_BYTES % (NW * 1024) == 0,
                  "a half stage must be whole 1 KB windows per wave");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
    static_assert(kDmaRB == 128, "128-byte stage rows");
};

// The B group order and A read plan of cross_gemm_soloq_kernel (below).
template <int L, bool TRI> struct SoloQPlan {
    static constexpr int NG = 2 * L, D = 3;
    // group p of a K step is B fragment (gj(p), p / L): heavy and light
    // groups of the triangle alternate
    static constexpr int gj(int pos) {
        constexpr int jo5[5] = {0, 4, 1, 3, 2}, jo4[4] = {0, 3, 1, 2};
        return L == 5 ? jo5[pos % 5] : jo4[pos % 4];
    }
    // the group after which A fragment row i is read for the next step: its
    // last use in the step, and not before the barrier group NG - D
    static constexpr int a_next(int i) {
        int last = 0;
        for (int pos = 0; pos < NG; ++pos)
            if (Pairs<L, TRI>::kept(i, gj(pos))) last = pos;
        return last > NG - D ? last : NG - D;
    }
};
static_assert(SoloQPlan<5, true>::a_next(4) == 7 && SoloQPlan<5, true>::a_next(3) == 7 &&
                  SoloQPlan<5, true>::a_next(2) == 9 && SoloQPlan<5, false>::a_next(4) == 9 &&
                  SoloQPlan<4, true>::a_next(3) == 5 && SoloQPlan<4, true>::a_next(0) == 7,
              "solo read plan");

// ---------------------------------------------------------------------------
// The solo configuration on 16 x 16 MFMAs (int8, fp16, bf16 slices), for
// num_splits L = 5 and the triangle at 4: 64 x 64 tiles, 4 waves (one per
// SIMD), wave (x, y) = (w / 2, w % 2) holding every kept pair of 32 x 32
// block (x, y) as 4 tiles of 16 x 16: acc[n][rh][ch] for pair n (i-major,
// j-minor), register e of lane l at row 16 rh + 4 (l / 16) + e, column 16 ch
// + l % 16 of the block.  L = 5, all 25 pairs: 100 tiles, 400 registers,
// pairs 0..15 in AGPRs and 16..24 in VGPRs; the triangles (60 and 40 tiles)
// and L = 4's 16 pairs all in AGPRs.  The MFMAs are inline assembly with the
// accumulator's file fixed (the compiler does not split accumulators between
// the files itself).  Per 64-byte K step a wave reads its 2 L A fragments (i,
// rh), resident through the step, and its 2 L B fragments (j, ch) through a
// ring (5 slots at L = 5, 4 at L = 4), B group p + 3 read while group p's
// MFMAs run; group p is B fragment (jo[p % L], p / L), jo = 0, 4, 1, 3, 2 (L
// = 4: 0, 3, 1, 2), so that any three groups of a triangle hold at least 12
// MFMAs.  The next step's A fragment (i, rh) is read after its last MFMA of
// the step, and not before group 2 L - 3, where the stage barrier sits.  The
// LDS holds two whole stages (2 x 16 L KB); DMA windows and the unchecked DMA
// of interior stages as in cross_gemm_ringq_kernel.  Hazards of the
// hand-placed MFMAs: results read only in the epilogue, after 64 wait states;
// an accumulator read as srcC first after its zero fill and the prologue
// barrier, and again only tens of MFMAs later.
// ---------------------------------------------------------------------------
template <typename ST, int L_, typename AccT, bool TRI>
__global__ __launch_bounds__(256, 1) void cross_gemm_soloq_kernel(GemmParams p, int group_m,
                                                                  uint32_t a_records,
                                                                  uint32_t b_records) {
    resolve_split_fail(p);
    using Sh = SoloShape<L_>;
    using MF = Mfma16<ST>;
    using Acc = typename MF::Acc;
    using OA = AccT;
    constexpr int L = Sh::L, BM = Sh::BM, BN = Sh::BN;
    using PS = Pairs<L, TRI>;
    constexpr int ES = (int)sizeof(ST);
    constexpr uint32_t kOOB = 0x80000000u;
    // DMA of stage kb + 2: P1 instructions after the barrier of stage kb, the
    // rest in groups 0 .. G0 - 1 of stage kb + 1's first step.  The triangle's
    // steps are 60 MFMAs long, and its DMA goes out earlier (8192^3, int8,
    // TFLOP/s end to end against (4, 10): (10, 4) 158.8, (12, 5) 156.8, (8, 5)
    // 156.7, (8, 3) 155.9, (8, 10) 153.7, (4, 5) 151.3, (4, 10) 149.5; all
    // pairs: (4, 10) 121.9, (8, 10) 121.4, (8, 5) 120.2, (4, 5) 118.9).
    constexpr int P1 = L == 5 ? (TRI ? 10 : 4) : (TRI ? 8 : 4);
    constexpr int G0 = L == 5 ? (TRI ? 4 : 10) : (TRI ? 3 : 8);
    constexpr int NAG = TRI || PS::N <= 16 ? PS::N : 16;   // pairs whose tiles sit in AGPRs
    constexpr int NG = 2 * L, D = 3;                       // B groups per step, read distance
    constexpr int R = NG % 5 == 0 ? 5 : 4;                 // B ring slots
    constexpr int NPA = 2 * L;                             // A fragments (i, rh)
    static_assert(Sh::NW == 4 && Sh::LA == 2 * L && Sh::LB == 2 * L && BM == 64 && BN == 64,
                  "the window arithmetic below is written for this shape");
    static_assert(NG % R == 0 && R > D && NAG * 4 * 4 <= 256, "ring; AGPR file");
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wx = wave >> 1, wy = wave & 1;

    const int64_t tiles_m = (p.M + BM - 1) / BM;
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t tiles = tiles_m * tiles_n;
    const int64_t g = xcd_remap_gemm(blockIdx.x, (int64_t)gridDim.x);
    const int64_t bidx = g / tiles;
    const int64_t t = g % tiles;
    const int64_t width = (int64_t)group_m * tiles_n;
    const int64_t first_m = (t / width) * group_m;
    const int64_t gsz = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
    const int64_t tm = first_m + (t % width) % gsz;
    const int64_t tn = (t % width) / gsz;
    const int64_t m0 = tm * BM, n0 = tn * BN;

    const uint32_t kbytes = (uint32_t)(p.K * ES);
    const int nkb = (int)((kbytes + kDmaRB - 1) / kDmaRB);

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.A + bidx * p.as_b * ES), (short)0, (int)a_records, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const char *)p.B + bidx * p.bs_b * ES), (short)0, (int)b_records, 0x00020000);

    // Stage DMA: 1 KB windows of 8 whole 128-byte rows (lane -> row lane / 8,
    // physical chunk lane % 8, which holds logical chunk c0 = (lane % 8) ^
    // (lane / 16) in an even window and c0 ^ 4 in an odd one); the stage's
    // windows r = 8 s + x (slice s, rows 8 x of the tile) sit at r KB of the A
    // and B regions.  Wave w fetches windows w + 4 q of each (q < 10: slice q
    // / 2, row window w + 4 (q % 2)): its windows share its parity, and their
    // sources are a base, plus a slice stride, plus 32 rows.
    const int64_t a_first = m0 + 8 * wave, b_first = n0 + 8 * wave;
    const uint32_t a_base = (uint32_t)__builtin_amdgcn_readfirstlane((int)((a_first * p.as_m) * ES));
    const uint32_t b_base = (uint32_t)__builtin_amdgcn_readfirstlane((int)((b_first * p.bs_n) * ES));
    const uint32_t a_sstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(p.as_l * ES));
    const uint32_t b_sstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(p.bs_l * ES));
    const uint32_t a_hstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(32 * p.as_m * ES));
    const uint32_t b_hstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)(32 * p.bs_n * ES));
    // rows of this wave's windows inside the operand (may be <= 0)
    const int a_rows0 = (int)(p.M - a_first < 8 ? p.M - a_first : 8);
    const int a_rows1 = (int)(p.M - a_first - 32 < 8 ? p.M - a_first - 32 : 8);
    const int b_rows0 = (int)(p.N - b_first < 8 ? p.N - b_first : 8);
    const int b_rows1 = (int)(p.N - b_first - 32 < 8 ? p.N - b_first - 32 : 8);
    uint32_t lane_src[2];   // [A, B]
    {
        const int c0 = (lane & 7) ^ (lane >> 4);
        const uint32_t chb = (uint32_t)((wave & 1) ? (c0 ^ 4) : c0) * 16;
        lane_src[0] = (uint32_t)((lane >> 3) * p.as_m * ES) + chb;
        lane_src[1] = (uint32_t)((lane >> 3) * p.bs_n * ES) + chb;
    }
    const int nkb_full = (int)(kbytes / kDmaRB);   // stages inside K
    auto buf = [&](int kb) { return smem + (kb & 1) * Sh::STAGE; };
    // DMA instruction q (< LA: A window q of this wave; else B window q - LA)
    // of stage kb; q is a constant at every call.  FAST: the window's rows and
    // the stage are known to lie inside the operand, and the uniform part of
    // the source is the instruction's scalar offset.
    auto issue = [&](int kb, int q, auto FAST) {
        const bool isa = q < Sh::LA;
        const int qq = isa ? q : q - Sh::LA;
        const uint32_t ub = (isa ? a_base + (uint32_t)(qq >> 1) * a_sstep + ((qq & 1) ? a_hstep : 0u)
                                 : b_base + (uint32_t)(qq >> 1) * b_sstep + ((qq & 1) ? b_hstep : 0u)) +
                            (uint32_t)kb * kDmaRB;
        const uint32_t lsrc = lane_src[isa ? 0 : 1];
        auto *ldsp = (__attribute__((address_space(3))) void *)(
            buf(kb) + (isa ? 0 : Sh::A_BYTES) + (wave + 4 * qq) * 1024);
        if constexpr (decltype(FAST)::value) {
            if (isa) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, lsrc, (int)ub, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, lsrc, (int)ub, 0, 0);
            return;
        }
        const int rows = isa ? ((qq & 1) ? a_rows1 : a_rows0) : ((qq & 1) ? b_rows1 : b_rows0);
        uint32_t vo;
        if (rows == 8 && kb < nkb_full) {
            vo = lsrc + ub;
        } else {
            const int kleft = (int)kbytes - kb * kDmaRB;   // > 0
            const int ln = lane_here();
            const int c0 = (ln & 7) ^ (ln >> 4);
            const int chb = ((wave & 1) ? (c0 ^ 4) : c0) * 16;
            vo = ((ln >> 3) < rows && chb < kleft) ? lsrc + ub : kOOB;
        }
        if (isa) __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, ldsp, 16, vo, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, ldsp, 16, vo, 0, 0, 0);
    };

    // The tile's scales (A's [L][BM], then B's [L][BN]: 2560 bytes) into the
    // buffer of stage nkb at the start of the last stage: instruction u (wave
    // u % 4) fetches entries 64 u .. 64 u + 63.
    char *const scl = buf(nkb);
    auto issue_scales = [&]() {
#pragma unroll
        for (int q = 0; q < Sh::SCQ; ++q) {
            const int u = q * Sh::NW + wave;
            if (u >= Sh::NSC) break;
            const bool isa = u < L * BM / 64;
            const int e = (isa ? u : u - L * BM / 64) * 64 + lane_here();
            const int s = isa ? e / BM : e / BN;                 // slice
            const int64_t rc = isa ? m0 + e % BM : n0 + e % BN;  // row of A / column of B
            const int64_t ext = isa ? ((int64_t)(L - 1) * p.sas_l + (p.M - 1) * p.sas_m + 1)
                                    : ((int64_t)(L - 1) * p.sbs_l + (p.N - 1) * p.sbs_n + 1);
            const bool ok = rc < (isa ? p.M : p.N);
            const uint32_t vo = ok ? (uint32_t)(((int64_t)s * (isa ? p.sas_l : p.sbs_l) +
                                                 rc * (isa ? p.sas_m : p.sbs_n)) * 4)
                                   : kOOB;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(isa ? p.sa + bidx * p.sas_b : p.sb + bidx * p.sbs_b), (short)0,
                (int)(ext * 4 < 0x7FFFFFFF ? ext * 4 : 0x7FFFFFFF), 0x00020000);
            auto *ldsp = (__attribute__((address_space(3))) void *)(scl + u * 256);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, ldsp, 4, vo, 0, 0, 0);
        }
    };
    const float *sa_lds = (const float *)scl, *sb_lds = (const float *)(scl + L * BM * 4);

    Acc acc[PS::N][2][2];
    static_for<PS::N>([&](auto n_) {
        constexpr int n = decltype(n_)::value;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            acc[n][x >> 1][x & 1] = MF::zero();
            // pinned where the hand-placed MFMAs keep it
            if constexpr (n < NAG) asm volatile("" : "+a"(acc[n][x >> 1][x & 1]));
            else asm volatile("" : "+v"(acc[n][x >> 1][x & 1]));
        }
    });
    asm volatile("s_nop 7" ::: "memory");

    // prologue: stages 0 and 1; stage 0 must land before the first reads
    constexpr std::false_type kChecked{};
    constexpr std::true_type kFast{};
#pragma unroll
    for (int q = 0; q < Sh::LPS; ++q) issue(0, q, kChecked);
    if (nkb > 1) {
#pragma unroll
        for (int q = 0; q < Sh::LPS; ++q) issue(1, q, kChecked);
        wait_vmcnt<Sh::LPS>();
    } else {
        wait_vmcnt<0>();
    }
    exec_barrier();

    // fragments: one lane address per region and K step, the fragment's row
    // its LDS read's immediate
    const int qrow = lane & 15;
    const int key = (qrow >> 1) & 7;
    int lane_rd[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) lane_rd[kk] = qrow * kDmaRB + (((4 * kk + (lane >> 4)) ^ key) << 4);
    const int smem_base = (int)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
    using lds_cptr = const __attribute__((address_space(3))) char *;
    const int a_org = wx * 32 * kDmaRB;
    const int b_org = Sh::A_BYTES + wy * 32 * kDmaRB;
    auto region = [&](int kb, int kk, int org) {
        const int u = __builtin_amdgcn_readfirstlane(smem_base + (kb & 1) * Sh::STAGE + org);
        return (lds_cptr)(uintptr_t)(u + lane_rd[kk]);
    };
    auto read_a = [&](lds_cptr ra, int pa) {   // A fragment pa = (i, rh)
        return *(const __attribute__((address_space(3))) i32x4 *)(
            ra + ((pa >> 1) * BM + 16 * (pa & 1)) * kDmaRB);
    };
    using QP = SoloQPlan<L, TRI>;
    auto read_b = [&](lds_cptr rb, int pos) {   // B fragment of group pos
        return *(const __attribute__((address_space(3))) i32x4 *)(
            rb + (QP::gj(pos) * BN + 16 * (pos / L)) * kDmaRB);
    };

    i32x4 fa[NPA];   // A fragments, resident through a K step
    i32x4 fb[R];     // B groups p .. p + 4 (p mod 5)

    // One K step: group pos runs the MFMAs of B fragment pos with every kept
    // A fragment and first reads B group pos + 3 (groups 7..9: groups 0..2 of
    // the next step, stage nkb_, step nkk).  With `bar`, group 7 starts behind
    // the stage barrier.  DMA instructions [lo, hi) of stage dkb go between
    // the MFMA slots of groups dg0 .. dg1 - 1 (LO, HI, DG0, DG1: compile-time
    // constants; FAST: as issue's).
    auto stepq = [&](int ckb, int ckk, int nkb_, int nkk, bool bar, int dkb, bool on, auto LO,
                     auto HI, auto DG0, auto DG1, auto FAST) __attribute__((always_inline)) {
        constexpr int lo = decltype(LO)::value, cnt = decltype(HI)::value - lo;
        constexpr int dg0 = decltype(DG0)::value, dg1 = decltype(DG1)::value;
        constexpr int span = (dg1 - dg0) * NPA;
        const lds_cptr rb_cur = region(ckb, ckk, b_org);
        static_for<NG>([&](auto pos_) {
            constexpr int pos = decltype(pos_)::value;
            if constexpr (pos + D < NG) {
                fb[(pos + D) % R] = read_b(rb_cur, pos + D);
            } else {
                if (pos == NG - D && bar) {
                    // stage nkb_ has landed (this wave's DMA, then every
                    // wave's through the barrier), and every wave's reads of
                    // stage ckb are complete before its buffer is refilled
                    wait_vmcnt<0>();
                    __builtin_amdgcn_s_waitcnt(0xC07F);
                    exec_barrier();
                }
                fb[(pos + D) % R] = read_b(region(nkb_, nkk, b_org), pos + D - NG);
            }
            constexpr int j = QP::gj(pos), ch = pos / L;
            static_for<NPA>([&](auto pa_) {
                constexpr int pa = decltype(pa_)::value;
                constexpr int i = pa >> 1, rh = pa & 1;
                if constexpr (PS::kept(i, j)) {
                    constexpr int n = PS::first(i) + j;
                    MF::template run<(n < NAG)>(acc[n][rh][ch], fa[pa], fb[pos % R]);
                }
                if constexpr (pos == QP::a_next(i)) fa[pa] = read_a(region(nkb_, nkk, a_org), pa);
                constexpr int n = (pos - dg0) * NPA + pa;
                static_for<cnt>([&](auto d_) {
                    // instruction lo + d goes after slot (d * span) / cnt of the span
                    constexpr int d = decltype(d_)::value;
                    if constexpr (pos >= dg0 && pos < dg1 && (d * span) / cnt == n) {
                        if (on) issue(dkb, lo + d, FAST);
                    }
                });
                __builtin_amdgcn_sched_barrier(0);
            });
        });
    };

    if (nkb > 0) {
        const lds_cptr ra0 = region(0, 0, a_org), rb0 = region(0, 0, b_org);
#pragma unroll
        for (int pa = 0; pa < NPA; ++pa) fa[pa] = read_a(ra0, pa);
#pragma unroll
        for (int pos = 0; pos < D; ++pos) fb[pos] = read_b(rb0, pos);
    }
    static_assert(kDmaRB / 64 == 2, "two 64-byte K steps per stage");
    if (nkb == 0) issue_scales();
    auto stage = [&](int kb, auto FAST) __attribute__((always_inline)) {
        // FAST stages are 1 .. nkb - 3: the tests below hold
        constexpr bool F = decltype(FAST)::value;
        const bool nb = F || kb + 1 < nkb, n2 = F || kb + 2 < nkb;
        // no DMA is outstanding in the last stage: its waits are unaffected
        if (!nb) issue_scales();
        // the rest of stage kb + 1 (stage 1 went out whole in the prologue)
        stepq(kb, 0, kb, 1, false, kb + 1, nb && (F || kb >= 1), std::integral_constant<int, P1>{},
              std::integral_constant<int, Sh::LPS>{}, std::integral_constant<int, 0>{},
              std::integral_constant<int, G0>{}, FAST);
        // groups 7..9 read stage kb + 1's step 0 (unused past the end) and
        // start stage kb + 2 in stage kb's buffer
        stepq(kb, 1, kb + 1, 0, nb, kb + 2, n2, std::integral_constant<int, 0>{},
              std::integral_constant<int, P1>{}, std::integral_constant<int, NG - D>{},
              std::integral_constant<int, NG>{}, FAST);
    };
    // Stages 1 .. kfast - 1 of a tile whose windows all lie inside M and N
    // issue all their DMA (stages kb + 1 and kb + 2 exist and lie inside K)
    // with no tests; the others test each instruction.
    const bool tile_full = a_rows0 == 8 && a_rows1 == 8 && b_rows0 == 8 && b_rows1 == 8;
    const int kfast = min(nkb - 2, nkb_full - 2);
    {
        int kb = 0;
        if (nkb > 0) stage(kb++, kChecked);
        if (tile_full)
            for (; kb < kfast; ++kb) stage(kb, kFast);
        for (; kb < nkb; ++kb) stage(kb, kChecked);
    }

    // the hand-placed MFMAs' results are read below: 64 wait states first
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");

    // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    exec_barrier();
    const int elane = lane_here();
    const int eq = elane & 15, eg = elane >> 4;
    const int64_t cbase = bidx * p.cs_b;
    float sbv[L][2];
#pragma unroll
    for (int j = 0; j < L; ++j)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) sbv[j][ch] = sb_lds[j * BN + wy * 32 + 16 * ch + eq];
    OA out[2][2][4];
#pragma unroll
    for (int rh = 0; rh < 2; ++rh)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
            for (int e = 0; e < 4; ++e) out[rh][ch][e] = (OA)0;
    static_for<L>([&](auto i_) {
        constexpr int i = decltype(i_)::value;
        f32x4 s4[2];
#pragma unroll
        for (int rh = 0; rh < 2; ++rh) s4[rh] = *(const f32x4 *)(sa_lds + i * BM + wx * 32 + 16 * rh + 4 * eg);
        static_for<L>([&](auto j_) {
            constexpr int j = decltype(j_)::value;
            if constexpr (PS::kept(i, j)) {
                constexpr int n = PS::first(i) + j;
#pragma unroll
                for (int rh = 0; rh < 2; ++rh)
#pragma unroll
                    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            // fl32(fl32(fl32(acc) * sa_i) * sb_j), summed i-major, j-minor
                            const float t1 = MF::to_f32(acc[n][rh][ch][e]) * s4[rh][e];
                            out[rh][ch][e] = out[rh][ch][e] + (OA)(t1 * sbv[j][ch]);
                        }
                __builtin_amdgcn_sched_barrier(0);
            }
        });
    });
#pragma unroll
    for (int rh = 0; rh < 2; ++rh)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
            const int64_t col = n0 + wy * 32 + 16 * ch + eq;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t row = m0 + wx * 32 + 16 * rh + 4 * eg + e;
                if (col < p.N && row < p.M) store_c(p, cbase + row * p.cs_m + col * p.cs_n, out[rh][ch][e]);
            }
        }
}

// ---------------------------------------------------------------------------
// Launch templates (host side)
// ---------------------------------------------------------------------------
// byte extent [0, bytes) one batch of a slice operand spans, or -1 if it does
// not fit the 31-bit buffer offsets of the DMA kernel.  The last row counts
// up to its 16-byte boundary: the kernels load 16-byte pieces, and a piece
// that crosses the buffer's end comes back zeroed as a whole, which would
// drop the row's last elements.  Those bytes exist and are zero: operands
// whose rows are not whole 16-byte pieces are the pack kernel's zero-padded
// copies (K * es is a multiple of 16 for every other operand).
static inline int64_t dma_extent(int64_t s_l, int64_t s_r, int L, int64_t rows, int64_t K, int es) {
    if (s_l < 0 || s_r < 0) return -1;
    const int64_t row_bytes = (K * es + 15) / 16 * 16;
    const int64_t e = ((int64_t)(L - 1) * s_l + (rows - 1) * s_r) * es + row_bytes;
    return (e < ((int64_t)1 << 31) - 64) ? e : -1;
}

// Raise a kernel's dynamic LDS limit (above the 64 KB default) once per
// device.  `done` is that kernel's bitmask of devices already set (bit d:
// device d); concurrent first calls may both set it, which is harmless.
static inline hipError_t set_lds_limit(const void *kern, int bytes, std::atomic<uint64_t> &done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = (dev >= 0 && dev < 64) ? (1ull << dev) : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
    return e;
}


template <typename ST, int L, int MI, int NI, typename AccT, bool TRI>
static hipError_t launch_dma(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    using Sh = DmaShape<L, MI, NI>;
    auto kern = cross_gemm_dma_kernel<ST, L, MI, NI, AccT, TRI>;
    static std::atomic<uint64_t> lds_set{0};   // devices whose LDS limit is raised
    if (hipError_t e = set_lds_limit((const void *)kern, Sh::LDS_BYTES, lds_set)) return e;
    const int es = (int)sizeof(ST);
    const int64_t ea = dma_extent(p.as_l, p.as_m, L, p.M, p.K, es);
    const int64_t eb = dma_extent(p.bs_l, p.bs_n, L, p.N, p.K, es);
    const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256), Sh::LDS_BYTES, st, p,
                       plan.group_m, (uint32_t)ea, (uint32_t)eb);
    return hipGetLastError();
}

template <typename ST, int L, typename AccT, bool TRI, int G = 1>
static hipError_t launch_kstep(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    using Sh = KStepShape<L, TRI, G>;
    auto kern = cross_gemm_kstep_kernel<ST, L, AccT, TRI, G>;
    static std::atomic<uint64_t> lds_set{0};   // devices whose LDS limit is raised
    if (hipError_t e = set_lds_limit((const void *)kern, Sh::LDS_BYTES, lds_set)) return e;
    const int es = (int)sizeof(ST);
    const int64_t ea = dma_extent(p.as_l, p.as_m, L, p.M, p.K, es);
    const int64_t eb = dma_extent(p.bs_l, p.bs_n, L, p.N, p.K, es);
    const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256 * G), Sh::LDS_BYTES, st, p,
                       plan.group_m, (uint32_t)ea, (uint32_t)eb);
    return hipGetLastError();
}

template <typename ST, int L, typename AccT, int R, bool TRI = false>
static hipError_t launch_pair(const GemmParams &p, const GemmPlan &plan, hipStream_t st, int i0,
                              int cont) {
    using Sh = PairShape<L, R>;
    auto kern = cross_gemm_pair_kernel<ST, L, AccT, R, TRI>;
    static std::atomic<uint64_t> lds_set{0};   // devices whose LDS limit is raised
    if (hipError_t e = set_lds_limit((const void *)kern, Sh::LDS_BYTES, lds_set)) return e;
    const int es = (int)sizeof(ST);
    const int64_t ea = dma_extent(p.as_l, p.as_m, L, p.M, p.K, es);
    const int64_t eb = dma_extent(p.bs_l, p.bs_n, L, p.N, p.K, es);
    const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(512), Sh::LDS_BYTES, st, p,
                       plan.group_m, (uint32_t)ea, (uint32_t)eb, i0, cont);
    return hipGetLastError();
}

template <typename ST, int L, typename AccT>
static hipError_t launch_ring(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    constexpr int W = (L <= 2) ? 2 : 1;
    // int8 / fp16 / bf16 slices: the 16 x 16 MFMA form (same tiles, pair
    // groups and split-K hand-over; fp32 slices keep the 32 x 32 x 2 one)
    constexpr bool kQ = !std::is_same<ST, float>::value;
    using Sh = std::conditional_t<kQ, RingQShape<L, W>, RingShape<L, W>>;
    auto kern = [] {
        if constexpr (kQ) return cross_gemm_ringq_kernel<ST, L, W, AccT>;
        else return cross_gemm_ring_kernel<ST, L, AccT, W>;
    }();
    static_assert(Sh::BM == 64 * W && Sh::BN == 64 * W, "the planner's tile size");
    static std::atomic<uint64_t> lds_set{0};   // devices whose LDS limit is raised
    if (hipError_t e = set_lds_limit((const void *)kern, Sh::LDS_BYTES, lds_set)) return e;
    const int es = (int)sizeof(ST);
    const int64_t ea = dma_extent(p.as_l, p.as_m, L, p.M, p.K, es);
    const int64_t eb = dma_extent(p.bs_l, p.bs_n, L, p.N, p.K, es);
    const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
    if (tiles == 0) return hipSuccess;
    const int64_t ranges = p.ksplit > 1 ? p.ksplit : 1;
    hipLaunchKernelGGL(kern, dim3((unsigned)(tiles * ranges)), dim3(512), Sh::LDS_BYTES, st, p,
                       plan.group_m, (uint32_t)ea, (uint32_t)eb);
    return hipGetLastError();
}

template <typename ST, typename AccT, bool TRI>
static hipError_t launch_wide(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    using Sh = WideShape;
    // int8 / fp16 / bf16 slices: the 16 x 16 MFMA form (fp32 slices keep the
    // 32 x 32 x 2 one)
    auto kern = [] {
        if constexpr (std::is_same<ST, float>::value) return cross_gemm_wide_kernel<ST, AccT, TRI>;
        else return cross_gemm_wideq_kernel<ST, AccT, TRI>;
    }();
    static std::atomic<uint64_t> lds_set{0};   // devices whose LDS limit is raised
    if (hipError_t e = set_lds_limit((const void *)kern, Sh::LDS_BYTES, lds_set)) return e;
    const int es = (int)sizeof(ST);
    const int64_t ea = dma_extent(p.as_l, p.as_m, Sh::L, p.M, p.K, es);
    const int64_t eb = dma_extent(p.bs_l, p.bs_n, Sh::L, p.N, p.K, es);
    const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
    if (tiles == 0) return hipSuccess;
    const int64_t ranges = p.ksplit > 1 ? p.ksplit : 1;
    hipLaunchKernelGGL(kern, dim3((unsigned)(tiles * ranges)), dim3(512), Sh::LDS_BYTES, st, p,
                       plan.group_m, (uint32_t)ea, (uint32_t)eb);
    return hipGetLastError();
}

template <typename ST, typename AccT, bool TRI>
static hipError_t launch_wide4(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    using Sh = Wide4Shape;
    // int8 / fp16 / bf16 slices: the 16 x 16 form (the same tile, pairs and bits; fp32 slices keep
    // the 32 x 32 x 2 one)
    auto kern = [] {
        if constexpr (std::is_same<ST, float>::value) return cross_gemm_wide4_kernel<ST, AccT, TRI>;
        else return cross_gemm_wide4q_kernel<ST, AccT, TRI>;
    }();
    static std::atomic<uint64_t> lds_set{0};   // devices whose LDS limit is raised
    if (hipError_t e = set_lds_limit((const void *)kern, Sh::LDS_BYTES, lds_set)) return e;
    const int es = (int)sizeof(ST);
    const int64_t ea = dma_extent(p.as_l, p.as_m, Sh::L, p.M, p.K, es);
    const int64_t eb = dma_extent(p.bs_l, p.bs_n, Sh::L, p.N, p.K, es);
    const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(512), Sh::LDS_BYTES, st, p,
                       plan.group_m, (uint32_t)ea, (uint32_t)eb);
    return hipGetLastError();
}

template <typename ST, int L, typename AccT, bool TRI>
static hipError_t launch_solo(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    if constexpr (std::is_same<ST, float>::value) {
        return hipErrorInvalidValue;   // no fp32-slice form
    } else {
        using Sh = SoloShape<L>;
        auto kern = cross_gemm_soloq_kernel<ST, L, AccT, TRI>;
        static std::atomic<uint64_t> lds_set{0};   // devices whose LDS limit is raised
        if (hipError_t e = set_lds_limit((const void *)kern, Sh::LDS_BYTES, lds_set)) return e;
        const int es = (int)sizeof(ST);
        const int64_t ea = dma_extent(p.as_l, p.as_m, Sh::L, p.M, p.K, es);
        const int64_t eb = dma_extent(p.bs_l, p.bs_n, Sh::L, p.N, p.K, es);
        const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
        if (tiles == 0) return hipSuccess;
        hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256), Sh::LDS_BYTES, st, p,
                           plan.group_m, (uint32_t)ea, (uint32_t)eb);
        return hipGetLastError();
    }
}

// num_splits = 5..8: launches over consecutive i-rows (at most 16 pairs each,
// so a wave group still holds 8 pairs), in i-major order, each continuing the
// fp64 sum from C.  int8 / fp16 / bf16 slices with an fp64 outer accumulator.
template <typename ST, int L, typename AccT>
static hipError_t launch_chunks(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    if constexpr (!std::is_same<AccT, double>::value || std::is_same<ST, float>::value) {
        return hipErrorInvalidValue;
    } else {
        constexpr int R = (L == 5) ? 3 : 2;   // rows per launch (16 / L, at least 2)
        hipError_t e = hipSuccess;
        for (int i0 = 0; i0 < L && e == hipSuccess; i0 += R) {
            const int cont = i0 > 0;
            if (L - i0 >= R) e = launch_pair<ST, L, AccT, R>(p, plan, st, i0, cont);
            else if constexpr (L % R != 0) e = launch_pair<ST, L, AccT, L % R>(p, plan, st, i0, cont);
        }
        return e;
    }
}

// TRI: the triangular pair set, which the kernels that hold every pair of a
// block in one wave sum (staged, dma, ad, kstep, wide, solo5), wide4 and the
// pair-split kernel over all i-rows in one launch (L = 3..5); the ring kernel
// is not instantiated for it, and the planner does not choose it.
template <typename ST, int L, int MI, int NI, typename AccT, bool TRI>
static hipError_t launch_one(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    if constexpr (!TRI) {
        if constexpr (L >= 3) {
            if (plan.kind == kGemmPair) return launch_pair<ST, L, AccT, L>(p, plan, st, 0, 0);
        }
        if constexpr (L >= 2 && L <= 4) {
            if (plan.kind == kGemmRing) return launch_ring<ST, L, AccT>(p, plan, st);
        }
    } else {
        if constexpr (L >= 3) {
            // one launch over the kept pairs of all i-rows
            if (plan.kind == kGemmPair) return launch_pair<ST, L, AccT, L, true>(p, plan, st, 0, 0);
        }
        if (plan.kind == kGemmPair || plan.kind == kGemmRing) return hipErrorInvalidValue;
    }
    if constexpr (L == 4) {
        if (plan.kind == kGemmWide4) return launch_wide4<ST, AccT, TRI>(p, plan, st);
    }
    if constexpr (L == 3) {
        if (plan.kind == kGemmWide) return launch_wide<ST, AccT, TRI>(p, plan, st);
    }
    if (plan.kind == kGemmDMA) return launch_dma<ST, L, MI, NI, AccT, TRI>(p, plan, st);
    using Sh = GemmShape<L, MI, NI>;
    auto kern = cross_gemm_kernel<ST, L, MI, NI, AccT, TRI>;
    static std::atomic<uint64_t> lds_set{0};   // devices whose LDS limit is raised
    if (hipError_t e = set_lds_limit((const void *)kern, Sh::LDS_BYTES, lds_set)) return e;
    const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256), Sh::LDS_BYTES, st, p,
                       plan.group_m);
    return hipGetLastError();
}

template <typename ST, int L, typename AccT, bool TRI>
static hipError_t launch_L(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    // (fp32 slices at L = 4: no hand-placed MFMA, so no K-step kernel)
    if constexpr (L <= 4 && !(L == 4 && std::is_same_v<ST, float>)) {
        if (plan.kind == kGemmKStep) return launch_kstep<ST, L, AccT, TRI>(p, plan, st);
    }
    if constexpr (L >= 2 && L <= 4) {
        if (plan.kind == kGemmKStep2) return launch_kstep<ST, L, AccT, TRI, 2>(p, plan, st);
    }
    const int key = plan.mi * 10 + plan.ni;
    if constexpr (L == 1) {
        switch (key) {
        case 24: return launch_one<ST, 1, 2, 4, AccT, TRI>(p, plan, st);
        case 22: return launch_one<ST, 1, 2, 2, AccT, TRI>(p, plan, st);
        case 12: return launch_one<ST, 1, 1, 2, AccT, TRI>(p, plan, st);
        case 11: return launch_one<ST, 1, 1, 1, AccT, TRI>(p, plan, st);
        }
    } else if constexpr (L == 2) {
        switch (key) {
        case 22: return launch_one<ST, 2, 2, 2, AccT, TRI>(p, plan, st);
        case 12: return launch_one<ST, 2, 1, 2, AccT, TRI>(p, plan, st);
        case 11: return launch_one<ST, 2, 1, 1, AccT, TRI>(p, plan, st);
        }
    } else if constexpr (L <= 4) {
        if constexpr (L == 4)
            if (plan.kind == kGemmSolo) return launch_solo<ST, 4, AccT, TRI>(p, plan, st);
        if (key == 11) return launch_one<ST, L, 1, 1, AccT, TRI>(p, plan, st);
    } else if constexpr (L == 5) {
        if (plan.kind == kGemmSolo) return launch_solo<ST, 5, AccT, TRI>(p, plan, st);
        if constexpr (!TRI) return launch_chunks<ST, L, AccT>(p, plan, st);
        // the 15 kept pairs split 8 / 7 over the wave groups: one launch
        else if (plan.kind == kGemmPair && !std::is_same_v<ST, float>)
            return launch_pair<ST, 5, AccT, 5, true>(p, plan, st, 0, 0);
    } else if constexpr (!TRI) {
        return launch_chunks<ST, L, AccT>(p, plan, st);
    }
    return hipErrorInvalidValue;
}

template <typename ST, typename AccT, bool TRI>
static hipError_t launch_st(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t st) {
    switch (L) {
    case 1: return launch_L<ST, 1, AccT, false>(p, plan, st);   // one pair either way
    case 2: return launch_L<ST, 2, AccT, TRI>(p, plan, st);
    case 3: return launch_L<ST, 3, AccT, TRI>(p, plan, st);
    case 4: return launch_L<ST, 4, AccT, TRI>(p, plan, st);
    case 5: return launch_L<ST, 5, AccT, TRI>(p, plan, st);
    case 6: return launch_L<ST, 6, AccT, TRI>(p, plan, st);
    case 7: return launch_L<ST, 7, AccT, TRI>(p, plan, st);
    case 8: return launch_L<ST, 8, AccT, TRI>(p, plan, st);
    }
    return hipErrorInvalidValue;
}

// the entry point of one slice dtype's unit (ozk_gemm_<dtype>.hip)
template <typename ST>
static hipError_t launch_typed(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t st) {
    const bool acc64 = p.out_dtype == 0;
    if (p.tri) return acc64 ? launch_st<ST, double, true>(p, plan, L, st)
                            : launch_st<ST, float, true>(p, plan, L, st);
    return acc64 ? launch_st<ST, double, false>(p, plan, L, st)
                 : launch_st<ST, float, false>(p, plan, L, st);
}
}  // namespace ozk
