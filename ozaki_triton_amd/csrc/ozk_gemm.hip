// ozk_gemm.hip -- the fused cross-GEMM of ozaki_triton.py:306-452 as an
// LDS-staged MFMA kernel for gfx950.
//
//   C[m, n] = sum_{i<L} sum_{j<L} fl32(fl32(fl32(acc_ij[m, n]) * sa_i[m]) * sb_j[n])
//   acc_ij  = A_i[m, :] . B_j[:, n]        (int8: exact int32, fp16: fp32 MFMA)
//   the outer sum runs i-major, j-minor from +0 in the output's accumulator
//   dtype (fp64 for fp64 inputs, fp32 for fp32), exactly as the reference.
//
// Design (one workgroup = 256 lanes = 4 waves in a 2 x 2 grid):
//   * Every wave owns a (32*MI) x (32*NI) block of C and ALL L*L slice pairs
//     for it, so each output element's L*L accumulators live in one lane and
//     the ordered epilogue needs no cross-wave traffic.
//   * v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_f16: 32 bytes of K per row
//     per instruction, 16 accumulator registers per lane.
//   * Both operands are K-contiguous ([L, M, K] and B^T = [L, N, K]); a stage
//     holds 128 bytes of K for all L*(BM+BN) rows, staged global -> VGPR ->
//     LDS with the next stage's loads in flight during the current MFMAs
//     (double-buffered LDS, one barrier per stage).  16-byte chunks are
//     XOR-swizzled by (row & 7) so ds_read_b128 / ds_write_b128 are
//     bank-conflict free.
//   * int8 products are exact integers, so the order in which K is fed to
//     the MFMA cannot change acc_ij: the int8 result is bit-identical to the
//     reference for any tiling.
//   * Workgroups are remapped so each XCD (own L2) processes a contiguous
//     range of tiles, grouped GROUP_M tile-rows at a time.
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
    OZK_DEV static Acc zero() { return Acc{0}; }
    OZK_DEV static Acc run(i32x4 a, i32x4 b, Acc c) {
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
    }
    OZK_DEV static float to_f32(int x) { return (float)x; }   // RNE int32 -> fp32
};
template <> struct Mfma<_Float16> {
    using Acc = f32x16;
    OZK_DEV static Acc zero() { return Acc{0.0f}; }
    OZK_DEV static Acc run(i32x4 a, i32x4 b, Acc c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    OZK_DEV static float to_f32(float x) { return x; }
};

template <typename OutT> struct OutAcc;
template <> struct OutAcc<double> { using T = double; };
template <> struct OutAcc<float> { using T = float; };

OZK_DEV int64_t xcd_remap_gemm(int64_t g, int64_t n) {
    const int64_t q = n / 8;
    if (g >= q * 8) return g;
    return (g % 8) * q + g / 8;
}

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

OZK_DEV int swz(int row, int chunk) { return row * kRowBytes + ((chunk ^ (row & 7)) << 4); }

template <typename ST, int L, int MI, int NI, typename OutT>
__global__ __launch_bounds__(256, 1) void cross_gemm_kernel(GemmParams p, int group_m) {
    using Sh = GemmShape<L, MI, NI>;
    using MF = Mfma<ST>;
    using Acc = typename MF::Acc;
    using OA = typename OutAcc<OutT>::T;
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
                            acc[i][j][a][c] = MF::run(af[i][a], bf[j][c], acc[i][j][a][c]);
        }
        if (more) store_stage(smem + ((kb + 1) & 1) * Sh::STAGE, stg);
        __syncthreads();
    }

    // ---- epilogue: ordered outer accumulation, ozaki_triton.py:420-452 ----
    const float *sab = p.sa + bidx * p.sas_b;
    const float *sbb = p.sb + bidx * p.sbs_b;
    OutT *Cb = (OutT *)p.C + bidx * p.cs_b;
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
                            const float x = MF::to_f32(acc[i][j][a][c][r]);
                            const float t1 = x * sai;
                            const float t2 = t1 * sbv[j];
                            out = out + (OA)t2;
                        }
                    }
                    Cb[row * p.cs_m + col * p.cs_n] = (OutT)out;
                }
            }
        }
    }
}

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
        } else {
            ((uint16_t *)p.dst)[idx] = (k < p.K) ? ((const uint16_t *)p.src)[so] : (uint16_t)0;
        }
    }
}

// num_splits == 0: the reference's kernel stores its zero-initialised outer
// accumulator (ozaki_triton.py:426,452), so C is all zeros.
template <typename OutT>
__global__ __launch_bounds__(256) void zero_c_kernel(GemmParams p) {
    const int64_t total = p.batch * p.M * p.N;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t n = idx % p.N;
        const int64_t m = (idx / p.N) % p.M;
        const int64_t b = idx / (p.N * p.M);
        ((OutT *)p.C)[b * p.cs_b + m * p.cs_m + n * p.cs_n] = (OutT)0;
    }
}

hipError_t launch_zero_c(const GemmParams &p, int out_dtype, hipStream_t st) {
    const int64_t total = p.batch * p.M * p.N;
    if (total == 0) return hipSuccess;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (out_dtype == 0) hipLaunchKernelGGL(zero_c_kernel<double>, dim3((unsigned)blocks), dim3(256), 0, st, p);
    else hipLaunchKernelGGL(zero_c_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st, p);
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
GemmPlan plan_gemm(const GemmParams &p, int L, int slice_dtype) {
    (void)slice_dtype;
    GemmPlan plan{1, 1, 8};
    int mi = 1, ni = 1;
    if (L <= 1) { mi = 2; ni = 4; }
    else if (L == 2) { mi = 2; ni = 2; }
    auto nt = [&](int a, int c) {
        return p.batch * ((p.M + 64 * a - 1) / (64 * a)) * ((p.N + 64 * c - 1) / (64 * c));
    };
    // a grid smaller than two waves of 256 CUs loses more to idle CUs than the
    // larger tile gains in reuse
    while ((mi > 1 || ni > 1) && nt(mi, ni) < 512) {
        if (ni >= mi && ni > 1) ni /= 2;
        else mi /= 2;
    }
    plan.mi = mi;
    plan.ni = ni;
    plan.group_m = 8;
    return plan;
}

template <typename ST, int L, int MI, int NI, typename OutT>
static hipError_t launch_one(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    using Sh = GemmShape<L, MI, NI>;
    auto kern = cross_gemm_kernel<ST, L, MI, NI, OutT>;
    static bool attr_set = false;   // idempotent; a racing second set is harmless
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void *)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           Sh::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int64_t tiles = p.batch * ((p.M + Sh::BM - 1) / Sh::BM) * ((p.N + Sh::BN - 1) / Sh::BN);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256), Sh::LDS_BYTES, st, p,
                       plan.group_m);
    return hipGetLastError();
}

template <typename ST, int L, typename OutT>
static hipError_t launch_L(const GemmParams &p, const GemmPlan &plan, hipStream_t st) {
    const int key = plan.mi * 10 + plan.ni;
    if constexpr (L == 1) {
        switch (key) {
        case 24: return launch_one<ST, 1, 2, 4, OutT>(p, plan, st);
        case 22: return launch_one<ST, 1, 2, 2, OutT>(p, plan, st);
        case 12: return launch_one<ST, 1, 1, 2, OutT>(p, plan, st);
        case 11: return launch_one<ST, 1, 1, 1, OutT>(p, plan, st);
        }
    } else if constexpr (L == 2) {
        switch (key) {
        case 22: return launch_one<ST, 2, 2, 2, OutT>(p, plan, st);
        case 12: return launch_one<ST, 2, 1, 2, OutT>(p, plan, st);
        case 11: return launch_one<ST, 2, 1, 1, OutT>(p, plan, st);
        }
    } else {
        if (key == 11) return launch_one<ST, L, 1, 1, OutT>(p, plan, st);
    }
    return hipErrorInvalidValue;
}

template <typename ST, typename OutT>
static hipError_t launch_st(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t st) {
    switch (L) {
    case 1: return launch_L<ST, 1, OutT>(p, plan, st);
    case 2: return launch_L<ST, 2, OutT>(p, plan, st);
    case 3: return launch_L<ST, 3, OutT>(p, plan, st);
    case 4: return launch_L<ST, 4, OutT>(p, plan, st);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemm(const GemmParams &p, const GemmPlan &plan, int L, int slice_dtype,
                       int out_dtype, hipStream_t st) {
    if (slice_dtype == 4 && out_dtype == 0) return launch_st<int8_t, double>(p, plan, L, st);
    if (slice_dtype == 4 && out_dtype == 1) return launch_st<int8_t, float>(p, plan, L, st);
    if (slice_dtype == 2 && out_dtype == 0) return launch_st<_Float16, double>(p, plan, L, st);
    if (slice_dtype == 2 && out_dtype == 1) return launch_st<_Float16, float>(p, plan, L, st);
    return hipErrorInvalidValue;
}

}  // namespace ozk
