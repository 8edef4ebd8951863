// ozk_split.hip -- the split of ozaki_triton.py:137-211 as bandwidth-bound
// gfx950 kernels.
//
// For every operand row (a row of A, or a column of B seen through B^T) and
// every level l < L:
//   mu  = max(1e-38f, fl32(max_k |src_k|))
//   E   = ceil(log2_f32(mu)),  s = 2^(E - alpha)          (scales[b, l, row])
//   q   = src / s (in RES = fp64 for fp64 input, else fp32)
//   slice = int8: trunc(clamp(fl(q +/- 0.5), -128, 127));  fp16: RN(q)
//   src <- fl32(src - slice * s)   (the reference's fp32 residual buffer)
//
// Three kernels:
//   split_rows_kernel   row-resident, for K-contiguous rows (A).  A group of
//                       64*GW lanes owns one row; the row stays in VGPRs across
//                       all levels, so X is read from HBM once and each slice
//                       written once.
//   split_strip_kernel  column-strip-resident, for row-contiguous operands
//                       (the B^T view).  A workgroup owns W adjacent columns of
//                       B for all K; loads are 16 B per lane along N, and each
//                       lane holds 4 consecutive k per column so that int8 /
//                       fp16 slices leave as 4-/8-byte stores along K.
//   split_generic_kernel any strides and any K: one workgroup per row,
//                       multi-pass over K with an fp32 residual in workspace
//                       (the reference's own traffic pattern).
#include "ozk_common.h"
#include "ozk_internal.h"

namespace ozk {

typedef double dbl2 __attribute__((ext_vector_type(2)));
typedef float flt4 __attribute__((ext_vector_type(4)));

template <typename XT> struct ResOf;
template <> struct ResOf<double> { using R = double; };
template <> struct ResOf<float> { using R = float; };

OZK_DEV ScaleF64 make_scale(int e_minus_alpha, double) { return make_scale_f64(e_minus_alpha); }
OZK_DEV ScaleF32 make_scale(int e_minus_alpha, float) { return make_scale_f32(e_minus_alpha); }

// Quantise one value.  Returns the slice bit pattern (int8 in the low byte or
// fp16 bits) and writes the dequantised slice value (exact in R) to *deq.
template <typename ST> struct Quant;
template <> struct Quant<int8_t> {
    template <typename R> OZK_DEV static uint32_t run(R q, R *deq) {
        int v = quant_i8(q);
        *deq = (R)v;
        return (uint32_t)v & 0xFFu;
    }
};
template <> struct Quant<_Float16> {
    OZK_DEV static uint32_t run(double q, double *deq) {
        uint32_t h = f64_to_f16_bits(q);
        *deq = (double)f16_bits_to_f32(h);
        return h;
    }
    OZK_DEV static uint32_t run(float q, float *deq) {
        uint32_t h = f32_to_f16_bits(q);
        *deq = f16_bits_to_f32(h);
        return h;
    }
};

// fl32(src - deq * s) evaluated in R, then widened back to R.
OZK_DEV double next_residual(double src, double deq, float s) {
    double prod = deq * (double)s;
    return (double)(float)(src - prod);
}
OZK_DEV float next_residual(float src, float deq, float s) {
    float prod = deq * s;
    return src - prod;
}

// Store 4 consecutive slice values (k .. k+3) of one row.
template <typename ST> struct Store4;
template <> struct Store4<int8_t> {
    OZK_DEV static void run(void *base, int64_t off, const uint32_t v[4]) {
        uint32_t w = v[0] | (v[1] << 8) | (v[2] << 16) | (v[3] << 24);
        *(uint32_t *)((int8_t *)base + off) = w;
    }
};
template <> struct Store4<_Float16> {
    OZK_DEV static void run(void *base, int64_t off, const uint32_t v[4]) {
        uint64_t w = (uint64_t)v[0] | ((uint64_t)v[1] << 16) | ((uint64_t)v[2] << 32) |
                     ((uint64_t)v[3] << 48);
        *(uint64_t *)((_Float16 *)base + off) = w;
    }
};
template <typename ST> OZK_DEV void store1(void *base, int64_t off, uint32_t v) {
    if (sizeof(ST) == 1) ((uint8_t *)base)[off] = (uint8_t)v;
    else ((uint16_t *)base)[off] = (uint16_t)v;
}

// Load 4 consecutive elements (16-byte aligned for float, two 16-byte loads
// for double).
OZK_DEV void load4(const double *p, double v[4]) {
    dbl2 a = *(const dbl2 *)p;
    dbl2 b = *(const dbl2 *)(p + 2);
    v[0] = a.x; v[1] = a.y; v[2] = b.x; v[3] = b.y;
}
OZK_DEV void load4(const float *p, float v[4]) {
    flt4 a = *(const flt4 *)p;
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
}
// Load VEC = 16 / sizeof(XT) consecutive elements with one 16-byte load.
OZK_DEV void loadvec(const double *p, double v[2]) {
    dbl2 a = *(const dbl2 *)p;
    v[0] = a.x; v[1] = a.y;
}
OZK_DEV void loadvec(const float *p, float v[4]) {
    flt4 a = *(const flt4 *)p;
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
}

OZK_DEV float wave_max(float m) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    return m;
}

// ---------------------------------------------------------------------------
// Row-resident split.  Block = RPB groups of G = 64*GW lanes; group g owns
// global row blockIdx.x*RPB + g.  Lane t of a group holds elements
// (c*G + t)*4 + {0..3} for c < NC, so each wave load covers 1 KB (fp64: 2 KB)
// of contiguous row and each wave store 256 B (int8) of contiguous slice.
// Requirements (checked on the host): xs_k == 1, ss_k == 1, K % 4 == 0, X rows
// 16-byte aligned, slice rows 4-byte (int8) / 8-byte (fp16) aligned,
// K <= 4 * NC * G.
// ---------------------------------------------------------------------------
template <typename XT, typename ST, int GW, int RPB, int NC>
__global__ __launch_bounds__(64 * GW * RPB) void split_rows_kernel(SplitParams p) {
    using R = typename ResOf<XT>::R;
    constexpr int G = 64 * GW;
    constexpr int NE = 4 * NC;
    __shared__ float red[2][RPB][GW];

    const int tid = threadIdx.x;
    const int grp = tid / G;
    const int t = tid % G;
    const int wave = t / 64;
    const int64_t nrows = p.batch * p.rows;
    const int64_t grow = (int64_t)blockIdx.x * RPB + grp;
    const bool active = grow < nrows;
    const int64_t b = active ? grow / p.rows : 0;
    const int64_t r = active ? grow % p.rows : 0;

    const XT *xrow = (const XT *)p.X + b * p.xs_b + r * p.xs_r;
    const int64_t srow = b * p.ss_b + r * p.ss_r;

    R v[NE];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int64_t e0 = ((int64_t)c * G + t) * 4;
        XT tmp[4];
        if (active && e0 < p.K) {
            load4(xrow + e0, tmp);
        } else {
            tmp[0] = tmp[1] = tmp[2] = tmp[3] = (XT)0;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) v[c * 4 + u] = (R)tmp[u];
    }

    for (int l = 0; l < p.L; ++l) {
        // sweep 0: row max
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < NE; ++e) m = fmaxf(m, (float)fabs(v[e]));
        m = wave_max(m);
        if (GW > 1) {
            if ((t & 63) == 0) red[l & 1][grp][wave] = m;
            __syncthreads();
#pragma unroll
            for (int w = 0; w < GW; ++w) m = fmaxf(m, red[l & 1][grp][w]);
        }
        const float mu = fmaxf(1e-38f, m);
        const int ema = ceil_log2_f32(mu) - p.alpha;
        const float s = pow2f(ema);
        const auto sc = make_scale(ema, R(0));
        if (active && t == 0) p.scales[b * p.cs_b + l * p.cs_l + r * p.cs_r] = s;

        // sweep 1: quantise, store, residual
        const bool upd = (l + 1 < p.L);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int64_t e0 = ((int64_t)c * G + t) * 4;
            uint32_t qv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                R deq;
                const R q = sc.apply(v[c * 4 + u]);
                qv[u] = Quant<ST>::run(q, &deq);
                if (upd) v[c * 4 + u] = next_residual(v[c * 4 + u], deq, s);
            }
            if (active && e0 < p.K) Store4<ST>::run(p.slices, srow + l * p.ss_l + e0, qv);
        }
    }
}

// ---------------------------------------------------------------------------
// Column-strip-resident split for operands whose rows are contiguous
// (xs_r == 1): the B^T view, where a "row" is a column of B.  The workgroup
// owns W = 2*VEC adjacent columns.  Lane t: column group cg = t % 2 (VEC
// columns read with one 16-byte load), k-quad kq = t / 2; it holds
// k = 4*(kq + g*NT/2) + {0..3} for g < KPT/4.  Per-column maxima reduce over
// lanes of equal cg (xor 2..32) and then over waves through LDS.
// Strips are mapped to workgroups XCD-aware: the strips sharing a cache line
// are consecutive on one XCD.
// Requirements (host-checked): xs_r == 1, ss_k == 1, rows % VEC == 0, xs_k %
// VEC == 0, X 16-byte aligned, K % 4 == 0, slice rows 4-/8-byte aligned,
// K <= KPT * NT / 2.
// ---------------------------------------------------------------------------
OZK_DEV int64_t xcd_remap(int64_t g, int64_t n) {
    // hardware dispatches workgroup g to XCD g % 8; give each XCD a contiguous
    // range of logical ids (the tail beyond a multiple of 8 keeps its id)
    const int64_t q = n / 8;
    if (g >= q * 8) return g;
    return (g % 8) * q + g / 8;
}

template <typename XT, typename ST, int NT, int KPT>
__global__ __launch_bounds__(NT) void split_strip_kernel(SplitParams p) {
    using R = typename ResOf<XT>::R;
    constexpr int VEC = 16 / (int)sizeof(XT);
    constexpr int W = 2 * VEC;
    constexpr int NQ = NT / 2;      // k-quads per sweep
    constexpr int NG = KPT / 4;     // k-quads per lane
    constexpr int NW = NT / 64;
    __shared__ float red[2][NW][W];

    const int tid = threadIdx.x;
    const int cg = tid & 1;
    const int kq = tid >> 1;
    const int wave = tid / 64;
    const int64_t strips_per_b = (p.rows + W - 1) / W;
    const int64_t sidx = xcd_remap(blockIdx.x, (int64_t)gridDim.x);
    const int64_t b = sidx / strips_per_b;
    const int64_t col0 = (sidx % strips_per_b) * W + cg * VEC;
    const bool colok = col0 < p.rows;   // rows % VEC == 0: whole group valid

    const XT *xb = (const XT *)p.X + b * p.xs_b + col0;

    R v[NG][4][VEC];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
        for (int dk = 0; dk < 4; ++dk) {
            const int64_t k = 4 * ((int64_t)kq + (int64_t)g * NQ) + dk;
            XT tmp[VEC];
            if (colok && k < p.K) {
                loadvec(xb + k * p.xs_k, tmp);
            } else {
#pragma unroll
                for (int u = 0; u < VEC; ++u) tmp[u] = (XT)0;
            }
#pragma unroll
            for (int u = 0; u < VEC; ++u) v[g][dk][u] = (R)tmp[u];
        }
    }

    for (int l = 0; l < p.L; ++l) {
        float m[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) m[u] = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u) m[u] = fmaxf(m[u], (float)fabs(v[g][dk][u]));
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
#pragma unroll
            for (int off = 32; off >= 2; off >>= 1) m[u] = fmaxf(m[u], __shfl_xor(m[u], off, 64));
        }
        if ((tid & 63) < 2) {
#pragma unroll
            for (int u = 0; u < VEC; ++u) red[l & 1][wave][cg * VEC + u] = m[u];
        }
        __syncthreads();
        float s[VEC];
        decltype(make_scale(0, R(0))) sc[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
            float mm = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) mm = fmaxf(mm, red[l & 1][w][cg * VEC + u]);
            const float mu = fmaxf(1e-38f, mm);
            const int ema = ceil_log2_f32(mu) - p.alpha;
            s[u] = pow2f(ema);
            sc[u] = make_scale(ema, R(0));
        }
        if (colok && kq == 0) {
#pragma unroll
            for (int u = 0; u < VEC; ++u)
                p.scales[b * p.cs_b + l * p.cs_l + (col0 + u) * p.cs_r] = s[u];
        }
        const bool upd = (l + 1 < p.L);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int64_t k0 = 4 * ((int64_t)kq + (int64_t)g * NQ);
            uint32_t qv[VEC][4];
#pragma unroll
            for (int dk = 0; dk < 4; ++dk) {
#pragma unroll
                for (int u = 0; u < VEC; ++u) {
                    R deq;
                    const R q = sc[u].apply(v[g][dk][u]);
                    qv[u][dk] = Quant<ST>::run(q, &deq);
                    if (upd) v[g][dk][u] = next_residual(v[g][dk][u], deq, s[u]);
                }
            }
            if (colok && k0 < p.K) {
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    Store4<ST>::run(p.slices, b * p.ss_b + l * p.ss_l + (col0 + u) * p.ss_r + k0,
                                    qv[u]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Generic split: one workgroup of 256 lanes per row, any strides, any K.
// Level l reads src (X for l = 0, else the fp32 residual workspace) twice:
// once for the row max, once to quantise; lane t always touches k = t + 256*i,
// so a lane re-reads only residuals it wrote itself.
// ---------------------------------------------------------------------------
template <typename XT, typename ST>
__global__ __launch_bounds__(256) void split_generic_kernel(SplitParams p) {
    using R = typename ResOf<XT>::R;
    __shared__ float red[2][4];
    const int t = threadIdx.x;
    const int64_t grow = blockIdx.x;
    const int64_t b = grow / p.rows;
    const int64_t r = grow % p.rows;
    const XT *xrow = (const XT *)p.X + b * p.xs_b + r * p.xs_r;
    float *res = p.resid + (b * p.rows + r) * p.K;
    const int64_t srow = b * p.ss_b + r * p.ss_r;

    for (int l = 0; l < p.L; ++l) {
        float m = 0.0f;
        for (int64_t k = t; k < p.K; k += 256) {
            const R x = (l == 0) ? (R)xrow[k * p.xs_k] : (R)res[k];
            m = fmaxf(m, (float)fabs(x));
        }
        m = wave_max(m);
        if ((t & 63) == 0) red[l & 1][t / 64] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[l & 1][0], red[l & 1][1]), fmaxf(red[l & 1][2], red[l & 1][3]));
        const float mu = fmaxf(1e-38f, m);
        const int ema = ceil_log2_f32(mu) - p.alpha;
        const float s = pow2f(ema);
        const auto sc = make_scale(ema, R(0));
        if (t == 0) p.scales[b * p.cs_b + l * p.cs_l + r * p.cs_r] = s;
        const bool upd = (l + 1 < p.L);
        for (int64_t k = t; k < p.K; k += 256) {
            const R x = (l == 0) ? (R)xrow[k * p.xs_k] : (R)res[k];
            R deq;
            const uint32_t qv = Quant<ST>::run(sc.apply(x), &deq);
            store1<ST>(p.slices, srow + l * p.ss_l + k * p.ss_k, qv);
            if (upd) res[k] = (float)next_residual(x, deq, s);
        }
    }
}

// ---------------------------------------------------------------------------
// Transpose of a row-contiguous operand (xs_r == 1, the B^T view) into a
// K-contiguous workspace [batch, rows, K], for K too long for the strip
// kernel; the row kernel then splits the workspace.  64 x 64 tiles through
// LDS: loads are 16 bytes per lane along the rows, stores 16 bytes along K.
// ---------------------------------------------------------------------------
template <typename XT>
__global__ __launch_bounds__(256) void transpose_kernel(const XT *__restrict__ X, int64_t batch,
                                                        int64_t rows, int64_t K, int64_t xs_b,
                                                        int64_t xs_k, XT *__restrict__ T) {
    constexpr int TILE = 64;
    constexpr int VEC = 16 / (int)sizeof(XT);
    __shared__ XT tile[TILE][TILE + 1];
    const int64_t tiles_r = (rows + TILE - 1) / TILE;
    const int64_t tiles_k = (K + TILE - 1) / TILE;
    const int64_t tb = blockIdx.x;
    const int64_t b = tb / (tiles_r * tiles_k);
    const int64_t rem = tb % (tiles_r * tiles_k);
    const int64_t r0 = (rem % tiles_r) * TILE;
    const int64_t k0 = (rem / tiles_r) * TILE;
    const XT *xb = X + b * xs_b;
    // load: lane covers VEC consecutive rows of one k
    constexpr int LPR = TILE / VEC;              // lanes per k-row of the tile
    constexpr int KPP = 256 / LPR;               // k-rows per pass
    const int lr = threadIdx.x % LPR, lk = threadIdx.x / LPR;
#pragma unroll
    for (int kk = 0; kk < TILE; kk += KPP) {
        const int64_t k = k0 + kk + lk;
        const int64_t r = r0 + lr * VEC;
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
            XT v = (XT)0;
            if (k < K && r + u < rows) v = xb[k * xs_k + r + u];
            tile[kk + lk][lr * VEC + u] = v;
        }
    }
    __syncthreads();
    // store: lane covers VEC consecutive k of one row
    XT *tb_out = T + b * rows * K;
#pragma unroll
    for (int rr = 0; rr < TILE; rr += KPP) {
        const int64_t r = r0 + rr + lk;
        const int64_t k = k0 + lr * VEC;
        if (r < rows) {
#pragma unroll
            for (int u = 0; u < VEC; ++u)
                if (k + u < K) tb_out[r * K + k + u] = tile[lr * VEC + u][rr + lk];
        }
    }
}

// ---------------------------------------------------------------------------
// Planning and launch.
// Row variants (GW waves per row, RPB rows per block, NC chunks): capacity
// 4*NC*64*GW elements.  fp64 rows keep at most 32 values per lane.
// ---------------------------------------------------------------------------
struct RowCfg { int gw, rpb, nc; };
static const RowCfg kRowCfgs[] = {
    {1, 4, 1},    // K <= 256
    {1, 4, 2},    // K <= 512
    {1, 4, 4},    // K <= 1024
    {4, 1, 2},    // K <= 2048
    {4, 1, 4},    // K <= 4096
    {4, 1, 8},    // K <= 8192
    {8, 1, 8},    // K <= 16384
    {16, 1, 8},   // K <= 32768
    {16, 1, 16},  // K <= 65536 (fp32 only)
};
static const int kNumRowCfgs = sizeof(kRowCfgs) / sizeof(kRowCfgs[0]);

struct StripCfg { int nt, kpt; };
static const StripCfg kStripCfgs[] = {
    {256, 8},     // K <= 1024
    {512, 8},     // K <= 2048
    {1024, 8},    // K <= 4096
    {1024, 16},   // K <= 8192
};
static const int kNumStripCfgs = sizeof(kStripCfgs) / sizeof(kStripCfgs[0]);

static bool aligned(const void *ptr, int64_t bytes) {
    return ((uintptr_t)ptr % (uintptr_t)bytes) == 0;
}

SplitPlan plan_split(const SplitParams &p, int x_dtype, int slice_dtype) {
    const int xsz = (x_dtype == 0) ? 8 : 4;
    const int ssz = (slice_dtype == 4) ? 1 : 2;
    const bool k4 = (p.K % 4) == 0;
    const bool slice_ok = p.ss_k == 1 && aligned(p.slices, 4 * ssz) &&
                          (p.ss_r * ssz) % (4 * ssz) == 0 && (p.ss_l * ssz) % (4 * ssz) == 0 &&
                          (p.ss_b * ssz) % (4 * ssz) == 0;
    if (k4 && slice_ok && p.xs_k == 1 && aligned(p.X, 16) && (p.xs_r * xsz) % 16 == 0 &&
        (p.xs_b * xsz) % 16 == 0) {
        for (int i = 0; i < kNumRowCfgs; ++i) {
            const RowCfg &c = kRowCfgs[i];
            if (x_dtype == 0 && c.nc > 8) continue;
            if (p.K <= (int64_t)4 * c.nc * 64 * c.gw) return {kSplitRows, i};
        }
    }
    const int vec = 16 / xsz;
    if (k4 && slice_ok && p.xs_r == 1 && p.rows % vec == 0 && aligned(p.X, 16) &&
        (p.xs_k * xsz) % 16 == 0 && (p.xs_b * xsz) % 16 == 0) {
        for (int i = 0; i < kNumStripCfgs; ++i) {
            const StripCfg &c = kStripCfgs[i];
            if (p.K <= (int64_t)c.kpt * c.nt / 2) return {kSplitStrip, i};
        }
    }
    // row-contiguous operand with a K too long for a resident strip: transpose
    // into the workspace, then the row kernel (if the row fits)
    if (k4 && slice_ok && p.xs_r == 1) {
        for (int i = 0; i < kNumRowCfgs; ++i) {
            const RowCfg &c = kRowCfgs[i];
            if (x_dtype == 0 && c.nc > 8) continue;
            if (p.K <= (int64_t)4 * c.nc * 64 * c.gw) return {kSplitTransposeRows, i};
        }
    }
    return {kSplitGeneric, 0};
}

size_t split_workspace_bytes(const SplitParams &p, const SplitPlan &plan, int x_dtype) {
    const int64_t n = p.batch * p.rows * p.K;
    if (plan.path == kSplitTransposeRows) return (size_t)(n * (x_dtype == 0 ? 8 : 4));
    if (plan.path == kSplitGeneric && p.L > 1) return (size_t)(n * 4);
    return 0;
}

template <typename XT, typename ST>
static hipError_t launch_rows(const SplitParams &p, int v, hipStream_t st) {
    const int64_t nrows = p.batch * p.rows;
#define OZK_ROWS(GW, RPB, NC)                                                               \
    hipLaunchKernelGGL((split_rows_kernel<XT, ST, GW, RPB, NC>),                            \
                       dim3((unsigned)((nrows + RPB - 1) / RPB)), dim3(64 * GW * RPB), 0, st, p)
    switch (v) {
    case 0: OZK_ROWS(1, 4, 1); break;
    case 1: OZK_ROWS(1, 4, 2); break;
    case 2: OZK_ROWS(1, 4, 4); break;
    case 3: OZK_ROWS(4, 1, 2); break;
    case 4: OZK_ROWS(4, 1, 4); break;
    case 5: OZK_ROWS(4, 1, 8); break;
    case 6: OZK_ROWS(8, 1, 8); break;
    case 7: OZK_ROWS(16, 1, 8); break;
    case 8:
        if constexpr (sizeof(XT) == 4) { OZK_ROWS(16, 1, 16); }
        else return hipErrorInvalidValue;
        break;
    default: return hipErrorInvalidValue;
    }
#undef OZK_ROWS
    return hipGetLastError();
}

template <typename XT, typename ST>
static hipError_t launch_strip(const SplitParams &p, int v, hipStream_t st) {
    constexpr int W = 2 * (16 / (int)sizeof(XT));
    const int64_t nstrips = p.batch * ((p.rows + W - 1) / W);
#define OZK_STRIP(NT, KPT)                                                                  \
    hipLaunchKernelGGL((split_strip_kernel<XT, ST, NT, KPT>), dim3((unsigned)nstrips),      \
                       dim3(NT), 0, st, p)
    switch (v) {
    case 0: OZK_STRIP(256, 8); break;
    case 1: OZK_STRIP(512, 8); break;
    case 2: OZK_STRIP(1024, 8); break;
    case 3: OZK_STRIP(1024, 16); break;
    default: return hipErrorInvalidValue;
    }
#undef OZK_STRIP
    return hipGetLastError();
}

template <typename XT, typename ST>
static hipError_t launch_typed(const SplitParams &p, const SplitPlan &plan, hipStream_t st) {
    switch (plan.path) {
    case kSplitRows: return launch_rows<XT, ST>(p, plan.variant, st);
    case kSplitStrip: return launch_strip<XT, ST>(p, plan.variant, st);
    case kSplitTransposeRows: {
        XT *T = (XT *)p.resid;   // workspace [batch, rows, K]
        const int64_t tiles = p.batch * ((p.rows + 63) / 64) * ((p.K + 63) / 64);
        hipLaunchKernelGGL((transpose_kernel<XT>), dim3((unsigned)tiles), dim3(256), 0, st,
                           (const XT *)p.X, p.batch, p.rows, p.K, p.xs_b, p.xs_k, T);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        SplitParams q = p;
        q.X = T;
        q.xs_b = p.rows * p.K;
        q.xs_r = p.K;
        q.xs_k = 1;
        return launch_rows<XT, ST>(q, plan.variant, st);
    }
    default:
        hipLaunchKernelGGL((split_generic_kernel<XT, ST>), dim3((unsigned)(p.batch * p.rows)),
                           dim3(256), 0, st, p);
        return hipGetLastError();
    }
}

hipError_t launch_split(const SplitParams &p, const SplitPlan &plan, int x_dtype,
                        int slice_dtype, hipStream_t st) {
    if (p.batch * p.rows == 0 || p.L == 0) return hipSuccess;
    if (x_dtype == 0 && slice_dtype == 4) return launch_typed<double, int8_t>(p, plan, st);
    if (x_dtype == 0 && slice_dtype == 2) return launch_typed<double, _Float16>(p, plan, st);
    if (x_dtype == 1 && slice_dtype == 4) return launch_typed<float, int8_t>(p, plan, st);
    if (x_dtype == 1 && slice_dtype == 2) return launch_typed<float, _Float16>(p, plan, st);
    return hipErrorInvalidValue;
}

}  // namespace ozk
