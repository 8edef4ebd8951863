// ozk_split.hip -- the split of ozaki_triton.py:137-211 as gfx950 kernels.
//
// For every operand row (a row of A, or a column of B seen through B^T) and
// every level l < L:
//   mu  = max(1e-38f, fl32(max_k |src_k|))
//   E   = ceil(log2_f32(mu)),  s = 2^(E - alpha)          (scales[b, l, row])
//   q   = src / s (in RES = fp64 for fp64 input, else fp32)
//   slice = int8: trunc(clamp(fl(q +/- 0.5), -128, 127));  fp16: RN(q)
//   src <- fl32(src - slice * s)   (the reference's fp32 residual buffer)
//
// Arithmetic per element (bit-identical to the above, fewer instructions):
//   level 0, fp64 input   q = x * 2^(alpha-E) and t = fl64(q +/- 0.5) in fp64;
//                         residual fma(-slice, s, x) rounded to fp64 then fp32
//                         (the product is exact, so this is fl32(fl64(x - slice*s))).
//   level >= 1, fp64 input: src is an fp32 residual r.  q = r * 2^(alpha-E)
//                         is exact in fp32 (or below 2^-126, where the slice
//                         is 0 either way), so q is computed with ldexp in
//                         fp32; fl64(q +/- 0.5) is exact, and trunc of it
//                         equals trunc(fl32(q +/- c)) with c = 0.5 - 2^-25
//                         for every fp32 q (c keeps q = 0.5 - 2^-25 from
//                         rounding up to 1; for |q| >= 0.5 subtracting 2^-25
//                         moves no sum across an integer).  The residual
//                         r - slice*s is exact in fp32 (for |q| >= 0.5 it is a
//                         multiple of ulp(r) not above |r|; else it is r), so
//                         one fp32 fma gives it.
//   fp32 input (RES = fp32): q = ldexp(x, alpha-E) is the correctly rounded
//                         quotient; t = fl32(q +/- 0.5) as in the reference;
//                         residual fma(-slice, s, x) = fl32(x - fl32(slice*s))
//                         because slice*s is exact.
//   fp16 slices: RN(q) from fp64 at level 0 of fp64 input (integer rounding);
//                elsewhere q is an fp32 value and the hardware RNE conversion
//                rounds it once; slice*s is exact in fp32 in every case.
//
// Kernels:
//   split_rows_kernel   row-resident, for K-contiguous rows (A).  A group of
//                       64*GW lanes owns one row; the row stays in VGPRs across
//                       all levels, so X is read from HBM once and each slice
//                       written once.
//   split_rows_coop_kernel  rows longer than 16384: K chunks of a row in
//                       separate workgroups that exchange the level maxima
//                       through the workspace.
//   split_coop_kernel   column groups of row-contiguous operands (the B^T
//                       view), 128-byte row segments wide, cut along K over
//                       several workgroups that exchange the level maxima
//                       through the workspace; X read once, slices written
//                       once (the default for columns of 64 KB and more, up
//                       to 32 K chunks).
//   split_strip_kernel  column-strip-resident, for row-contiguous operands
//                       with columns under 64 KB.  A workgroup owns the VEC
//                       adjacent columns one 16-byte load covers, for all K;
//                       each lane holds 4 consecutive k of every column so that
//                       int8 / fp16 slices leave as 4-/8-byte stores along K.
//                       Its 16-byte row pieces touch a cache line per 16 bytes
//                       read, which longer columns pay for.
//   transpose_kernel    + a row kernel: columns longer than the cooperative
//                       kernel takes, transposed into the workspace first.
//   split_generic_kernel any strides and any K: one workgroup per row,
//                       multi-pass over K, each level's residual recomputed
//                       from the input (no workspace).
#include "ozk_common.h"
#include "ozk_internal.h"

#include <atomic>
#include <stdlib.h>
#include <string.h>

namespace ozk {

typedef double dbl2 __attribute__((ext_vector_type(2)));
typedef float flt4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Per-level constants from the row maximum m (wave-uniform).
// ---------------------------------------------------------------------------
struct LevelScale {
    float s;       // 2^(E - alpha), the stored scale
    int up;        // alpha - E
    double s64;    // s as double
    double inv64;  // 2^(alpha - E) as double (always a normal double)
};
OZK_DEV LevelScale level_scale(float m, int alpha) {
    const float mu = fmaxf(1e-38f, m);
    const int ema = ceil_log2_f32(mu) - alpha;
    LevelScale c;
    c.s = pow2f(ema);
    c.up = -ema;
    c.s64 = (double)c.s;
    c.inv64 = pow2d(-ema);
    // a row with an infinite entry has m = inf, for which the reference's
    // exp2(ceil(log2(m)) - alpha) is inf: that scale is stored as it is, so
    // the row's terms in C come out non-finite (its slices carry no meaning)
    if (!(m <= 3.402823466e38f)) c.s = m;
    return c;
}

// Quantisation of one value at one level.  MODE: kQF64 = level 0 of fp64
// input; kQExact = level >= 1 of fp64 input (fp32 residuals, exact fp32
// arithmetic); kQF32 = every level of fp32 input.  Returns the slice bits
// (int8 value in the low byte, or fp16 bits) and writes the fp32 residual.
enum { kQF64 = 0, kQExact = 1, kQF32 = 2 };
template <typename ST, int MODE> struct Quant;

template <> struct Quant<int8_t, kQF64> {
    OZK_DEV static uint32_t run(double x, const LevelScale &c, float *res) {
        const double q = x * c.inv64;
        // |q| <= 2^7 (1 + 2^-18): the sum stays above -129, so truncation
        // alone gives the reference's lower clamp
        double t = fmin(q + __builtin_copysign(0.5, q), 127.0);
        t = (q == q) ? t : 0.0;   // NaN quantises to 0
        const int k = (int)t;
        *res = (float)__builtin_fma(-(double)k, c.s64, x);
        return (uint32_t)k;
    }
};
template <> struct Quant<int8_t, kQExact> {
    OZK_DEV static uint32_t run(float r, const LevelScale &c, float *res) {
        const float q = __builtin_ldexpf(r, c.up);
        float t = fminf(__builtin_truncf(q + __builtin_copysignf(0x1.fffffep-2f, q)), 127.0f);
        t = (q == q) ? t : 0.0f;   // NaN quantises to 0
        *res = __builtin_fmaf(-t, c.s, r);
        return (uint32_t)(int)t;
    }
};
template <> struct Quant<int8_t, kQF32> {
    OZK_DEV static uint32_t run(float x, const LevelScale &c, float *res) {
        const float q = __builtin_ldexpf(x, c.up);
        float t = __builtin_truncf(
            __builtin_amdgcn_fmed3f(q + __builtin_copysignf(0.5f, q), -128.0f, 127.0f));
        t = (q == q) ? t : 0.0f;   // NaN quantises to 0
        *res = __builtin_fmaf(-t, c.s, x);
        return (uint32_t)(int)t;
    }
};
template <> struct Quant<_Float16, kQF64> {
    OZK_DEV static uint32_t run(double x, const LevelScale &c, float *res) {
        const double q = x * c.inv64;
        const uint32_t h = f64_to_f16_bits(q);
        const double d = (double)f16_bits_to_f32(h);
        *res = (float)__builtin_fma(-d, c.s64, x);
        return h;
    }
};
template <int MODE> struct QuantF16F32 {
    OZK_DEV static uint32_t run(float x, const LevelScale &c, float *res) {
        const float q = __builtin_ldexpf(x, c.up);
        const _Float16 h = (_Float16)q;
        *res = __builtin_fmaf(-(float)h, c.s, x);
        return (uint32_t)__builtin_bit_cast(uint16_t, h);
    }
};
template <> struct Quant<_Float16, kQExact> : QuantF16F32<kQExact> {};
template <> struct Quant<_Float16, kQF32> : QuantF16F32<kQF32> {};

// bfloat16 slices: one RNE rounding of q to 8 significant bits (integer code
// from fp64 at level 0 of fp64 input; from the exact fp32 q elsewhere)
template <> struct Quant<__bf16, kQF64> {
    OZK_DEV static uint32_t run(double x, const LevelScale &c, float *res) {
        const double q = x * c.inv64;
        const uint32_t h = f64_to_bf16_bits(q);
        const double d = (double)bf16_bits_to_f32(h);
        *res = (float)__builtin_fma(-d, c.s64, x);
        return h;
    }
};
template <int MODE> struct QuantBF16F32 {
    OZK_DEV static uint32_t run(float x, const LevelScale &c, float *res) {
        const float q = __builtin_ldexpf(x, c.up);
        const uint32_t h = f32_to_bf16_bits(q);
        *res = __builtin_fmaf(-bf16_bits_to_f32(h), c.s, x);
        return h;
    }
};
template <> struct Quant<__bf16, kQExact> : QuantBF16F32<kQExact> {};
template <> struct Quant<__bf16, kQF32> : QuantBF16F32<kQF32> {};

// fp32 slices: the slice is q rounded once to fp32 (exact when RES is fp32 or
// at levels >= 1, where q is an fp32 value or below 2^-126 either way)
template <> struct Quant<float, kQF64> {
    OZK_DEV static uint32_t run(double x, const LevelScale &c, float *res) {
        const float q = (float)(x * c.inv64);
        *res = (float)__builtin_fma(-(double)q, c.s64, x);
        return __float_as_uint(q);
    }
};
template <int MODE> struct QuantF32F32 {
    OZK_DEV static uint32_t run(float x, const LevelScale &c, float *res) {
        const float q = __builtin_ldexpf(x, c.up);
        *res = __builtin_fmaf(-q, c.s, x);
        return __float_as_uint(q);
    }
};
template <> struct Quant<float, kQExact> : QuantF32F32<kQExact> {};
template <> struct Quant<float, kQF32> : QuantF32F32<kQF32> {};

template <typename XT> struct Modes;
template <> struct Modes<double> { static constexpr int first = kQF64, rest = kQExact; };
template <> struct Modes<float> { static constexpr int first = kQF32, rest = kQF32; };

// Store 4 consecutive slice values (k .. k+3) of one row.
template <typename ST> struct Store4;
template <> struct Store4<int8_t> {
    OZK_DEV static void run(void *base, int64_t off, const uint32_t v[4]) {
        const uint32_t w = __builtin_amdgcn_perm(v[1], v[0], 0x0c0c0400u) |
                           __builtin_amdgcn_perm(v[3], v[2], 0x04000c0cu);
        *(uint32_t *)((int8_t *)base + off) = w;
    }
};
struct Store4Half {
    OZK_DEV static void run(void *base, int64_t off, const uint32_t v[4]) {
        const uint32_t lo = v[0] | (v[1] << 16), hi = v[2] | (v[3] << 16);
        *(uint64_t *)((uint16_t *)base + off) = (uint64_t)lo | ((uint64_t)hi << 32);
    }
};
template <> struct Store4<_Float16> : Store4Half {};
template <> struct Store4<__bf16> : Store4Half {};
template <> struct Store4<float> {
    OZK_DEV static void run(void *base, int64_t off, const uint32_t v[4]) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        *(u32x4 *)((uint32_t *)base + off) = u32x4{v[0], v[1], v[2], v[3]};
    }
};
template <typename ST> OZK_DEV void store1(void *base, int64_t off, uint32_t v) {
    if constexpr (sizeof(ST) == 1) ((uint8_t *)base)[off] = (uint8_t)v;
    else if constexpr (sizeof(ST) == 2) ((uint16_t *)base)[off] = (uint16_t)v;
    else ((uint32_t *)base)[off] = v;
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

OZK_DEV float absf(double x) { return (float)fabs(x); }   // fl32(|x|)
OZK_DEV float absf(float x) { return fabsf(x); }

// Maximum of non-negative values over the 64 lanes of a wave, returned
// wave-uniform.  DPP row reductions, then the row broadcasts of GFX9.
template <int CTRL, int ROWS> OZK_DEV float dpp_max(float v) {
    const int o = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS,
                                              0xF, false);
    return fmaxf(v, __int_as_float(o));
}
OZK_DEV float wave_max(float v) {
    v = dpp_max<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_max<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_max<0x141, 0xF>(v);   // row_half_mirror
    v = dpp_max<0x140, 0xF>(v);   // row_mirror: every lane holds its row's max
    v = dpp_max<0x142, 0xA>(v);   // row_bcast15 into rows 1 and 3
    v = dpp_max<0x143, 0xC>(v);   // row_bcast31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Workgroup barrier for LDS exchanges: completes this wave's LDS accesses,
// then s_barrier.  Unlike __syncthreads() it does not wait for outstanding
// global stores (the previous level's slices).
OZK_DEV void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

// ---------------------------------------------------------------------------
// Row-resident split.  Block = RPB groups of G = 64*GW lanes; group g owns
// global row blockIdx.x*RPB + g.  Lane t of a group holds elements
// (c*G + t)*4 + {0..3} for c < NC, so each wave load covers 1 KB (fp64: 2 KB)
// of contiguous row and each wave store 256 B (int8) of contiguous slice.
// Level 0 quantises the input values; levels >= 1 the fp32 residuals.
// Requirements (checked on the host): xs_k == 1, ss_k == 1, K % 4 == 0, X rows
// 16-byte aligned, slice rows 4-byte (int8) / 8-byte (fp16) aligned,
// K <= 4 * NC * G.
// ---------------------------------------------------------------------------
template <int GW, int RPB>
OZK_DEV float row_max(float m, float (*red)[RPB][GW], int buf, int grp, int t) {
    m = wave_max(m);
    if constexpr (GW > 1) {
        if ((t & 63) == 0) red[buf][grp][t / 64] = m;
        lds_barrier();
        float r = red[buf][grp][0];
#pragma unroll
        for (int w = 1; w < GW; ++w) r = fmaxf(r, red[buf][grp][w]);
        m = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(r)));
    }
    return m;
}

// The body of the row kernel for row block `block` (its workgroup, or a
// workgroup of split_pair_kernel); red: LDS for the row maxima.
template <typename XT, typename ST, int GW, int RPB, int NC>
OZK_DEV void split_rows_body(const SplitParams &p, int64_t block, float (*red)[RPB][GW]) {
    constexpr int G = 64 * GW;
    constexpr int NE = 4 * NC;

    const int tid = threadIdx.x;
    const int grp = tid / G;
    const int t = tid % G;
    const int64_t nrows = p.batch * p.rows;
    const int64_t grow = block * RPB + grp;
    const bool active = grow < nrows;
    const int64_t b = active ? grow / p.rows : 0;
    const int64_t r = active ? grow % p.rows : 0;

    const XT *xrow = (const XT *)p.X + b * p.xs_b + r * p.xs_r;
    const int64_t srow = b * p.ss_b + r * p.ss_r;
    float *srow_scale = p.scales + b * p.cs_b + r * p.cs_r;

    XT v[NE];
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
        for (int u = 0; u < 4; ++u) v[c * 4 + u] = tmp[u];
    }

    // level 0 on the input values
    float w[NE];
    {
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < NE; ++e) m = fmaxf(m, absf(v[e]));
        const LevelScale c = level_scale(row_max<GW, RPB>(m, red, 0, grp, t), p.alpha);
        if (active && t == 0) srow_scale[0] = c.s;
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) {
            const int64_t e0 = ((int64_t)ch * G + t) * 4;
            uint32_t qv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                qv[u] = Quant<ST, Modes<XT>::first>::run(v[ch * 4 + u], c, &w[ch * 4 + u]);
            if (active && e0 < p.K) Store4<ST>::run(p.slices, srow + e0, qv);
        }
    }
    // levels >= 1 on the fp32 residuals (the last level's update is unused)
    for (int l = 1; l < p.L; ++l) {
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < NE; ++e) m = fmaxf(m, fabsf(w[e]));
        const LevelScale c = level_scale(row_max<GW, RPB>(m, red, l & 1, grp, t), p.alpha);
        if (active && t == 0) srow_scale[l * p.cs_l] = c.s;
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) {
            const int64_t e0 = ((int64_t)ch * G + t) * 4;
            uint32_t qv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                qv[u] = Quant<ST, Modes<XT>::rest>::run(w[ch * 4 + u], c, &w[ch * 4 + u]);
            if (active && e0 < p.K) Store4<ST>::run(p.slices, srow + l * p.ss_l + e0, qv);
        }
    }
}

template <typename XT, typename ST, int GW, int RPB, int NC>
__global__ __launch_bounds__(64 * GW * RPB) void split_rows_kernel(SplitParams p) {
    __shared__ float red[2][RPB][GW];
    split_rows_body<XT, ST, GW, RPB, NC>(p, blockIdx.x, red);
}

// ---------------------------------------------------------------------------
// Column-strip-resident split for operands whose rows are contiguous
// (xs_r == 1): the B^T view, where a "row" is a column of B.  The workgroup
// owns the VEC = 16 / sizeof(XT) adjacent columns one 16-byte load covers.
// Lane t holds k = 4*(t + g*NT) + {0..3} for g < KPT/4, all VEC columns, so a
// wave load reads 64 rows x 16 B and every column's maximum reduces over the
// whole workgroup.  A strip is at most 128 KB of registers, so two or three
// workgroups share a CU and one's loads overlap another's arithmetic.
// Strips are mapped to workgroups XCD-aware: the 8 strips sharing a 128-byte
// line are consecutive on one XCD.
// Requirements (host-checked): xs_r == 1, ss_k == 1, rows % VEC == 0, xs_k %
// VEC == 0, X 16-byte aligned, K % 4 == 0, slice rows 4-/8-byte aligned,
// K <= KPT * NT.
// ---------------------------------------------------------------------------
OZK_DEV int64_t xcd_remap(int64_t g, int64_t n) {
    // hardware dispatches workgroup g to XCD g % 8; give each XCD a contiguous
    // range of logical ids (the tail beyond a multiple of 8 keeps its id)
    const int64_t q = n / 8;
    if (g >= q * 8) return g;
    return (g % 8) * q + g / 8;
}

template <int NW, int VEC>
OZK_DEV void strip_max(float m[VEC], float (*red)[NW][VEC], int buf, int tid) {
#pragma unroll
    for (int u = 0; u < VEC; ++u) m[u] = wave_max(m[u]);
    if constexpr (NW > 1) {
        if ((tid & 63) == 0) {
#pragma unroll
            for (int u = 0; u < VEC; ++u) red[buf][tid / 64][u] = m[u];
        }
        lds_barrier();
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
            float r = red[buf][0][u];
#pragma unroll
            for (int w = 1; w < NW; ++w) r = fmaxf(r, red[buf][w][u]);
            m[u] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(r)));
        }
    }
}

template <typename XT, typename ST, int NT, int KPT>
OZK_DEV void split_strip_body(const SplitParams &p, int64_t sidx,
                              float (*red)[NT / 64][16 / sizeof(XT)]) {
    constexpr int VEC = 16 / (int)sizeof(XT);
    constexpr int NG = KPT / 4;     // k-quads per lane
    constexpr int NW = NT / 64;

    const int tid = threadIdx.x;
    const int64_t strips_per_b = p.rows / VEC;
    const int64_t b = sidx / strips_per_b;
    const int64_t col0 = (sidx % strips_per_b) * VEC;

    const XT *xb = (const XT *)p.X + b * p.xs_b + col0;
    const int64_t sbase = b * p.ss_b + col0 * p.ss_r;
    float *sc_base = p.scales + b * p.cs_b + col0 * p.cs_r;

    XT v[NG][4][VEC];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
        for (int dk = 0; dk < 4; ++dk) {
            const int64_t k = 4 * ((int64_t)tid + (int64_t)g * NT) + dk;
            XT tmp[VEC];
            if (k < p.K) {
                loadvec(xb + k * p.xs_k, tmp);
            } else {
#pragma unroll
                for (int u = 0; u < VEC; ++u) tmp[u] = (XT)0;
            }
#pragma unroll
            for (int u = 0; u < VEC; ++u) v[g][dk][u] = tmp[u];
        }
    }

    float w[NG][4][VEC];
    {
        float m[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) m[u] = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u) m[u] = fmaxf(m[u], absf(v[g][dk][u]));
        strip_max<NW, VEC>(m, red, 0, tid);
        LevelScale c[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) c[u] = level_scale(m[u], p.alpha);
        if (tid == 0) {
#pragma unroll
            for (int u = 0; u < VEC; ++u) sc_base[u * p.cs_r] = c[u].s;
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int64_t k0 = 4 * ((int64_t)tid + (int64_t)g * NT);
            uint32_t qv[VEC][4];
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    qv[u][dk] = Quant<ST, Modes<XT>::first>::run(v[g][dk][u], c[u], &w[g][dk][u]);
            if (k0 < p.K) {
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    Store4<ST>::run(p.slices, sbase + u * p.ss_r + k0, qv[u]);
            }
        }
    }
    for (int l = 1; l < p.L; ++l) {
        float m[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) m[u] = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u) m[u] = fmaxf(m[u], fabsf(w[g][dk][u]));
        strip_max<NW, VEC>(m, red, l & 1, tid);
        LevelScale c[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) c[u] = level_scale(m[u], p.alpha);
        if (tid == 0) {
#pragma unroll
            for (int u = 0; u < VEC; ++u) sc_base[l * p.cs_l + u * p.cs_r] = c[u].s;
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int64_t k0 = 4 * ((int64_t)tid + (int64_t)g * NT);
            uint32_t qv[VEC][4];
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    qv[u][dk] = Quant<ST, Modes<XT>::rest>::run(w[g][dk][u], c[u], &w[g][dk][u]);
            if (k0 < p.K) {
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    Store4<ST>::run(p.slices, sbase + l * p.ss_l + u * p.ss_r + k0, qv[u]);
            }
        }
    }
}

template <typename XT, typename ST, int NT, int KPT>
__global__ __launch_bounds__(NT) void split_strip_kernel(SplitParams p) {
    __shared__ float red[2][NT / 64][16 / sizeof(XT)];
    split_strip_body<XT, ST, NT, KPT>(p, xcd_remap(blockIdx.x, (int64_t)gridDim.x), red);
}

// ---------------------------------------------------------------------------
// Column split shared by a group of workgroups (row-contiguous operands, the
// B^T view).  A 16-byte load per lane covers only 16 bytes of a row, so a
// strip one load wide (split_strip_kernel) touches one cache line per 16
// bytes read; reads of 128-byte row segments run at copy speed.  A strip of
// SW = 128 / sizeof(XT) columns over all of K does not fit one CU, so it is
// cut along K into P chunks of CH rows, one workgroup each, and the level
// maxima are combined through global memory.  A column group is SEG 16-byte
// pieces of each row: 128 bytes (SEG = 8), or 32 bytes (SEG = 2, when forced)
// for columns too long for 32 chunks of those, whose chunks then hold 4x the
// rows with the same registers (65536-long fp32 columns: 32 chunks of 2048):
//   * workgroup g = blockIdx.x is member g % P of column group g / P (batch
//     b, columns col0 .. col0 + SW, SW = SEG * VEC); lane t covers the VEC
//     columns col0 + VEC * (t % SEG) + {0..VEC-1} and the rows
//     member * CH + 4 * (t / SEG + RPP * j) + {0..3}, j < RPL / 4, RPP = 256 /
//     SEG, so a wave load covers 64 / SEG whole row segments and a lane holds
//     4 consecutive k of each column (4- / 8-byte slice stores along K);
//   * per level, wave 0 stores the workgroup's column maxima into
//     slot[group][level][member][SW], one 64-bit word each (the tag 1 in the
//     high half, the fp32 maximum in the low half), with agent-scope stores,
//     and polls the P * SW words of its group and level with agent-scope
//     loads until all carry the tag.  Every word validates itself, so no
//     fence (no L2 write-back or invalidation) is needed;
//   * the members of a group are consecutive workgroup ids, and the planner
//     keeps P at most 8 below the workgroups one XCD holds (the residency
//     limit before plan_split_raw), so every group becomes resident and its
//     waits end.  A wait is still bounded (2 s of the 100 MHz real-time
//     counter): a member that gives up sets the launch's status word and
//     member 0 stores NaN scales.  After ozk_split the poison kernel then
//     makes every scale of the split NaN and records the failure in the
//     sticky device status (ozk_device_status); in a matmul the cross-GEMM
//     reads the status word instead, writes NaN for C and records it.
// slot and the status word after it must be zero at launch (the launcher
// clears them first).
// ---------------------------------------------------------------------------
constexpr int kCoopNT = 256;
constexpr int kCoopMaxP = 32;
constexpr int64_t kCoopMinColumnBytes = 64 * 1024;
// rows kernel shared by workgroups: 256 lanes, 64 (fp32) or 32 (fp64) values
// per lane, for rows longer than 16384 elements, at most 64 chunks by its own
// layout (one polling lane each) and 56 by the residency limit on MI355X
constexpr int kRowsCoopVariant = 100;
constexpr int64_t kRowsCoopMinK = 16384;
constexpr int kRowsCoopMaxP = 64;
constexpr uint64_t kCoopTickLimit = 200000000ull;   // 2 s of the 100 MHz counter
constexpr uint64_t kCoopTag = 1ull << 32;               // high word of a published maximum

__global__ __launch_bounds__(256) void zero_u64_kernel(uint64_t *p, int64_t n) {
    for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

// Sticky device status: bit 0 = a cooperative wait gave up since the last
// clear (read and cleared by read_device_status).
__device__ uint32_t g_device_status = 0;

// After a cooperative launch: if any member gave up its wait (status != 0),
// every scale of the split becomes NaN, so no entry of C computed from it can
// pass for a valid result, and the sticky device status records it.
__global__ __launch_bounds__(256) void poison_scales_kernel(const uint32_t *status, float *scales,
                                                            int64_t batch, int L, int64_t rows,
                                                            int64_t cs_b, int64_t cs_l,
                                                            int64_t cs_r) {
    if (*status == 0) return;
    const int64_t n = batch * L * rows;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        const int64_t r = i % rows, l = (i / rows) % L, b = i / (rows * L);
        scales[b * cs_b + l * cs_l + r * cs_r] = __int_as_float(0x7fc00000);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_fetch_or(&g_device_status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// LDS of one cooperative column workgroup
template <typename XT, int SEG> struct CoopShared {
    static constexpr int VEC = 16 / (int)sizeof(XT);
    float red[kCoopNT / 64][SEG][VEC];
    float fin[SEG * VEC];
    int bad;
};

// The body of the cooperative column kernel for logical workgroup g (member
// g % P of column group g / P): its own workgroup, or one of split_pair_kernel.
template <typename XT, typename ST, int RPL, int SEG>
OZK_DEV void split_coop_body(const SplitParams &p, uint64_t *slot, int P, uint32_t want_tag,
                             uint64_t tick_limit, uint32_t *status, int64_t g,
                             CoopShared<XT, SEG> &sh) {
    constexpr int NT = kCoopNT, NG = RPL / 4;
    constexpr int VEC = 16 / (int)sizeof(XT);
    constexpr int SW = SEG * VEC;        // columns per group
    constexpr int RPP = NT / SEG;        // row quads per pass
    constexpr int NW = NT / 64;
    static_assert(SEG == 8 || SEG == 2, "128- or 32-byte row segments");
    auto &red = sh.red;
    auto &fin = sh.fin;
    int &bad = sh.bad;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int seg = t % SEG, ro = t / SEG;
    const int member = (int)(g % P);
    const int64_t grp = g / P;
    const int64_t nstr = (p.rows + SW - 1) / SW;
    const int64_t b = grp / nstr;
    const int64_t col0 = (grp % nstr) * SW;
    const int64_t mycol = col0 + seg * VEC;
    const bool cvalid = mycol < p.rows;   // rows % VEC == 0: all VEC columns or none
    const int64_t kbase = (int64_t)member * (RPP * RPL);

    const XT *xb = (const XT *)p.X + b * p.xs_b + mycol;
    XT v[NG][4][VEC];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
#pragma unroll
        for (int dk = 0; dk < 4; ++dk) {
            const int64_t k = kbase + 4 * (ro + RPP * j) + dk;
            XT tmp[VEC];
            if (cvalid && k < p.K) {
                loadvec(xb + k * p.xs_k, tmp);
            } else {
#pragma unroll
                for (int u = 0; u < VEC; ++u) tmp[u] = (XT)0;
            }
#pragma unroll
            for (int u = 0; u < VEC; ++u) v[j][dk][u] = tmp[u];
        }
    }
    if (t == 0) bad = 0;

    // maximum over the group of the lane maxima m (fl32 values >= 0), per column
    auto group_max = [&](float m[VEC], int l) {
#pragma unroll
        for (int u = 0; u < VEC; ++u)
#pragma unroll
            for (int x = SEG; x < 64; x *= 2) m[u] = fmaxf(m[u], __shfl_xor(m[u], x));
        if (lane < SEG) {
#pragma unroll
            for (int u = 0; u < VEC; ++u) red[wave][lane][u] = m[u];
        }
        lds_barrier();
        float r = 0.0f;
        if (t < SW) {
            r = red[0][t / VEC][t % VEC];
#pragma unroll
            for (int w = 1; w < NW; ++w) r = fmaxf(r, red[w][t / VEC][t % VEC]);
        }
        if (P > 1 && wave == 0) {
            // publish this member's maxima, then poll until every member's
            // word of this level carries the tag (words already seen are not
            // read again)
            uint64_t *sl = slot + (grp * p.L + l) * (int64_t)P * SW;
            if (t < SW)
                __hip_atomic_store(sl + (int64_t)member * SW + t, kCoopTag | __float_as_uint(r),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int nw = P * SW;
            uint64_t seen = 0;
            const uint64_t want = (lane < nw) ? (((nw - 1 - lane) / 64 >= 63)
                                                     ? ~0ull
                                                     : (2ull << ((nw - 1 - lane) / 64)) - 1)
                                              : 0;
            float q = 0.0f;
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                for (int n = 0; n < (nw + 63) / 64; ++n) {
                    const int i = lane + 64 * n;
                    if (i < nw && !((seen >> n) & 1)) {
                        const uint64_t w64 =
                            __hip_atomic_load(sl + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if ((uint32_t)(w64 >> 32) == want_tag) {
                            seen |= 1ull << n;
                            q = fmaxf(q, __uint_as_float((uint32_t)w64));
                        }
                    }
                }
                if (__all(seen == want)) break;
                if (__builtin_amdgcn_s_memrealtime() - t0 >= tick_limit) {
                    if (lane == 0) {
                        bad = 1;
                        __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                    }
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            // lane i holds the maximum of column i % SW over members i / SW + 64 / SW * n
            r = q;
#pragma unroll
            for (int x = SW; x < 64; x *= 2) r = fmaxf(r, __shfl_xor(r, x));
        }
        if (t < SW) fin[t] = r;
        lds_barrier();
#pragma unroll
        for (int u = 0; u < VEC; ++u) m[u] = fin[seg * VEC + u];
    };
    // scales of level l (member 0 stores them; NaN after a wait that ran out)
    auto store_scales = [&](int l) {
        if (member == 0 && t < SW && col0 + t < p.rows) {
            const LevelScale c = level_scale(fin[t], p.alpha);
            p.scales[b * p.cs_b + l * p.cs_l + (col0 + t) * p.cs_r] =
                bad ? __int_as_float(0x7fc00000) : c.s;
        }
    };
    const int64_t sbase = b * p.ss_b + mycol * p.ss_r;

    float w[NG][4][VEC];
    {
        float m[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) m[u] = 0.0f;
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u) m[u] = fmaxf(m[u], absf(v[j][dk][u]));
        group_max(m, 0);
        store_scales(0);
        LevelScale c[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) c[u] = level_scale(m[u], p.alpha);
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const int64_t k0 = kbase + 4 * (ro + RPP * j);
            uint32_t qv[VEC][4];
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    qv[u][dk] = Quant<ST, Modes<XT>::first>::run(v[j][dk][u], c[u], &w[j][dk][u]);
            if (cvalid && k0 < p.K) {
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    Store4<ST>::run(p.slices, sbase + u * p.ss_r + k0, qv[u]);
            }
            // the residuals here, not at their first use (the level-1 maximum):
            // sunk there, every input and every slice value are live at once
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u) asm volatile("" : "+v"(w[j][dk][u]));
        }
    }
    for (int l = 1; l < p.L; ++l) {
        float m[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) m[u] = 0.0f;
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u) m[u] = fmaxf(m[u], fabsf(w[j][dk][u]));
        group_max(m, l);
        store_scales(l);
        LevelScale c[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) c[u] = level_scale(m[u], p.alpha);
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const int64_t k0 = kbase + 4 * (ro + RPP * j);
            uint32_t qv[VEC][4];
#pragma unroll
            for (int dk = 0; dk < 4; ++dk)
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    qv[u][dk] = Quant<ST, Modes<XT>::rest>::run(w[j][dk][u], c[u], &w[j][dk][u]);
            if (cvalid && k0 < p.K) {
#pragma unroll
                for (int u = 0; u < VEC; ++u)
                    Store4<ST>::run(p.slices, sbase + l * p.ss_l + u * p.ss_r + k0, qv[u]);
            }
        }
    }
}

template <typename XT, typename ST, int RPL, int SEG>
__global__ __launch_bounds__(kCoopNT) void split_coop_kernel(SplitParams p, uint64_t *slot, int P,
                                                             uint32_t want_tag,
                                                             uint64_t tick_limit,
                                                             uint32_t *status) {
    __shared__ CoopShared<XT, SEG> sh;
    split_coop_body<XT, ST, RPL, SEG>(p, slot, P, want_tag, tick_limit, status, blockIdx.x, sh);
}

// ---------------------------------------------------------------------------
// Both splits of a matmul in one launch, where A's rows take a 256-lane row
// configuration (4 waves per row) and B's columns the cooperative column
// kernel with 128-byte groups (fp64 operands, 4096 <= K <= 8192: config 3).
// The grid runs in periods of P + KA workgroups: the P members of one
// column group of B, then KA row blocks of A.  The row blocks never wait, so
// they keep CUs busy while column groups wait on their exchanges, and the
// two splits cost one launch.  The members of a group stay consecutive
// workgroup ids, which the cooperative kernel's residency argument needs
// (row blocks between groups retire without waiting).
// ---------------------------------------------------------------------------
template <typename XT, typename ST, int RPL, int NC>
__global__ __launch_bounds__(kCoopNT) void split_pair_kernel(SplitParams pb, uint64_t *slot, int P,
                                                             uint32_t want_tag,
                                                             uint64_t tick_limit,
                                                             uint32_t *status, SplitParams pa,
                                                             int ka) {
    __shared__ CoopShared<XT, 8> sh;
    __shared__ float red[2][1][4];
    const int64_t period = (int64_t)P + ka;
    const int64_t q = blockIdx.x / period;
    const int pos = (int)(blockIdx.x % period);
    if (pos < P) {
        split_coop_body<XT, ST, RPL, 8>(pb, slot, P, want_tag, tick_limit, status, q * P + pos, sh);
    } else {
        const int64_t ab = q * ka + (pos - P);
        if (ab < pa.batch * pa.rows) split_rows_body<XT, ST, 4, 1, NC>(pa, ab, red);
    }
}

// ---------------------------------------------------------------------------
// Both splits of a matmul in one launch where B's columns take the 256-lane
// strip kernel and A's rows a 256-lane row configuration (K <= 8192; the
// shapes where neither split alone fills the chip).  The first nstrips
// workgroups are B's strips, in the strip kernel's XCD order (hardware puts
// workgroup g on XCD g % 8 from the first id on), the rest A's row blocks.
// Neither waits on another workgroup.
// ---------------------------------------------------------------------------
template <typename XT, typename ST, int KPT, int GW, int RPB, int NC>
__global__ __launch_bounds__(256) void split_duo_kernel(SplitParams pb, int64_t nstrips,
                                                        SplitParams pa) {
    static_assert(64 * GW * RPB == 256, "a 256-lane row configuration");
    __shared__ float red_s[2][4][16 / sizeof(XT)];
    __shared__ float red_r[2][RPB][GW];
    if ((int64_t)blockIdx.x < nstrips)
        split_strip_body<XT, ST, 256, KPT>(pb, xcd_remap(blockIdx.x, nstrips), red_s);
    else
        split_rows_body<XT, ST, GW, RPB, NC>(pa, (int64_t)blockIdx.x - nstrips, red_r);
}

// ---------------------------------------------------------------------------
// Row split shared by workgroups, for K-contiguous rows too long for one
// workgroup per row to keep a CU busy (rows over 16384 elements: one
// 1024-lane workgroup per CU, whose loads then never overlap another's
// arithmetic).  Workgroup g takes K chunk g % P of row g / P: CHR = 4 * NC *
// 64 * GW elements, laid out per lane as in split_rows_kernel.  Per level the
// workgroup's row maximum is combined over the P chunks through tagged words as
// in split_coop_kernel: slot[row][level][P], one word per chunk (lane i of
// wave 0 polls chunk i's word; P <= 64).
// ---------------------------------------------------------------------------
template <typename XT, typename ST, int GW, int NC>
__global__ __launch_bounds__(64 * GW) void split_rows_coop_kernel(SplitParams p, uint64_t *slot,
                                                                  int P, uint32_t want_tag,
                                                                  uint64_t tick_limit,
                                                                  uint32_t *status) {
    constexpr int G = 64 * GW;
    constexpr int NE = 4 * NC;
    constexpr int CHR = NE * G;
    __shared__ float red[2][1][GW];
    __shared__ float fin[2];
    __shared__ int bad;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int64_t g = blockIdx.x;
    const int member = (int)(g % P);
    const int64_t grow = g / P;
    const int64_t b = grow / p.rows, r = grow % p.rows;
    const int64_t kbase = (int64_t)member * CHR;
    const int64_t kleft = p.K - kbase;   // this chunk's elements inside the row (> 0)
    const XT *xrow = (const XT *)p.X + b * p.xs_b + r * p.xs_r + kbase;
    const int64_t srow = b * p.ss_b + r * p.ss_r + kbase;
    float *srow_scale = p.scales + b * p.cs_b + r * p.cs_r;

    XT v[NE];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int64_t e0 = ((int64_t)c * G + t) * 4;
        XT tmp[4];
        if (e0 < kleft) {
            load4(xrow + e0, tmp);
        } else {
            tmp[0] = tmp[1] = tmp[2] = tmp[3] = (XT)0;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) v[c * 4 + u] = tmp[u];
    }
    if (t == 0) bad = 0;

    // the row's maximum at level l (wave-uniform)
    auto rmax = [&](float m, int l) {
        m = row_max<GW, 1>(m, red, l & 1, 0, t);
        if (P > 1) {
            if (wave == 0) {
                uint64_t *sl = slot + (grow * p.L + l) * (int64_t)P;
                if (lane == 0)
                    __hip_atomic_store(sl + member, kCoopTag | __float_as_uint(m), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                bool seen = lane >= P;
                float q = 0.0f;
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                for (;;) {
                    if (!seen) {
                        const uint64_t w64 =
                            __hip_atomic_load(sl + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if ((uint32_t)(w64 >> 32) == want_tag) {
                            seen = true;
                            q = __uint_as_float((uint32_t)w64);
                        }
                    }
                    if (__all(seen)) break;
                    if (__builtin_amdgcn_s_memrealtime() - t0 >= tick_limit) {
                        if (lane == 0) {
                            bad = 1;
                            __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                        }
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                q = wave_max(q);
                if (lane == 0) fin[l & 1] = q;
            }
            lds_barrier();
            m = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(fin[l & 1])));
        }
        return m;
    };
    auto store_scale = [&](int l, const LevelScale &c) {
        if (member == 0 && t == 0) srow_scale[l * p.cs_l] = bad ? __int_as_float(0x7fc00000) : c.s;
    };

    float w[NE];
    {
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < NE; ++e) m = fmaxf(m, absf(v[e]));
        const LevelScale c = level_scale(rmax(m, 0), p.alpha);
        store_scale(0, c);
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) {
            const int64_t e0 = ((int64_t)ch * G + t) * 4;
            uint32_t qv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                qv[u] = Quant<ST, Modes<XT>::first>::run(v[ch * 4 + u], c, &w[ch * 4 + u]);
            if (e0 < kleft) Store4<ST>::run(p.slices, srow + e0, qv);
            // the residuals here, not at their first use (see split_coop_kernel)
#pragma unroll
            for (int u = 0; u < 4; ++u) asm volatile("" : "+v"(w[ch * 4 + u]));
        }
    }
    for (int l = 1; l < p.L; ++l) {
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < NE; ++e) m = fmaxf(m, fabsf(w[e]));
        const LevelScale c = level_scale(rmax(m, l), p.alpha);
        store_scale(l, c);
#pragma unroll
        for (int ch = 0; ch < NC; ++ch) {
            const int64_t e0 = ((int64_t)ch * G + t) * 4;
            uint32_t qv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                qv[u] = Quant<ST, Modes<XT>::rest>::run(w[ch * 4 + u], c, &w[ch * 4 + u]);
            if (e0 < kleft) Store4<ST>::run(p.slices, srow + l * p.ss_l + e0, qv);
        }
    }
}

// ---------------------------------------------------------------------------
// Generic split: one workgroup of 256 lanes per row, any strides, any K, no
// workspace.  Level l sweeps the row twice (maximum, then quantise).  The
// level-l source of an element is recomputed from the input with the scales
// of levels < l, kept in LDS: the same chain of quantisations as the
// reference's residual buffer (ozaki_triton.py:208-211), so the same bits,
// with L(L+1) reads of the input instead of a residual written and re-read.
// ---------------------------------------------------------------------------
template <typename XT, typename ST>
__global__ __launch_bounds__(256) void split_generic_kernel(SplitParams p) {
    __shared__ float red[2][1][4];
    __shared__ LevelScale cs[kMaxLevels];
    const int t = threadIdx.x;
    const int64_t grow = blockIdx.x;
    const int64_t b = grow / p.rows;
    const int64_t r = grow % p.rows;
    const XT *xrow = (const XT *)p.X + b * p.xs_b + r * p.xs_r;
    const int64_t srow = b * p.ss_b + r * p.ss_r;

    // the fp32 residual entering level l >= 1 of input value x
    auto resid = [&](XT x, int l) {
        float rr;
        (void)Quant<ST, Modes<XT>::first>::run(x, cs[0], &rr);
        for (int j = 1; j < l; ++j) (void)Quant<ST, Modes<XT>::rest>::run(rr, cs[j], &rr);
        return rr;
    };
    for (int l = 0; l < p.L; ++l) {
        float m = 0.0f;
        for (int64_t k = t; k < p.K; k += 256) {
            const XT x = xrow[k * p.xs_k];
            m = fmaxf(m, l == 0 ? absf(x) : fabsf(resid(x, l)));
        }
        const LevelScale c = level_scale(row_max<4, 1>(m, red, l & 1, 0, t), p.alpha);
        if (t == 0) {
            cs[l] = c;
            p.scales[b * p.cs_b + l * p.cs_l + r * p.cs_r] = c.s;
        }
        __syncthreads();
        for (int64_t k = t; k < p.K; k += 256) {
            const XT x = xrow[k * p.xs_k];
            float rr;
            const uint32_t qv = (l == 0) ? Quant<ST, Modes<XT>::first>::run(x, c, &rr)
                                         : Quant<ST, Modes<XT>::rest>::run(resid(x, l), c, &rr);
            store1<ST>(p.slices, srow + l * p.ss_l + k * p.ss_k, qv);
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
                                                        int64_t xs_k, XT *__restrict__ T,
                                                        int vec_loads) {
    constexpr int TILE = 64;
    constexpr int VEC = 16 / (int)sizeof(XT);
    typedef XT vec_t __attribute__((ext_vector_type(VEC)));
    __shared__ XT tile[TILE][TILE + 1];
    const int64_t tiles_r = (rows + TILE - 1) / TILE;
    const int64_t tiles_k = (K + TILE - 1) / TILE;
    const int64_t tb = blockIdx.x;
    const int64_t b = tb / (tiles_r * tiles_k);
    const int64_t rem = tb % (tiles_r * tiles_k);
    const int64_t r0 = (rem % tiles_r) * TILE;
    const int64_t k0 = (rem / tiles_r) * TILE;
    const XT *xb = X + b * xs_b;
    // load: a lane covers VEC consecutive rows of one k (one 16-byte load when
    // the host found every such group 16-byte aligned and it lies inside)
    constexpr int LPR = TILE / VEC;              // lanes per k-row of the tile
    constexpr int KPP = 256 / LPR;               // k-rows per pass
    const int lr = threadIdx.x % LPR, lk = threadIdx.x / LPR;
#pragma unroll
    for (int kk = 0; kk < TILE; kk += KPP) {
        const int64_t k = k0 + kk + lk;
        const int64_t r = r0 + lr * VEC;
        XT v[VEC];
        if (vec_loads && k < K && r + VEC <= rows) {
            const vec_t w = *(const vec_t *)(xb + k * xs_k + r);
#pragma unroll
            for (int u = 0; u < VEC; ++u) v[u] = w[u];
        } else {
#pragma unroll
            for (int u = 0; u < VEC; ++u)
                v[u] = (k < K && r + u < rows) ? xb[k * xs_k + r + u] : (XT)0;
        }
#pragma unroll
        for (int u = 0; u < VEC; ++u) tile[kk + lk][lr * VEC + u] = v[u];
    }
    __syncthreads();
    // store: a lane covers VEC consecutive k of one row (K % VEC == 0, checked
    // on the host, and T rows start 16-byte aligned)
    XT *tb_out = T + b * rows * K;
#pragma unroll
    for (int rr = 0; rr < TILE; rr += KPP) {
        const int64_t r = r0 + rr + lk;
        const int64_t k = k0 + lr * VEC;
        if (r < rows && k < K) {
            vec_t w;
#pragma unroll
            for (int u = 0; u < VEC; ++u) w[u] = tile[lr * VEC + u][rr + lk];
            *(vec_t *)(tb_out + r * K + k) = w;
        }
    }
}

// ---------------------------------------------------------------------------
// Exact conversion of a narrow input (fp16 / bf16 / int8, any strides) into
// an fp32 copy [batch, rows, K] in the workspace.  A thread converts 4
// consecutive k of one row; rows run fastest when the operand's rows are
// contiguous (the B^T view), so loads stay coalesced either way.
// ---------------------------------------------------------------------------
template <typename XT>
__global__ __launch_bounds__(256) void convert_kernel(const XT *__restrict__ X, int64_t batch,
                                                      int64_t rows, int64_t K, int64_t xs_b,
                                                      int64_t xs_r, int64_t xs_k,
                                                      float *__restrict__ T, int rows_fast) {
    const int64_t kq = (K + 3) / 4;
    const int64_t total = batch * rows * kq;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        int64_t r, q;
        if (rows_fast) {
            r = i % rows;
            q = (i / rows) % kq;
        } else {
            q = i % kq;
            r = (i / kq) % rows;
        }
        const int64_t b = i / (rows * kq);
        const XT *src = X + b * xs_b + r * xs_r;
        float *dst = T + (b * rows + r) * K;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t k = 4 * q + u;
            if (k < K) dst[k] = (float)src[k * xs_k];
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
// capacity K <= nt * kpt; a lane holds kpt * VEC values: at most 64 (fp64:
// VEC = 2, kpt <= 32; fp32: VEC = 4, kpt <= 16)
static const StripCfg kStripCfgs[] = {
    {256, 4},     // K <= 1024
    {256, 8},     // K <= 2048
    {256, 16},    // K <= 4096
    {256, 32},    // K <= 8192  (fp64)
    {512, 16},    // K <= 8192  (fp32)
    {512, 32},    // K <= 16384 (fp64)
    {1024, 16},   // K <= 16384 (fp32)
};
static const int kNumStripCfgs = sizeof(kStripCfgs) / sizeof(kStripCfgs[0]);

// rows per lane of split_coop_kernel (64 values per lane: 32 rows of fp64,
// 16 of fp32), the members (K chunks of 32 * rpl rows) of a column group, and
// the workspace: the published maxima [groups][L][P][SW], 8 bytes each (none
// for P = 1)
static int coop_rpl(int xsz) { return 64 / (16 / xsz); }
static int64_t coop_members(int64_t K, int xsz, int seg) {
    const int64_t ch = (int64_t)kCoopNT / seg * coop_rpl(xsz);
    return K <= 0 ? 1 : (K + ch - 1) / ch;
}
static int64_t coop_slots(const SplitParams &p, int xsz, int seg) {
    const int64_t P = coop_members(p.K, xsz, seg);
    if (P <= 1) return 0;
    const int64_t sw = seg * (16 / xsz);
    const int64_t groups = p.batch * ((p.rows + sw - 1) / sw);
    return groups * p.L * P * sw;
}

static int64_t rows_coop_chunk(int xsz) { return xsz == 8 ? 4 * 8 * 256 : 4 * 16 * 256; }
static int64_t rows_coop_members(int64_t K, int xsz) {
    const int64_t ch = rows_coop_chunk(xsz);
    return K <= 0 ? 1 : (K + ch - 1) / ch;
}
static int64_t rows_coop_slots(const SplitParams &p, int xsz) {
    const int64_t P = rows_coop_members(p.K, xsz);
    return P > 1 ? p.batch * p.rows * p.L * P : 0;
}
// exchange words plus the launch's status word (none without an exchange)
static size_t slot_bytes(int64_t nslots) { return nslots > 0 ? (size_t)(nslots + 1) * 8 : 0; }
static size_t rows_coop_slot_bytes(const SplitParams &p, int xsz) {
    return slot_bytes(rows_coop_slots(p, xsz));
}
static size_t round256(size_t x) { return (x + 255) / 256 * 256; }

static bool aligned(const void *ptr, int64_t bytes) {
    return ((uintptr_t)ptr % (uintptr_t)bytes) == 0;
}

static int dtype_size(int code) {
    switch (code) {
    case 0: return 8;           // f64
    case 1: return 4;           // f32
    case 2: case 3: return 2;   // f16, bf16
    default: return 1;          // i8
    }
}

// layout of the fp32 copy a narrow input (fp16 / bf16 / int8) is split from
static SplitParams converted_params(const SplitParams &p) {
    SplitParams q = p;
    q.xs_b = p.rows * p.K;
    q.xs_r = p.K;
    q.xs_k = 1;
    return q;
}

// ---------------------------------------------------------------------------
// Residency limit of the cooperative kernels.  The members of a group are
// consecutive workgroup ids and workgroups are dispatched in id order.  While
// the group of the oldest unfinished workgroup is not wholly resident, every
// workgroup that holds back the next id is a member of that group: the ids
// before it have finished, the next id is the group's own.  If the hardware
// sends each id to a fixed XCD, that XCD is full of members; if to any XCD
// with room, every XCD is.  Either way the group has more members than one
// XCD holds, so a group of at most that many (less a margin of 8) always
// becomes resident and its waits end.  One XCD holds the kernels' occupancy
// (the fewest workgroups per CU over every kernel that waits) times its CUs:
// 32 on gfx950, or all of a smaller partition.  Asked once per device; where
// the runtime cannot say (no device: a workspace query on a host without a
// GPU) MI355X's figure is assumed: 2 workgroups per CU (the kernels with
// 169-205 VGPRs, one wave per SIMD each, fit twice in 512), so 64 per XCD
// and at most 56 members (the row kernel's 64 chunks are cut to 56).
// ---------------------------------------------------------------------------
constexpr int kCusPerXcd = 32;
constexpr int kMi355xResident = 2 * kCusPerXcd;

template <typename Kern> static void min_occupancy(Kern kernel, int &occ, bool &ok) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kCoopNT, 0) != hipSuccess ||
        n <= 0) {
        ok = false;
        return;
    }
    occ = n < occ ? n : occ;
}

template <typename ST> static void coop_occupancy(int &occ, bool &ok) {
    min_occupancy(split_rows_coop_kernel<double, ST, 4, 8>, occ, ok);
    min_occupancy(split_rows_coop_kernel<float, ST, 4, 16>, occ, ok);
    min_occupancy(split_coop_kernel<double, ST, 32, 8>, occ, ok);
    min_occupancy(split_coop_kernel<double, ST, 32, 2>, occ, ok);
    min_occupancy(split_coop_kernel<float, ST, 16, 8>, occ, ok);
    min_occupancy(split_coop_kernel<float, ST, 16, 2>, occ, ok);
    min_occupancy(split_pair_kernel<double, ST, 32, 4>, occ, ok);
    min_occupancy(split_pair_kernel<double, ST, 32, 8>, occ, ok);
}

int coop_resident_per_xcd() {
    if (debug_overrides().coop_resident > 0) return debug_overrides().coop_resident;
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kMi355xResident;
    int r = cached[dev].load(std::memory_order_relaxed);
    if (r > 0) return r;
    int cus = 0, occ = 1 << 20;
    bool ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ==
                  hipSuccess && cus > 0;
    if (ok) {
        coop_occupancy<int8_t>(occ, ok);
        coop_occupancy<_Float16>(occ, ok);
        coop_occupancy<__bf16>(occ, ok);
        coop_occupancy<float>(occ, ok);
    }
    if (!ok) {
        (void)hipGetLastError();   // a failed query is not a launch error
        return kMi355xResident;
    }
    r = occ * (cus < kCusPerXcd ? cus : kCusPerXcd);
    cached[dev].store(r, std::memory_order_relaxed);
    return r;
}

// the most members a cooperative group may have on the current device (at
// least 1: a group of one never waits)
static int64_t coop_member_limit(int64_t kernel_max) {
    const int64_t r = (int64_t)coop_resident_per_xcd() - 8;
    return r < 1 ? 1 : (r < kernel_max ? r : kernel_max);
}

static SplitPlan plan_split_raw(const SplitParams &p, int x_dtype, int slice_dtype) {
    // narrow inputs: the reference loads them into its fp32 RES exactly
    // (ozaki_triton.py:188), so they are converted into the workspace first and
    // split as fp32 (X is replaced by the workspace at launch, which is 16-byte
    // aligned; the plan of the copy is taken with that assumption)
    if (x_dtype >= 2) return {kSplitConvert, 0};
    const int xsz = dtype_size(x_dtype);
    const int ssz = dtype_size(slice_dtype);
    const bool k4 = (p.K % 4) == 0;
    const bool slice_ok = p.ss_k == 1 && aligned(p.slices, 4 * ssz) &&
                          (p.ss_r * ssz) % (4 * ssz) == 0 && (p.ss_l * ssz) % (4 * ssz) == 0 &&
                          (p.ss_b * ssz) % (4 * ssz) == 0;
    // the test hooks (include/ozaki_amd_debug.h) steer column operands to the
    // coop / strip / transpose / generic path, or force one of the two row
    // kernels; a path whose requirements fail is not taken
    const int force = debug_overrides().split;
    auto forced = [&](int which) { return force == which; };
    // long rows: the row kernel shared by workgroups
    const bool rows_coop = rows_coop_members(p.K, xsz) <= coop_member_limit(kRowsCoopMaxP) &&
                           (forced(kForceSplitRowsCoop) || (!forced(kForceSplitRows) && p.K > kRowsCoopMinK));
    if (k4 && slice_ok && p.xs_k == 1 && aligned(p.X, 16) && (p.xs_r * xsz) % 16 == 0 &&
        (p.xs_b * xsz) % 16 == 0 && !forced(kForceSplitGeneric)) {
        if (rows_coop) return {kSplitRows, kRowsCoopVariant};
        for (int i = 0; i < kNumRowCfgs; ++i) {
            const RowCfg &c = kRowCfgs[i];
            if (x_dtype == 0 && c.nc > 8) continue;
            if (p.K <= (int64_t)4 * c.nc * 64 * c.gw) return {kSplitRows, i};
        }
    }
    const int vec = 16 / xsz;
    const bool cols_ok = k4 && slice_ok && p.xs_r == 1 && p.rows % vec == 0 && aligned(p.X, 16) &&
                         (p.xs_k * xsz) % 16 == 0 && (p.xs_b * xsz) % 16 == 0;
    // columns of 64 KB and more: the cooperative kernel (the strip kernel's
    // 16-byte row pieces cost more than the exchange from there on; measured
    // over K = 1024..16384, N = 1024..8192, fp64 / fp32), and fp64 columns of
    // 32 KB into 1 or 2 int8 slices when there are at least 2048 of them
    // (alone, 0.90-0.94x the strip kernel's time at K = 4096, N = 2048..8192;
    // 1.04x at N = 1024; fp16 slices gain nothing there, fp32 columns below
    // 64 KB lose 1.1-1.3x).  With 3 or more slices the strip kernel and A's
    // rows share one launch (split_duo_kernel), and the whole call is faster
    // that way: at K = 4096, 4 slices, 83.3 / 370.8 / 1163 us against 89.2 /
    // 394.2 / 1197 for M x N = 128 x 2048, 1024 x 4096, 2048 x 8192, while 1
    // slice is 7-11% slower and 2 even.  A forced coop takes it for any length
    // it holds
    const int64_t coop_max = coop_member_limit(kCoopMaxP);
    const bool coop_fits = cols_ok && coop_members(p.K, xsz, 8) <= coop_max;
    // columns too long for 32 chunks of 128-byte groups: 32-byte groups, whose
    // chunks hold 4x the rows, when the cooperative kernel is forced.  By
    // default such columns are transposed instead: at config 5 (fp32, K =
    // 65536, 32 chunks of 2048 rows) the 32-byte groups took 0.255-0.265 ms
    // against 0.216 ms for the transpose path, the exchange waiting on 32
    // members per group.
    const bool coop2_fits = cols_ok && !coop_fits && coop_members(p.K, xsz, 2) <= coop_max;
    const bool other = forced(kForceSplitStrip) || forced(kForceSplitTranspose) || forced(kForceSplitGeneric);
    const bool coop_long = p.K * xsz >= kCoopMinColumnBytes ||
                           (xsz == 8 && ssz == 1 && p.L <= 2 &&
                            p.K * xsz >= kCoopMinColumnBytes / 2 && p.batch * p.rows >= 2048);
    if (coop_fits && (forced(kForceSplitCoop) || (!other && coop_long))) return {kSplitCoop, 8};
    if (coop2_fits && forced(kForceSplitCoop)) return {kSplitCoop, 2};
    if (cols_ok && !forced(kForceSplitTranspose) && !forced(kForceSplitGeneric)) {
        for (int i = 0; i < kNumStripCfgs; ++i) {
            const StripCfg &c = kStripCfgs[i];
            if (c.kpt * vec > 64) continue;
            if (p.K <= (int64_t)c.kpt * c.nt) return {kSplitStrip, i};
        }
    }
    // row-contiguous operand with a K too long for a resident strip: transpose
    // into the workspace, then the row kernel (if the row fits)
    if (k4 && slice_ok && p.xs_r == 1 && (p.K * xsz) % 16 == 0 && !forced(kForceSplitGeneric)) {
        if (rows_coop) return {kSplitTransposeRows, kRowsCoopVariant};
        for (int i = 0; i < kNumRowCfgs; ++i) {
            const RowCfg &c = kRowCfgs[i];
            if (x_dtype == 0 && c.nc > 8) continue;
            if (p.K <= (int64_t)4 * c.nc * 64 * c.gw) return {kSplitTransposeRows, i};
        }
    }
    return {kSplitGeneric, 0};
}


SplitPlan plan_split(const SplitParams &p, int x_dtype, int slice_dtype) {
    const SplitPlan plan = plan_split_raw(p, x_dtype, slice_dtype);
    if (aligned(p.X, 16) && aligned(p.slices, 16)) return plan;   // the aligned plan
    // other pointers: no more scratch than the workspace queries reserve for
    // aligned ones, which see no pointers (the generic kernel needs none)
    SplitParams q = p;
    q.X = (const void *)(uintptr_t)256;
    q.slices = (void *)(uintptr_t)256;
    const SplitPlan ref = plan_split_raw(q, x_dtype, slice_dtype);
    if (split_workspace_bytes(p, plan, x_dtype, slice_dtype) >
        split_workspace_bytes(q, ref, x_dtype, slice_dtype))
        return {kSplitGeneric, 0};
    return plan;
}

// plan of the fp32 copy of a narrow input (its X is the 16-byte aligned
// workspace: `aligned` in plan_split must see an aligned pointer)
static SplitPlan converted_plan(const SplitParams &p, int slice_dtype) {
    SplitParams q = converted_params(p);
    q.X = (const void *)(uintptr_t)256;
    return plan_split(q, 1, slice_dtype);
}

size_t split_workspace_bytes(const SplitParams &p, const SplitPlan &plan, int x_dtype,
                             int slice_dtype) {
    const int64_t n = p.batch * p.rows * p.K;
    if (plan.path == kSplitConvert) {
        const SplitPlan inner = converted_plan(p, slice_dtype);
        const size_t in = split_workspace_bytes(converted_params(p), inner, 1, slice_dtype);
        return in ? round256((size_t)(n * 4)) + in : (size_t)(n * 4);
    }
    if (plan.path == kSplitTransposeRows) {
        const size_t tb = (size_t)(n * dtype_size(x_dtype));
        if (plan.variant != kRowsCoopVariant) return tb;
        return round256(tb) + rows_coop_slot_bytes(p, dtype_size(x_dtype));
    }
    if (plan.path == kSplitRows && plan.variant == kRowsCoopVariant)
        return rows_coop_slot_bytes(p, dtype_size(x_dtype));
    if (plan.path == kSplitCoop) return slot_bytes(coop_slots(p, dtype_size(x_dtype), plan.variant));
    return 0;
}

// Clears n exchange words and the status word after them.
static hipError_t clear_slots(uint64_t *slot, int64_t n, hipStream_t st) {
    const int64_t zb = (n + 256) / 256 < 2048 ? (n + 256) / 256 : 2048;
    hipLaunchKernelGGL(zero_u64_kernel, dim3((unsigned)zb), dim3(256), 0, st, slot, n + 1);
    return hipGetLastError();
}

// Follows a cooperative launch whose status word is `status` (see
// poison_scales_kernel).
static hipError_t launch_poison(const SplitParams &p, const uint64_t *status, hipStream_t st) {
    if (p.fail_out) {   // the cross-GEMM that follows checks the word instead
        *p.fail_out = (const uint32_t *)status;
        return hipSuccess;
    }
    const int64_t n = p.batch * p.L * p.rows;
    const int64_t nb = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
    hipLaunchKernelGGL(poison_scales_kernel, dim3((unsigned)nb), dim3(256), 0, st,
                       (const uint32_t *)status, p.scales, p.batch, p.L, p.rows, p.cs_b, p.cs_l,
                       p.cs_r);
    return hipGetLastError();
}

// The tag a wait looks for and its time limit: the test hook makes every wait
// look for a tag that is never written and give up at its first check, so
// the timeout path runs with no wait longer than one poll.
struct WaitRule {
    uint32_t tag;
    uint64_t ticks;
};
static WaitRule wait_rule() {
    const bool force = debug_overrides().coop_timeout != 0;
    return {(uint32_t)(kCoopTag >> 32) + (force ? 1u : 0u), force ? 0ull : kCoopTickLimit};
}

template <typename XT, typename ST>
static hipError_t launch_rows_coop(const SplitParams &p, uint64_t *slot, hipStream_t st) {
    const int xsz = (int)sizeof(XT);
    const int64_t P = rows_coop_members(p.K, xsz);
    const int64_t n = rows_coop_slots(p, xsz);
    uint32_t *status = nullptr;
    if (P > 1) {
        if (hipError_t e = clear_slots(slot, n, st)) return e;
        status = (uint32_t *)(slot + n);
    }
    const WaitRule w = wait_rule();
    const dim3 grid((unsigned)(p.batch * p.rows * P)), block(256);
    if constexpr (sizeof(XT) == 8)
        hipLaunchKernelGGL((split_rows_coop_kernel<XT, ST, 4, 8>), grid, block, 0, st, p, slot,
                           (int)P, w.tag, w.ticks, status);
    else
        hipLaunchKernelGGL((split_rows_coop_kernel<XT, ST, 4, 16>), grid, block, 0, st, p, slot,
                           (int)P, w.tag, w.ticks, status);
    if (hipError_t e = hipGetLastError()) return e;
    return P > 1 ? launch_poison(p, slot + n, st) : hipSuccess;
}

template <typename XT, typename ST>
static hipError_t launch_rows(const SplitParams &p, int v, hipStream_t st, uint64_t *slot) {
    if (v == kRowsCoopVariant) return launch_rows_coop<XT, ST>(p, slot, st);
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
    constexpr int VEC = 16 / (int)sizeof(XT);
    const int64_t nstrips = p.batch * (p.rows / VEC);   // rows % VEC == 0
#define OZK_STRIP(NT, KPT)                                                                  \
    hipLaunchKernelGGL((split_strip_kernel<XT, ST, NT, KPT>), dim3((unsigned)nstrips),      \
                       dim3(NT), 0, st, p)
    switch (v) {
    case 0: OZK_STRIP(256, 4); break;
    case 1: OZK_STRIP(256, 8); break;
    case 2: OZK_STRIP(256, 16); break;
    case 3:
        if constexpr (VEC == 2) { OZK_STRIP(256, 32); } else return hipErrorInvalidValue;
        break;
    case 4: OZK_STRIP(512, 16); break;
    case 5:
        if constexpr (VEC == 2) { OZK_STRIP(512, 32); } else return hipErrorInvalidValue;
        break;
    case 6: OZK_STRIP(1024, 16); break;
    default: return hipErrorInvalidValue;
    }
#undef OZK_STRIP
    return hipGetLastError();
}

template <typename XT, typename ST>
static hipError_t launch_typed(const SplitParams &p, const SplitPlan &plan, hipStream_t st) {
    switch (plan.path) {
    case kSplitRows: return launch_rows<XT, ST>(p, plan.variant, st, (uint64_t *)p.resid);
    case kSplitStrip: return launch_strip<XT, ST>(p, plan.variant, st);
    case kSplitCoop: {
        const int seg = plan.variant;   // 16-byte pieces per row of a column group
        const int64_t sw = seg * (16 / (int)sizeof(XT));
        const int64_t groups = p.batch * ((p.rows + sw - 1) / sw);
        const int64_t P = coop_members(p.K, (int)sizeof(XT), seg);
        uint64_t *slot = nullptr;
        uint32_t *status = nullptr;
        const int64_t n = coop_slots(p, (int)sizeof(XT), seg);
        if (P > 1) {
            slot = (uint64_t *)p.resid;
            if (hipError_t e = clear_slots(slot, n, st)) return e;
            status = (uint32_t *)(slot + n);
        }
        const dim3 grid((unsigned)(groups * P)), block(kCoopNT);
        constexpr int RPL = 64 / (16 / (int)sizeof(XT));
        const WaitRule w = wait_rule();
        if (seg == 8)
            hipLaunchKernelGGL((split_coop_kernel<XT, ST, RPL, 8>), grid, block, 0, st, p, slot,
                               (int)P, w.tag, w.ticks, status);
        else if (seg == 2)
            hipLaunchKernelGGL((split_coop_kernel<XT, ST, RPL, 2>), grid, block, 0, st, p, slot,
                               (int)P, w.tag, w.ticks, status);
        else
            return hipErrorInvalidValue;
        if (hipError_t e = hipGetLastError()) return e;
        return P > 1 ? launch_poison(p, slot + n, st) : hipSuccess;
    }
    case kSplitTransposeRows: {
        XT *T = (XT *)p.resid;   // workspace [batch, rows, K]
        const int64_t tiles = p.batch * ((p.rows + 63) / 64) * ((p.K + 63) / 64);
        const int64_t xsz = (int64_t)sizeof(XT);
        const int vec_loads = aligned(p.X, 16) && (p.xs_k * xsz) % 16 == 0 &&
                              (p.xs_b * xsz) % 16 == 0;
        hipLaunchKernelGGL((transpose_kernel<XT>), dim3((unsigned)tiles), dim3(256), 0, st,
                           (const XT *)p.X, p.batch, p.rows, p.K, p.xs_b, p.xs_k, T, vec_loads);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        SplitParams q = p;
        q.X = T;
        q.xs_b = p.rows * p.K;
        q.xs_r = p.K;
        q.xs_k = 1;
        // the exchange words of the shared row kernel follow the transposed copy
        const size_t tb = (size_t)(p.batch * p.rows * p.K) * sizeof(XT);
        return launch_rows<XT, ST>(q, plan.variant, st, (uint64_t *)((char *)p.resid + round256(tb)));
    }
    default:
        hipLaunchKernelGGL((split_generic_kernel<XT, ST>), dim3((unsigned)(p.batch * p.rows)),
                           dim3(256), 0, st, p);
        return hipGetLastError();
    }
}

template <typename XT>
static hipError_t launch_convert(const SplitParams &p, float *T, hipStream_t st) {
    const int64_t total = p.batch * p.rows * ((p.K + 3) / 4);
    if (total == 0) return hipSuccess;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const int rows_fast = (p.xs_r == 1 && p.xs_k != 1);
    hipLaunchKernelGGL((convert_kernel<XT>), dim3((unsigned)blocks), dim3(256), 0, st,
                       (const XT *)p.X, p.batch, p.rows, p.K, p.xs_b, p.xs_r, p.xs_k, T,
                       rows_fast);
    return hipGetLastError();
}

template <typename ST>
static hipError_t launch_slice(const SplitParams &p, const SplitPlan &plan, int x_dtype,
                               int slice_dtype, hipStream_t st) {
    if (x_dtype == 0) return launch_typed<double, ST>(p, plan, st);
    if (x_dtype == 1) return launch_typed<float, ST>(p, plan, st);
    // narrow input: convert into the workspace, then split the fp32 copy (any
    // scratch that split needs follows the copy)
    float *T = p.resid;
    hipError_t e;
    if (x_dtype == 2) e = launch_convert<_Float16>(p, T, st);
    else if (x_dtype == 3) e = launch_convert<__bf16>(p, T, st);
    else e = launch_convert<int8_t>(p, T, st);
    if (e != hipSuccess) return e;
    SplitParams q = converted_params(p);
    q.X = T;
    q.resid = (float *)((char *)T + round256((size_t)(p.batch * p.rows * p.K) * 4));
    const SplitPlan inner = plan_split(q, 1, slice_dtype);
    return launch_typed<float, ST>(q, inner, st);
}

hipError_t launch_split(const SplitParams &p, const SplitPlan &plan, int x_dtype,
                        int slice_dtype, hipStream_t st) {
    if (p.batch * p.rows == 0 || p.L == 0) return hipSuccess;
    switch (slice_dtype) {
    case 4: return launch_slice<int8_t>(p, plan, x_dtype, slice_dtype, st);
    case 2: return launch_slice<_Float16>(p, plan, x_dtype, slice_dtype, st);
    case 3: return launch_slice<__bf16>(p, plan, x_dtype, slice_dtype, st);
    case 1: return launch_slice<float>(p, plan, x_dtype, slice_dtype, st);
    }
    return hipErrorInvalidValue;
}

// split_pair_kernel's row configurations: variants 4 and 5 of kRowCfgs (4
// waves per row, K <= 4096 / 8192)
static int pair_nc(const SplitPlan &a) {
    return a.path == kSplitRows ? (a.variant == 4 ? 4 : a.variant == 5 ? 8 : 0) : 0;
}

bool split_pair_ok(const SplitPlan &plan_a, const SplitPlan &plan_b, int x_dtype) {
    return x_dtype == 0 && pair_nc(plan_a) != 0 && plan_b.path == kSplitCoop &&
           plan_b.variant == 8 && debug_overrides().split == kForceSplitNone;
}

template <typename ST>
static hipError_t launch_pair_typed(const SplitParams &pa, const SplitPlan &plan_a,
                                    const SplitParams &pb, hipStream_t st) {
    using XT = double;
    constexpr int RPL = 64 / (16 / (int)sizeof(XT));
    const int64_t sw = 8 * (16 / (int)sizeof(XT));
    const int64_t groups = pb.batch * ((pb.rows + sw - 1) / sw);
    const int64_t P = coop_members(pb.K, (int)sizeof(XT), 8);
    const int64_t n = coop_slots(pb, (int)sizeof(XT), 8);
    uint64_t *slot = nullptr;
    uint32_t *status = nullptr;
    if (P > 1) {
        slot = (uint64_t *)pb.resid;
        if (hipError_t e = clear_slots(slot, n, st)) return e;
        status = (uint32_t *)(slot + n);
    }
    const int64_t na = pa.batch * pa.rows;
    const int64_t ka = groups > 0 ? (na + groups - 1) / groups : 0;
    const dim3 grid((unsigned)(groups * (P + ka))), block(kCoopNT);
    const WaitRule w = wait_rule();
    if (pair_nc(plan_a) == 4)
        hipLaunchKernelGGL((split_pair_kernel<XT, ST, RPL, 4>), grid, block, 0, st, pb, slot,
                           (int)P, w.tag, w.ticks, status, pa, (int)ka);
    else
        hipLaunchKernelGGL((split_pair_kernel<XT, ST, RPL, 8>), grid, block, 0, st, pb, slot,
                           (int)P, w.tag, w.ticks, status, pa, (int)ka);
    if (hipError_t e = hipGetLastError()) return e;
    return P > 1 ? launch_poison(pb, slot + n, st) : hipSuccess;
}

hipError_t launch_split_pair(const SplitParams &pa, const SplitPlan &plan_a,
                             const SplitParams &pb, const SplitPlan &plan_b, int x_dtype,
                             int slice_dtype, hipStream_t st) {
    if (!split_pair_ok(plan_a, plan_b, x_dtype)) return hipErrorInvalidValue;
    if (pa.batch * pa.rows == 0 || pb.batch * pb.rows == 0 || pa.L == 0) return hipSuccess;
    switch (slice_dtype) {
    case 4: return launch_pair_typed<int8_t>(pa, plan_a, pb, st);
    case 2: return launch_pair_typed<_Float16>(pa, plan_a, pb, st);
    case 3: return launch_pair_typed<__bf16>(pa, plan_a, pb, st);
    case 1: return launch_pair_typed<float>(pa, plan_a, pb, st);
    }
    return hipErrorInvalidValue;
}

// split_duo_kernel's pairs of strip configuration (kStripCfgs, 256 lanes) and
// row configuration (kRowCfgs, 256 lanes): the ones plan_split takes for one K
bool split_duo_ok(const SplitPlan &plan_a, const SplitPlan &plan_b, int x_dtype) {
    if ((x_dtype != 0 && x_dtype != 1) || debug_overrides().split != kForceSplitNone) return false;
    if (plan_a.path != kSplitRows || plan_b.path != kSplitStrip) return false;
    const int s = plan_b.variant, r = plan_a.variant;
    return (s == 0 && r >= 0 && r <= 2) || (s == 1 && r == 3) || (s == 2 && r == 4) ||
           (s == 3 && r == 5 && x_dtype == 0);
}

template <typename XT, typename ST>
static hipError_t launch_duo_typed(const SplitParams &pa, int r, const SplitParams &pb, int s,
                                   hipStream_t st) {
    constexpr int VEC = 16 / (int)sizeof(XT);
    const int64_t nstrips = pb.batch * (pb.rows / VEC);   // rows % VEC == 0 (strip plan)
    const int64_t nrows = pa.batch * pa.rows;
#define OZK_DUO(KPT, GW, RPB, NC)                                                            \
    hipLaunchKernelGGL((split_duo_kernel<XT, ST, KPT, GW, RPB, NC>),                          \
                       dim3((unsigned)(nstrips + (nrows + RPB - 1) / RPB)), dim3(256), 0, st, pb, \
                       nstrips, pa)
    switch (s * 10 + r) {
    case 0: OZK_DUO(4, 1, 4, 1); break;
    case 1: OZK_DUO(4, 1, 4, 2); break;
    case 2: OZK_DUO(4, 1, 4, 4); break;
    case 13: OZK_DUO(8, 4, 1, 2); break;
    case 24: OZK_DUO(16, 4, 1, 4); break;
    case 35:
        if constexpr (VEC == 2) { OZK_DUO(32, 4, 1, 8); } else return hipErrorInvalidValue;
        break;
    default: return hipErrorInvalidValue;
    }
#undef OZK_DUO
    return hipGetLastError();
}

template <typename XT>
static hipError_t launch_duo_x(const SplitParams &pa, int r, const SplitParams &pb, int s,
                               int slice_dtype, hipStream_t st) {
    switch (slice_dtype) {
    case 4: return launch_duo_typed<XT, int8_t>(pa, r, pb, s, st);
    case 2: return launch_duo_typed<XT, _Float16>(pa, r, pb, s, st);
    case 3: return launch_duo_typed<XT, __bf16>(pa, r, pb, s, st);
    case 1: return launch_duo_typed<XT, float>(pa, r, pb, s, st);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_split_duo(const SplitParams &pa, const SplitPlan &plan_a, const SplitParams &pb,
                            const SplitPlan &plan_b, int x_dtype, int slice_dtype,
                            hipStream_t st) {
    if (!split_duo_ok(plan_a, plan_b, x_dtype)) return hipErrorInvalidValue;
    if (pa.batch * pa.rows == 0 || pb.batch * pb.rows == 0 || pa.L == 0) return hipSuccess;
    return x_dtype == 0 ? launch_duo_x<double>(pa, plan_a.variant, pb, plan_b.variant, slice_dtype, st)
                        : launch_duo_x<float>(pa, plan_a.variant, pb, plan_b.variant, slice_dtype, st);
}

uint32_t *device_status_word() {
    static std::atomic<uint32_t *> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    uint32_t *ptr = cached[dev].load(std::memory_order_acquire);
    if (!ptr) {
        void *addr = nullptr;
        if (hipGetSymbolAddress(&addr, HIP_SYMBOL(g_device_status)) != hipSuccess) return nullptr;
        ptr = (uint32_t *)addr;
        cached[dev].store(ptr, std::memory_order_release);
    }
    return ptr;
}

hipError_t read_device_status(unsigned *out, bool clear, hipStream_t st) {
    uint32_t v = 0;
    hipError_t e = hipMemcpyFromSymbolAsync(&v, HIP_SYMBOL(g_device_status), sizeof(v), 0,
                                            hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess && clear && v != 0) {
        const uint32_t zero = 0;
        e = hipMemcpyToSymbolAsync(HIP_SYMBOL(g_device_status), &zero, sizeof(zero), 0,
                                   hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
    }
    *out = v;
    return e;
}

}  // namespace ozk
