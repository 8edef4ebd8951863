/*
 * ozaki_oracle.c -- CPU restatement of the Ozaki-scheme split and cross-GEMM of
 * WhFanatic/Ozaki_triton (ozaki_triton.py), written in plain C.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (ozaki_triton_amd, libozaki_amd.so) never links or calls it.
 *
 * Semantics followed (all citations are /root/reference files):
 *   - compute_split_bits ........................ ozaki_triton.py:76-98
 *   - residual compute dtype RES = fp64 for fp64 input else fp32
 *                                                 ozaki_triton.py:69-73,227
 *   - residual buffer always fp32 (every stored residual is rounded to fp32)
 *                                                 ozaki_triton.py:233,211
 *   - row max  mu = max(1e-38f, fl32(max_k |src_k|))   ozaki_triton.py:172,192
 *   - scale    s  = exp2(ceil(log2(mu)) - alpha) in fp32  ozaki_triton.py:174
 *     log2 is the correctly rounded float32 log2 (what the Triton interpreter's
 *     numpy log2 returns); ceil() of it has the integer closed form in
 *     ozo_ceil_log2_f32 below.
 *   - q = src / s in RES                          ozaki_triton.py:196
 *   - int8 slice: trunc(clip(fl(q +/- 0.5), -128, 127))  ozaki_triton.py:199-200
 *   - fp16 / bf16 / fp32 slice: single round-to-nearest-even from RES
 *                                                 ozaki_triton.py:202
 *   - inputs fp16 / bf16 / int8 are converted exactly to the fp32 RES
 *                                                 ozaki_triton.py:188,190
 *   - residual  r = src - (RES)slice * (RES)s, stored as fp32 for l < L-1
 *                                                 ozaki_triton.py:208-211
 *   - cross-GEMM: acc_ij = A_i . B_j (int32 exact for int8, fp32 hardware for
 *     fp16); t_ij = fl32(fl32(fl32(acc_ij) * sa_i) * sb_j);
 *     out = 0; for i: for j: out = fl_OUTACC(out + t_ij); C = (out dtype) out,
 *     where the final cast rounds to nearest even for fp16 / bf16 output and
 *     truncates toward zero, saturating, for int8 output (the NVIDIA
 *     float-to-integer conversion the reference's tl.store performs)
 *                                                 ozaki_triton.py:357-452
 *
 * Must be compiled with -ffp-contract=off (no fused multiply-add may merge a
 * multiply and an add whose intermediate the reference rounds) and without
 * -ffast-math; x86-64 SSE arithmetic gives IEEE binary32/binary64 results.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* dtype codes shared with include/ozaki_amd.h */
enum { OZO_F64 = 0, OZO_F32 = 1, OZO_F16 = 2, OZO_BF16 = 3, OZO_I8 = 4, OZO_I32 = 5 };

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* alpha rule: ozaki_triton.py:87-98.  Returns alpha, or a value < 1 when the
 * reference's assert would fire, or -1000 for an unsupported accumulator.     */
int ozo_compute_split_bits(int64_t n, int slice_dtype, int dot_accum_dtype)
{
    int acc_bits;
    if (dot_accum_dtype == OZO_I32) acc_bits = 31;
    else if (dot_accum_dtype == OZO_F32) acc_bits = 23;
    else return -1000;
    int slice_bits;
    switch (slice_dtype) {
    case OZO_F32: slice_bits = 23; break;
    case OZO_F16: slice_bits = 10; break;
    case OZO_BF16: slice_bits = 7; break;
    case OZO_I8: slice_bits = 7; break;
    default: return -1000;
    }
    /* int((acc_bits - log2(n)) / 2): Python int() truncates toward zero */
    double a = ((double)acc_bits - log2((double)n)) / 2.0;
    int alpha = (int)a;   /* C cast truncates toward zero as well */
    if (alpha > slice_bits) alpha = slice_bits;
    return alpha;
}

/* ------------------------------------------------------------------------ */
/* ceil(RN_f32(log2(mu))) for a positive finite float mu >= 1e-38f.
 * mu = 2^k (1 + j 2^-23):  j == 0 -> k ; 1 <= j <= J(k) -> k (log2 rounds down
 * onto the integer k) ; otherwise k + 1.  J(k) = floor(2^(p-1) ln 2) with
 * 2^p <= k < 2^(p+1) for k >= 4, 2^p < |k| <= 2^(p+1) for k <= -5, and J = 0 for
 * -4 <= k <= 3.  Subnormal mu in [1e-38f, 2^-126): log2 lies in (-126.24, -126),
 * so the ceiling is -126 whatever the rounding.                                */
static const int ozo_J_by_p[7] = {0, 0, 1, 2, 5, 11, 22};

int ozo_band_J(int k)
{
    int p;
    if (k >= 4) { p = 0; while ((2 << p) <= k) ++p; }            /* 2^p <= k < 2^(p+1) */
    else if (k <= -5) { int a = -k; p = 0; while ((2 << p) < a) ++p; } /* 2^p < a <= 2^(p+1) */
    else return 0;
    return ozo_J_by_p[p];
}

int ozo_ceil_log2_f32(float mu)
{
    uint32_t u = f32_bits(mu);
    int be = (int)(u >> 23) & 0xFF;
    uint32_t j = u & 0x7FFFFFu;
    if (be == 0) return -126;
    int k = be - 127;
    if (j == 0) return k;
    if ((int)j <= ozo_band_J(k)) return k;
    return k + 1;
}

/* exact 2^e as a float for e in [-149, 127] (subnormal for e < -126) */
float ozo_pow2f(int e)
{
    if (e >= -126) return bits_f32((uint32_t)(e + 127) << 23);
    return bits_f32(1u << (e + 149));
}

/* scale of one row: ozaki_triton.py:174.  A row holding +-inf has mu = inf,
 * where the reference's exp2(ceil(log2(mu)) - alpha) is inf (log2(inf) = inf,
 * ozaki_triton.py:173-176); the closed form above covers finite mu only. */
float ozo_scale_from_max(float mu, int alpha)
{
    if (!(mu <= FLT_MAX)) return mu;
    return ozo_pow2f(ozo_ceil_log2_f32(mu) - alpha);
}

/* ------------------------------------------------------------------------ */
/* Round-to-nearest-even binary64 -> binary16 in one step (no double rounding
 * through binary32).  Returns the fp16 bit pattern.                           */
uint16_t ozo_f64_to_f16(double x)
{
    uint64_t u; memcpy(&u, &x, 8);
    uint16_t s = (uint16_t)((u >> 48) & 0x8000u);
    int be = (int)((u >> 52) & 0x7FF);
    uint64_t m = u & 0xFFFFFFFFFFFFFull;
    if (be == 0x7FF) return (uint16_t)(s | (m ? 0x7E00u : 0x7C00u));
    if (be == 0) return s;                       /* |x| < 2^-1022 -> 0 */
    uint64_t sig = (1ull << 52) | m;             /* x = sig * 2^(e-52) */
    int e = be - 1023;
    int qe = (e < -14 ? -14 : e) - 10;           /* fp16 quantum 2^qe */
    int shift = qe - (e - 52);                   /* >= 42 */
    if (shift > 63) return s;                    /* |x| < 2^-35: rounds to 0 */
    uint64_t n = sig >> shift;
    uint64_t rem = sig & ((1ull << shift) - 1);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (n & 1u))) ++n;
    uint32_t b = (e <= -14) ? (uint32_t)n : (uint32_t)(((e + 14) << 10) + n);
    if (b >= 0x7C00u) b = 0x7C00u;
    return (uint16_t)(s | b);
}

double ozo_f16_to_f64(uint16_t h)
{
    int s = h >> 15, be = (h >> 10) & 0x1F, m = h & 0x3FF;
    double v;
    if (be == 0x1F) v = m ? NAN : INFINITY;
    else if (be == 0) v = ldexp((double)m, -24);
    else v = ldexp((double)(1024 + m), be - 25);
    return s ? -v : v;
}

/* Round-to-nearest-even binary64 -> bfloat16 in one step.  bfloat16 has
 * binary32's exponent range and 8 significant bits: quantum 2^(e-7) for a
 * normal value, 2^-133 below 2^-126.  Returns the bit pattern.                */
uint16_t ozo_f64_to_bf16(double x)
{
    uint64_t u; memcpy(&u, &x, 8);
    uint16_t s = (uint16_t)((u >> 48) & 0x8000u);
    int be = (int)((u >> 52) & 0x7FF);
    uint64_t m = u & 0xFFFFFFFFFFFFFull;
    if (be == 0x7FF) return (uint16_t)(s | (m ? 0x7FC0u : 0x7F80u));
    if (be == 0) return s;
    uint64_t sig = (1ull << 52) | m;
    int e = be - 1023;
    int qe = (e < -126 ? -126 : e) - 7;
    int shift = qe - (e - 52);                   /* >= 45 */
    if (shift > 63) return s;
    uint64_t n = sig >> shift;
    uint64_t rem = sig & ((1ull << shift) - 1);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (n & 1u))) ++n;
    uint32_t b = (e <= -126) ? (uint32_t)n : (uint32_t)(((e + 126) << 7) + n);
    if (b >= 0x7F80u) b = 0x7F80u;
    return (uint16_t)(s | b);
}

double ozo_bf16_to_f64(uint16_t h)
{
    int s = h >> 15, be = (h >> 7) & 0xFF, m = h & 0x7F;
    double v;
    if (be == 0xFF) v = m ? NAN : INFINITY;
    else if (be == 0) v = ldexp((double)m, -133);
    else v = ldexp((double)(128 + m), be - 134);
    return s ? -v : v;
}

/* an input element as a double (exact for every input dtype) */
static inline double load_x(const void *X, int dt, int64_t off)
{
    switch (dt) {
    case OZO_F64: return ((const double *)X)[off];
    case OZO_F32: return (double)((const float *)X)[off];
    case OZO_F16: return ozo_f16_to_f64(((const uint16_t *)X)[off]);
    case OZO_BF16: return ozo_bf16_to_f64(((const uint16_t *)X)[off]);
    default: return (double)((const int8_t *)X)[off];
    }
}

/* ------------------------------------------------------------------------ */
/* Split one operand.
 * X: logical [rows, K] with element strides (stride_r, stride_k), dtype x_dtype
 *    (any input dtype; fp16 / bf16 as bit patterns).
 * slices: [L, rows, K] contiguous, dtype slice_dtype (int8, fp16 / bf16 bits,
 *    or fp32).
 * scales: [L, rows] contiguous fp32.
 * Follows ozaki_triton.py:157-211 for one batch.  Returns 0, or -1 on a bad
 * argument, -2 on allocation failure.                                          */
static void quant_store(void *slices, int slice_dtype, size_t idx, double q, int res64,
                        double *deq)
{
    if (slice_dtype == OZO_I8) {
        double t;
        if (res64) {
            t = (q >= 0) ? q + 0.5 : q - 0.5;
        } else {
            float qf = (float)q;                 /* q is already an fp32 value */
            float tf = (qf >= 0) ? qf + 0.5f : qf - 0.5f;
            t = tf;
        }
        /* tl.clamp(x, -128, 127) then cast to int8 (fptosi: toward zero).
         * A NaN input quantises to 0: the Triton interpreter's np.clip keeps
         * the NaN and its astype(int8) gives 0 on x86-64; what a GPU build of
         * the reference gives is not pinned by any of its tests.            */
        if (t != t) t = 0.0;
        if (t < -128.0) t = -128.0;
        if (t > 127.0) t = 127.0;
        int8_t v = (int8_t)(int)t;
        ((int8_t *)slices)[idx] = v;
        *deq = (double)v;
    } else if (slice_dtype == OZO_F16) {
        uint16_t h = ozo_f64_to_f16(q);          /* q is exact in double for fp32 RES */
        ((uint16_t *)slices)[idx] = h;
        *deq = ozo_f16_to_f64(h);
    } else if (slice_dtype == OZO_BF16) {
        uint16_t h = ozo_f64_to_bf16(q);
        ((uint16_t *)slices)[idx] = h;
        *deq = ozo_bf16_to_f64(h);
    } else {                                     /* OZO_F32 */
        float f = (float)q;                      /* RNE (exact for fp32 RES) */
        ((float *)slices)[idx] = f;
        *deq = (double)f;
    }
}

int ozo_split(const void *X, int x_dtype, int64_t rows, int64_t K, int64_t stride_r,
              int64_t stride_k, int L, int alpha, int slice_dtype, void *slices,
              float *scales)
{
    if (x_dtype < OZO_F64 || x_dtype > OZO_I8 || slice_dtype < OZO_F32 || slice_dtype > OZO_I8 ||
        L < 0 || rows < 0 || K < 0)
        return -1;
    const int res64 = (x_dtype == OZO_F64);
    float *R = (float *)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
    if (!R) return -2;
    for (int64_t r = 0; r < rows; ++r) {
        for (int l = 0; l < L; ++l) {
            /* sweep 0: row max (ozaki_triton.py:172,192) */
            float mu = 1e-38f;
            for (int64_t k = 0; k < K; ++k) {
                float a;
                if (l == 0) {
                    a = (float)fabs(load_x(X, x_dtype, r * stride_r + k * stride_k));
                } else {
                    a = fabsf(R[k]);
                }
                if (a > mu) mu = a;
            }
            float s = ozo_scale_from_max(mu, alpha);
            scales[(size_t)l * rows + r] = s;
            /* sweep 1: quantise, store slice, update residual (:193-211) */
            for (int64_t k = 0; k < K; ++k) {
                size_t idx = ((size_t)l * rows + r) * (size_t)K + k;
                double deq;
                if (res64) {
                    double src = (l == 0) ? load_x(X, x_dtype, r * stride_r + k * stride_k)
                                          : (double)R[k];
                    double q = src / (double)s;
                    quant_store(slices, slice_dtype, idx, q, 1, &deq);
                    if (l < L - 1) {
                        double rr = src - deq * (double)s;
                        R[k] = (float)rr;
                    }
                } else {
                    float src = (l == 0) ? (float)load_x(X, x_dtype, r * stride_r + k * stride_k)
                                         : R[k];
                    float q = src / s;
                    quant_store(slices, slice_dtype, idx, (double)q, 0, &deq);
                    if (l < L - 1) {
                        float prod = (float)deq * s;
                        float rr = src - prod;
                        R[k] = rr;
                    }
                }
            }
        }
    }
    free(R);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Exact int8 dot product.  Partial sums of at most 2^16 products of magnitude
 * <= 2^14 fit int32; the chunks are added in int64.  target_clones lets the
 * same binary use the widest integer SIMD of whatever host runs it.           */
__attribute__((target_clones("arch=skylake-avx512", "avx2", "default")))
int64_t ozo_dot_i8(const int8_t *a, const int8_t *b, int64_t K)
{
    int64_t total = 0;
    for (int64_t k0 = 0; k0 < K; k0 += 65536) {
        int64_t k1 = (k0 + 65536 < K) ? k0 + 65536 : K;
        int32_t s = 0;
        for (int64_t k = k0; k < k1; ++k) s += (int32_t)a[k] * (int32_t)b[k];
        total += s;
    }
    return total;
}

/* ------------------------------------------------------------------------ */
/* The final cast of the fp32 outer accumulator to a non-fp64 output dtype
 * (ozaki_triton.py:452).                                                      */
static void store_out(void *C, int out_dtype, int64_t idx, float out)
{
    switch (out_dtype) {
    case OZO_F32: ((float *)C)[idx] = out; break;
    case OZO_F16: ((uint16_t *)C)[idx] = ozo_f64_to_f16((double)out); break;
    case OZO_BF16: ((uint16_t *)C)[idx] = ozo_f64_to_bf16((double)out); break;
    default: {                                   /* OZO_I8 */
        float t = isnan(out) ? 0.0f : truncf(out);
        if (t < -128.0f) t = -128.0f;
        if (t > 127.0f) t = 127.0f;
        ((int8_t *)C)[idx] = (int8_t)(int)t;
    }
    }
}

/* ------------------------------------------------------------------------ */
/* Cross-GEMM for one batch.
 * As: [L, M, K] contiguous slices, Bs: [L, N, K] contiguous slices (B^T per
 * slice: the physical layout ozaki_matmul produces, ozaki_triton.py:593-595).
 * sa: [L, M] fp32, sb: [L, N] fp32.  C: [M, N] contiguous, dtype out_dtype
 * (any input dtype); the outer accumulator is fp64 for fp64 output else fp32
 * (ozaki_triton.py:69-73,474).
 * int8 slices: acc_ij is the exact integer dot product (int32 never overflows
 * under the alpha rule, ozaki_triton.py:95); returns -3 if it would.
 * fp16 / bf16 / fp32 slices: acc_ij is the binary64 dot product of the exact
 * slice values, i.e. an (almost) exact reference for the fp32 hardware
 * accumulation, which a GPU kernel can only match within a tolerance.         */
int ozo_cross_gemm_pairs(const void *As, const void *Bs, const float *sa, const float *sb,
                         int64_t M, int64_t N, int64_t K, int L, int slice_dtype, void *C,
                         int out_dtype, int pairs, int skip_pair);

int ozo_cross_gemm(const void *As, const void *Bs, const float *sa, const float *sb,
                   int64_t M, int64_t N, int64_t K, int L, int slice_dtype, void *C,
                   int out_dtype)
{
    return ozo_cross_gemm_pairs(As, Bs, sa, sb, M, N, K, L, slice_dtype, C, out_dtype, 0, -1);
}

/* The same with the term of pair i * L + j == skip_pair left out of the outer
 * sum: a deliberately wrong result, which tests use to show that their checks
 * catch a dropped slice pair (skip_pair = -1: the correct result).            */
int ozo_cross_gemm_skip(const void *As, const void *Bs, const float *sa, const float *sb,
                        int64_t M, int64_t N, int64_t K, int L, int slice_dtype, void *C,
                        int out_dtype, int skip_pair)
{
    return ozo_cross_gemm_pairs(As, Bs, sa, sb, M, N, K, L, slice_dtype, C, out_dtype, 0,
                                skip_pair);
}

/* pairs = 0: every pair (i, j), the reference's sum.  pairs = 1: only the
 * pairs with i + j <= L - 1 (not in the reference: the triangular pair set of
 * this library's ozk_cross_gemm_pairs / ozk_matmul_pairs), the same terms in
 * the same i-major / j-minor order with the others left out.                 */
int ozo_cross_gemm_pairs(const void *As, const void *Bs, const float *sa, const float *sb,
                         int64_t M, int64_t N, int64_t K, int L, int slice_dtype, void *C,
                         int out_dtype, int pairs, int skip_pair)
{
    if (pairs != 0 && pairs != 1) return -1;
    if (slice_dtype < OZO_F32 || slice_dtype > OZO_I8 || out_dtype < OZO_F64 ||
        out_dtype > OZO_I8 || L < 0)
        return -1;
    const int out64 = (out_dtype == OZO_F64);
    double *Bf = NULL, *Af = NULL;
    if (slice_dtype != OZO_I8) {
        Af = (double *)malloc(sizeof(double) * (size_t)(L * M * K + 1));
        Bf = (double *)malloc(sizeof(double) * (size_t)(L * N * K + 1));
        if (!Af || !Bf) { free(Af); free(Bf); return -2; }
        for (int64_t t = 0; t < (int64_t)L * M * K; ++t) Af[t] = load_x(As, slice_dtype, t);
        for (int64_t t = 0; t < (int64_t)L * N * K; ++t) Bf[t] = load_x(Bs, slice_dtype, t);
    }
    float *acc = (float *)malloc(sizeof(float) * (size_t)(L * L + 1));
    if (!acc) { free(Af); free(Bf); return -2; }
    int rc = 0;
    for (int64_t m = 0; m < M && rc == 0; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            for (int i = 0; i < L; ++i) {
                for (int j = 0; j < L; ++j) {
                    float accf;
                    if (slice_dtype == OZO_I8) {
                        const int8_t *a = (const int8_t *)As + ((size_t)i * M + m) * K;
                        const int8_t *b = (const int8_t *)Bs + ((size_t)j * N + n) * K;
                        int64_t s = ozo_dot_i8(a, b, K);
                        if (s > INT32_MAX || s < INT32_MIN) { rc = -3; }
                        accf = (float)(int32_t)s;          /* int32 -> fp32, RNE */
                    } else {
                        const double *a = Af + ((size_t)i * M + m) * K;
                        const double *b = Bf + ((size_t)j * N + n) * K;
                        double s = 0.0;
                        for (int64_t k = 0; k < K; ++k) s += a[k] * b[k];
                        accf = (float)s;
                    }
                    acc[i * L + j] = accf;
                }
            }
            if (out64) {
                double out = 0.0;
                for (int i = 0; i < L; ++i) {
                    float si = sa[(size_t)i * M + m];
                    for (int j = 0; j < L; ++j) {
                        if (i * L + j == skip_pair || (pairs == 1 && i + j > L - 1)) continue;
                        float t1 = acc[i * L + j] * si;
                        float t2 = t1 * sb[(size_t)j * N + n];
                        out = out + (double)t2;
                    }
                }
                ((double *)C)[m * N + n] = out;
            } else {
                float out = 0.0f;
                for (int i = 0; i < L; ++i) {
                    float si = sa[(size_t)i * M + m];
                    for (int j = 0; j < L; ++j) {
                        if (i * L + j == skip_pair || (pairs == 1 && i + j > L - 1)) continue;
                        float t1 = acc[i * L + j] * si;
                        float t2 = t1 * sb[(size_t)j * N + n];
                        out = out + t2;
                    }
                }
                store_out(C, out_dtype, m * N + n, out);
            }
        }
    }
    free(acc); free(Af); free(Bf);
    return rc;
}

/* Integer-only helper for the int8 path: acc[i][j][m][n] = A_i[m,:] . B_j[n,:]
 * exactly, returned as int64 (lets a test check the int32 range and compare a
 * GPU int32 accumulator independently of the epilogue).                       */
int ozo_int8_pair_dots(const int8_t *As, const int8_t *Bs, int64_t M, int64_t N, int64_t K,
                       int L, int64_t *out)
{
    for (int i = 0; i < L; ++i)
        for (int j = 0; j < L; ++j)
            for (int64_t m = 0; m < M; ++m)
                for (int64_t n = 0; n < N; ++n) {
                    const int8_t *a = As + ((size_t)i * M + m) * K;
                    const int8_t *b = Bs + ((size_t)j * N + n) * K;
                    out[(((size_t)i * L + j) * M + m) * N + n] = ozo_dot_i8(a, b, K);
                }
    return 0;
}

/* Array form of ozo_f64_to_f16 (lets a test compare many values at once). */
void ozo_f64_to_f16_array(const double *x, uint16_t *out, int64_t n)
{
    for (int64_t t = 0; t < n; ++t) out[t] = ozo_f64_to_f16(x[t]);
}

/* Array form of ozo_ceil_log2_f32. */
void ozo_ceil_log2_f32_array(const float *x, int32_t *out, int64_t n)
{
    for (int64_t t = 0; t < n; ++t) out[t] = ozo_ceil_log2_f32(x[t]);
}

/* Array forms of the bfloat16 conversions. */
void ozo_f64_to_bf16_array(const double *x, uint16_t *out, int64_t n)
{
    for (int64_t t = 0; t < n; ++t) out[t] = ozo_f64_to_bf16(x[t]);
}

void ozo_bf16_to_f64_array(const uint16_t *h, double *out, int64_t n)
{
    for (int64_t t = 0; t < n; ++t) out[t] = ozo_bf16_to_f64(h[t]);
}
