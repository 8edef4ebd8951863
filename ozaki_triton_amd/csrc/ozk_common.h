// ozk_common.h -- device arithmetic shared by the split and cross-GEMM kernels.
//
// Every helper reproduces one rounding step of the reference exactly (IEEE
// binary32/binary64, round-to-nearest-even, denormals kept).  The library is
// compiled with -ffp-contract=off so that no multiply-add pair is fused where
// the reference rounds the product.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define OZK_DEV __device__ __forceinline__

namespace ozk {

// ---------------------------------------------------------------------------
// Exponent rule of ozaki_triton.py:174: E = ceil(log2(mu)) where log2 is the
// correctly rounded float32 log2 (the value numpy's float32 log2 returns).
// For normal mu = 2^k (1 + j 2^-23) the result is k when j == 0 or j <= J(k),
// else k + 1.  J(k) = floor(2^(p-1) ln 2): p = floor(log2 k) for k >= 4,
// p = ceil(log2 |k|) - 1 for k <= -5, J = 0 for -4 <= k <= 3; byte p of
// kBandJ holds J for that p (p = 2..6 -> 1, 2, 5, 11, 22).  mu is never below
// 1e-38f (ozaki_triton.py:172), so a subnormal mu lies in [1e-38f, 2^-126) and
// its ceiling is -126.
// ---------------------------------------------------------------------------
constexpr uint64_t kBandJ = 0x00160B0502010000ull;

OZK_DEV int ceil_log2_f32(float mu) {
    uint32_t u = __float_as_uint(mu);
    int be = (int)((u >> 23) & 0xFFu);
    uint32_t j = u & 0x7FFFFFu;
    if (be == 0) return -126;
    int k = be - 127;
    int p = -1;
    if (k >= 4) p = 31 - __clz(k);                 // floor(log2 k)
    else if (k <= -5) p = 31 - __clz(-k - 1);       // ceil(log2 |k|) - 1
    int J = (p >= 0) ? (int)((kBandJ >> (8 * p)) & 0xFFu) : 0;
    return (j == 0u || (int)j <= J) ? k : k + 1;
}

// exact 2^e as float, e in [-149, 127]
OZK_DEV float pow2f(int e) {
    return (e >= -126) ? __uint_as_float((uint32_t)(e + 127) << 23)
                       : __uint_as_float(1u << (e + 149));
}

// exact 2^e as double, e in [-1022, 1023]
OZK_DEV double pow2d(int e) {
    return __longlong_as_double((long long)(e + 1023) << 52);
}

// Single round-to-nearest-even conversion of a binary64 value to binary16 (bit
// pattern), written with integer arithmetic: one rounding from fp64, which a
// conversion through fp32 would not give.
OZK_DEV uint32_t f64_to_f16_bits(double x) {
    uint64_t u = (uint64_t)__double_as_longlong(x);
    uint32_t s = (uint32_t)((u >> 48) & 0x8000u);
    int be = (int)((u >> 52) & 0x7FF);
    uint64_t m = u & 0xFFFFFFFFFFFFFull;
    if (be == 0x7FF) return s | (m ? 0x7E00u : 0x7C00u);
    if (be == 0) return s;
    uint64_t sig = (1ull << 52) | m;
    int e = be - 1023;
    int qe = (e < -14 ? -14 : e) - 10;
    int shift = qe - (e - 52);
    if (shift > 63) return s;
    uint64_t n = sig >> shift;
    uint64_t rem = sig & ((1ull << shift) - 1ull);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (n & 1ull))) ++n;
    uint32_t b = (e <= -14) ? (uint32_t)n : (uint32_t)(((e + 14) << 10) + (int)n);
    if (b >= 0x7C00u) b = 0x7C00u;
    return s | b;
}
// Single round-to-nearest-even conversion of a binary64 value to bfloat16 (bit
// pattern).  bfloat16 has binary32's exponent range and 8 significant bits:
// quantum 2^(e-7) for a normal value, 2^-133 below 2^-126.
OZK_DEV uint32_t f64_to_bf16_bits(double x) {
    uint64_t u = (uint64_t)__double_as_longlong(x);
    uint32_t s = (uint32_t)((u >> 48) & 0x8000u);
    int be = (int)((u >> 52) & 0x7FF);
    uint64_t m = u & 0xFFFFFFFFFFFFFull;
    if (be == 0x7FF) return s | (m ? 0x7FC0u : 0x7F80u);
    if (be == 0) return s;
    uint64_t sig = (1ull << 52) | m;
    int e = be - 1023;
    int qe = (e < -126 ? -126 : e) - 7;
    int shift = qe - (e - 52);          // >= 45
    if (shift > 63) return s;
    uint64_t n = sig >> shift;
    uint64_t rem = sig & ((1ull << shift) - 1ull);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (n & 1ull))) ++n;
    uint32_t b = (e <= -126) ? (uint32_t)n : (uint32_t)(((e + 126) << 7) + (int)n);
    if (b >= 0x7F80u) b = 0x7F80u;
    return s | b;
}
// Round-to-nearest-even binary32 -> bfloat16 bits for finite x: add half an
// ulp of the kept part (minus one on even) and drop the low 16 bits; a carry
// out of the mantissa steps the exponent, up to infinity.
OZK_DEV uint32_t f32_to_bf16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
OZK_DEV float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// exact binary16 -> binary32 (every binary16 value is a binary32 value)
OZK_DEV float f16_bits_to_f32(uint32_t h) {
    uint32_t s = (h & 0x8000u) << 16;
    uint32_t be = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (be == 0x1F) return __uint_as_float(s | 0x7F800000u | (m << 13));
    if (be == 0) {
        // subnormal: m * 2^-24, exact in binary32
        float v = (float)m * 5.9604644775390625e-08f;
        return s ? -v : v;
    }
    return __uint_as_float(s | ((be + 112u) << 23) | (m << 13));
}

}  // namespace ozk
