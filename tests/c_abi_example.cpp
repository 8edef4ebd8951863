// c_abi_example.cpp -- a plain C++ caller of libozaki_amd.so (no Python, no
// torch): one FP64 -> INT8 Ozaki product with 4 slices of A[96, 1000] and
// B[1000, 80], taken
//   (1) in one call, ozk_matmul, on one caller workspace, and
//   (2) as the reference's three launches: ozk_split of A's rows, ozk_split of
//       B's columns through the B^T view, ozk_cross_gemm on the slices.
// The two results must agree bit for bit (int8 slice products are exact), and
// match a CPU fp64 matmul to the Ozaki scheme's accuracy at 4 slices.
// K = 1000 bytes per int8 slice row is not a whole number of 16-byte pieces,
// so the cross-GEMM goes through its packed copy.  Built by build() in
// __graft_entry__.py; run by tests/test_gpu_parity.py.  Exit status 0 = pass.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../include/ozaki_amd.h"

#define CHECK_HIP(x)                                                                       \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                   \
            return 2;                                                                      \
        }                                                                                  \
    } while (0)
#define CHECK_OZK(x)                                                                       \
    do {                                                                                   \
        int s_ = (x);                                                                      \
        if (s_ != OZK_OK) {                                                                \
            std::fprintf(stderr, "%s: %s\n", #x, ozk_strerror(s_));                        \
            return 3;                                                                      \
        }                                                                                  \
    } while (0)

int main() {
    const int64_t M = 96, N = 80, K = 1000;
    const int L = 4;
    std::vector<double> A(M * K), B(K * N), C1(M * N), C2(M * N);
    uint64_t state = 0x9e3779b97f4a7c15ull;
    auto uniform = [&]() {   // 64-bit LCG, 53-bit uniform in [-1, 1)
        state = state * 6364136223846793005ull + 1442695040888963407ull;
        return (double)(state >> 11) * (1.0 / 9007199254740992.0) * 2.0 - 1.0;
    };
    for (int64_t m = 0; m < M; ++m) {
        const double e = std::ldexp(1.0, (int)(m % 17) - 8);   // per-row exponents
        for (int64_t k = 0; k < K; ++k) A[m * K + k] = uniform() * e;
    }
    for (auto &x : B) x = uniform();

    int alpha = 0;
    CHECK_OZK(ozk_compute_split_bits(K, OZK_I8, OZK_I32, &alpha));
    double *dA, *dB, *dC1, *dC2;
    CHECK_HIP(hipMalloc(&dA, A.size() * 8));
    CHECK_HIP(hipMalloc(&dB, B.size() * 8));
    CHECK_HIP(hipMalloc(&dC1, C1.size() * 8));
    CHECK_HIP(hipMalloc(&dC2, C2.size() * 8));
    CHECK_HIP(hipMemcpy(dA, A.data(), A.size() * 8, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(dB, B.data(), B.size() * 8, hipMemcpyHostToDevice));
    hipStream_t st;
    CHECK_HIP(hipStreamCreate(&st));

    // (1) one call
    const int64_t a_st[3] = {M * K, K, 1}, b_st[3] = {K * N, N, 1}, c_st[3] = {M * N, N, 1};
    size_t ws_bytes = 0;
    CHECK_OZK(ozk_matmul_workspace_bytes(OZK_F64, 1, M, N, K, a_st, b_st, L, OZK_I8, &ws_bytes));
    void *dWs = nullptr;
    CHECK_HIP(hipMalloc(&dWs, ws_bytes));
    CHECK_OZK(ozk_matmul(dA, a_st, dB, b_st, OZK_F64, 1, M, N, K, L, OZK_I8, dC1, c_st, dWs,
                         ws_bytes, nullptr, st));

    // (2) split A, split B^T, cross-GEMM
    const int64_t bt_st[3] = {K * N, 1, N};
    const int64_t as_st[4] = {L * M * K, M * K, K, 1}, bs_st[4] = {L * N * K, N * K, K, 1};
    const int64_t sa_st[3] = {L * M, M, 1}, sb_st[3] = {L * N, N, 1};
    int8_t *dAs, *dBs;
    float *dsa, *dsb;
    CHECK_HIP(hipMalloc(&dAs, L * M * K));
    CHECK_HIP(hipMalloc(&dBs, L * N * K));
    CHECK_HIP(hipMalloc(&dsa, L * M * 4));
    CHECK_HIP(hipMalloc(&dsb, L * N * 4));
    size_t wa = 0, wb = 0, wg = 0;
    CHECK_OZK(ozk_split_workspace_bytes(OZK_F64, 1, M, K, a_st, L, OZK_I8, as_st, &wa));
    CHECK_OZK(ozk_split_workspace_bytes(OZK_F64, 1, N, K, bt_st, L, OZK_I8, bs_st, &wb));
    const int64_t b_view[4] = {L * N * K, N * K, 1, K};   // [L, K, N] view of the [L, N, K] slices
    CHECK_OZK(ozk_cross_gemm_workspace_bytes(1, M, N, K, L, OZK_I8, dAs, as_st, dBs, b_view, &wg));
    size_t wmax = wa > wb ? wa : wb;
    wmax = wmax > wg ? wmax : wg;
    void *dW2 = nullptr;
    if (wmax) CHECK_HIP(hipMalloc(&dW2, wmax));
    CHECK_OZK(ozk_split(dA, OZK_F64, 1, M, K, a_st, L, alpha, OZK_I8, dAs, as_st, dsa, sa_st,
                        wa ? dW2 : nullptr, wa, st));
    CHECK_OZK(ozk_split(dB, OZK_F64, 1, N, K, bt_st, L, alpha, OZK_I8, dBs, bs_st, dsb, sb_st,
                        wb ? dW2 : nullptr, wb, st));
    CHECK_OZK(ozk_cross_gemm(dAs, as_st, dBs, b_view, dsa, sa_st, dsb, sb_st, 1, M, N, K, L,
                             OZK_I8, dC2, OZK_F64, c_st, wg ? dW2 : nullptr, wg, st));
    CHECK_HIP(hipStreamSynchronize(st));
    CHECK_HIP(hipMemcpy(C1.data(), dC1, C1.size() * 8, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(C2.data(), dC2, C2.size() * 8, hipMemcpyDeviceToHost));

    if (std::memcmp(C1.data(), C2.data(), C1.size() * 8) != 0) {
        std::fprintf(stderr, "ozk_matmul and split + cross_gemm differ\n");
        return 4;
    }
    double num = 0.0, den = 0.0;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            double ref = 0.0;
            for (int64_t k = 0; k < K; ++k) ref += A[m * K + k] * B[k * N + n];
            const double d = C1[m * N + n] - ref;
            num += d * d;
            den += ref * ref;
        }
    const double rel = std::sqrt(num / den);
    if (!(rel < 1e-8)) {
        std::fprintf(stderr, "rel err %.3e too large\n", rel);
        return 5;
    }
    std::printf("c_abi_example ok: alpha %d, workspace %zu bytes, rel err vs fp64 %.3e\n", alpha,
                ws_bytes, rel);
    void *bufs[] = {dA, dB, dC1, dC2, dWs, dAs, dBs, dsa, dsb, dW2};
    for (void *b : bufs)
        if (b) CHECK_HIP(hipFree(b));
    CHECK_HIP(hipStreamDestroy(st));
    return 0;
}
