// mfma_power_probe: the MFMA rate of v_mfma_i32_32x32x32_i8 streams as more
// of the cross-GEMM's data movement is added, and the shader clock it runs at.
//
// Measurement tool for the cross-GEMM's roofline (not part of the library).
// Every case runs one workgroup of 8 waves per CU (two waves per SIMD), each
// wave holding 12 accumulator tiles fed by 3 A and 4 B fragments, as the
// num_splits 4 cross-GEMM kernel (cross_gemm_wide4_kernel) does.  Cases:
//   const        constant operands, no memory traffic
//   random_regs  operands changed by one add per dword each iteration
//   lds          operands read from the LDS (random bytes): 7 fragment reads
//                per 12 MFMAs, the kernel's ratio
//   lds_dma      as lds, plus global -> LDS DMA at the kernel's rate (five 1 KB
//                instructions per wave per 24 MFMAs) from a 4 MiB buffer that
//                stays in L2
//   lds_dma_miss as lds_dma with one window in five from a 1 GiB buffer (L2
//                misses: the kernel's L2 fetch is about 19% of its requests)
//   zeros        lds_dma_miss with every operand and buffer byte zero
// Each case prints one JSON line: the MFMA rate as a fraction of the dense
// INT8 peak (5.0 POP/s: 32 cycles per MFMA per SIMD at 2.4 GHz), the shader
// clock (s_memtime cycles over the 100 MHz s_memrealtime counter, averaged
// over the CUs of the last launch) and the issue share at that clock.
//
// Bounds: LDS offsets are masked to the allocated sizes; global reads go
// through buffer resources whose num_records is the buffer size, with offsets
// reduced modulo it; the final stores index grid * block lanes of buffers
// sized to match.  Usage: mfma_power_probe [--quick]
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

#define CHECK(x)                                                                        \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess) {                                                         \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            return 1;                                                                   \
        }                                                                               \
    } while (0)

constexpr int kNA = 3, kNB = 4;        // fragments per wave
constexpr int kThreads = 512;          // 8 waves
constexpr int kOpLds = 64 * 1024;      // operand region of the LDS
constexpr int kDmaLds = 64 * 1024;     // DMA target region
enum Mode { kConst = 0, kRegs = 1, kLds = 2, kLdsDma = 3 };

__device__ __forceinline__ uint32_t mix(uint32_t x) {
    x ^= x >> 16; x *= 0x7feb352du; x ^= x >> 15; x *= 0x846ca68bu; x ^= x >> 16;
    return x;
}

// miss_every: 0 = every DMA window from the small buffer, n = one in n from
// the large one.  zero: all operands zero.
template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void probe(int iters, const int8_t *small_buf,
                                                     uint32_t small_bytes, const int8_t *big_buf,
                                                     uint32_t big_bytes, int miss_every, int zero,
                                                     int *out, unsigned long long *clk) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    unsigned long long t0 = 0, r0 = 0;
    if (tid == 0) {
        t0 = __builtin_amdgcn_s_memtime();
        r0 = __builtin_amdgcn_s_memrealtime();
    }
    for (int o = tid * 16; o < kOpLds; o += kThreads * 16) {
        i32x4 v;
        for (int c = 0; c < 4; ++c) v[c] = zero ? 0 : (int)mix(o * 4 + c + 977 * blockIdx.x);
        *(i32x4 *)(smem + o) = v;
    }
    __syncthreads();
    i32x4 a[kNA], b[kNB];
    for (int u = 0; u < kNA; ++u)
        for (int c = 0; c < 4; ++c)
            a[u][c] = MODE == kConst ? 0x01020304 + u : (zero ? 0 : (int)mix(tid * 64 + u * 4 + c));
    for (int j = 0; j < kNB; ++j)
        for (int c = 0; c < 4; ++c)
            b[j][c] = MODE == kConst ? 0x05060708 + j
                                     : (zero ? 0 : (int)mix(tid * 64 + 32 + j * 4 + c));
    i32x16 acc[kNA][kNB];
    for (int u = 0; u < kNA; ++u)
        for (int j = 0; j < kNB; ++j) acc[u][j] = i32x16{0};

    const __amdgpu_buffer_rsrc_t rs_small =
        __builtin_amdgcn_make_buffer_rsrc((void *)small_buf, (short)0, (int)small_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs_big =
        __builtin_amdgcn_make_buffer_rsrc((void *)big_buf, (short)0, (int)big_bytes, 0x00020000);
    const uint32_t nsmall = small_bytes / 1024, nbig = big_bytes / 1024;   // 1 KB windows
    uint32_t ws = mix(blockIdx.x * 8 + wave) % nsmall, wb = mix(blockIdx.x * 8 + wave + 7) % nbig;
    int dma_count = 0;
    const int smem_base = (int)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
    int rd = (wave * 8192) & (kOpLds - 1);
    for (int it = 0; it < iters; ++it) {
        if (MODE >= kLds) {
#pragma unroll
            for (int u = 0; u < kNA; ++u) {
                const int off = (rd + u * 1024) & (kOpLds - 1);
                a[u] = *(const __attribute__((address_space(3))) i32x4 *)(uintptr_t)(
                    smem_base + off + lane * 16);
            }
#pragma unroll
            for (int j = 0; j < kNB; ++j) {
                const int off = (rd + (kNA + j) * 1024) & (kOpLds - 1);
                b[j] = *(const __attribute__((address_space(3))) i32x4 *)(uintptr_t)(
                    smem_base + off + lane * 16);
            }
            rd = (rd + (kNA + kNB) * 1024 + 4096) & (kOpLds - 1);
        }
        if (MODE == kLdsDma) {
            // 2 or 3 windows per iteration: 5 per 24 MFMAs
            const int nd = 2 + (it & 1);
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                if (d >= nd) break;
                auto *ldsp = (__attribute__((address_space(3))) void *)(
                    smem + kOpLds + (((wave * 3 + d) * 1024) & (kDmaLds - 1)));
                const bool miss = miss_every > 0 && (dma_count % miss_every) == 0;
                if (miss) {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_big, ldsp, 16, wb * 1024u + lane * 16u,
                                                             0, 0, 0);
                    wb += 8 * 256 + 1;
                    if (wb >= nbig) wb -= nbig;
                } else {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_small, ldsp, 16,
                                                             ws * 1024u + lane * 16u, 0, 0, 0);
                    ws += 8 * 256 + 1;
                    if (ws >= nsmall) ws -= nsmall;
                }
                ++dma_count;
            }
        }
#pragma unroll
        for (int j = 0; j < kNB; ++j)
#pragma unroll
            for (int u = 0; u < kNA; ++u)
                acc[u][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[u], b[j], acc[u][j], 0, 0, 0);
        if (MODE == kRegs) {
#pragma unroll
            for (int u = 0; u < kNA; ++u)
                for (int c = 0; c < 4; ++c) a[u][c] = (int)((uint32_t)a[u][c] + 0x9E3779B9u + 2u * u);
#pragma unroll
            for (int j = 0; j < kNB; ++j)
                for (int c = 0; c < 4; ++c) b[j][c] = (int)((uint32_t)b[j][c] + 0x7F4A7C15u + 2u * j);
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): every DMA landed
    int s = 0;
    for (int u = 0; u < kNA; ++u)
        for (int j = 0; j < kNB; ++j)
            for (int r = 0; r < 16; ++r) s += acc[u][j][r];
    out[blockIdx.x * kThreads + tid] = s;
    __syncthreads();
    if (tid == 0) {
        clk[blockIdx.x * 2 + 0] = __builtin_amdgcn_s_memtime() - t0;
        clk[blockIdx.x * 2 + 1] = __builtin_amdgcn_s_memrealtime() - r0;
    }
}

struct Ctx {
    int cus;
    double rtc_hz;
    int8_t *small_buf, *big_buf;
    uint32_t small_bytes, big_bytes;
    int8_t *zero_small, *zero_big;
    int *out;
    unsigned long long *clk;
};

template <int MODE>
int run_case(const char *name, const Ctx &c, int iters, int launches, int warm, int miss_every,
             int zero) {
    const size_t lds = kOpLds + (MODE == kLdsDma ? kDmaLds : 0);
    auto k = probe<MODE>;
    CHECK(hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds));
    const int8_t *sb = zero ? c.zero_small : c.small_buf, *bb = zero ? c.zero_big : c.big_buf;
    // untimed launches first (about 0.1 s): the clock settles to the load
    for (int w = 0; w < warm; ++w)
        hipLaunchKernelGGL(k, dim3(c.cus), dim3(kThreads), lds, 0, iters, sb, c.small_bytes, bb,
                           c.big_bytes, miss_every, zero, c.out, c.clk);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    CHECK(hipEventRecord(e0));
    for (int l = 0; l < launches; ++l)
        hipLaunchKernelGGL(k, dim3(c.cus), dim3(kThreads), lds, 0, iters, sb, c.small_bytes, bb,
                           c.big_bytes, miss_every, zero, c.out, c.clk);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    std::vector<unsigned long long> h((size_t)c.cus * 2);
    CHECK(hipMemcpy(h.data(), c.clk, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
    double cyc = 0, rt = 0;
    for (int i = 0; i < c.cus; ++i) {
        cyc += (double)h[2 * i];
        rt += (double)h[2 * i + 1];
    }
    const double ghz = cyc / (rt / c.rtc_hz) / 1e9;
    // MFMAs per SIMD: 2 waves x 12 per iteration
    const double mfma_per_simd = (double)launches * iters * kNA * kNB * 2.0;
    const double frac = (32.0 / 2.4e9) / (ms * 1e-3 / mfma_per_simd);
    printf("{\"case\": \"%s\", \"ms\": %.3f, \"frac_of_int8_peak\": %.4f, \"clock_GHz\": %.3f, "
           "\"mfma_issue_share\": %.4f}\n",
           name, ms, frac, ghz, frac * 2.4 / ghz);
    fflush(stdout);
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
    return 0;
}

int main(int argc, char **argv) {
    const bool quick = argc > 1 && strcmp(argv[1], "--quick") == 0;
    Ctx c{};
    CHECK(hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, 0));
    int rtc_khz = 0;
    CHECK(hipDeviceGetAttribute(&rtc_khz, hipDeviceAttributeWallClockRate, 0));
    c.rtc_hz = rtc_khz > 0 ? rtc_khz * 1e3 : 1e8;
    c.small_bytes = 4u << 20;
    c.big_bytes = quick ? (256u << 20) : (1u << 30);
    CHECK(hipMalloc(&c.small_buf, c.small_bytes));
    CHECK(hipMalloc(&c.big_buf, c.big_bytes));
    CHECK(hipMalloc(&c.zero_small, c.small_bytes));
    CHECK(hipMalloc(&c.zero_big, c.big_bytes));
    CHECK(hipMemset(c.zero_small, 0, c.small_bytes));
    CHECK(hipMemset(c.zero_big, 0, c.big_bytes));
    {
        std::vector<uint32_t> h(c.big_bytes / 4);
        uint32_t x = 12345;
        for (auto &v : h) {
            x ^= x << 13;
            x ^= x >> 17;
            x ^= x << 5;
            v = x;
        }
        CHECK(hipMemcpy(c.big_buf, h.data(), c.big_bytes, hipMemcpyHostToDevice));
        CHECK(hipMemcpy(c.small_buf, h.data(), c.small_bytes, hipMemcpyHostToDevice));
    }
    CHECK(hipMalloc(&c.out, (size_t)c.cus * kThreads * sizeof(int)));
    CHECK(hipMalloc(&c.clk, (size_t)c.cus * 2 * sizeof(unsigned long long)));
    printf("{\"cus\": %d, \"wall_clock_MHz\": %.1f, \"quick\": %s}\n", c.cus, c.rtc_hz / 1e6,
           quick ? "true" : "false");
    // about 10 ms per launch at the peak rate; 30 launches after 10 (quick: 5
    // of 2 ms after 50)
    const int iters = quick ? 6144 : 32768, launches = quick ? 5 : 30, warm = quick ? 50 : 10;
    int rc = 0;
    rc |= run_case<kConst>("const", c, iters, launches, warm, 0, 0);
    rc |= run_case<kRegs>("random_regs", c, iters, launches, warm, 0, 0);
    rc |= run_case<kLds>("lds", c, iters, launches, warm, 0, 0);
    rc |= run_case<kLdsDma>("lds_dma", c, iters, launches, warm, 0, 0);
    rc |= run_case<kLdsDma>("lds_dma_miss", c, iters, launches, warm, 5, 0);
    rc |= run_case<kLdsDma>("zeros", c, iters, launches, warm, 5, 1);
    CHECK(hipFree(c.small_buf));
    CHECK(hipFree(c.big_buf));
    CHECK(hipFree(c.zero_small));
    CHECK(hipFree(c.zero_big));
    CHECK(hipFree(c.out));
    CHECK(hipFree(c.clk));
    return rc;
}
