// ozk_internal.h -- parameter blocks and launchers shared between the C ABI
// layer (ozk_api.cpp) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ozk {

constexpr int kMaxLevels = 8;   // most slices a split or cross-GEMM takes (OZK_MAX_SPLITS)

// Kernel choices forced by the test hooks of include/ozaki_amd_debug.h.  They
// live in thread-local storage: a setting applies to calls made from the host
// thread that set it, and nothing else (no environment variable is read).
enum ForceGemm { kForceGemmNone = -1 };   // else a GemmKind
enum ForceSplit {
    kForceSplitNone = -1,
    kForceSplitCoop = 0,
    kForceSplitStrip = 1,
    kForceSplitTranspose = 2,
    kForceSplitGeneric = 3,
    kForceSplitRows = 4,
    kForceSplitRowsCoop = 5
};
struct DebugOverrides {
    int gemm = kForceGemmNone;
    int split = kForceSplitNone;
    int coop_timeout = 0;   // 1: every cooperative wait gives up at once (its timeout path)
    int ksplit = 0;         // > 0: split-K ranges of the ring and wide kernels (0: the planner's)
    int coop_resident = 0;  // > 0: workgroups one XCD holds for the cooperative split kernels
                            // (0: the current device's)
};
DebugOverrides &debug_overrides();

// One split launch: X [batch, rows, K] -> slices [batch, L, rows, K] and
// scales [batch, L, rows].  All strides in elements.
struct SplitParams {
    const void *X;
    int64_t batch, rows, K;
    int64_t xs_b, xs_r, xs_k;
    int L, alpha;
    void *slices;
    int64_t ss_b, ss_l, ss_r, ss_k;
    float *scales;
    int64_t cs_b, cs_l, cs_r;
    float *resid;  // workspace: exchange words of the cooperative kernels, the
                   // transposed operand [batch, rows, K] (transpose + row path) or
                   // the fp32 copy of a narrow input
    // null: a cooperative launch is followed by its poison kernel (NaN scales
    // and the device status if a wait gave up).  Else the launcher runs no
    // poison kernel and stores the launch's status word here (left alone if
    // the plan has no cooperative launch): the cross-GEMM that follows on
    // the same stream takes the check over (GemmParams::split_fail).
    const uint32_t **fail_out;
};

enum SplitPath {
    kSplitRows = 0,
    kSplitStrip = 1,
    kSplitGeneric = 2,
    kSplitTransposeRows = 3,
    kSplitConvert = 4,  // narrow input: exact fp32 copy in the workspace, then the fp32 plan
    kSplitCoop = 5      // column strips of 128-byte row segments cut along K, the level
                        // maxima combined through the workspace
};

// Chooses the split kernel for p (x_dtype: 0 = f64, 1 = f32, 2 = f16,
// 3 = bf16, 4 = i8; slice: 1 = f32, 2 = f16, 3 = bf16, 4 = i8).  Returns the path and, for the resident paths, the variant index.
struct SplitPlan {
    SplitPath path;
    int variant;
};
// The plan depends on the pointers X and slices only through alignment.  The
// workspace queries see no pointers and size for 256-byte aligned ones; a plan
// for other pointers never needs more scratch than that (it falls back to the
// generic kernel, which needs none).
SplitPlan plan_split(const SplitParams &p, int x_dtype, int slice_dtype);
// scratch the plan needs: the exchange words of the cooperative kernels and
// their status word, the transposed operand (transpose + row path), the fp32
// copy of a narrow input (none for the row, strip and generic kernels)
size_t split_workspace_bytes(const SplitParams &p, const SplitPlan &plan, int x_dtype,
                             int slice_dtype);
hipError_t launch_split(const SplitParams &p, const SplitPlan &plan, int x_dtype,
                        int slice_dtype, hipStream_t stream);
// Workgroups one XCD of the current device holds for the cooperative split
// kernels (the debug override, if set); a cooperative group has at most this
// many members minus 8
int coop_resident_per_xcd();
// Both splits of a matmul in one launch (split_pair_kernel): A's rows by a
// 4-wave row configuration and B's columns by the cooperative kernel, fp64
// input, no split kernel forced by the test hooks.  pb.resid holds B's
// exchange words (A needs no scratch).
bool split_pair_ok(const SplitPlan &plan_a, const SplitPlan &plan_b, int x_dtype);
hipError_t launch_split_pair(const SplitParams &pa, const SplitPlan &plan_a, const SplitParams &pb,
                             const SplitPlan &plan_b, int x_dtype, int slice_dtype,
                             hipStream_t stream);
// both splits in one launch where B takes the 256-lane strip kernel and A a
// 256-lane row configuration
bool split_duo_ok(const SplitPlan &plan_a, const SplitPlan &plan_b, int x_dtype);
hipError_t launch_split_duo(const SplitParams &pa, const SplitPlan &plan_a, const SplitParams &pb,
                            const SplitPlan &plan_b, int x_dtype, int slice_dtype, hipStream_t st);

// Sticky device status (per device): bit 0 is set when a cooperative split
// wait gave up (the split's scales are then NaN).  read_device_status waits
// for `stream`, reads the word of the current device and clears it if asked.
hipError_t read_device_status(unsigned *out, bool clear, hipStream_t stream);
// Device address of the current device's sticky status word (asked once per
// device), for kernels that record a failure themselves; null on error.
uint32_t *device_status_word();

// One cross-GEMM launch.  A slices [batch, L, M, K] and B slices presented as
// [batch, L, N, K] (K-contiguous rows of B^T).  Strides in elements of the
// slice dtype; scales and C strides in their own elements.
struct GemmParams {
    const void *A;
    const void *B;
    int64_t as_b, as_l, as_m;   // A: k stride is 1
    int64_t bs_b, bs_l, bs_n;   // B^T: k stride is 1
    const float *sa;
    const float *sb;
    int64_t sas_b, sas_l, sas_m;
    int64_t sbs_b, sbs_l, sbs_n;
    void *C;
    int64_t cs_b, cs_m, cs_n;
    int64_t batch, M, N, K;
    int out_dtype;              // C's dtype code: 0 f64 (fp64 outer accumulator), else
                                // f32 / f16 / bf16 / i8 (fp32 outer accumulator)
    int tri;                    // 1: sum only the pairs i + j <= L - 1 (OZK_PAIRS_TRIANGULAR)
    // split-K (ring and wide kernels): a tile's 128-byte K stages are cut into
    // ksplit ranges of kb_per_split stages, one workgroup each; ksplit <= 1:
    // none.  kpart holds the ranges' raw accumulators, kcount one arrival
    // counter per tile (zero at launch).
    int ksplit;
    int kb_per_split;
    uint32_t *kpart;
    uint32_t *kcount;
    // Status words of the cooperative splits that ran before this launch on
    // the same stream in place of their poison kernels (SplitParams::fail_out),
    // or null.  Non-zero in either: every C entry is stored as NaN (0 in an
    // int8 C) and workgroup 0 sets bit 0 of *dev_status, the device's sticky
    // status.
    const uint32_t *split_fail[2];
    uint32_t *dev_status;
    int failed;   // set on the device from the split_fail words at kernel entry
};

enum GemmKind {
    kGemmStaged = 0,  // global -> VGPR -> LDS, 2 x 2 waves (any operand extent)
    kGemmDMA = 1,     // LDS-DMA ring for A and B, 2 x 2 waves
                      // (2: unused)
    kGemmPair = 3,    // LDS-DMA ring, 8 waves: 2 x 2 blocks x 2 halves of the slice pairs
    kGemmRing = 4,    // the pair split over a five-slot ring of half stages, DMA spread
                      // between the MFMAs (num_splits 3 and 4)
    kGemmWide = 5,    // num_splits 3: 64 x 128 tiles, 8 waves each holding all 9 pairs
                      // of a 32 x 32 block, two whole stages in the LDS
    kGemmWide4 = 6,   // num_splits 4: 96 x 64 tiles, 8 waves of 12 accumulator tiles
                      // (3 A x 4 B fragments), two whole stages in the LDS
    kGemmSolo = 7,    // num_splits 5 (and 4 on the triangle): 64 x 64 tiles, 4 waves (one
                      // per SIMD) each holding every pair of a 32 x 32 block, two whole
                      // stages in the LDS
    kGemmKStep = 8,   // num_splits 1-4 on small grids: 32 x 32 tiles, 4 waves, wave w takes
                      // K step w of every stage and all pairs; summed through the LDS
    kGemmKStep2 = 9   // the same with 8 waves: two pair groups, two waves per SIMD (L = 2..4)
};
struct GemmPlan {
    int mi, ni;       // 2 x 2 kernels: wave tile = (32*mi) x (32*ni)
    int group_m;      // tile-row group for L2 reuse
    int kind;         // GemmKind; the LDS-DMA kernels need 31-bit operand extents
    int ksplit;       // split-K ranges per tile (1: none)
    int kb_per_split; // 128-byte K stages per range
};
// cus: compute units of the device (0: ask the current device, once per device)
GemmPlan plan_gemm(const GemmParams &p, int L, int slice_dtype, int cus = 0);
// Workspace of a split-K plan: the ranges' accumulators and the tile counters
// (0 without split-K), and where they go in it (256-byte aligned offsets).
size_t splitk_bytes(const GemmParams &p, const GemmPlan &plan, int L);
// Points p at the split-K buffers in ws and clears the counters (a fill
// kernel, no memset: the call may be captured in a graph).
hipError_t setup_splitk(GemmParams &p, const GemmPlan &plan, int L, void *ws, hipStream_t stream);
hipError_t launch_gemm(const GemmParams &p, const GemmPlan &plan, int L, int slice_dtype,
                       hipStream_t stream);
// the same for one slice dtype (one translation unit each)
hipError_t launch_gemm_i8(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t stream);
hipError_t launch_gemm_f16(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t stream);
hipError_t launch_gemm_bf16(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t stream);
hipError_t launch_gemm_f32(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t stream);

hipError_t launch_zero_c(const GemmParams &p, hipStream_t stream);

// Packs slices [batch, L, rows, K] (any strides) into a K-contiguous buffer
// [batch, L, rows, Kp] with Kp = K rounded up to 16 bytes and zero padding.
struct PackParams {
    const void *src;
    int64_t s_b, s_l, s_r, s_k;
    void *dst;
    int64_t batch, L, rows, K, Kp;
    int esize;
};
hipError_t launch_pack(const PackParams &p, hipStream_t stream);

}  // namespace ozk
