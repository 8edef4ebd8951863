// ozk_api.cpp -- the extern "C" boundary of libozaki_amd.so (include/ozaki_amd.h).
//
// Host-side only: argument validation, path planning and the launches.  No
// device memory is allocated here; scratch comes from the caller's workspace.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <string.h>

#include <atomic>

#include "../../include/ozaki_amd.h"
#include "../../include/ozaki_amd_debug.h"
#include "ozk_internal.h"

namespace ozk {
DebugOverrides &debug_overrides() {
    static thread_local DebugOverrides d;
    return d;
}
}  // namespace ozk

namespace {

// the reference's _INPUT_DTYPES and _SLICE_DTYPE_INFO (ozaki_triton.py:35-48)
bool is_input_dtype(int d) {
    return d == OZK_F64 || d == OZK_F32 || d == OZK_F16 || d == OZK_BF16 || d == OZK_I8;
}
bool is_slice_dtype(int d) { return d == OZK_F32 || d == OZK_F16 || d == OZK_BF16 || d == OZK_I8; }
int slice_size(int d) { return d == OZK_I8 ? 1 : d == OZK_F32 ? 4 : 2; }
int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

int hip_status(hipError_t e) { return e == hipSuccess ? OZK_OK : OZK_ERR_LAUNCH; }

// A known pair set; the triangular one for at most 5 slices (no kernel sums
// it over more: with the reference's fp32 residual buffer a sixth slice adds
// no accuracy).
bool pair_set_ok(int pairs, int L) {
    if (pairs == OZK_PAIRS_ALL) return true;
    return pairs == OZK_PAIRS_TRIANGULAR && L <= 5;
}

// Split-K buffers (plus 256 bytes of alignment slack) of the cross-GEMM of
// K-contiguous slice operands with these strides, 0 when the plan has no
// split-K; the larger of the two pair sets' plans, so that the workspace
// queries need no pair set.  Planned for 256 CUs: a device with fewer plans
// no more ranges.
size_t splitk_need(int64_t batch, int64_t M, int64_t N, int64_t K, int L, int sd,
                   int64_t as_l, int64_t as_m, int64_t bs_l, int64_t bs_n, int out_dtype) {
    if (L < 1 || L > 4 || batch * M * N == 0) return 0;
    ozk::GemmParams gp{};
    gp.as_l = as_l;
    gp.as_m = as_m;
    gp.bs_l = bs_l;
    gp.bs_n = bs_n;
    gp.batch = batch;
    gp.M = M;
    gp.N = N;
    gp.K = K;
    gp.out_dtype = out_dtype;
    size_t b = 0;
    for (int tri = 0; tri <= (L >= 2 ? 1 : 0); ++tri) {
        gp.tri = tri;
        const size_t bt = ozk::splitk_bytes(gp, ozk::plan_gemm(gp, L, sd, 256), L);
        if (bt > b) b = bt;
    }
    return b ? b + 256 : 0;
}

ozk::SplitParams make_split_params(const void *X, int64_t batch, int64_t rows, int64_t K,
                                   const int64_t xs[3], int L, int alpha, void *slices,
                                   const int64_t ss[4], float *scales, const int64_t cs[3]) {
    ozk::SplitParams p;
    p.X = X;
    p.batch = batch;
    p.rows = rows;
    p.K = K;
    p.xs_b = xs[0];
    p.xs_r = xs[1];
    p.xs_k = xs[2];
    p.L = L;
    p.alpha = alpha;
    p.slices = slices;
    p.ss_b = ss[0];
    p.ss_l = ss[1];
    p.ss_r = ss[2];
    p.ss_k = ss[3];
    p.scales = scales;
    p.cs_b = cs[0];
    p.cs_l = cs[1];
    p.cs_r = cs[2];
    p.resid = nullptr;
    p.fail_out = nullptr;
    return p;
}

// Bytes of the packed copy of one slice operand, or 0 when it is already in
// the layout the MFMA kernel reads: K-contiguous, 16-byte aligned rows/planes.
int64_t pack_bytes(const void *ptr, const int64_t s[4], int64_t batch, int L, int64_t rows,
                   int64_t K, int es, bool is_b) {
    // a_strides = (b, l, m, k); b_strides = (b, l, k, n)
    const int64_t sk = is_b ? s[2] : s[3];
    const int64_t sr = is_b ? s[3] : s[2];
    const bool ok = sk == 1 && ((uintptr_t)ptr % 16) == 0 && (sr * es) % 16 == 0 &&
                    (s[1] * es) % 16 == 0 && (s[0] * es) % 16 == 0 && (K * es) % 16 == 0;
    if (ok || rows == 0 || K == 0 || L == 0) return 0;
    const int64_t kp = round_up(K * es, 16) / es;
    return round_up(batch * L * rows * kp * es, 256);
}

}  // namespace

extern "C" {

const char *ozk_strerror(int status) {
    switch (status) {
    case OZK_OK: return "ok";
    case OZK_ERR_NULL: return "required pointer is NULL";
    case OZK_ERR_DTYPE: return "unsupported dtype combination";
    case OZK_ERR_SPLITS: return "num_splits out of range";
    case OZK_ERR_SHAPE: return "invalid shape";
    case OZK_ERR_ALPHA: return "alpha < 1: K too large to split safely";
    case OZK_ERR_WORKSPACE: return "workspace missing, too small or not 16-byte aligned";
    case OZK_ERR_LAUNCH: return "HIP launch failed";
    case OZK_ERR_ACCUM: return "unsupported dot accumulator dtype";
    case OZK_ERR_DEVICE_WAIT:
        return "a cooperative split wait gave up on the device (its scales and C are NaN)";
    case OZK_ERR_TOO_LARGE: return "the call needs more scratch than OZK_STATIC_SCRATCH_BYTES";
    default: return "unknown status";
    }
}

int ozk_version(void) { return 300; }   // 0.3.0: the *_pairs calls

int ozk_device_status(int clear, int *status_out, void *stream) {
    if (!status_out) return OZK_ERR_NULL;
    unsigned v = 0;
    if (ozk::read_device_status(&v, clear != 0, (hipStream_t)stream) != hipSuccess)
        return OZK_ERR_LAUNCH;
    *status_out = v ? OZK_ERR_DEVICE_WAIT : OZK_OK;
    return OZK_OK;
}

int ozk_compute_split_bits(int64_t n, int slice_dtype, int dot_accum_dtype, int *alpha_out) {
    if (!alpha_out) return OZK_ERR_NULL;
    int acc_bits;
    if (dot_accum_dtype == OZK_I32) acc_bits = 31;
    else if (dot_accum_dtype == OZK_F32) acc_bits = 23;
    else return OZK_ERR_ACCUM;
    int slice_bits;
    switch (slice_dtype) {
    case OZK_F32: slice_bits = 23; break;
    case OZK_F16: slice_bits = 10; break;
    case OZK_BF16: slice_bits = 7; break;
    case OZK_I8: slice_bits = 7; break;
    default: return OZK_ERR_DTYPE;
    }
    if (n <= 0) return OZK_ERR_SHAPE;   // log2(0) raises in the reference
    const double a = ((double)acc_bits - log2((double)n)) / 2.0;
    int alpha = (int)a;                 // int(): truncation toward zero
    if (alpha > slice_bits) alpha = slice_bits;
    *alpha_out = alpha;
    return alpha >= 1 ? OZK_OK : OZK_ERR_ALPHA;
}

int ozk_split_workspace_bytes(int x_dtype, int64_t batch, int64_t rows, int64_t K,
                              const int64_t x_strides[3], int num_splits, int slice_dtype,
                              const int64_t slice_strides[4], size_t *bytes_out) {
    if (!bytes_out || !x_strides || !slice_strides) return OZK_ERR_NULL;
    if (!is_input_dtype(x_dtype) || !is_slice_dtype(slice_dtype)) return OZK_ERR_DTYPE;
    if (num_splits < 0 || num_splits > OZK_MAX_SPLITS) return OZK_ERR_SPLITS;
    if (batch < 0 || rows < 0 || K < 0) return OZK_ERR_SHAPE;
    *bytes_out = 0;
    if (num_splits == 0) return OZK_OK;
    // the plan depends on pointer alignment only through 16-byte checks; a
    // 256-byte aligned stand-in pointer gives the plan of any aligned tensor
    ozk::SplitParams p = make_split_params((const void *)256, batch, rows, K, x_strides,
                                           num_splits, 1, (void *)256, slice_strides, nullptr,
                                           x_strides);
    const ozk::SplitPlan plan = ozk::plan_split(p, x_dtype, slice_dtype);
    *bytes_out = ozk::split_workspace_bytes(p, plan, x_dtype, slice_dtype);
    return OZK_OK;
}

int ozk_split(const void *X, int x_dtype, int64_t batch, int64_t rows, int64_t K,
              const int64_t x_strides[3], int num_splits, int alpha, int slice_dtype,
              void *slices, const int64_t slice_strides[4], float *scales,
              const int64_t scale_strides[3], void *workspace, size_t workspace_bytes,
              void *stream) {
    if (!x_strides || !slice_strides || !scale_strides) return OZK_ERR_NULL;
    if (!is_input_dtype(x_dtype) || !is_slice_dtype(slice_dtype)) return OZK_ERR_DTYPE;
    if (num_splits < 0 || num_splits > OZK_MAX_SPLITS) return OZK_ERR_SPLITS;
    if (batch < 0 || rows < 0 || K < 0) return OZK_ERR_SHAPE;
    if (num_splits > 0 && alpha < 1) return OZK_ERR_ALPHA;
    if (batch * rows == 0 || num_splits == 0) return OZK_OK;
    if (!X || !slices || !scales) return OZK_ERR_NULL;
    ozk::SplitParams p = make_split_params(X, batch, rows, K, x_strides, num_splits, alpha,
                                           slices, slice_strides, scales, scale_strides);
    const ozk::SplitPlan plan = ozk::plan_split(p, x_dtype, slice_dtype);
    const size_t need = ozk::split_workspace_bytes(p, plan, x_dtype, slice_dtype);
    if (need > 0) {
        if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16 != 0)
            return OZK_ERR_WORKSPACE;
        p.resid = (float *)workspace;
    }
    return hip_status(ozk::launch_split(p, plan, x_dtype, slice_dtype, (hipStream_t)stream));
}

int ozk_cross_gemm_workspace_bytes(int64_t batch, int64_t M, int64_t N, int64_t K,
                                   int num_splits, int slice_dtype, const void *A_slices,
                                   const int64_t a_strides[4], const void *B_slices,
                                   const int64_t b_strides[4], size_t *bytes_out) {
    if (!bytes_out || !a_strides || !b_strides) return OZK_ERR_NULL;
    if (!is_slice_dtype(slice_dtype)) return OZK_ERR_DTYPE;
    if (num_splits < 0 || num_splits > OZK_MAX_SPLITS) return OZK_ERR_SPLITS;
    if (batch < 0 || M < 0 || N < 0 || K < 0) return OZK_ERR_SHAPE;
    const int es = slice_size(slice_dtype);
    const int64_t a = pack_bytes(A_slices, a_strides, batch, num_splits, M, K, es, false);
    const int64_t b = pack_bytes(B_slices, b_strides, batch, num_splits, N, K, es, true);
    // and, for grids too small to fill the chip, the split-K buffers (the
    // call runs without split-K when the workspace lacks them)
    const int64_t kp = round_up(K * es, 16) / es;
    const size_t sk = splitk_need(batch, M, N, K, num_splits, slice_dtype,
                                  a ? M * kp : a_strides[1], a ? kp : a_strides[2],
                                  b ? N * kp : b_strides[1], b ? kp : b_strides[3], OZK_F64);
    *bytes_out = (size_t)(a + b) + sk;
    return OZK_OK;
}

static int cross_gemm_impl(const void *A_slices, const int64_t a_strides[4], const void *B_slices,
                   const int64_t b_strides[4], const float *A_scales,
                   const int64_t sa_strides[3], const float *B_scales,
                   const int64_t sb_strides[3], int64_t batch, int64_t M, int64_t N, int64_t K,
                   int num_splits, int slice_dtype, int pairs, void *C, int out_dtype,
                   const int64_t c_strides[3], void *workspace, size_t workspace_bytes,
                   void *stream, const uint32_t *const split_fail[2] = nullptr) {
    if (!a_strides || !b_strides || !sa_strides || !sb_strides || !c_strides)
        return OZK_ERR_NULL;
    if (!is_slice_dtype(slice_dtype) || !is_input_dtype(out_dtype)) return OZK_ERR_DTYPE;
    if (num_splits < 0 || num_splits > OZK_MAX_SPLITS || !pair_set_ok(pairs, num_splits))
        return OZK_ERR_SPLITS;
    if (batch < 0 || M < 0 || N < 0 || K < 0) return OZK_ERR_SHAPE;
    if (batch * M * N == 0) return OZK_OK;
    if (!C) return OZK_ERR_NULL;
    hipStream_t st = (hipStream_t)stream;

    ozk::GemmParams p{};
    p.sa = A_scales;
    p.sb = B_scales;
    p.sas_b = sa_strides[0];
    p.sas_l = sa_strides[1];
    p.sas_m = sa_strides[2];
    p.sbs_b = sb_strides[0];
    p.sbs_l = sb_strides[1];
    p.sbs_n = sb_strides[2];
    p.C = C;
    p.cs_b = c_strides[0];
    p.cs_m = c_strides[1];
    p.cs_n = c_strides[2];
    p.batch = batch;
    p.M = M;
    p.N = N;
    p.K = K;
    p.out_dtype = out_dtype;
    // one slice is one pair in either set
    p.tri = pairs == OZK_PAIRS_TRIANGULAR && num_splits >= 2;
    p.split_fail[0] = split_fail ? split_fail[0] : nullptr;
    p.split_fail[1] = split_fail ? split_fail[1] : nullptr;
    p.dev_status = nullptr;
    p.failed = 0;
    if ((p.split_fail[0] || p.split_fail[1]) && !(p.dev_status = ozk::device_status_word()))
        return OZK_ERR_LAUNCH;
    if (num_splits == 0) return hip_status(ozk::launch_zero_c(p, st));
    if (!A_slices || !B_slices || !A_scales || !B_scales) return OZK_ERR_NULL;

    const int es = slice_size(slice_dtype);
    const int64_t abytes = pack_bytes(A_slices, a_strides, batch, num_splits, M, K, es, false);
    const int64_t bbytes = pack_bytes(B_slices, b_strides, batch, num_splits, N, K, es, true);
    if (abytes + bbytes > 0 && (!workspace || workspace_bytes < (size_t)(abytes + bbytes) ||
                                (uintptr_t)workspace % 16 != 0))
        return OZK_ERR_WORKSPACE;
    const int64_t kp = round_up(K * es, 16) / es;
    char *ws = (char *)workspace;

    if (abytes > 0) {
        ozk::PackParams pk{A_slices, a_strides[0], a_strides[1], a_strides[2], a_strides[3],
                           ws, batch, num_splits, M, K, kp, es};
        hipError_t e = ozk::launch_pack(pk, st);
        if (e != hipSuccess) return OZK_ERR_LAUNCH;
        p.A = ws;
        p.as_b = num_splits * M * kp;
        p.as_l = M * kp;
        p.as_m = kp;
        ws += abytes;
    } else {
        p.A = A_slices;
        p.as_b = a_strides[0];
        p.as_l = a_strides[1];
        p.as_m = a_strides[2];
    }
    if (bbytes > 0) {
        ozk::PackParams pk{B_slices, b_strides[0], b_strides[1], b_strides[3], b_strides[2],
                           ws, batch, num_splits, N, K, kp, es};
        hipError_t e = ozk::launch_pack(pk, st);
        if (e != hipSuccess) return OZK_ERR_LAUNCH;
        p.B = ws;
        p.bs_b = num_splits * N * kp;
        p.bs_l = N * kp;
        p.bs_n = kp;
    } else {
        p.B = B_slices;
        p.bs_b = b_strides[0];
        p.bs_l = b_strides[1];
        p.bs_n = b_strides[3];
    }
    ozk::GemmPlan plan = ozk::plan_gemm(p, num_splits, slice_dtype);
    // more than 4 slices, operands within the 31-bit offsets of the LDS-DMA
    // kernels: 5 int8 / fp16 / bf16 slices in one launch (any C dtype); 6 to
    // 8 (or a forced pair-split kernel) into an fp64 C, which holds the
    // partial sum between the i-row launches
    if (num_splits > 4) {
        const bool solo = plan.kind == ozk::kGemmSolo;
        // (the triangular set sums all its pairs in one launch, so any C)
        const bool pair = plan.kind == ozk::kGemmPair && slice_dtype != OZK_F32 &&
                          (out_dtype == OZK_F64 || p.tri);
        if (!solo && !pair) return OZK_ERR_SPLITS;
    }
    // split-K buffers after the packed operands, 256-byte aligned, when the
    // workspace holds them (else the plan runs without split-K)
    void *skws = nullptr;
    if (const size_t skb = ozk::splitk_bytes(p, plan, num_splits)) {
        const uintptr_t base = (uintptr_t)workspace;
        const uintptr_t start = (base + (uintptr_t)(abytes + bbytes) + 255) / 256 * 256;
        if (workspace && start + skb <= base + workspace_bytes) skws = (void *)start;
        else plan.ksplit = 1;
    }
    if (hipError_t e = ozk::setup_splitk(p, plan, num_splits, skws, st)) return hip_status(e);
    return hip_status(ozk::launch_gemm(p, plan, num_splits, slice_dtype, st));
}

int ozk_cross_gemm(const void *A_slices, const int64_t a_strides[4], const void *B_slices,
                   const int64_t b_strides[4], const float *A_scales,
                   const int64_t sa_strides[3], const float *B_scales,
                   const int64_t sb_strides[3], int64_t batch, int64_t M, int64_t N, int64_t K,
                   int num_splits, int slice_dtype, void *C, int out_dtype,
                   const int64_t c_strides[3], void *workspace, size_t workspace_bytes,
                   void *stream) {
    return cross_gemm_impl(A_slices, a_strides, B_slices, b_strides, A_scales, sa_strides,
                           B_scales, sb_strides, batch, M, N, K, num_splits, slice_dtype,
                           OZK_PAIRS_ALL, C, out_dtype, c_strides, workspace, workspace_bytes,
                           stream);
}

int ozk_cross_gemm_pairs(const void *A_slices, const int64_t a_strides[4], const void *B_slices,
                         const int64_t b_strides[4], const float *A_scales,
                         const int64_t sa_strides[3], const float *B_scales,
                         const int64_t sb_strides[3], int64_t batch, int64_t M, int64_t N,
                         int64_t K, int num_splits, int slice_dtype, int pairs, void *C,
                         int out_dtype, const int64_t c_strides[3], void *workspace,
                         size_t workspace_bytes, void *stream) {
    return cross_gemm_impl(A_slices, a_strides, B_slices, b_strides, A_scales, sa_strides,
                           B_scales, sb_strides, batch, M, N, K, num_splits, slice_dtype, pairs,
                           C, out_dtype, c_strides, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// The whole ozaki_matmul below its Python checks (ozaki_triton.py:565-606):
// alpha, the split of B through its transposed view and of A, and the
// cross-GEMM, enqueued on one stream from one call; everything temporary
// (slices, scales, scratch) lives in the caller's workspace:
//   [A slices][A scales][B slices][B scales][split scratch][pack scratch],
// each region 256-byte aligned.  A broadcast operand (batch stride 0) is split
// once.
// ---------------------------------------------------------------------------
namespace {

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct MatmulLayout {
    int alpha;
    int64_t bA, bB;                                 // split batches (1 when broadcast)
    size_t a_sl, a_sc, b_sl, b_sc, scratch, pack;   // byte offsets
    size_t scratch_bytes;                           // split scratch reserved
    size_t splitk;                                  // cross-GEMM split-K buffers (after pack)
    size_t total;
    int64_t bt_strides[3];                          // B^T view of B
    int64_t ga[4], gb[4], gsa[3], gsb[3];           // cross-GEMM strides of the slices
};

int matmul_layout(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                  const int64_t as[3], const int64_t bs[3], int L, int sd, int pairs,
                  MatmulLayout *o) {
    if (!is_input_dtype(dtype) || !is_slice_dtype(sd)) return OZK_ERR_DTYPE;
    if (batch < 0 || M < 0 || N < 0 || K < 0) return OZK_ERR_SHAPE;
    // alpha for every num_splits, 0 included: the reference calls
    // compute_split_bits before splitting (ozaki_triton.py:580), so K = 0
    // (log2(0)) and alpha < 1 fail whatever the slice count
    o->alpha = 0;
    {
        const int st = ozk_compute_split_bits(K, sd, sd == OZK_I8 ? OZK_I32 : OZK_F32, &o->alpha);
        if (st != OZK_OK) return st;
    }
    if (L < 0 || L > OZK_MAX_SPLITS || !pair_set_ok(pairs, L)) return OZK_ERR_SPLITS;
    // more than 4 slices: 5 int8 / fp16 / bf16 slices into any C; 6 to 8 into
    // an fp64 C only
    if (L > 4 && (sd == OZK_F32 || (L > 5 && dtype != OZK_F64))) return OZK_ERR_SPLITS;
    if (L > 4) {
        // and a kernel that takes them (the LDS-DMA kernels' 31-bit operand
        // extents), known before anything is enqueued
        const int64_t es = slice_size(sd), kp = (K * es + 15) / 16 * 16 / es;
        ozk::GemmParams gp{};
        gp.as_l = M * kp; gp.as_m = kp; gp.bs_l = N * kp; gp.bs_n = kp;
        gp.batch = batch; gp.M = M; gp.N = N; gp.K = K; gp.out_dtype = dtype;
        gp.tri = pairs == OZK_PAIRS_TRIANGULAR;
        const int kind = ozk::plan_gemm(gp, L, sd, 256).kind;
        if (kind != ozk::kGemmSolo &&
            !(kind == ozk::kGemmPair && (dtype == OZK_F64 || gp.tri)))
            return OZK_ERR_SPLITS;
    }
    o->bA = (batch > 1 && as[0] != 0) ? batch : 1;
    o->bB = (batch > 1 && bs[0] != 0) ? batch : 1;
    o->bt_strides[0] = bs[0];
    o->bt_strides[1] = bs[2];
    o->bt_strides[2] = bs[1];
    const int64_t ss = slice_size(sd);
    const int64_t asl[4] = {L * M * K, M * K, K, 1}, bsl[4] = {L * N * K, N * K, K, 1};
    size_t off = 0;
    o->a_sl = off; off = align256(off + (size_t)(o->bA * L * M * K * ss));
    o->a_sc = off; off = align256(off + (size_t)(o->bA * L * M * 4));
    o->b_sl = off; off = align256(off + (size_t)(o->bB * L * N * K * ss));
    o->b_sc = off; off = align256(off + (size_t)(o->bB * L * N * 4));
    // the split scratch is sized for 256-byte aligned operands; plan_split
    // keeps the plan of any other pointer within that (ozk_matmul checks it)
    size_t scratch = 0;
    if (L > 0) {
        const int64_t dummy3[3] = {0, 0, 0};
        ozk::SplitParams pa = make_split_params((const void *)256, o->bA, M, K, as, L, o->alpha,
                                                (void *)256, asl, nullptr, dummy3);
        ozk::SplitParams pb = make_split_params((const void *)256, o->bB, N, K, o->bt_strides,
                                                L, o->alpha, (void *)256, bsl, nullptr, dummy3);
        const size_t wa = ozk::split_workspace_bytes(pa, ozk::plan_split(pa, dtype, sd), dtype, sd);
        const size_t wb = ozk::split_workspace_bytes(pb, ozk::plan_split(pb, dtype, sd), dtype, sd);
        scratch = wa > wb ? wa : wb;
    }
    o->scratch = off; off = align256(off + scratch);
    o->scratch_bytes = scratch;
    // cross-GEMM view of the slices (a batch-1 split is broadcast); they are
    // K-contiguous from a 256-byte aligned base, so only a row length that is
    // not a multiple of 16 bytes needs the packed copy
    const int64_t ga[4] = {o->bA == 1 ? 0 : L * M * K, M * K, K, 1};
    const int64_t gb[4] = {o->bB == 1 ? 0 : L * N * K, N * K, 1, K};
    const int64_t gsa[3] = {o->bA == 1 ? 0 : L * M, M, 1};
    const int64_t gsb[3] = {o->bB == 1 ? 0 : L * N, N, 1};
    for (int t = 0; t < 4; ++t) { o->ga[t] = ga[t]; o->gb[t] = gb[t]; }
    for (int t = 0; t < 3; ++t) { o->gsa[t] = gsa[t]; o->gsb[t] = gsb[t]; }
    const int64_t pk = pack_bytes((const void *)256, ga, batch, L, M, K, (int)ss, false) +
                       pack_bytes((const void *)256, gb, batch, L, N, K, (int)ss, true);
    o->pack = off; off = align256(off + (size_t)pk);
    // the split-K buffers of a grid too small to fill the chip follow the
    // pack region (the cross-GEMM runs without them when they are missing)
    const int64_t kp = round_up(K * ss, 16) / ss;
    o->splitk = splitk_need(batch, M, N, K, L, sd, M * kp, kp, N * kp, kp, dtype);
    o->total = off + o->splitk;
    return OZK_OK;
}

int record(void *const *events, int i, hipStream_t st) {
    if (!events || !events[i]) return OZK_OK;
    return hipEventRecord((hipEvent_t)events[i], st) == hipSuccess ? OZK_OK : OZK_ERR_LAUNCH;
}

}  // namespace

int ozk_matmul_workspace_bytes(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                               const int64_t a_strides[3], const int64_t b_strides[3],
                               int num_splits, int slice_dtype, size_t *bytes_out) {
    if (!bytes_out || !a_strides || !b_strides) return OZK_ERR_NULL;
    MatmulLayout lay;
    const int st = matmul_layout(dtype, batch, M, N, K, a_strides, b_strides, num_splits,
                                 slice_dtype, OZK_PAIRS_ALL, &lay);
    if (st != OZK_OK) return st;
    *bytes_out = (batch * M * N == 0 || num_splits == 0) ? 0 : lay.total;
    return OZK_OK;
}

int ozk_matmul(const void *A, const int64_t a_strides[3], const void *B,
               const int64_t b_strides[3], int dtype, int64_t batch, int64_t M, int64_t N,
               int64_t K, int num_splits, int slice_dtype, void *C, const int64_t c_strides[3],
               void *workspace, size_t workspace_bytes, void *const events[4], void *stream) {
    return ozk_matmul_pairs(A, a_strides, B, b_strides, dtype, batch, M, N, K, num_splits,
                            slice_dtype, OZK_PAIRS_ALL, C, c_strides, workspace,
                            workspace_bytes, events, stream);
}

int ozk_matmul_pairs(const void *A, const int64_t a_strides[3], const void *B,
                     const int64_t b_strides[3], int dtype, int64_t batch, int64_t M, int64_t N,
                     int64_t K, int num_splits, int slice_dtype, int pairs, void *C,
                     const int64_t c_strides[3], void *workspace, size_t workspace_bytes,
                     void *const events[4], void *stream) {
    if (!a_strides || !b_strides || !c_strides) return OZK_ERR_NULL;
    MatmulLayout lay;
    const int lst = matmul_layout(dtype, batch, M, N, K, a_strides, b_strides, num_splits,
                                  slice_dtype, pairs, &lay);
    if (lst != OZK_OK) return lst;
    if (batch * M * N == 0) return OZK_OK;
    if (!C) return OZK_ERR_NULL;
    hipStream_t st = (hipStream_t)stream;
    const int L = num_splits;
    if (L == 0) {
        // the reference's kernel stores its zero-initialised accumulator
        const int64_t z4[4] = {0, 0, 0, 0}, z3[3] = {0, 0, 0};
        return cross_gemm_impl(nullptr, z4, nullptr, z4, nullptr, z3, nullptr, z3, batch, M, N,
                               K, 0, slice_dtype, OZK_PAIRS_ALL, C, dtype, c_strides, nullptr, 0,
                               stream);
    }
    if (!A || !B) return OZK_ERR_NULL;
    // the split-K buffers at the end are optional
    if (!workspace || workspace_bytes < lay.total - lay.splitk || (uintptr_t)workspace % 256 != 0)
        return OZK_ERR_WORKSPACE;
    char *ws = (char *)workspace;
    const int64_t asl[4] = {L * M * K, M * K, K, 1}, bsl[4] = {L * N * K, N * K, K, 1};
    const int64_t asc[3] = {L * M, M, 1}, bsc[3] = {L * N, N, 1};
    int e;
    // split B through its transposed view, then A (ozaki_triton.py:588-599)
    ozk::SplitParams pb = make_split_params(B, lay.bB, N, K, lay.bt_strides, L, lay.alpha,
                                            ws + lay.b_sl, bsl, (float *)(ws + lay.b_sc), bsc);
    const ozk::SplitPlan plan_b = ozk::plan_split(pb, dtype, slice_dtype);
    ozk::SplitParams pa = make_split_params(A, lay.bA, M, K, a_strides, L, lay.alpha,
                                            ws + lay.a_sl, asl, (float *)(ws + lay.a_sc), asc);
    const ozk::SplitPlan plan_a = ozk::plan_split(pa, dtype, slice_dtype);
    if (ozk::split_workspace_bytes(pb, plan_b, dtype, slice_dtype) > lay.scratch_bytes ||
        ozk::split_workspace_bytes(pa, plan_a, dtype, slice_dtype) > lay.scratch_bytes)
        return OZK_ERR_WORKSPACE;
    pb.resid = pa.resid = (float *)(ws + lay.scratch);
    // The status words of the cooperative split launches go to the
    // cross-GEMM, which stores a NaN C and sets the device status if a wait
    // gave up, in place of the poison kernels after those launches.  A's split
    // runs last, so its word survives until then; B's word is the last 8
    // bytes of B's share of the scratch, and survives A's split where A's
    // share ends before it (else B keeps its poison kernel).  Both splits in
    // one launch: B's word, the only one.
    const uint32_t *split_fail[2] = {nullptr, nullptr};
    const size_t wa = ozk::split_workspace_bytes(pa, plan_a, dtype, slice_dtype);
    const size_t wb = ozk::split_workspace_bytes(pb, plan_b, dtype, slice_dtype);
    if (ozk::split_pair_ok(plan_a, plan_b, dtype)) {
        pb.fail_out = &split_fail[1];
    } else {
        pa.fail_out = &split_fail[0];
        if (wa + 8 <= wb) pb.fail_out = &split_fail[1];
    }
    if ((e = record(events, 0, st)) != OZK_OK) return e;
    if (ozk::split_pair_ok(plan_a, plan_b, dtype)) {
        // both in one launch; the second event marks the same point (the B
        // phase then reads as empty, the A phase as both splits)
        if ((e = record(events, 1, st)) != OZK_OK) return e;
        if (hipError_t he = ozk::launch_split_pair(pa, plan_a, pb, plan_b, dtype, slice_dtype, st))
            return hip_status(he);
    } else if (ozk::split_duo_ok(plan_a, plan_b, dtype)) {
        // B's strips and A's row blocks in one launch (the same event rule)
        if ((e = record(events, 1, st)) != OZK_OK) return e;
        if (hipError_t he = ozk::launch_split_duo(pa, plan_a, pb, plan_b, dtype, slice_dtype, st))
            return hip_status(he);
    } else {
        if (hipError_t he = ozk::launch_split(pb, plan_b, dtype, slice_dtype, st))
            return hip_status(he);
        if ((e = record(events, 1, st)) != OZK_OK) return e;
        if (hipError_t he = ozk::launch_split(pa, plan_a, dtype, slice_dtype, st))
            return hip_status(he);
    }
    if ((e = record(events, 2, st)) != OZK_OK) return e;
    // cross-GEMM over the K-contiguous slices
    e = cross_gemm_impl(ws + lay.a_sl, lay.ga, ws + lay.b_sl, lay.gb,
                        (const float *)(ws + lay.a_sc), lay.gsa, (const float *)(ws + lay.b_sc),
                        lay.gsb, batch, M, N, K, L, slice_dtype, pairs, C, dtype, c_strides,
                        ws + lay.pack, workspace_bytes - lay.pack, stream, split_fail);
    if (e != OZK_OK) return e;
    return record(events, 3, st);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// ozk_matmul_static: ozk_matmul on a library-owned scratch buffer, for callers
// that cannot allocate.  `scratch` is a file-scope device array; every device
// holds its own copy at its own address.  In host code the array's name is
// only a stand-in for the symbol, so its device address is asked once per
// device (hipGetSymbolAddress, with that device current) and only that
// address is handed to the kernels.  Every region the kernels read is written
// by the same call first, and the exchange words of the cooperative splits
// are cleared by a fill kernel at each launch, so nothing depends on what an
// earlier call left in the array.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[OZK_STATIC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxDevices];   // device address of `scratch`, per device

int static_scratch(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return OZK_ERR_LAUNCH;
    void *ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!ptr) {
        // first call on this device (concurrent first calls store the same address)
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
            return OZK_ERR_LAUNCH;
        g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
    *out = ptr;
    return OZK_OK;
}
}  // namespace

extern "C" int ozk_matmul_static(const void *A, const int64_t a_strides[3], const void *B,
                                 const int64_t b_strides[3], int dtype, int64_t batch,
                                 int64_t M, int64_t N, int64_t K, int num_splits,
                                 int slice_dtype, void *C, const int64_t c_strides[3],
                                 void *const events[4], void *stream) {
    if (!a_strides || !b_strides || !c_strides) return OZK_ERR_NULL;
    MatmulLayout lay;
    const int lst = matmul_layout(dtype, batch, M, N, K, a_strides, b_strides, num_splits,
                                  slice_dtype, OZK_PAIRS_ALL, &lay);
    if (lst != OZK_OK) return lst;
    if (batch * M * N == 0 || num_splits == 0)   // no workspace used
        return ozk_matmul(A, a_strides, B, b_strides, dtype, batch, M, N, K, num_splits,
                          slice_dtype, C, c_strides, nullptr, 0, events, stream);
    // split-K buffers are optional: the call needs the rest, and takes them
    // only if they fit too
    if (lay.total - lay.splitk > OZK_STATIC_SCRATCH_BYTES) return OZK_ERR_TOO_LARGE;
    void *ws = nullptr;
    if (const int e = static_scratch(&ws)) return e;
    return ozk_matmul(A, a_strides, B, b_strides, dtype, batch, M, N, K, num_splits,
                      slice_dtype, C, c_strides, ws, OZK_STATIC_SCRATCH_BYTES, events, stream);
}

// ---------------------------------------------------------------------------
// Test hooks (include/ozaki_amd_debug.h)
// ---------------------------------------------------------------------------
namespace {
struct Named {
    const char *name;
    int code;
};
const Named kGemmNames[] = {{"staged", ozk::kGemmStaged}, {"dma", ozk::kGemmDMA},
                            {"pair", ozk::kGemmPair},
                            {"ring", ozk::kGemmRing},     {"wide", ozk::kGemmWide},
                            {"wide4", ozk::kGemmWide4},   {"solo", ozk::kGemmSolo},
                            {"kstep", ozk::kGemmKStep},   {"kstep2", ozk::kGemmKStep2},
                            {"solo5", ozk::kGemmSolo}};   // an earlier name of "solo"
const Named kSplitNames[] = {{"coop", ozk::kForceSplitCoop},
                             {"strip", ozk::kForceSplitStrip},
                             {"transpose", ozk::kForceSplitTranspose},
                             {"generic", ozk::kForceSplitGeneric},
                             {"rows", ozk::kForceSplitRows},
                             {"rowscoop", ozk::kForceSplitRowsCoop}};
template <size_t N> int lookup(const Named (&t)[N], const char *name, int none, int *out) {
    if (!name || !*name) {
        *out = none;
        return OZK_OK;
    }
    for (size_t i = 0; i < N; ++i)
        if (strcmp(t[i].name, name) == 0) {
            *out = t[i].code;
            return OZK_OK;
        }
    return OZK_ERR_DTYPE;
}
template <size_t N> const char *name_of(const Named (&t)[N], int code) {
    for (size_t i = 0; i < N; ++i)
        if (t[i].code == code) return t[i].name;
    return "?";
}
}  // namespace

extern "C" {

int ozk_debug_force_gemm_kernel(const char *name) {
    return lookup(kGemmNames, name, ozk::kForceGemmNone, &ozk::debug_overrides().gemm);
}

int ozk_debug_force_gemm_ksplit(int ranges) {
    if (ranges < 0) return OZK_ERR_SPLITS;
    ozk::debug_overrides().ksplit = ranges;
    return OZK_OK;
}

int ozk_debug_force_split_kernel(const char *name) {
    return lookup(kSplitNames, name, ozk::kForceSplitNone, &ozk::debug_overrides().split);
}

int ozk_debug_force_coop_timeout(int on) {
    ozk::debug_overrides().coop_timeout = on != 0;
    return OZK_OK;
}

int ozk_debug_coop_residency(int force, int *resident_out) {
    if (force >= 0) ozk::debug_overrides().coop_resident = force;
    if (resident_out) *resident_out = ozk::coop_resident_per_xcd();
    return OZK_OK;
}

int ozk_debug_gemm_kernel(int64_t batch, int64_t M, int64_t N, int64_t K, int num_splits,
                          int slice_dtype, int cus, const char **name_out, int *ksplit_out) {
    return ozk_debug_gemm_kernel_pairs(batch, M, N, K, num_splits, slice_dtype, OZK_PAIRS_ALL,
                                       cus, name_out, ksplit_out);
}

int ozk_debug_gemm_kernel_pairs(int64_t batch, int64_t M, int64_t N, int64_t K, int num_splits,
                                int slice_dtype, int pairs, int cus, const char **name_out,
                                int *ksplit_out) {
    if (!name_out) return OZK_ERR_NULL;
    if (!is_slice_dtype(slice_dtype)) return OZK_ERR_DTYPE;
    if (num_splits < 1 || num_splits > OZK_MAX_SPLITS || !pair_set_ok(pairs, num_splits))
        return OZK_ERR_SPLITS;
    if (batch < 0 || M < 0 || N < 0 || K < 0) return OZK_ERR_SHAPE;
    ozk::GemmParams p{};
    const int64_t es = slice_size(slice_dtype);
    const int64_t kp = round_up(K * es, 16) / es;
    p.A = p.B = (const void *)(uintptr_t)256;
    p.as_m = kp;
    p.as_l = M * kp;
    p.as_b = num_splits * M * kp;
    p.bs_n = kp;
    p.bs_l = N * kp;
    p.bs_b = num_splits * N * kp;
    p.batch = batch;
    p.M = M;
    p.N = N;
    p.K = K;
    p.out_dtype = OZK_F64;
    p.tri = pairs == OZK_PAIRS_TRIANGULAR && num_splits >= 2;
    const ozk::GemmPlan plan = ozk::plan_gemm(p, num_splits, slice_dtype, cus);
    *name_out = name_of(kGemmNames, plan.kind);
    if (ksplit_out) *ksplit_out = plan.ksplit;
    return OZK_OK;
}

int ozk_debug_split_kernel(const void *X, int x_dtype, int64_t batch, int64_t rows, int64_t K,
                           const int64_t x_strides[3], int num_splits, int slice_dtype,
                           const void *slices, const int64_t slice_strides[4],
                           const char **name_out, size_t *bytes_out) {
    if (!name_out || !bytes_out || !x_strides || !slice_strides) return OZK_ERR_NULL;
    if (!is_input_dtype(x_dtype) || !is_slice_dtype(slice_dtype)) return OZK_ERR_DTYPE;
    if (num_splits < 1 || num_splits > OZK_MAX_SPLITS) return OZK_ERR_SPLITS;
    if (batch < 0 || rows < 0 || K < 0) return OZK_ERR_SHAPE;
    const int64_t dummy3[3] = {0, 0, 0};
    ozk::SplitParams p = make_split_params(X, batch, rows, K, x_strides, num_splits, 1,
                                           const_cast<void *>(slices), slice_strides, nullptr,
                                           dummy3);
    const ozk::SplitPlan plan = ozk::plan_split(p, x_dtype, slice_dtype);
    *bytes_out = ozk::split_workspace_bytes(p, plan, x_dtype, slice_dtype);
    switch (plan.path) {
    case ozk::kSplitRows: *name_out = plan.variant == 100 ? "rowscoop" : "rows"; break;
    case ozk::kSplitStrip: *name_out = "strip"; break;
    case ozk::kSplitCoop: *name_out = "coop"; break;
    case ozk::kSplitTransposeRows:
        *name_out = plan.variant == 100 ? "transposerowscoop" : "transpose";
        break;
    case ozk::kSplitConvert: *name_out = "convert"; break;
    default: *name_out = "generic";
    }
    return OZK_OK;
}

}  // extern "C"
