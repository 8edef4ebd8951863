/*
 * ozaki_amd.h -- C ABI of the MI355X-native Ozaki-scheme matmul (libozaki_amd.so).
 *
 * The reference (WhFanatic/Ozaki_triton) has no FFI: its hot path sits behind
 * the Python functions of ozaki_triton.py and, below them, the Triton launch
 * ABI of two JIT kernels.  Each entry point here replaces one of those launch
 * sites; the Python package ozaki_triton_amd binds them with ctypes.
 *
 * Conventions
 *   - Plain pointers to device memory, sizes and element strides (int64, in
 *     elements of the tensor they describe).  A batch stride may be 0
 *     (broadcast operand).
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).  All
 *     work is enqueued asynchronously on it; nothing synchronises the host.
 *   - Return 0 on success and a negative OZK_ERR_* code on failure;
 *     ozk_strerror() names the code.  Argument checks run on the host before
 *     anything is enqueued, so a rejected call has no device side effect.
 *   - No device memory is allocated.  Scratch space comes from the caller
 *     through (workspace, workspace_bytes), 16-byte aligned; *_workspace_bytes() says
 *     how much.
 *   - Calls are re-entrant and thread-safe.  The only process-wide state is,
 *     per cross-GEMM kernel, an atomic record of the devices on which its
 *     dynamic-LDS limit has been raised (hipFuncSetAttribute, once per device),
 *     each device's compute-unit count (asked once), and the sticky device
 *     status word (ozk_device_status).
 */
#ifndef OZAKI_AMD_H
#define OZAKI_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes (torch dtype names in comments) */
enum {
    OZK_F64 = 0,  /* torch.float64 */
    OZK_F32 = 1,  /* torch.float32 */
    OZK_F16 = 2,  /* torch.float16 */
    OZK_BF16 = 3, /* torch.bfloat16 */
    OZK_I8 = 4,   /* torch.int8 */
    OZK_I32 = 5   /* torch.int32 */
};

/* status codes */
enum {
    OZK_OK = 0,
    OZK_ERR_NULL = -1,        /* a required pointer is NULL */
    OZK_ERR_DTYPE = -2,       /* dtype combination not supported */
    OZK_ERR_SPLITS = -3,      /* num_splits outside [0, OZK_MAX_SPLITS], or > 4 with a
                                 cross-GEMM that cannot take it; or (the *_pairs
                                 calls) an unknown pair set, or the triangular set
                                 with more than 5 slices */
    OZK_ERR_SHAPE = -4,       /* negative size, or K mismatch */
    OZK_ERR_ALPHA = -5,       /* alpha < 1 (K too large for the accumulator) */
    OZK_ERR_WORKSPACE = -6,   /* workspace missing, too small or not 16-byte aligned */
    OZK_ERR_LAUNCH = -7,      /* a HIP launch failed (hipGetLastError) */
    OZK_ERR_ACCUM = -8,       /* unsupported dot accumulator dtype */
    OZK_ERR_DEVICE_WAIT = -9, /* (ozk_device_status) a cooperative split wait on the
                                 device gave up; that split's scales, and so the C
                                 computed from them, are NaN -- except in an int8 C,
                                 whose conversion maps NaN to 0: there C is 0, and
                                 only this status tells it from a valid result */
    OZK_ERR_TOO_LARGE = -10   /* (ozk_matmul_static) the call needs more scratch than
                                 OZK_STATIC_SCRATCH_BYTES */
};

/* The reference's ozaki_matmul asserts num_splits <= 4 (ozaki_triton.py:563),
 * a limit of its kernel's hard-coded accumulators.  The calls here take up to
 * 8 slices; with more than 4, the cross-GEMM needs int8 / fp16 / bf16 slices,
 * and with more than 5 an fp64 C (OZK_ERR_SPLITS otherwise). */
#define OZK_MAX_SPLITS 8

/* Name of a status code (static string). */
const char *ozk_strerror(int status);

/* ABI version: major * 10000 + minor * 100 + patch. */
int ozk_version(void);

/*
 * Sticky device status -- no counterpart in the reference, whose kernels have
 * no bounded waits.  The cooperative split kernels (long columns of B, long
 * rows of A) combine their level maxima across workgroups with waits bounded
 * at 2 s.  A wait that gives up sets a per-device status word and marks what
 * the split feeds: after ozk_split every scale of that split is NaN; after
 * ozk_matmul every entry of C is NaN (0 in an int8 C, see
 * OZK_ERR_DEVICE_WAIT), never a silently wrong value.  This call
 * waits for `stream`, reads the current device's word into *status_out
 * (OZK_OK or OZK_ERR_DEVICE_WAIT) and clears it when `clear` is non-zero.
 * Calls are asynchronous, so a failure is seen by the first status read
 * after the call that failed.
 */
int ozk_device_status(int clear, int *status_out, void *stream);

/*
 * compute_split_bits -- replaces ozaki_triton.py:76-98.
 *   alpha = min(int((acc_bits - log2 n) / 2), slice_bits), acc_bits 31 for an
 *   int32 dot accumulator and 23 for fp32.  Writes alpha (which may be < 1) to
 *   *alpha_out; returns OZK_ERR_ALPHA when alpha < 1 (the reference asserts),
 *   OZK_ERR_ACCUM / OZK_ERR_DTYPE for an unknown accumulator / slice dtype.
 */
int ozk_compute_split_bits(int64_t n, int slice_dtype, int dot_accum_dtype, int *alpha_out);

/*
 * Split -- replaces the launch of split_matrix_kernel in split_matrix
 * (ozaki_triton.py:214-256; kernel 137-211).
 *   X       [batch, rows, K]      x_dtype any of OZK_F64 / F32 / F16 / BF16 / I8
 *                                 (ozaki_triton.py:42-48), strides x_strides
 *   slices  [batch, L, rows, K]   slice_dtype OZK_I8 / F16 / BF16 / F32, strides
 *                                 slice_strides
 *   scales  [batch, L, rows]      fp32, strides scale_strides
 * For each row: L levels of (row max -> power-of-two scale -> quantise ->
 * residual), in fp64 for fp64 input and fp32 otherwise (narrow inputs convert
 * exactly), with the residual rounded to fp32 between levels exactly as the
 * reference's fp32 residual buffer does.  B is split through its transposed
 * view (rows = columns of B, x_strides = {K*N, 1, N}).
 * Workspace (ozk_split_workspace_bytes()): 0 bytes for K-contiguous fp64 /
 * fp32 rows up to 16384 long and for odd layouts; for row-contiguous operands
 * (the B^T view) 8 bytes per column group (128 bytes of a row), level and K
 * chunk of 512 or 1024 rows, through which the workgroups of a column group
 * exchange their level maxima (likewise per row, level and chunk for longer
 * rows), plus a status word; an fp32 copy of a narrow input, or a transposed
 * copy of a long column operand.  The query sees no pointers: it sizes for
 * 16-byte aligned X and slices, and a call with other pointers needs no more.
 */
int ozk_split_workspace_bytes(int x_dtype, int64_t batch, int64_t rows, int64_t K,
                              const int64_t x_strides[3], int num_splits, int slice_dtype,
                              const int64_t slice_strides[4], size_t *bytes_out);

int ozk_split(const void *X, int x_dtype, int64_t batch, int64_t rows, int64_t K,
              const int64_t x_strides[3], int num_splits, int alpha, int slice_dtype,
              void *slices, const int64_t slice_strides[4], float *scales,
              const int64_t scale_strides[3], void *workspace, size_t workspace_bytes,
              void *stream);

/*
 * Cross-GEMM -- replaces the launch of cross_gemm_kernel in cross_gemm
 * (ozaki_triton.py:455-498; kernel 306-452).
 *   A_slices [batch, L, M, K]  strides a_strides
 *   B_slices [batch, L, K, N]  strides b_strides (logical K x N; ozaki_matmul
 *                              passes a K-contiguous view, b_strides[2] == 1)
 *   A_scales [batch, L, M] fp32, B_scales [batch, L, N] fp32
 *   C        [batch, M, N]  out_dtype OZK_F64 (fp64 outer accumulator) or
 *                           OZK_F32 / F16 / BF16 / I8 (fp32 outer accumulator,
 *                           stored rounded to nearest even, or for I8 truncated
 *                           toward zero and saturated)
 *   C = sum_{i,j} fl32(fl32(fl32(A_i B_j) * sa_i) * sb_j), summed i-major,
 *   j-minor from 0 in the outer accumulator.  int8 slices use an exact int32
 *   dot (MFMA i8); fp16 / bf16 / fp32 slices an fp32-accumulated dot (MFMA f16,
 *   bf16, f32).
 * Workspace: 0 bytes when both slice operands are K-contiguous with 16-byte
 * aligned rows; otherwise ozk_cross_gemm_workspace_bytes() for a packed copy.
 */
int ozk_cross_gemm_workspace_bytes(int64_t batch, int64_t M, int64_t N, int64_t K,
                                   int num_splits, int slice_dtype,
                                   const void *A_slices, const int64_t a_strides[4],
                                   const void *B_slices, const int64_t b_strides[4],
                                   size_t *bytes_out);

int ozk_cross_gemm(const void *A_slices, const int64_t a_strides[4], const void *B_slices,
                   const int64_t b_strides[4], const float *A_scales,
                   const int64_t sa_strides[3], const float *B_scales,
                   const int64_t sb_strides[3], int64_t batch, int64_t M, int64_t N, int64_t K,
                   int num_splits, int slice_dtype, void *C, int out_dtype,
                   const int64_t c_strides[3], void *workspace, size_t workspace_bytes,
                   void *stream);

/*
 * Pair sets -- no counterpart in the reference, whose cross-GEMM always sums
 * all L x L slice pairs (ozaki_triton.py:403-447).
 *   OZK_PAIRS_ALL         every pair (i, j): the reference's sum, bit for bit.
 *   OZK_PAIRS_TRIANGULAR  only the pairs with i + j <= L - 1, L (L + 1) / 2 of
 *                         them, summed in the same i-major / j-minor order from
 *                         the same t_ij.  Pair (i, j) carries about
 *                         2^(-alpha (i + j)) of C's magnitude, so the terms left
 *                         out are of the size of the split's own truncation
 *                         error: 5 int8 slices on 15 pairs reach the accuracy of
 *                         25 pairs (fp64 inputs, K = 8192: rel-err 4.31e-10
 *                         against 4.26e-10), with fewer products than 4 slices
 *                         on all 16 pairs (2.8e-9).  Takes 1 to 5 slices.
 * The *_pairs calls take the set as an extra argument and are otherwise the
 * calls above (the same workspace queries cover both sets).
 */
enum { OZK_PAIRS_ALL = 0, OZK_PAIRS_TRIANGULAR = 1 };

int ozk_cross_gemm_pairs(const void *A_slices, const int64_t a_strides[4], const void *B_slices,
                         const int64_t b_strides[4], const float *A_scales,
                         const int64_t sa_strides[3], const float *B_scales,
                         const int64_t sb_strides[3], int64_t batch, int64_t M, int64_t N,
                         int64_t K, int num_splits, int slice_dtype, int pairs, void *C,
                         int out_dtype, const int64_t c_strides[3], void *workspace,
                         size_t workspace_bytes, void *stream);

/*
 * Matmul -- replaces ozaki_matmul below its Python checks (ozaki_triton.py:
 * 565-606): alpha (compute_split_bits), the split of B through its transposed
 * view and of A, and the fused cross-GEMM, enqueued on `stream` by one call.
 *   A [batch, M, K], strides a_strides; B [batch, K, N], strides b_strides;
 *   a batch stride of 0 broadcasts that operand (it is split once).
 *   dtype: the input dtype of A and B, which is also C's (any input dtype).
 *   C [batch, M, N], strides c_strides.
 * Everything temporary lives in `workspace` (256-byte aligned,
 * ozk_matmul_workspace_bytes() long), so the call allocates nothing and may be
 * captured in a HIP graph.  events: NULL, or 4 hipEvent_t (each may be NULL)
 * recorded on `stream` before the B split, before the A split, before the
 * cross-GEMM and after it (where both splits run in one launch, the first
 * two mark the same point).  Returns OZK_ERR_ALPHA when K is too large for
 * the slice dtype (the reference asserts) and OZK_ERR_SHAPE for K = 0 (the
 * reference's log2(0) raises).
 */
int ozk_matmul_workspace_bytes(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                               const int64_t a_strides[3], const int64_t b_strides[3],
                               int num_splits, int slice_dtype, size_t *bytes_out);

int ozk_matmul(const void *A, const int64_t a_strides[3], const void *B,
               const int64_t b_strides[3], int dtype, int64_t batch, int64_t M, int64_t N,
               int64_t K, int num_splits, int slice_dtype, void *C, const int64_t c_strides[3],
               void *workspace, size_t workspace_bytes, void *const events[4], void *stream);

/* ozk_matmul with a pair set (OZK_PAIRS_*, above); ozk_matmul_workspace_bytes
 * sizes its workspace. */
int ozk_matmul_pairs(const void *A, const int64_t a_strides[3], const void *B,
                     const int64_t b_strides[3], int dtype, int64_t batch, int64_t M, int64_t N,
                     int64_t K, int num_splits, int slice_dtype, int pairs, void *C,
                     const int64_t c_strides[3], void *workspace, size_t workspace_bytes,
                     void *const events[4], void *stream);

/*
 * Matmul without a workspace -- no counterpart in the reference.  For callers
 * that cannot allocate device memory at all (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): ozk_matmul with its
 * workspace taken from a library-owned device array of OZK_STATIC_SCRATCH_BYTES,
 * one per device, held until the process ends.  The caller still passes the
 * inputs and C.  A call that needs more than that, not counting the optional
 * split-K buffers (ozk_matmul_workspace_bytes() includes them), returns
 * OZK_ERR_TOO_LARGE before anything is enqueued; split-K buffers that do not
 * fit as well are left out (the same bits, from unsplit tiles).  The call allocates
 * nothing (no hipMalloc, hipFree or allocating library routine).  All calls on
 * one device share its array: calls that overlap on one device (other streams
 * or threads, without ordering between them) race and give wrong results.
 */
#define OZK_STATIC_SCRATCH_BYTES ((size_t)64 << 20)

int ozk_matmul_static(const void *A, const int64_t a_strides[3], const void *B,
                      const int64_t b_strides[3], int dtype, int64_t batch, int64_t M,
                      int64_t N, int64_t K, int num_splits, int slice_dtype, void *C,
                      const int64_t c_strides[3], void *const events[4], void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OZAKI_AMD_H */
