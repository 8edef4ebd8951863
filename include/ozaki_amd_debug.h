/*
 * ozaki_amd_debug.h -- test hooks of libozaki_amd.so.
 *
 * None of these has a counterpart in the reference (WhFanatic/Ozaki_triton):
 * its kernels are chosen by an autotuner and it has no bounded waits.  They
 * exist so that tests can run every kernel and every error path, and so that
 * tools can name the kernel a call would use.  Product code never needs them.
 *
 * The force settings live in thread-local storage: they apply to calls made
 * from the host thread that set them, and to nothing else.  The library reads
 * no environment variable.
 */
#ifndef OZAKI_AMD_DEBUG_H
#define OZAKI_AMD_DEBUG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Force the cross-GEMM kernel of later calls on this thread: one of "staged",
 * "dma", "pair", "ring", "wide", "wide4", "solo" ("solo5" too), "kstep",
 * "kstep2", or NULL / "" for the planner's choice.  A kernel that cannot take a call (operand
 * extents, slice count) is not used for it.  Returns OZK_ERR_DTYPE for an
 * unknown name.
 */
int ozk_debug_force_gemm_kernel(const char *name);

/*
 * Force the split kernel of later calls on this thread: "coop", "strip",
 * "transpose", "generic" (column operands), "rows", "rowscoop" (row
 * operands), or NULL / "" for the planner's choice.  A path whose layout
 * requirements fail is not taken.  Returns OZK_ERR_DTYPE for an unknown name.
 */
int ozk_debug_force_split_kernel(const char *name);

/*
 * on != 0: every cooperative split wait of later calls on this thread gives
 * up at its first check (it looks for a tag that is never written), so the
 * timeout path runs: after ozk_split the split's scales become NaN, after
 * ozk_matmul C does (0 for an int8 C), and the sticky device status is set
 * (ozk_device_status).  No kernel waits longer than one poll.
 */
int ozk_debug_force_coop_timeout(int on);

/*
 * The workgroups one XCD holds for the cooperative split kernels (their
 * occupancy per CU times the CUs of one XCD, 32 on gfx950), written to
 * *resident_out (may be NULL).  The split planner gives a cooperative group
 * at most that many members minus 8, so that every group becomes resident.
 * force > 0: later plans on this thread assume `force` instead; 0: the
 * current device's figure again; < 0: no change.
 */
int ozk_debug_coop_residency(int force, int *resident_out);

/*
 * Force the split-K ranges of later calls on this thread whose cross-GEMM
 * runs the ring or the wide kernel: each tile's K is cut into `ranges` (at
 * most one per 128 bytes of K), one workgroup each, when the call's
 * workspace holds the split-K buffers (ozk_cross_gemm_workspace_bytes and
 * ozk_matmul_workspace_bytes size them for the forced count); 0 for the
 * planner's choice, 1 for none.
 */
int ozk_debug_force_gemm_ksplit(int ranges);

/*
 * The cross-GEMM kernel the planner would choose for K-contiguous,
 * 16-byte aligned slice operands of this shape, as a name ("dma", "ring",
 * "wide", "wide4", "solo", "kstep", "kstep2", "pair", "staged") written to
 * *name_out (a static string), and its split-K ranges per tile to *ksplit_out (1: none;
 * may be NULL).  cus: compute units to plan for (0: those of the current
 * device).
 */
int ozk_debug_gemm_kernel(int64_t batch, int64_t M, int64_t N, int64_t K, int num_splits,
                          int slice_dtype, int cus, const char **name_out, int *ksplit_out);

/* The same for a pair set (OZK_PAIRS_ALL or OZK_PAIRS_TRIANGULAR). */
int ozk_debug_gemm_kernel_pairs(int64_t batch, int64_t M, int64_t N, int64_t K, int num_splits,
                                int slice_dtype, int pairs, int cus, const char **name_out,
                                int *ksplit_out);

/*
 * The split path the planner would choose for an operand described as in
 * ozk_split (X and slices are only inspected for their alignment, never
 * read), as a name ("rows", "rowscoop", "coop", "strip", "transpose",
 * "transposerowscoop", "generic", "convert") written to *name_out (a static
 * string), and the workspace bytes that plan needs to *bytes_out.
 */
int ozk_debug_split_kernel(const void *X, int x_dtype, int64_t batch, int64_t rows, int64_t K,
                           const int64_t x_strides[3], int num_splits, int slice_dtype,
                           const void *slices, const int64_t slice_strides[4],
                           const char **name_out, size_t *bytes_out);

#ifdef __cplusplus
}
#endif

#endif /* OZAKI_AMD_DEBUG_H */
