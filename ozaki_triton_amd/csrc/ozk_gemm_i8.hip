// ozk_gemm_i8.hip -- cross-GEMM kernels with int8_t slices (one translation
// unit per slice dtype, compiled in parallel).
#include "ozk_gemm_kernels.h"

namespace ozk {

hipError_t launch_gemm_i8(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t st) {
    return p.out_dtype == 0 ? launch_st<int8_t, double>(p, plan, L, st)
                            : launch_st<int8_t, float>(p, plan, L, st);
}

}  // namespace ozk
