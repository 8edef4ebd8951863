// ozk_gemm_i8.hip -- cross-GEMM kernels with int8_t slices (one translation
// unit per slice dtype, compiled in parallel).
#include "ozk_gemm_kernels.h"

namespace ozk {

hipError_t launch_gemm_i8(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t st) {
    return launch_typed<int8_t>(p, plan, L, st);
}

}  // namespace ozk
