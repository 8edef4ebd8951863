// ozk_gemm_f16.hip -- cross-GEMM kernels with _Float16 slices (one translation
// unit per slice dtype, compiled in parallel).
#include "ozk_gemm_kernels.h"

namespace ozk {

hipError_t launch_gemm_f16(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t st) {
    return launch_typed<_Float16>(p, plan, L, st);
}

}  // namespace ozk
