// ozk_gemm_f32.hip -- cross-GEMM kernels with float slices (one translation
// unit per slice dtype, compiled in parallel).
#include "ozk_gemm_kernels.h"

namespace ozk {

hipError_t launch_gemm_f32(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t st) {
    return launch_typed<float>(p, plan, L, st);
}

}  // namespace ozk
