// ozk_gemm_bf16.hip -- cross-GEMM kernels with __bf16 slices (one translation
// unit per slice dtype, compiled in parallel).
#include "ozk_gemm_kernels.h"

namespace ozk {

hipError_t launch_gemm_bf16(const GemmParams &p, const GemmPlan &plan, int L, hipStream_t st) {
    return launch_typed<__bf16>(p, plan, L, st);
}

}  // namespace ozk
