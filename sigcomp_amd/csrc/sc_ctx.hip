// sc_ctx.hip -- k_mlp_context for one output mode (built with
// -DSC_CTX_MODE=0: int8 logits, 1: int32 CDF tables).
#include "sc_kernels.h"

#ifndef SC_CTX_MODE
#error "build with -DSC_CTX_MODE=0 or 1"
#endif

namespace sc {

template <>
void launch_mlp_context<SC_CTX_MODE>(const ModelDev &M, unsigned grid, hipStream_t s, const int64_t *ctx,
                                     int64_t rows, int8_t *logits, int32_t *cdf, int32_t *status) {
    auto *kern = M.pipe == CORE_PIPE_UNI ? k_mlp_context<SC_CTX_MODE, CORE_PIPE_UNI>
                 : M.pipe == CORE_PIPE   ? k_mlp_context<SC_CTX_MODE, CORE_PIPE>
                                         : k_mlp_context<SC_CTX_MODE, CORE_PLAIN>;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(THREADS), 0, s, M, ctx, rows, logits, cdf, status);
}

}  // namespace sc
