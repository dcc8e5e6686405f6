// sc_comp.hip -- k_compress_mlp (teacher-forced MLP fused with the
// frequency step) for the per-tensor pipelined core and the plain core.
#include "sc_kernels.h"

namespace sc {

void launch_compress_mlp(const ModelDev &M, unsigned grid, hipStream_t s, const uint8_t *tokens, int64_t n_chunks,
                         const int32_t *tile_start, const int4 *desc, int64_t max_desc, uint2 *pairs) {
    // compress runs the pipelined core only with per-tensor constants (the
    // bundled checkpoints); other models take the plain core
    auto *kern = M.pipe == CORE_PIPE_UNI ? k_compress_mlp<CORE_PIPE_UNI> : k_compress_mlp<CORE_PLAIN>;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(THREADS), 0, s, M, tokens, n_chunks, tile_start, desc, max_desc,
                       pairs);
}

}  // namespace sc
