// sc_dec.hip -- k_decompress for one workgroup size (built with
// -DSC_DEC_RT=1..5: 32 * SC_DEC_RT chunks per workgroup).
#include "sc_kernels.h"

#ifndef SC_DEC_RT
#error "build with -DSC_DEC_RT=1..5"
#endif

namespace sc {

template <>
void launch_decompress<SC_DEC_RT>(const ModelDev &M, unsigned grid, hipStream_t s, const uint32_t *words,
                                  const int64_t *woff, const int32_t *wcnt, const int32_t *len, int64_t count,
                                  uint8_t *tokens, const int64_t *toff, int32_t *st, DecState *state,
                                  int32_t t_begin, int32_t t_end, int64_t n_second) {
    constexpr int RT = SC_DEC_RT;
    // the pipelined core holds at most 128 rows (4 row tiles)
    auto *kern = M.pipe == CORE_PIPE_UNI && RT <= 4 ? k_decompress<RT, (RT <= 4 ? CORE_PIPE_UNI : CORE_PLAIN)>
                                                    : k_decompress<RT, CORE_PLAIN>;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(THREADS), 0, s, M, words, woff, wcnt, len, count, tokens, toff, st,
                       state, t_begin, t_end, n_second, (uint8_t *)nullptr, 0);
}

}  // namespace sc
