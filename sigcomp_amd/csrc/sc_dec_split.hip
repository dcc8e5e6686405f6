// sc_dec_split.hip -- the split decode of small batches (k_decompress with
// 4 or 8 workgroups per 32-chunk group sharing layer 0).
#include "sc_kernels.h"

namespace sc {

hipError_t launch_decompress_split(const ModelDev &M, int p, unsigned groups, hipStream_t s, const uint32_t *words,
                                   const int64_t *woff, const int32_t *wcnt, const int32_t *len, int64_t count,
                                   uint8_t *tokens, const int64_t *toff, int32_t *st, DecState *state,
                                   int32_t t_begin, int32_t t_end, uint8_t *xch, int32_t spin_max) {
    int64_t n_second = 0;
    void *args[] = {(void *)&M, (void *)&words, (void *)&woff, (void *)&wcnt, (void *)&len, (void *)&count,
                    (void *)&tokens, (void *)&toff, (void *)&st, (void *)&state, (void *)&t_begin,
                    (void *)&t_end, (void *)&n_second, (void *)&xch, (void *)&spin_max};
    // cooperative: every workgroup of the grid is resident at once (the
    // groups' workgroups wait for each other)
    const void *kern = p == 8 ? (const void *)k_decompress<1, CORE_PIPE_UNI, 8>
                              : (const void *)k_decompress<1, CORE_PIPE_UNI, 4>;
    return hipLaunchCooperativeKernel(kern, dim3(groups * (p == 8 ? 8 : 4)), dim3(THREADS), args, 0, s);
}

}  // namespace sc
