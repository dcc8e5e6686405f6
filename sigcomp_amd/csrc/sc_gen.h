// sc_gen.h -- host entry points of the codec for architectures the
// specialised kernels do not cover (sc_gen.hip).  The model's layers are
// packed in 32 x 32 MFMA fragments zero padded to whole tiles, with
// per-channel requant blocks (ModelDev::pipe == CORE_GENERIC).
#pragma once

#include <string>

#include "sc_kernels.h"

namespace sc {

constexpr int R_GEN_TILE = R_TILE;              // steps per compress tile descriptor (k_tile_table)
constexpr int64_t GEN_BATCH_ROWS = 1 << 16;     // rows per launch batch at most
constexpr int64_t GEN_SCRATCH_BYTES = 1 << 30;  // scratch per call at most (batches shrink for wide models)

// Scratch memory of these calls comes from hipMallocAsync / hipFreeAsync on
// the call's stream.  Return SC_OK or SC_ERR_HIP with `err` set.

// sc_mlp_forward / sc_mlp_forward_cdf (exactly one of logits, cdf non-null).
int gen_mlp_forward(const ModelDev &M, const int64_t *ctx, int64_t rows, int8_t *logits, int32_t *cdf,
                    int32_t *status, hipStream_t s, std::string &err);
// sc_compress_chunks between the tile table and k_encode_pairs: the (cum,
// freq) pair of every token of the tiles (max_tiles: a host-side bound on
// the tile count, whose exact value is tile_start[n_chunks] on the device).
int gen_compress(const ModelDev &M, const uint8_t *tokens, const int32_t *tile_start, int64_t n_chunks,
                 const int4 *desc, int64_t max_tiles, uint2 *pairs, hipStream_t s, std::string &err);
// sc_decompress_chunks: `state` holds n_chunks DecState; max_len = the
// longest chunk.
int gen_decompress(const ModelDev &M, const uint32_t *words, const int64_t *word_off, const int32_t *word_cnt,
                   const int32_t *lengths, int64_t n_chunks, uint8_t *tokens, const int64_t *tok_off,
                   int32_t *status, DecState *state, int32_t max_len, hipStream_t s, std::string &err);

}  // namespace sc
