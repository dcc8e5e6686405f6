/*
 * sigcomp_hip.h -- C ABI of the MI355X (gfx950) SigComp codec library.
 *
 * libsigcomp_hip.so holds hand-written HIP kernels for the codec hot path of
 * SigComp (BioinfoSZU/SigComp v1.1.0): the integer-quantised MLP entropy model
 * on int8 MFMA with fused requantisation, the fused int8-logits -> frequency /
 * CDF step, the range encoder and decoder, and the batched autoregressive
 * decode loop.  Every entry point below names the reference interface it
 * replaces (paths relative to the reference's sigcomp/ package).
 *
 * Conventions
 *  - Pointers documented "device" are HIP device pointers owned by the caller
 *    (the library never frees caller memory).  "host" pointers are read during
 *    the call only.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).  All
 *    work is stream-ordered; no call waits for the device, except
 *    sc_decompress_chunks when it is not given the lengths on the host.
 *  - Return value: SC_OK or an SC_ERR_* code for argument / HIP errors found
 *    at launch time; sc_last_error() describes the last failure of the calling
 *    thread.  Data-dependent failures (an out-of-range token, an encoder
 *    capacity overflow, an invalid range stream) are reported through the
 *    caller's device `status` arrays with the SC_STATUS_* codes, since they
 *    are known only after the kernels ran.
 *  - A model handle is read-only after sc_model_create: calls on several
 *    streams or host threads may share it.  Each call's mutable device state
 *    lives in memory the caller passes (workspace, state and output arrays);
 *    calls that share such memory must not overlap.
 *
 * Architectures: any window W, embedding 257 x E and chain of n_layers
 * (1..16) linear layers from W * E inputs to 256 logits, as the reference's
 * GPU codec takes (quant_mlp_export.py:21-101,215-269).  The bundled one
 * (window 64, embedding 257 x 128, layer 0 8192 -> 512, n_layers - 2 hidden
 * layers 512 -> 512, last layer 512 -> 256: both bundled checkpoints,
 * quant_mlp_export.py:211-213, cpu_int_inference.py:395-445) runs the
 * specialised persistent kernels; any other runs the generic path (one
 * launch per stage, scratch memory from hipMallocAsync on the call's
 * stream), with identical results for any model.
 */
#ifndef SIGCOMP_HIP_H
#define SIGCOMP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SC_OK 0
#define SC_ERR_ARG 1
#define SC_ERR_HIP 2
#define SC_ERR_UNSUPPORTED 3

/* Per-row / per-stream status codes written to device status arrays. */
#define SC_STATUS_OK 0
#define SC_STATUS_CAPACITY 1        /* encoder output capacity exceeded (OverflowError) */
#define SC_STATUS_INVALID_STREAM 2  /* decoder: scale == 0 or quantile >= 2**24 (ValueError) */
#define SC_STATUS_BAD_TOKEN 3       /* context token outside [0, 256] (ValueError) */
#define SC_STATUS_SYNC_TIMEOUT 4    /* decoder: the workgroups sharing a small decode's layer 0
                                       waited too long for each other (RuntimeError; tokens
                                       unspecified) */

#define SC_VOCAB 256
#define SC_SOS 256

typedef struct sc_model sc_model;

/* One quantised linear layer, host arrays, nn.Linear layout.
 * y = clamp(((x . W^T + bias) * m0) >> shift, relu ? 0 : -128, 127). */
typedef struct {
    int32_t n, k;
    const int8_t *weight;   /* [n, k] */
    const int32_t *bias;    /* [n]    */
    const int64_t *m0;      /* [n], each in [0, 2**31] (per-tensor models repeat one value) */
    const int32_t *shift;   /* [n], each in [0, 63] */
    int32_t relu;
} sc_layer_desc;

/* Last error message of the calling thread (never NULL). */
const char *sc_last_error(void);

/* Library version string. */
const char *sc_version(void);

/* Upload an integer model to `device` and pack its weights in MFMA fragment
 * order.  Replaces QuantMLPCompression.__init__ + convert_ptq_to_gpu_pipeline
 * (quant_mlp_export.py:215-269,180-200) after the host has derived the
 * integer constants (cpu_int_inference.py:395-445); `exp_lut` is the 256-entry
 * integer exp table of build_integer_exp_lut (gpu_entropy_coding.py:8-22). */
int sc_model_create(const int8_t *emb, int32_t emb_rows, int32_t emb_dim, int32_t window,
                    const sc_layer_desc *layers, int32_t n_layers, const int64_t *exp_lut,
                    int32_t device, sc_model **out);
int sc_model_destroy(sc_model *model);

/* Device copy of the model's exp LUT (uint64 [256]); owned by the model. */
const uint64_t *sc_model_lut(const sc_model *model);

/* MLP core the model runs on: 2 = pipelined core with per-tensor requant
 * (every layer's constants satisfy m0 < 2**31 and shift >= 32 after the
 * m0 = 2**31 rewrite, ReLU on every layer but the last, and one m0 and
 * shift per layer, as in both bundled checkpoints;
 * tiles of up to 128 rows; every kernel), 1 = pipelined core with
 * per-channel constants (the explicit-context kernels; compress and
 * decompress run the plain core), 0 = plain core (any model of the bundled
 * architecture; also selected by SC_HIP_PLAIN_CORE=1 in the environment at
 * sc_model_create), 3 = generic path (any other architecture).  All give
 * identical results.  No reference counterpart (diagnostic). */
int sc_model_core(const sc_model *model);

/* MLP forward on explicit context windows: ctx int64 [rows, 64] (device,
 * tokens in [0, 256]) -> logits int8 [rows, 256] (device).  Replaces
 * GPUBitExactMLPDecoder._ar_step (quant_mlp_export.py:133-138) = int8
 * embedding gather + 9 x bit_exact_linear_kernel launches
 * (quant_mlp_export.py:21-110).  status: device int32 [1], set to
 * SC_STATUS_BAD_TOKEN if any token is out of range (never cleared). */
int sc_mlp_forward(const sc_model *model, const int64_t *ctx, int64_t rows, int8_t *logits,
                   int32_t *status, void *stream);

/* MLP forward fused with the logits -> CDF step: ctx int64 [rows, 64] ->
 * cdf int32 [rows, 257] (cdf[0] = 0, cdf[256] = 2**24).  Equals
 * int8_logits_to_cdf(_ar_step(ctx)) (gpu_entropy_coding.py:25-51,
 * cpu_entropy_coding.py:73-110) without materialising the logits. */
int sc_mlp_forward_cdf(const sc_model *model, const int64_t *ctx, int64_t rows, int32_t *cdf,
                       int32_t *status, void *stream);

/* int8 logits [rows, 256] + LUT (device uint64/int64 [256]) -> int64 CDF
 * [rows, 257].  Replaces int8_logits_to_cdf (gpu_entropy_coding.py:25-51). */
int sc_logits_to_cdf(const int8_t *logits, int64_t rows, const uint64_t *lut, int64_t *cdf,
                     void *stream);

/* Range encoder state, one entry per stream (device arrays [B]).
 * Mirrors GpuRangeStepEncoder's tensors (gpu_entropy_coding.py:255-267). */
typedef struct {
    uint64_t *lower;        /* init 0            */
    uint64_t *range;        /* init 2**64 - 1    */
    int32_t *inverted;      /* init 0            */
    uint32_t *first;        /* init 0            */
    int32_t *write_pos;     /* init 0            */
    int32_t *status;        /* init 0            */
} sc_encoder_state;

/* One encoder step for every stream b with t < valid_lens[b]: frequencies
 * from logits[b] (int8 [B, 256]) and the LUT, then the range-coder update
 * with symbols[b] (int64 [B]); words go to words[b * max_words + pos].
 * From 2**18 streams the step runs as a kernel that codes 64 streams per
 * wavefront (results identical; SC_HIP_STEP_WIDE=0 or 1 in the environment
 * forces the small-batch or the large-batch kernel, as does sc_decode_step).
 * Replaces GpuRangeStepEncoder.encode_step_int8 / _range_encode_step_int8_kernel
 * (gpu_entropy_coding.py:270-280,137-252). */
int sc_encode_step(const int8_t *logits, const uint64_t *lut, const int64_t *symbols,
                   const int64_t *valid_lens, int64_t t, int64_t B, const sc_encoder_state *state,
                   uint32_t *words, int64_t max_words, void *stream);

/* Flush every stream (GpuRangeStepEncoder.seal / _range_seal_kernel,
 * gpu_entropy_coding.py:282-290,78-134).  Sealing twice emits nothing more. */
int sc_encode_seal(int64_t B, const sc_encoder_state *state, uint32_t *words, int64_t max_words,
                   void *stream);

/* Range decoder state (device arrays [B]); mirrors GpuRangeDecoder's tensors
 * (gpu_entropy_coding.py:400-442). */
typedef struct {
    uint64_t *lower;        /* init 0                                   */
    uint64_t *range;        /* init 2**64 - 1                           */
    uint64_t *point;        /* init: first two words, big word first    */
    int64_t *read_pos;      /* index into words of the next word        */
    const int64_t *end_pos; /* one past the stream's last word          */
    int32_t *status;        /* init 0                                   */
} sc_decoder_state;

/* One decoder step: symbols_out[b] (int64 [B]) = decoded symbol, or 256 for
 * streams with t >= valid_lens[b] or a failed stream.  Replaces
 * GpuRangeDecoder.decode_step_int8 / _range_decode_step_int8_kernel
 * (gpu_entropy_coding.py:444-454,306-397). */
int sc_decode_step(const int8_t *logits, const uint64_t *lut, const int64_t *valid_lens, int64_t t,
                   int64_t B, const sc_decoder_state *state, const uint32_t *words,
                   int64_t *symbols_out, void *stream);

/* Bytes of device workspace sc_compress_chunks needs for n_tokens tokens in
 * n_chunks chunks (a tile table, 4 bytes per chunk, tile descriptors, 16
 * bytes per 128 tokens and per chunk, and 8 bytes per token). */
int64_t sc_compress_workspace_bytes(int64_t n_tokens, int64_t n_chunks);

/* Compress n_chunks independent token chunks (teacher-forced MLP over every
 * step fused with the logits -> frequency step, then the range encoder and
 * seal).  Chunk c: lengths[c] tokens (uint8) at tokens + tok_off[c]; chunks
 * are disjoint and lie inside the n_tokens-byte token array; its u32
 * words go to words + word_off[c] (capacity word_cap[c] >= lengths[c] + 2 is
 * always sufficient); word_cnt[c] and status[c] are written.  All arrays
 * device.  Replaces QuantMLPCompression.compress_chunks /
 * _compress_chunks_gpu_ar (quant_mlp_export.py:271-323) and produces the
 * chunk bytes of CPUQuantMLPCompression.compress_chunks
 * (cpu_compression.py:178-257). */
int sc_compress_chunks(const sc_model *model, const uint8_t *tokens, const int64_t *tok_off,
                       const int32_t *lengths, int64_t n_chunks, int64_t n_tokens,
                       uint32_t *words, const int64_t *word_off, const int32_t *word_cap,
                       int32_t *word_cnt, int32_t *status, void *workspace,
                       int64_t workspace_bytes, void *stream);

/* Copy each chunk's word_cnt[c] words from words + word_off[c] to
 * out + out_off[c] (device arrays), e.g. from sc_compress_chunks' capacity
 * slots into a dense buffer before the device -> host copy.  Replaces the
 * full-buffer transfer of GpuRangeStepEncoder.get_compressed
 * (gpu_entropy_coding.py:292-303). */
int sc_gather_words(const uint32_t *words, const int64_t *word_off, const int32_t *word_cnt, int64_t n_chunks,
                    uint32_t *out, const int64_t *out_off, void *stream);

/* Measurement hook, no counterpart in the reference: n_groups workgroups of
 * 4 wavefronts each issue iters * 64 v_mfma_i32_32x32x32_i8 (65,536 int ops
 * each) on register operands taken from ops (device, 8192 bytes: 4 A and 4 B
 * fragments of 64 lanes x 16 bytes), with no memory traffic in the loop; out
 * (device, n_groups * 256 * 16 int32) receives the accumulator sums.  Timed
 * by the caller, it gives the int8 MFMA rate the GPU sustains at its power
 * limit for that operand data (the practical ceiling of the MLP kernels). */
int sc_mfma_burn_i8(const int8_t *ops, int32_t iters, int32_t n_groups, int32_t *out, void *stream);

/* Bytes of device workspace sc_decompress_chunks needs for n_chunks chunks:
 * the coder state of every chunk between step segments (40 bytes per chunk),
 * the launch plan's four length statistics, and the exchange buffers of a
 * split decode (32 KiB per 32 chunks, at most 64 such groups, and 32 bytes of
 * step flags per group), each part 256-byte aligned. */
int64_t sc_decompress_workspace_bytes(int64_t n_chunks);

/* Decompress n_chunks chunks with persistent kernels: every workgroup owns a
 * tile of chunks and runs the autoregressive loop for them (MLP step, fused
 * frequency step and decoder step per token, context kept on chip), in
 * launches of 256 steps; the coder state of each chunk is carried between
 * them in `workspace` (device, at least sc_decompress_workspace_bytes).
 * Chunk c: word_cnt[c] words at words + word_off[c] -> lengths[c] tokens at
 * tokens + tok_off[c]; status[c] is written (SC_STATUS_INVALID_STREAM on a
 * corrupt stream, whose tokens are then unspecified).  Device arrays:
 * words, word_off, word_cnt, lengths, tokens, tok_off, status, workspace.
 * `lengths_host` is an optional host copy of `lengths` (the reference's
 * list_of_lengths is host data): with it the launch plan is computed on the
 * host and the call only enqueues work on `stream`; with NULL the plan's
 * length statistics are computed on the device and read back, so the call
 * waits for the work already queued on `stream`; on a stream under graph
 * capture that wait is not possible, and lengths_host NULL is SC_ERR_ARG
 * before anything is enqueued (the capture stays valid).  Chunks sorted by
 * descending length (as QuantMLPCompression passes them) give the shortest
 * schedule: the shortest chunks are then left over after the full waves of
 * workgroups and follow the shortest chunks of the last full wave in the
 * same rows.  A launch of at most 64 groups of 32 chunks runs split: 8
 * workgroups per group (4 when the CUs cannot hold 8) share layer 0 and
 * wait for each other every step (a cooperative launch, so all are
 * resident; a bounded wait, SC_STATUS_SYNC_TIMEOUT when it expires), except
 * on a stream under graph capture.  Replaces
 * QuantMLPCompression.decompress_chunks / _decompress_chunks_gpu
 * (quant_mlp_export.py:325-377); output equals
 * CPUQuantMLPCompression.decompress_chunks (cpu_compression.py:259-332). */
int sc_decompress_chunks(const sc_model *model, const uint32_t *words, const int64_t *word_off,
                         const int32_t *word_cnt, const int32_t *lengths, int64_t n_chunks,
                         uint8_t *tokens, const int64_t *tok_off, int32_t *status,
                         const int32_t *lengths_host, void *workspace, int64_t workspace_bytes,
                         void *stream);

/* sc_decompress_chunks with options (a bitwise or of SC_DEC_OPT_*; any other
 * bit is SC_ERR_ARG).  SC_DEC_OPT_NO_SPLIT: every launch runs unsplit (one
 * workgroup per 32-chunk tile, no wait between workgroups), as
 * QuantMLPCompression.decompress_flat re-runs the chunks of a split launch
 * that reported SC_STATUS_SYNC_TIMEOUT.  Replaces the same reference call
 * as sc_decompress_chunks (quant_mlp_export.py:325-377). */
#define SC_DEC_OPT_NO_SPLIT 1
int sc_decompress_chunks_opts(const sc_model *model, const uint32_t *words, const int64_t *word_off,
                              const int32_t *word_cnt, const int32_t *lengths, int64_t n_chunks,
                              uint8_t *tokens, const int64_t *tok_off, int32_t *status,
                              const int32_t *lengths_host, void *workspace, int64_t workspace_bytes,
                              int32_t options, void *stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  sc_decompress_chunks with its workspace replaced by a
 * static device array the library holds on each GPU it runs on until the
 * process ends (SC_STATIC_DEC_MAX_CHUNKS chunks of coder state and the
 * split decode's exchange buffers, 4.6 MiB);
 * the call allocates nothing.  n_chunks above SC_STATIC_DEC_MAX_CHUNKS ->
 * SC_ERR_ARG.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (on different streams or threads) race.  With
 * lengths_host NULL the call waits for its stream, as sc_decompress_chunks
 * does (and is SC_ERR_ARG under graph capture).  Models of the bundled architecture only (SC_ERR_UNSUPPORTED for a
 * generic model, whose path allocates scratch memory). */
#define SC_STATIC_DEC_MAX_CHUNKS 65536
int sc_decompress_chunks_static(const sc_model *model, const uint32_t *words, const int64_t *word_off,
                                const int32_t *word_cnt, const int32_t *lengths, int64_t n_chunks,
                                uint8_t *tokens, const int64_t *tok_off, int32_t *status,
                                const int32_t *lengths_host, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SIGCOMP_HIP_H */
